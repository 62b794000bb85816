// Wave-level page selection shared by the selection kernels and the fused
// attention prologue.  Reference semantics: src/flashquest/eager/selection.py:65-126.
#pragma once

#include "fq_common.h"

namespace fq {

FQ_DEV int k_for(float r, int P, int k_max) {
    // selection.py:103: ceil(fp32(r) * fp32(P)) clamped to [0, P]
    float kf = ceilf(__fmul_rn(r, (float)P));
    int k = kf <= 0.f ? 0 : (kf >= (float)P ? P : (int)kf);
    if (k_max >= 0 && k > k_max) k = k_max;
    return k;
}

// Marks the k largest of keys (lane holds key[j] of page 64 j + lane; ties to the
// lower page index) into qm |= bit.  The k-th largest key is found bit by bit
// with wave-wide counts (ballots, scalar popcounts); ties are ranked by ballots.
// The k-th largest of the wave's 64 C keys (k >= 1), found bit by bit: T keeps
// the largest prefix that at least k keys reach.  Wave-uniform, no LDS.
template <int C>
FQ_DEV uint32_t wave_kth_largest(const uint32_t (&key)[C], int k) {
    uint32_t T = 0;
    for (int bitpos = 31; bitpos >= 0; --bitpos) {
        const uint32_t cand = T | (1u << bitpos);
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < C; ++j) cnt += __popcll(__ballot(key[j] >= cand));
        if (cnt >= k) T = cand;
    }
    return T;
}

template <int C>
FQ_DEV uint32_t wave_kth_hist(const uint32_t (&key)[C], int k, uint32_t* hist, bool* exact = nullptr);

// hist: 256 words of LDS used by this wave only (wave_kth_hist's digit counts).
template <int C>
FQ_DEV void wave_topk(const uint32_t (&key)[C], uint8_t (&qm)[C], int k, uint8_t bit, uint32_t* hist) {
    if (k <= 0) return;
    bool exact;
    const uint32_t T = wave_kth_hist<C>(key, k, hist, &exact);
    if (exact) {         // exactly k keys >= T: no ties to rank
#pragma unroll
        for (int j = 0; j < C; ++j)
            if (key[j] >= T) qm[j] |= bit;
        return;
    }
    // T is the k-th largest key; keys above it are in, ties fill the rest by index
    int gt = 0;
#pragma unroll
    for (int j = 0; j < C; ++j) gt += __popcll(__ballot(key[j] > T));
    int take_eq = k - gt;
#pragma unroll
    for (int j = 0; j < C; ++j) {
        if (key[j] > T) qm[j] |= bit;
        const uint64_t eq = __ballot(key[j] == T);
        const int rank = (int)lanes_below(eq);
        if (key[j] == T && rank < take_eq) qm[j] |= bit;
        take_eq -= __popcll(eq);
    }
}

template <int C>
FQ_DEV int wave_list_group(uint8_t (&qm)[C], int P, int nrep, int num_sinks, int window, int* entries,
                           uint8_t* mask_out);

// One KV group's selection by one wave (P <= 64 C): scores of row r at
// sc[r * P + p] (nrep rows per query head, or one summed row), top-k per
// query head or once per KV head with the group's largest retention, forced
// sink / window pages (selection.py:110-117), then the ascending union list
// entries[i] = page | selecting-heads << 16 (LDS or global) and, if mask_out,
// the per-head boolean rows mask_out[r * P + p].  Returns the list length.
template <int C>
FQ_DEV int wave_select_group(const float* sc, int P, int nrep, int mode, const float* retention, int k_max,
                             int num_sinks, int window, int* entries, uint8_t* mask_out, uint32_t* hist) {
    const int lane = lane_id();
    uint32_t key[C];
    uint8_t qm[C];
#pragma unroll
    for (int j = 0; j < C; ++j) qm[j] = 0;
    // Every row's loads are issued one row ahead, and the first row's together
    // with the retention load, so the wave waits for memory once per row at most.
    float v[2][C];
    auto fetch = [&](int buf, int r) {
#pragma unroll
        for (int j = 0; j < C; ++j) v[buf][j] = sc[r * P + min(64 * j + lane, P - 1)];
    };
    auto make_keys = [&](int buf) {
#pragma unroll
        for (int j = 0; j < C; ++j) key[j] = 64 * j + lane < P ? sortable_key(v[buf][j]) : 0u;  // 0: below every score
    };
    const float ret_l = retention[min(lane, nrep - 1)];      // lane r: head r's retention
    fetch(0, 0);
    const uint8_t all_bits = (uint8_t)((1u << nrep) - 1u);
    if (mode == FQ_SELECT_PER_Q_HEAD) {
        for (int r = 0; r < nrep; ++r) {
            if (r + 1 < nrep) fetch((r + 1) & 1, r + 1);
            make_keys(r & 1);
            wave_topk<C>(key, qm, k_for(__shfl(ret_l, r, 64), P, k_max), (uint8_t)(1u << r), hist);
        }
    } else {
        float rmax = 0.f;
        for (int r = 0; r < nrep; ++r) rmax = fmaxf(rmax, __shfl(ret_l, r, 64));
        make_keys(0);
        wave_topk<C>(key, qm, k_for(rmax, P, k_max), all_bits, hist);
    }
    return wave_list_group<C>(qm, P, nrep, num_sinks, window, entries, mask_out);
}

// The end of wave_select_group: qm[j] holds the selection bits (bit r: query
// row r) of page 64 j + lane; forces the sink and window pages into every row,
// writes the ascending entry list (page | bits << 16) and, if mask_out, the
// per-row mask; returns the list length.
template <int C>
FQ_DEV int wave_list_group(uint8_t (&qm)[C], int P, int nrep, int num_sinks, int window, int* entries,
                           uint8_t* mask_out) {
    const int lane = lane_id();
    const uint8_t all_bits = (uint8_t)((1u << nrep) - 1u);
    const int ns = num_sinks < P ? num_sinks : P;
    const int wnd = window < P ? window : P;
    int n = 0;
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const int i = 64 * j + lane;
        if (i < P && (i < ns || (wnd > 0 && i >= P - wnd))) qm[j] |= all_bits;
        const bool f = i < P && qm[j] != 0;
        const uint64_t bal = __ballot(f);
        if (f) entries[n + (int)lanes_below(bal)] = i | ((int)qm[j] << 16);
        n += __popcll(bal);
        if (mask_out && i < P)
            for (int r = 0; r < nrep; ++r) mask_out[(int64_t)r * P + i] = (qm[j] >> r) & 1;
    }
    return n;
}

// Quest page score (criticality.py:128-163) of one page for NR query rows, by
// the 16 lanes of a DPP row, each owning 8 channels (q values in registers).
// The fp32 order is fixed (and restated by the CPU oracle): a lane starts from
// its first product (rounded) and adds the other 7 by fused multiply-adds, one
// rounding each (fp16 metadata feeds v_fma_mix_f32 with no conversion); lanes
// combine by the DPP butterfly in row_sum<16>, score = t1 + t2 * levels (15 for
// INT4 metadata, criticality.py:161; 255 for INT8, criticality.py:123).
// emit(r, score) runs on all 16 lanes with the same value.
template <int NR, typename MT, typename Emit>
FQ_DEV void score_page_regs(const uint4& sv, const uint4& mv, const float (&qr)[NR][8], const float (&qp)[NR][8],
                            Emit emit, float levels = 15.0f) {
    float sf[8], mf[8];
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
    const uint32_t mw[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        sf[2 * j] = half_to_f<MT>(sw[j]);
        sf[2 * j + 1] = half_to_f<MT>(sw[j] >> 16);
        mf[2 * j] = half_to_f<MT>(mw[j]);
        mf[2 * j + 1] = half_to_f<MT>(mw[j] >> 16);
    }
    float t1[NR], t2[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        t1[r] = __fmul_rn(qr[r][0], mf[0]);
        t2[r] = __fmul_rn(qp[r][0], sf[0]);
#pragma unroll
        for (int j = 1; j < 8; ++j) {
            t1[r] = __builtin_fmaf(qr[r][j], mf[j], t1[r]);
            t2[r] = __builtin_fmaf(qp[r][j], sf[j], t2[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        t1[r] = row_sum<16>(t1[r]);
        t2[r] = row_sum<16>(t2[r]);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) emit(r, __fadd_rn(t1[r], __fmul_rn(t2[r], levels)));
}

// The forced pages of a P-page row (selection.py:110-117): sinks [0, ns) and
// the window [start, P) with start = max(ns, P - window), in ascending order;
// forced entry f is page f (f < ns) or start + f - ns.
struct ForcedPages {
    int ns, start, count;
    FQ_DEV bool contains(int i) const { return i < ns || i >= start; }
    FQ_DEV int index(int i) const { return i < ns ? i : ns + i - start; }
    FQ_DEV int page(int f) const { return f < ns ? f : start + f - ns; }
};
FQ_DEV ForcedPages forced_pages(int P, int num_sinks, int window) {
    ForcedPages fp;
    fp.ns = num_sinks < P ? (num_sinks > 0 ? num_sinks : 0) : P;
    const int wnd = window < P ? (window > 0 ? window : 0) : P;
    fp.start = P - wnd > fp.ns ? P - wnd : fp.ns;
    fp.count = fp.ns + P - fp.start;
    return fp;
}

// Workgroup-wide selection for one KV group, same result as wave_select_group
// (P <= 64 C pages, NW waves).  keys[r * 64 C + p] holds sortable_key of row
// r's score of page p, and 0 (below every score) for p >= P.  Every wave loads
// every key (C per lane per row); wave r finds row r's k-th largest key with
// wave_kth_hist (no barrier inside; for one row only the last wave searches,
// so its SIMD is not shared with a partner wave doing the same search, and
// the last wave issues no forced-page loads before it); the thresholds meet
// in LDS, and every
// wave then ranks the ties and lists the pages.  Ties and forced pages follow
// wave_topk / wave_select_group; the entry list holds the forced pages first,
// then the other selected pages, each part ascending; wave w writes the entries
// of pages 64 j + lane with j = w (mod NW).  NROWS = 1: one top-k of the summed
// row with the group's largest retention (per_kv_head_sum); NROWS = nrep: one
// per query head.  ret_l: lane r holds query head r's retention.  All control
// flow is wave-uniform.  Ends with a barrier; returns the list length in
// every thread.
struct alignas(16) BlockSelectLds {
    uint32_t T[4];          // k-th largest key per row
    uint32_t hist[8][256];  // wave_kth_hist: one 256-bin digit histogram per wave
};

// DPP moves across a whole wave (gfx9 row broadcasts) and wave reductions
// built on them: no LDS traffic, only VALU latency.
template <int CTRL, int ROWS = 0xF> FQ_DEV int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xF, true);
}
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

// Inclusive prefix sum over lanes 0..lane.
FQ_DEV int wave_incl_sum(int v) {
    v += dpp_i<kDppRowShr1>(v);
    v += dpp_i<kDppRowShr2>(v);
    v += dpp_i<kDppRowShr4>(v);
    v += dpp_i<kDppRowShr8>(v);             // every row of 16 lanes scanned
    v += dpp_i<kDppRowBcast15, 0xA>(v);     // rows 1 and 3 add the row before's total
    v += dpp_i<kDppRowBcast31, 0xC>(v);     // rows 2 and 3 add rows 0-1's total
    return v;
}
// Wave-wide minimum / maximum of an unsigned value, returned wave-uniform.
FQ_DEV uint32_t wave_min_u32(uint32_t v) {
    int x = (int)v;
    x = (int)min((uint32_t)x, (uint32_t)__builtin_amdgcn_update_dpp(x, x, kDppXor1, 0xF, 0xF, false));
    x = (int)min((uint32_t)x, (uint32_t)__builtin_amdgcn_update_dpp(x, x, kDppXor2, 0xF, 0xF, false));
    x = (int)min((uint32_t)x, (uint32_t)__builtin_amdgcn_update_dpp(x, x, kDppHalfMirror, 0xF, 0xF, false));
    x = (int)min((uint32_t)x, (uint32_t)__builtin_amdgcn_update_dpp(x, x, kDppMirror, 0xF, 0xF, false));
    const uint32_t a = min((uint32_t)__builtin_amdgcn_readlane(x, 0), (uint32_t)__builtin_amdgcn_readlane(x, 16));
    const uint32_t b = min((uint32_t)__builtin_amdgcn_readlane(x, 32), (uint32_t)__builtin_amdgcn_readlane(x, 48));
    return min(a, b);
}
FQ_DEV uint32_t wave_max_u32(uint32_t v) {
    int x = (int)v;
    x = (int)max((uint32_t)x, (uint32_t)__builtin_amdgcn_update_dpp(x, x, kDppXor1, 0xF, 0xF, false));
    x = (int)max((uint32_t)x, (uint32_t)__builtin_amdgcn_update_dpp(x, x, kDppXor2, 0xF, 0xF, false));
    x = (int)max((uint32_t)x, (uint32_t)__builtin_amdgcn_update_dpp(x, x, kDppHalfMirror, 0xF, 0xF, false));
    x = (int)max((uint32_t)x, (uint32_t)__builtin_amdgcn_update_dpp(x, x, kDppMirror, 0xF, 0xF, false));
    const uint32_t a = max((uint32_t)__builtin_amdgcn_readlane(x, 0), (uint32_t)__builtin_amdgcn_readlane(x, 16));
    const uint32_t b = max((uint32_t)__builtin_amdgcn_readlane(x, 32), (uint32_t)__builtin_amdgcn_readlane(x, 48));
    return max(a, b);
}

// The k-th largest of the wave's 64 C keys (1 <= k <= 64 C) by one wave with
// no barrier: most-significant-digit radix selection in 8-bit digits, each
// digit's counts gathered in the wave's own 256-bin LDS histogram (hist: 256
// words used by this wave only) and located by a wave prefix sum.  The bits
// every key shares (the common prefix of the smallest and largest key) are
// skipped, and the search stops once the keys reaching the current prefix are
// exactly k (then T has exactly k keys >= T); otherwise T ends as the k-th
// largest key -- the contract the callers rely on: keys above T, then ties at
// T by page index, give the top k.  Wave-uniform; hist is left zeroed.
template <int C>
FQ_DEV uint32_t wave_kth_hist(const uint32_t (&key)[C], int k, uint32_t* hist, bool* exact) {
    const int lane = lane_id();
    // lo: the smallest key above 0.  Key 0 marks a slot past the last page
    // (below every score, never among the top k <= P), so leaving it out of
    // the common prefix only skips more leading bits when P < 64 C.
    uint32_t lo = key[0] ? key[0] : ~0u, hi = key[0];
#pragma unroll
    for (int j = 1; j < C; ++j) { lo = min(lo, key[j] ? key[j] : ~0u); hi = max(hi, key[j]); }
    lo = wave_min_u32(lo);
    if (lo > hi) lo = hi;            // no key above 0
    hi = wave_max_u32(hi);
    if (exact) *exact = false;
    if (lo == hi) return hi;
    int b = 31 - __clz(lo ^ hi);                    // bits above b are the same in every key
    uint32_t prefix = hi & ~((2u << b) - 1u);
    int need = k;                                   // keys still to take from those matching prefix above b
    uint32_t* const mine = hist + 252 - 4 * lane;   // lane l: digits 255 - 4l - m at mine[3 - m]
    *(uint4*)mine = make_uint4(0u, 0u, 0u, 0u);
    for (;;) {
        const int shift = b >= 7 ? b - 7 : 0;       // this pass's digit: bits [shift, b]
        const uint32_t dmask = (2u << (b - shift)) - 1u;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
        for (int j = 0; j < C; ++j)
            if ((((key[j] ^ prefix) >> b) >> 1) == 0u)
                __hip_atomic_fetch_add(&hist[(key[j] >> shift) & dmask], 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WAVEFRONT);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const uint4 h = *(const uint4*)mine;
        *(uint4*)mine = make_uint4(0u, 0u, 0u, 0u);
        const int c0 = (int)h.w, c1 = (int)h.z, c2 = (int)h.y, c3 = (int)h.x;   // digits 255-4l, -1, -2, -3
        const int tot = c0 + c1 + c2 + c3;
        const int incl = wave_incl_sum(tot);       // keys with digit >= 252 - 4l (lanes 0..l)
        const int above = incl - tot;
        const uint64_t hit = __ballot(incl >= need);
        const int ls = __builtin_amdgcn_readfirstlane((int)__builtin_ctzll(hit));   // the total is >= need
        // in lane ls (above < need <= incl): the first digit, from the top, that
        // brings the count to need; ab = keys above it, cd = keys on it
        int m = 3, ab = above + c0 + c1 + c2, cd = c3;
        if (above + c0 + c1 + c2 >= need) { m = 2; ab = above + c0 + c1; cd = c2; }
        if (above + c0 + c1 >= need) { m = 1; ab = above + c0; cd = c1; }
        if (above + c0 >= need) { m = 0; ab = above; cd = c0; }
        const int m_s = __builtin_amdgcn_readlane(m, ls);
        const int ab_s = __builtin_amdgcn_readlane(ab, ls);
        const int cd_s = __builtin_amdgcn_readlane(cd, ls);
        prefix |= (uint32_t)(255 - 4 * ls - m_s) << shift;
        need -= ab_s;
        if (cd_s == need) {          // exactly k keys are >= prefix
            if (exact) *exact = true;
            return prefix;
        }
        if (shift == 0) return prefix;
        b = shift - 1;
    }
}

template <int C, int NW, int NROWS, int NREP>
FQ_DEV int block_select_rows(const uint32_t* keys, int P, float ret_l, int k_max, int num_sinks, int window,
                             int* entries, BlockSelectLds& sl) {
    static_assert(NROWS <= NW && NROWS <= 4, "one wave per row; at most 4 rows");
    const int lane = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
    constexpr uint8_t kAll = (uint8_t)((1u << NREP) - 1u);
    uint32_t key[NROWS][C];
    int k[NROWS];
    uint32_t T[NROWS];
#pragma unroll
    for (int r = 0; r < NROWS; ++r)
#pragma unroll
        for (int j = 0; j < C; ++j) key[r][j] = keys[r * 64 * C + 64 * j + lane];
    float rmax = 0.f;
#pragma unroll
    for (int r = 0; r < NREP; ++r) rmax = fmaxf(rmax, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ret_l), r)));
#pragma unroll
    for (int r = 0; r < NROWS; ++r)
        k[r] = k_for(NROWS == 1 ? rmax : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ret_l), r)), P, k_max);
    bool exact = false;              // one row: exactly k keys >= T, no ties to rank
    if constexpr (NROWS == 1) {      // one row: the last wave finds the threshold, shared through LDS
        if (w == NW - 1) {
            bool ex = false;
            const uint32_t t = k[0] > 0 ? wave_kth_hist<C>(key[0], k[0], sl.hist[w], &ex) : 0u;
            if (lane == 0) { sl.T[0] = t; sl.T[1] = ex ? 1u : 0u; }
        }
        lds_barrier();
        T[0] = sl.T[0];
        exact = sl.T[1] != 0u;
    } else {                         // wave r finds row r's, shared through LDS
#pragma unroll
        for (int r = 0; r < NROWS; ++r) {
            if (w == r) {
                const uint32_t t = k[r] > 0 ? wave_kth_hist<C>(key[r], k[r], sl.hist[w]) : 0u;
                if (lane == 0) sl.T[r] = t;
            }
        }
        lds_barrier();
#pragma unroll
        for (int r = 0; r < NROWS; ++r) T[r] = sl.T[r];
    }
    // ties at T: the lowest page indices (wave_topk's rule); identical in every wave
    uint8_t qm[C];
#pragma unroll
    for (int j = 0; j < C; ++j) qm[j] = 0;
    if (exact) {         // uniform
#pragma unroll
        for (int j = 0; j < C; ++j) qm[j] = key[0][j] >= T[0] ? kAll : (uint8_t)0;
    } else
#pragma unroll
    for (int r = 0; r < NROWS; ++r) {
        if (k[r] <= 0) continue;
        const uint8_t bit = NROWS == 1 ? kAll : (uint8_t)(1u << r);
        int gt = 0;
#pragma unroll
        for (int j = 0; j < C; ++j) gt += __popcll(__ballot(key[r][j] > T[r]));
        int take_eq = k[r] - gt;
#pragma unroll
        for (int j = 0; j < C; ++j) {
            const uint64_t eq = __ballot(key[r][j] == T[r]);
            const bool in = key[r][j] > T[r] || (key[r][j] == T[r] && (int)lanes_below(eq) < take_eq);
            qm[j] |= in ? bit : (uint8_t)0;
            take_eq -= __popcll(eq);
        }
    }
    // The list: the forced pages first (ascending; forced_page() gives entry f
    // without the selection), then every other selected page ascending.
    const ForcedPages fp = forced_pages(P, num_sinks, window);
    int n = fp.count;
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const int i = 64 * j + lane;
        const bool forced = i < P && fp.contains(i);
        const bool f = i < P && !forced && qm[j] != 0;
        const uint64_t bal = __ballot(f);
        if (j % NW == w) {
            if (forced) entries[fp.index(i)] = i | ((int)kAll << 16);
            if (f) entries[n + (int)lanes_below(bal)] = i | ((int)qm[j] << 16);
        }
        n += __popcll(bal);
    }
    lds_barrier();
    return n;
}

// The group's selection as boolean rows mask[r * P + i] (query head r of the
// group, page i), from the entry list (page | selecting-heads << 16) of
// block_select_rows.  scratch: >= P bytes of LDS that nothing else uses any
// more; every thread of the NT-thread workgroup calls this (two barriers).
template <int NT, int NREP>
FQ_DEV void block_write_mask(const int* entries, int n, int P, uint8_t* scratch, uint8_t* mask, int tid) {
    for (int i = tid; i < P; i += NT) scratch[i] = 0;
    lds_barrier();
    for (int e = tid; e < n; e += NT) scratch[entries[e] & 0xFFFF] = (uint8_t)(entries[e] >> 16);
    lds_barrier();
    for (int i = tid; i < NREP * P; i += NT) {
        const int r = i / P, p = i - r * P;
        mask[i] = (scratch[p] >> r) & 1;
    }
}

template <int C, int NW, int NREP>
FQ_DEV int block_select_group(const uint32_t* keys, int P, int mode, float ret_l, int k_max, int num_sinks, int window,
                              int* entries, BlockSelectLds& sl) {
    if (mode == FQ_SELECT_PER_Q_HEAD)
        return block_select_rows<C, NW, NREP, NREP>(keys, P, ret_l, k_max, num_sinks, window, entries, sl);
    return block_select_rows<C, NW, 1, NREP>(keys, P, ret_l, k_max, num_sinks, window, entries, sl);
}

}  // namespace fq
