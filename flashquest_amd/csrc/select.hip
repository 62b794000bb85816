// Quest page scoring from INT4 K metadata, top-k page selection and the
// page-list builders that feed the attention kernel (gfx950).
//
// Reference semantics:
//   scoring   src/flashquest/eager/criticality.py:128-163
//   selection src/flashquest/eager/selection.py:65-126
//   compact   src/flashquest/eager/selection.py:129-164
#include "fused_common.h"
#include "select_common.h"

namespace fq {
namespace {

// Per-group selection state shared by the fused scoring kernel and the
// standalone selection kernel.
struct SelectLds {
    uint32_t keys[kMaxPages];
    uint8_t qmask[kMaxPages];
    int hist[256];
    int tmp[8];
};

// Marks the top-k of keys[0..P) into s.qmask (|= bit), ties to the lower index.
FQ_DEV void topk_into_qmask(SelectLds& s, const uint32_t* keys, int P, int k, uint8_t bit) {
    const int tid = threadIdx.x;
    if (k <= 0) return;
    if (k >= P) {
        for (int i = tid; i < P; i += kThreads) s.qmask[i] |= bit;
        __syncthreads();
        return;
    }
    int take_eq = 0;
    const uint32_t T = block_radix_select(keys, P, k, s.hist, s.tmp, &take_eq);
    // count of keys equal to T (all of them match the final prefix)
    const int n_eq = s.hist[T & 255u];
    if (take_eq >= n_eq) {
        for (int i = tid; i < P; i += kThreads)
            if (keys[i] >= T) s.qmask[i] |= bit;
        __syncthreads();
    } else {
        for (int i = tid; i < P; i += kThreads)
            if (keys[i] > T) s.qmask[i] |= bit;
        block_compact(P, [&](int i) { return keys[i] == T; },
                      [&](int i, int rank) { if (rank < take_eq) s.qmask[i] |= bit; }, s.tmp);
    }
}


FQ_DEV void force_pages(SelectLds& s, int P, int num_sinks, int window, uint8_t bits) {
    const int ns = num_sinks < P ? num_sinks : P;
    const int w = window < P ? window : P;
    for (int i = threadIdx.x; i < P; i += kThreads)
        if (i < ns || (w > 0 && i >= P - w)) s.qmask[i] |= bits;
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Scoring.  One workgroup scores `ppc` pages of one KV group for all of its
// query rows; NL = D/8 lanes cooperate on a page, each owning 8 channels.
// Order (matched by the CPU oracle): a lane starts from its first product and
// adds the other 7 left to right by fused multiply-adds, lanes combine by the
// 16-lane DPP butterfly; score = t1 + t2 * 15.
// ---------------------------------------------------------------------------
struct ScoreParams {
    Int4Cache c;
    const void* q; int q_dtype; int64_t q_s[5];   // l, b, h_q, s_q, d
    int Hq, nrep, Sq, rows;                       // rows = nrep * Sq
    float* scores; int64_t sc_s[4];              // user output (l*B+b, h_q, s_q, p) or null
    int ppc, nchunks;
    float* ws_scores;                             // [G][nrep][P] (per-q) or [G][1][P] (summed), or null
    int mode;
    int sum_rows;                                 // per_kv_head_sum: score the group's summed query (one row)
};

// Scores of one page for every query row (rows in LDS), computed by the NL lanes
// of a page; emit(r, score) runs on all of them with the same value.
template <int D, typename MT, typename Emit>
FQ_DEV void score_page(const uint4& sv, const uint4& mv, const float (*s_q)[D], const float (*s_qp)[D], int rows, float levels,
                       int lane_in_page, Emit emit) {
    constexpr int NL = D / 8;
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
    for (int r = 0; r < rows; ++r) {
        const float* qr = &s_q[r][lane_in_page * 8];
        const float* qp = &s_qp[r][lane_in_page * 8];
        float t1 = __fmul_rn(qr[0], mf[0]);
        float t2 = __fmul_rn(qp[0], sf[0]);
#pragma unroll
        for (int j = 1; j < 8; ++j) {
            t1 = __fadd_rn(t1, __fmul_rn(qr[j], mf[j]));
            t2 = __fadd_rn(t2, __fmul_rn(qp[j], sf[j]));
        }
        t1 = row_sum<NL>(t1);
        t2 = row_sum<NL>(t2);
        emit(r, __fadd_rn(t1, __fmul_rn(t2, levels)));
    }
}

// q rows of group g into LDS: s_q = q, s_qp = relu(q).  Every load is issued
// (clamped index, dtype branch outside) before the first is used.
template <int D>
FQ_DEV void load_q_rows(const ScoreParams& a, int l, int b, int h, float (*s_q)[D], float (*s_qp)[D]) {
    constexpr int kPer = kMaxRows * D / kThreads;
    const int n = a.rows * D;
    int64_t off[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = min((int)threadIdx.x + u * kThreads, n - 1);
        const int r = i / D, d = i % D;
        const int hq = h * a.nrep + r / a.Sq, sq = r % a.Sq;
        off[u] = l * a.q_s[0] + b * a.q_s[1] + hq * a.q_s[2] + sq * a.q_s[3] + d * a.q_s[4];
    }
    float v[kPer];
    if (a.q_dtype == FQ_F32) {
#pragma unroll
        for (int u = 0; u < kPer; ++u) v[u] = ((const float*)a.q)[off[u]];
    } else {
        uint32_t w[kPer];
#pragma unroll
        for (int u = 0; u < kPer; ++u) w[u] = ((const uint16_t*)a.q)[off[u]];
#pragma unroll
        for (int u = 0; u < kPer; ++u) v[u] = a.q_dtype == FQ_BF16 ? bf16_bits_to_f(w[u]) : f16_bits_to_f(w[u]);
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = threadIdx.x + u * kThreads;
        if (i < n) {
            s_q[i / D][i % D] = v[u];
            s_qp[i / D][i % D] = v[u] > 0.f ? v[u] : 0.f;
        }
    }
    if (a.sum_rows) {
        // row 0 <- (q_0 + q_1) + ... and (relu q_0 + relu q_1) + ..., heads in order
        __syncthreads();
        float qs = 0.f, ps = 0.f;
        if (threadIdx.x < D) {
            qs = s_q[0][threadIdx.x];
            ps = s_qp[0][threadIdx.x];
            for (int r = 1; r < a.rows; ++r) {
                qs = __fadd_rn(qs, s_q[r][threadIdx.x]);
                ps = __fadd_rn(ps, s_qp[r][threadIdx.x]);
            }
        }
        __syncthreads();
        if (threadIdx.x < D) {
            s_q[0][threadIdx.x] = qs;
            s_qp[0][threadIdx.x] = ps;
        }
    }
}

constexpr int kPasses = 4;                  // passes of PPP pages per scoring chunk

// NR > 0: D = 128 and exactly NR query rows, q held in registers; NR = 0: any rows.
template <int D, typename MT, int NR>
__global__ __launch_bounds__(kThreads) void score_kernel(ScoreParams a) {
    constexpr int NL = D / 8;
    constexpr int PPP = kThreads / NL;           // pages per pass
    __shared__ float s_q[kMaxRows][D];
    __shared__ float s_qp[kMaxRows][D];

    const Int4Cache& c = a.c;
    const int g = blockIdx.y;
    const int h = g % c.Hkv, b = (g / c.Hkv) % c.B, l = g / (c.Hkv * c.B);
    const int tid = threadIdx.x;
    const int lane_in_page = tid % NL;
    const int page_in_pass = tid / NL;
    const MT* ksc = (const MT*)c.ksc + l * c.ksc_s[0] + b * c.ksc_s[1] + h * c.ksc_s[2];
    const MT* kmn = (const MT*)c.kmn + l * c.kmn_s[0] + b * c.kmn_s[1] + h * c.kmn_s[2];
    float* ws_scores = a.ws_scores ? a.ws_scores + (int64_t)g * a.rows * c.P : nullptr;

    // The workgroup streams its chunk pass by pass (PPP pages per pass) with
    // kPasses passes of metadata in flight ahead of the one being scored (a
    // partial last pass re-reads the chunk's last page); no loads are issued
    // past the chunk's last pass, so the workgroup ends with nothing in flight.
    const int p_begin = blockIdx.x * a.ppc;
    const int p_end = min(c.P, p_begin + a.ppc);
    const int npass = (p_end - p_begin + PPP - 1) / PPP;
    uint4 sv[kPasses], mv[kPasses];
    auto fetch = [&](int u, int pass) {
        const int p = min(p_begin + pass * PPP + page_in_pass, p_end - 1);
        sv[u] = *(const uint4*)(ksc + p * c.ksc_s[3] + lane_in_page * 8);
        mv[u] = *(const uint4*)(kmn + p * c.kmn_s[3] + lane_in_page * 8);
    };
#pragma unroll
    for (int u = 0; u < kPasses; ++u)
        if (u < npass) fetch(u, u);          // uniform: no loads past the chunk's passes
    load_q_rows<D>(a, l, b, h, s_q, s_qp);
    __syncthreads();
    const float levels = c.bits == 8 ? 255.0f : 15.0f;     // INT8 / INT4 code range
    float qr[NR > 0 ? NR : 1][8], qp[NR > 0 ? NR : 1][8];
    if constexpr (NR > 0) {
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                qr[r][j] = s_q[r][lane_in_page * 8 + j];
                qp[r][j] = s_qp[r][lane_in_page * 8 + j];
            }
    }
    for (int pass0 = 0; pass0 < npass; pass0 += kPasses) {
#pragma unroll
        for (int u = 0; u < kPasses; ++u) {
            const int p = p_begin + (pass0 + u) * PPP + page_in_pass;
            if (pass0 + u < npass && p < p_end) {
                float acc_kv = 0.f;
                auto emit = [&](int r, float sc) {
                    if (lane_in_page == 0) {
                        const int hq = h * a.nrep + r / a.Sq, sq = r % a.Sq;
                        if (a.scores)
                            a.scores[(l * c.B + b) * a.sc_s[0] + hq * a.sc_s[1] + sq * a.sc_s[2] + p * a.sc_s[3]] = sc;
                        if (ws_scores && a.mode == FQ_SELECT_PER_Q_HEAD) ws_scores[r * c.P + p] = sc;
                    }
                    acc_kv = r == 0 ? sc : __fadd_rn(acc_kv, sc);
                };
                if constexpr (NR > 0) score_page_regs<NR, MT>(sv[u], mv[u], qr, qp, emit, levels);
                else score_page<D, MT>(sv[u], mv[u], s_q, s_qp, a.sum_rows ? 1 : a.rows, levels, lane_in_page, emit);
                if (ws_scores && a.mode == FQ_SELECT_PER_KV_HEAD_SUM && lane_in_page == 0)
                    ws_scores[p] = acc_kv;
            }
            if (pass0 + u + kPasses < npass) fetch(u, pass0 + u + kPasses);     // uniform
        }
    }
}

// ---------------------------------------------------------------------------
// Per-group selection for the fused decode: one workgroup per KV group reads
// the group's scores (written by score_kernel), selects pages per query head
// (or once per KV head), adds the forced pages and writes the ascending union
// page list (page | selecting-heads mask << 16) and its length.
// ---------------------------------------------------------------------------
struct GroupSelectParams {
    Workspace ws; int mode, nrep, Hkv, P;
    const float* retention; int num_sinks, window, k_max;
    int B; int64_t ret_ls;                        // retention row of group g: layer g / (B * Hkv), stride ret_ls
    uint8_t* mask_out;                            // (l, b, h_q, p) contiguous or null
};

// Group tail: forced pages, then the ascending union list (page | heads << 16),
// its length and (optionally) the boolean selection mask, from s.qmask.
FQ_DEV void finish_group(SelectLds& s, const GroupSelectParams& a, int g) {
    const int tid = threadIdx.x, P = a.P;
    const uint8_t all_bits = (uint8_t)((1u << a.nrep) - 1u);
    force_pages(s, P, a.num_sinks, a.window, all_bits);
    int* entries = a.ws.entries + (int64_t)g * P;
    const int n = block_compact(P, [&](int i) { return s.qmask[i] != 0; },
                                [&](int i, int rank) { entries[rank] = i | ((int)s.qmask[i] << 16); }, s.tmp);
    if (a.mask_out) {
        uint8_t* mo = a.mask_out + ((int64_t)g * a.nrep) * P;
        for (int i = tid; i < a.nrep * P; i += kThreads) {
            const int r = i / P, p = i % P;
            mo[(int64_t)r * P + p] = (s.qmask[p] >> r) & 1;
        }
    }
    if (tid == 0) a.ws.n_sel[g] = n;
}

// The retention of group g's query heads: (H_q,) for every layer, or row
// g / (B * Hkv) of an (L, H_q) array.
FQ_DEV const float* group_retention(const GroupSelectParams& a, int g) {
    return a.retention + (int64_t)(g / (a.B * a.Hkv)) * a.ret_ls + (g % a.Hkv) * a.nrep;
}

// Top-k per query head (row r's keys at keys + r * P) or once per KV head from
// the summed scores (keys[0..P)), into a cleared s.qmask; then the group tail.
FQ_DEV void select_group(SelectLds& s, const GroupSelectParams& a, int g, const uint32_t* keys) {
    const int P = a.P;
    const float* ret = group_retention(a, g);
    if (a.mode == FQ_SELECT_PER_Q_HEAD) {
        for (int r = 0; r < a.nrep; ++r)
            topk_into_qmask(s, keys + r * P, P, k_for(ret[r], P, a.k_max), (uint8_t)(1u << r));
    } else {
        float rmax = 0.f;
        for (int r = 0; r < a.nrep; ++r) rmax = fmaxf(rmax, ret[r]);
        topk_into_qmask(s, keys, P, k_for(rmax, P, a.k_max), (uint8_t)((1u << a.nrep) - 1u));
    }
    finish_group(s, a, g);
}

__global__ __launch_bounds__(kThreads) void select_groups_kernel(GroupSelectParams a) {
    __shared__ SelectLds s;
    const int g = blockIdx.x, tid = threadIdx.x, P = a.P;
    const float* sc = a.ws.scores + (int64_t)g * a.nrep * P;
    for (int i = tid; i < P; i += kThreads) s.qmask[i] = 0;
    if (a.mode == FQ_SELECT_PER_Q_HEAD) {
        // one row at a time through s.keys
        __syncthreads();
        const float* ret = group_retention(a, g);
        for (int r = 0; r < a.nrep; ++r) {
            for (int i = tid; i < P; i += kThreads) s.keys[i] = sortable_key(sc[r * P + i]);
            __syncthreads();
            topk_into_qmask(s, s.keys, P, k_for(ret[r], P, a.k_max), (uint8_t)(1u << r));
        }
        finish_group(s, a, g);
    } else {
        for (int i = tid; i < P; i += kThreads) s.keys[i] = sortable_key(sc[i]);
        __syncthreads();
        select_group(s, a, g, s.keys);
    }
}

// ---------------------------------------------------------------------------
// The same per-group selection with one wave per group and no workgroup
// barriers (wave_select_group, select_common.h).  Used for P <= 64 C; launched
// with one wave per workgroup, so that the groups spread over the CUs.
// ---------------------------------------------------------------------------
template <int C>
__global__ __launch_bounds__(kThreads) void select_groups_wave_kernel(GroupSelectParams a, int G) {
    __shared__ uint32_t s_hist[kThreads / 64][256];        // each wave's own radix-search counts
    const int g = blockIdx.x * (blockDim.x / 64) + wave_id();
    if (g >= G) return;                      // whole wave
    const int P = a.P;
    int* entries = a.ws.entries + (int64_t)g * P;
    uint8_t* mo = a.mask_out ? a.mask_out + ((int64_t)g * a.nrep) * P : nullptr;
    const int n = wave_select_group<C>(a.ws.scores + (int64_t)g * a.nrep * P, P, a.nrep, a.mode,
                                       group_retention(a, g), a.k_max, a.num_sinks, a.window, entries, mo,
                                       s_hist[wave_id()]);
    if (lane_id() == 0) a.ws.n_sel[g] = n;
}

// ---------------------------------------------------------------------------
// Top-k per query head with the rows spread over the waves of a workgroup:
// one group per 4-wave workgroup, wave w searches rows w, w + 4, ... (each a
// wave_topk of its own), the selection bits meet in LDS, and wave 0 lists the
// group as wave_select_group does (same entries, same mask).  P <= 64 C.
// ---------------------------------------------------------------------------
template <int C>
__global__ __launch_bounds__(kThreads) void select_groups_rows_kernel(GroupSelectParams a) {
    constexpr int NW = kThreads / 64;
    __shared__ uint32_t s_hist[NW][256];
    __shared__ uint8_t s_qm[NW][C][64];
    const int g = blockIdx.x, w = wave_id(), lane = lane_id(), P = a.P;
    const float* sc = a.ws.scores + (int64_t)g * a.nrep * P;
    const float* ret = group_retention(a, g);
    uint8_t qm[C];
#pragma unroll
    for (int j = 0; j < C; ++j) qm[j] = 0;
    for (int r = w; r < a.nrep; r += NW) {
        uint32_t key[C];
#pragma unroll
        for (int j = 0; j < C; ++j) {
            const int i = 64 * j + lane;
            key[j] = i < P ? sortable_key(sc[r * P + i]) : 0u;      // 0: below every score
        }
        wave_topk<C>(key, qm, k_for(ret[r], P, a.k_max), (uint8_t)(1u << r), s_hist[w]);
    }
#pragma unroll
    for (int j = 0; j < C; ++j) s_qm[w][j][lane] = qm[j];
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int j = 0; j < C; ++j)
        for (int v = 1; v < NW; ++v) qm[j] |= s_qm[v][j][lane];
    uint8_t* mo = a.mask_out ? a.mask_out + ((int64_t)g * a.nrep) * P : nullptr;
    const int n = wave_list_group<C>(qm, P, a.nrep, a.num_sinks, a.window, a.ws.entries + (int64_t)g * P, mo);
    if (lane == 0) a.ws.n_sel[g] = n;
}

// ---------------------------------------------------------------------------
// The same selection for few groups (a single layer's decode step): one
// 8-wave workgroup per group runs the in-LDS selection of the fused decode
// (block_select_group), so the group's rows are searched by 8 waves instead of
// one.  P <= 64 kSelC.  The list puts the forced pages first.
// ---------------------------------------------------------------------------
template <int NREP>
__global__ __launch_bounds__(512) void select_groups_block_kernel(GroupSelectParams a) {
    constexpr int NT = 512, NW = 8;
    __shared__ uint32_t s_key[NREP * 64 * kSelC];
    __shared__ BlockSelectLds s_bsel;
    __shared__ int s_ent[64 * kSelC];
    const int g = blockIdx.x, tid = threadIdx.x, P = a.P;
    const int rows = a.mode == FQ_SELECT_PER_KV_HEAD_SUM ? 1 : NREP;
    ScoreRowRegs<NREP, NT> srow;
    scores_load<NREP, NT>(srow, a.ws.scores + (int64_t)g * NREP * P, rows, P, tid);
    const float ret_l = group_retention(a, g)[min(lane_id(), NREP - 1)];     // lane r: head r's retention
    scores_to_keys<NREP, NT>(srow, s_key, rows, P, tid);
    __syncthreads();
    const int n = block_select_group<kSelC, NW, NREP>(s_key, P, a.mode, ret_l, a.k_max, a.num_sinks, a.window, s_ent,
                                                      s_bsel);
    int* entries = a.ws.entries + (int64_t)g * P;
    for (int i = tid; i < n; i += NT) entries[i] = s_ent[i];
    if (a.mask_out)       // uniform; the keys are no longer needed: their LDS is the scratch
        block_write_mask<NT, NREP>(s_ent, n, P, (uint8_t*)s_key, a.mask_out + (int64_t)g * NREP * P, tid);
    if (tid == 0) a.ws.n_sel[g] = n;
}

// ---------------------------------------------------------------------------
// Standalone selection: one workgroup per (b, h, s_q) score row.
// ---------------------------------------------------------------------------
struct SelectParams {
    const float* scores; int64_t sc_s[4];
    int B, H, Sq, P;
    const float* retention; int num_sinks, window, k_max;
    uint8_t* mask; int64_t m_s[4];
};

__global__ __launch_bounds__(kThreads) void select_rows_kernel(SelectParams a) {
    __shared__ SelectLds s;
    const int row = blockIdx.x;
    const int sq = row % a.Sq, h = (row / a.Sq) % a.H, b = row / (a.Sq * a.H);
    const int tid = threadIdx.x, P = a.P;
    const float* src = a.scores + b * a.sc_s[0] + h * a.sc_s[1] + sq * a.sc_s[2];
    for (int i = tid; i < P; i += kThreads) {
        s.keys[i] = sortable_key(src[i * a.sc_s[3]]);
        s.qmask[i] = 0;
    }
    __syncthreads();
    topk_into_qmask(s, s.keys, P, k_for(a.retention[h], P, a.k_max), 1);
    force_pages(s, P, a.num_sinks, a.window, 1);
    uint8_t* dst = a.mask + b * a.m_s[0] + h * a.m_s[1] + sq * a.m_s[2];
    for (int i = tid; i < P; i += kThreads) dst[i * a.m_s[3]] = s.qmask[i];
}

// mask row -> descending ids, -1 padded (selection.py:153-163)
struct CompactParams {
    const uint8_t* mask; int64_t m_s[4];
    int B, H, Sq, P, bucket;
    int32_t* ids;
};

__global__ __launch_bounds__(kThreads) void compact_ids_kernel(CompactParams a) {
    __shared__ int s_tmp[8];
    const int row = blockIdx.x;
    const int sq = row % a.Sq, h = (row / a.Sq) % a.H, b = row / (a.Sq * a.H);
    const uint8_t* src = a.mask + b * a.m_s[0] + h * a.m_s[1] + sq * a.m_s[2];
    int32_t* dst = a.ids + (int64_t)row * a.bucket;
    const int P = a.P, bucket = a.bucket;
    const int n = block_compact(P, [&](int i) { return src[(int64_t)(P - 1 - i) * a.m_s[3]] != 0; },
                                [&](int i, int rank) { if (rank < bucket) dst[rank] = P - 1 - i; },
                                s_tmp);
    for (int i = n + threadIdx.x; i < bucket; i += kThreads) dst[i] = -1;
}

// bool mask (l, b, h_q, p) -> per-group union list
struct UnionParams {
    const uint8_t* mask; int64_t m_s[4];
    const int32_t* ids; int64_t id_s[4]; int bucket;
    int L, B, Hkv, nrep, P;
    Workspace ws;
};

__global__ __launch_bounds__(kThreads) void union_from_mask_kernel(UnionParams a) {
    __shared__ uint8_t qm[kMaxPages];
    __shared__ int s_tmp[8];
    const int g = blockIdx.x;
    const int h = g % a.Hkv, b = (g / a.Hkv) % a.B, l = g / (a.Hkv * a.B);
    const int P = a.P;
    for (int i = threadIdx.x; i < P; i += kThreads) {
        uint32_t bits = 0;
        for (int r = 0; r < a.nrep; ++r) {
            const int hq = h * a.nrep + r;
            bits |= (a.mask[l * a.m_s[0] + b * a.m_s[1] + hq * a.m_s[2] + i * a.m_s[3]] != 0) << r;
        }
        qm[i] = (uint8_t)bits;
    }
    __syncthreads();
    int* entries = a.ws.entries + (int64_t)g * P;
    const int n = block_compact(P, [&](int i) { return qm[i] != 0; },
                                [&](int i, int rank) { entries[rank] = i | ((int)qm[i] << 16); }, s_tmp);
    if (threadIdx.x == 0) a.ws.n_sel[g] = n;
}

__global__ __launch_bounds__(kThreads) void union_from_ids_kernel(UnionParams a) {
    __shared__ uint32_t qm[kMaxPages];
    __shared__ int s_tmp[8];
    const int g = blockIdx.x;
    const int h = g % a.Hkv, b = (g / a.Hkv) % a.B, l = g / (a.Hkv * a.B);
    const int P = a.P;
    for (int i = threadIdx.x; i < P; i += kThreads) qm[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < a.nrep * a.bucket; i += kThreads) {
        const int r = i / a.bucket, j = i % a.bucket;
        const int hq = h * a.nrep + r;
        const int id = a.ids[l * a.id_s[0] + b * a.id_s[1] + hq * a.id_s[2] + j * a.id_s[3]];
        if (id >= 0 && id < P) atomicOr(&qm[id], 1u << r);
    }
    __syncthreads();
    int* entries = a.ws.entries + (int64_t)g * P;
    const int n = block_compact(P, [&](int i) { return qm[i] != 0; },
                                [&](int i, int rank) { entries[rank] = i | ((int)qm[i] << 16); }, s_tmp);
    if (threadIdx.x == 0) a.ws.n_sel[g] = n;
}

}  // namespace

// ---------------------------------------------------------------- launchers
hipError_t launch_score(const Int4Cache& c, const QueryArgs& q, int S_q, const int64_t* q4_s,
                        float* scores, const int64_t* sc4_s, const Workspace* ws, int select_mode,
                        const float* retention, int num_sinks, int window, int k_max,
                        uint8_t* mask_out, hipStream_t st, bool select_groups) {
    ScoreParams a{};
    a.c = c;
    a.q = q.q; a.q_dtype = q.q_dtype;
    // q strides: (l, b, h_q, s_q, d)
    a.q_s[0] = q.q_s[0]; a.q_s[1] = q4_s[0]; a.q_s[2] = q4_s[1]; a.q_s[3] = q4_s[2]; a.q_s[4] = q4_s[3];
    a.Hq = q.Hq; a.nrep = q.nrep; a.Sq = S_q; a.rows = q.nrep * S_q;
    a.scores = scores;
    if (sc4_s) for (int i = 0; i < 4; ++i) a.sc_s[i] = sc4_s[i];
    const int G = c.L * c.B * c.Hkv;
    // pages per chunk: about two workgroups per CU in one pass over the GPU,
    // each streaming a whole number of passes of ppp pages
    const int ppp = kThreads / (c.D / 8);
    int target_chunks = (512 + G - 1) / G;
    int ppc = (c.P + target_chunks - 1) / target_chunks;
    ppc = ((ppc + ppp - 1) / ppp) * ppp;
    if (ppc < ppp) ppc = ppp;
    a.ppc = ppc;
    a.nchunks = (c.P + ppc - 1) / ppc;
    a.ws_scores = ws ? ws->scores : nullptr;
    a.mode = select_mode;
    a.sum_rows = ws && select_mode == FQ_SELECT_PER_KV_HEAD_SUM && S_q == 1 && !scores;
    if (a.rows > kMaxRows || c.P > kMaxPages) return hipErrorInvalidValue;
    GroupSelectParams sp{};
    if (ws) {
        sp.ws = *ws; sp.mode = select_mode; sp.nrep = q.nrep; sp.Hkv = c.Hkv; sp.P = c.P;
        sp.retention = retention; sp.num_sinks = num_sinks; sp.window = window; sp.k_max = k_max;
        sp.mask_out = mask_out; sp.B = c.B; sp.ret_ls = q.ret_ls;
    }
    dim3 grid(a.nchunks, G);
#define FQ_SCORE(D_, MT_, NR_) hipLaunchKernelGGL((score_kernel<D_, MT_, NR_>), grid, dim3(kThreads), 0, st, a)
#define FQ_SCORE_NR(MT_)                                                   \
    switch (a.sum_rows ? 1 : a.rows) {                                     \
        case 1: FQ_SCORE(128, MT_, 1); break;                              \
        case 2: FQ_SCORE(128, MT_, 2); break;                              \
        case 3: FQ_SCORE(128, MT_, 3); break;                              \
        case 4: FQ_SCORE(128, MT_, 4); break;                              \
        default: FQ_SCORE(128, MT_, 0); break;                             \
    }
    if (c.D == 128) {
        if (c.meta_dtype == FQ_BF16) { FQ_SCORE_NR(bf16) } else { FQ_SCORE_NR(f16) }
    } else {
        if (c.meta_dtype == FQ_BF16) FQ_SCORE(64, bf16, 0); else FQ_SCORE(64, f16, 0);
    }
#undef FQ_SCORE_NR
#undef FQ_SCORE
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !ws || !select_groups) return e;
    if (G < 192 && c.P <= 64 * kSelC && q.nrep <= 4) {     // few groups: a workgroup per group
        switch (q.nrep) {
            case 1: hipLaunchKernelGGL(select_groups_block_kernel<1>, dim3(G), dim3(512), 0, st, sp); break;
            case 2: hipLaunchKernelGGL(select_groups_block_kernel<2>, dim3(G), dim3(512), 0, st, sp); break;
            case 3: hipLaunchKernelGGL(select_groups_block_kernel<3>, dim3(G), dim3(512), 0, st, sp); break;
            default: hipLaunchKernelGGL(select_groups_block_kernel<4>, dim3(G), dim3(512), 0, st, sp); break;
        }
    } else if (c.P > 64 * 8 && c.P <= 64 * 32 && q.nrep > 1 && select_mode == FQ_SELECT_PER_Q_HEAD) {
        if (c.P <= 64 * 16) hipLaunchKernelGGL(select_groups_rows_kernel<16>, dim3(G), dim3(kThreads), 0, st, sp);
        else hipLaunchKernelGGL(select_groups_rows_kernel<32>, dim3(G), dim3(kThreads), 0, st, sp);
    } else if (c.P <= 64 * 8) hipLaunchKernelGGL(select_groups_wave_kernel<8>, dim3(G), dim3(64), 0, st, sp, G);
    // one wave per workgroup: the groups spread over as many CUs as there are
    else if (c.P <= 64 * 16) hipLaunchKernelGGL(select_groups_wave_kernel<16>, dim3(G), dim3(64), 0, st, sp, G);
    else if (c.P <= 64 * 32) hipLaunchKernelGGL(select_groups_wave_kernel<32>, dim3(G), dim3(64), 0, st, sp, G);
    else hipLaunchKernelGGL(select_groups_kernel, dim3(G), dim3(kThreads), 0, st, sp);
    return hipGetLastError();
}

hipError_t launch_select_rows(const float* scores, const int64_t* sc_s, int B, int H, int S_q, int P,
                              const float* retention, int num_sinks, int window, int k_max,
                              uint8_t* mask, const int64_t* m_s, hipStream_t st) {
    SelectParams a{};
    a.scores = scores;
    for (int i = 0; i < 4; ++i) { a.sc_s[i] = sc_s[i]; a.m_s[i] = m_s[i]; }
    a.B = B; a.H = H; a.Sq = S_q; a.P = P;
    a.retention = retention; a.num_sinks = num_sinks; a.window = window; a.k_max = k_max;
    a.mask = mask;
    hipLaunchKernelGGL(select_rows_kernel, dim3(B * H * S_q), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_compact_ids(const uint8_t* mask, const int64_t* m_s, int B, int H, int S_q, int P,
                              int bucket, int32_t* ids, hipStream_t st) {
    CompactParams a{};
    a.mask = mask;
    for (int i = 0; i < 4; ++i) a.m_s[i] = m_s[i];
    a.B = B; a.H = H; a.Sq = S_q; a.P = P; a.bucket = bucket; a.ids = ids;
    hipLaunchKernelGGL(compact_ids_kernel, dim3(B * H * S_q), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_union_from_mask(const uint8_t* mask, const int64_t* m_s, int L, int B, int Hkv,
                                  int nrep, int P, const Workspace& ws, hipStream_t st) {
    UnionParams a{};
    a.mask = mask;
    for (int i = 0; i < 4; ++i) a.m_s[i] = m_s[i];
    a.L = L; a.B = B; a.Hkv = Hkv; a.nrep = nrep; a.P = P; a.ws = ws;
    hipLaunchKernelGGL(union_from_mask_kernel, dim3(L * B * Hkv), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_union_from_ids(const int32_t* ids, const int64_t* id_s, int bucket, int L, int B,
                                 int Hkv, int nrep, int P, const Workspace& ws, hipStream_t st) {
    UnionParams a{};
    a.ids = ids;
    for (int i = 0; i < 4; ++i) a.id_s[i] = id_s[i];
    a.bucket = bucket;
    a.L = L; a.B = B; a.Hkv = Hkv; a.nrep = nrep; a.P = P; a.ws = ws;
    hipLaunchKernelGGL(union_from_ids_kernel, dim3(L * B * Hkv), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace fq
