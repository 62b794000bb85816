// Sparse GQA decode attention over the INT8 cache on the gfx950 matrix cores.
// Semantics of flash_attn_sparse_fwd (src/flashquest/kernel/sparse_fwd.py:23-157):
// k = code * K_scale[p] + K_mn[p], v = code * V_scale[t] + V_mn[t] (codes
// 0..255, one byte per channel; K metadata per page and channel, V per token),
// base-2 online softmax, O = acc / l, lse = (m + log2 l) * ln2; an empty
// selection gives O = 0 and lse = -inf; tokens >= S are masked.
//
// The structure is the INT4 matrix-core kernel's (attn_mfma.hip): one
// 8-wave workgroup per KV group (or per balanced split of a group), which
// with FUSED scores its group's pages from the K page metadata (255 levels,
// criticality.py:77-125), selects them in LDS and attends them, wave w taking
// pages w, w + 8, ...  The page math:
//   q.k : v_mfma_i32_16x16x64_i8.  A = q_d * K_scale[p,d] as 3 balanced int8
//         digits of a 24-bit fixed-point number per page (rows 4r + digit);
//         B = code - 128 (the byte with its top bit flipped), so
//         q.k = sum A (code - 128) + 128 sum A + q.K_mn, the last two per head
//         and page on the VALU.  int32 accumulation is exact.
//   p.v : v_mfma_f32_16x16x32_f16.  A = p_t * V_scale[t] (/ a running bound
//         with bf16 metadata) split into fp16 parts hi = fp16(A) in rows r
//         and lo = fp16(A - hi) in rows 4 + r (the V metadata is per token,
//         so rows 4..7 are free), B = the codes as fp16 subnormals (bits =
//         code, value = code * 2^-24, exact); the two row sets are added at
//         the end, so each product carries A to 2^-22 relative (fp32-level,
//         like the reference's fp32 p * v); plus sum_t p_t V_mn[t].
// With 8-bit codes a page is twice the INT4 bytes, so the loads run half a
// page (32 tokens) ahead of the half being computed to keep both buffers in
// registers.
#include <algorithm>
#include <type_traits>

#include "attn_common.h"
#include "fused_common.h"

namespace fq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float f2v __attribute__((ext_vector_type(2)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

constexpr float kQkScale8 = 8323071.0f;      // 2^23 - 2^16 - 1: |X| <= this keeps 3 balanced digits in int8
constexpr float kSubnormal8 = 16777216.0f;   // 2^24
constexpr uint32_t kFlip8 = 0x80808080u;

struct Int8Params {
    Int4Cache c;
    QueryArgs q;
    Workspace ws;
    int splits;
    SelectArgs sel;
    TailArgs tail;          // tail.len > 0: attended (in_kernel: by split 0 of each group, else the split merge)
};

// Per-wave LDS operands: q.k A digits of the current page [k-step][row][k-group,
// swizzled][16 bytes]; p.v A of the current half page [row][k-group][16 bytes].
struct WaveLds8 {
    uint8_t aqk[2][16][4][16];
    uint8_t apv[16][4][16];
};
FQ_DEV int swz8(int row, int kg) { return kg ^ ((row >> 2) & 3); }

template <int I>
FQ_DEV uint32_t byte_of4(uint32_t y0, uint32_t y1, uint32_t y2, uint32_t y3) {
    constexpr uint32_t lo = 0x0C0C0000u | ((4u + I) << 8) | I;
    constexpr uint32_t hi = ((4u + I) << 24) | ((uint32_t)I << 16) | 0x0C0Cu;
    return __builtin_amdgcn_perm(y1, y0, lo) | __builtin_amdgcn_perm(y3, y2, hi);
}

// Half a page (tokens 32 hp .. 32 hp + 31): tiles T = 2 hp + t.
struct HalfBuf {
    uint4 kt[2][2];      // [t][k-step s]: K codes of token 16T + n16, bytes 64 s + 16 lg .. +15
    uint2 vw[8];         // [2 ai + jj]: V codes of token 16 (2 hp + jj) + 4 ai + lg, bytes 8 n16 .. +7
    uint32_t vs[2], vm[2];   // [t]: V scale / min (16-bit) of token 16T + n16
    uint2 ks, km;        // K scale / min of the lane's channels 4 (L & 31) .. +3 (the page's)
};

struct Int8Rsrc {
    __amdgpu_buffer_rsrc_t k, v, vs, vm, ks, km;
};

// Dense rows (128-byte codes, 2-byte V metadata, 256-byte K metadata rows):
// every offset is (lane part) + (page part) + an immediate.
FQ_DEV void load_half(HalfBuf& b, const Int8Rsrc& r, int p, int hp, int n16, int lg, int L) {
    const int kbase = p * 64 * 128 + n16 * 128 + 16 * lg;
    const int vbase = p * 64 * 128 + lg * 128 + 8 * n16;
    const int mbase = (p * 64 + n16) * 2;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int s = 0; s < 2; ++s) b.kt[t][s] = ld128(r.k, kbase + (32 * hp + 16 * t) * 128 + 64 * s);
#pragma unroll
    for (int i = 0; i < 8; ++i) b.vw[i] = ld64(r.v, vbase + (16 * (2 * hp + (i & 1)) + 4 * (i >> 1)) * 128);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        b.vs[t] = ld16(r.vs, mbase + (32 * hp + 16 * t) * 2);
        b.vm[t] = ld16(r.vm, mbase + (32 * hp + 16 * t) * 2);
    }
    b.ks = ld64(r.ks, p * 256 + 8 * (L & 31));
    b.km = ld64(r.km, p * 256 + 8 * (L & 31));
}

// HCH (FUSED only): head chunks, sel.head_chunks virtual KV heads per cache KV
// head (virtual head h = cache head hk * HC + chunk, NREP query heads each; q,
// outputs and retention follow h, the cache pages hk).  per_kv_head_sum then
// scores the summed query of all 2 NREP heads of the cache head, so every
// chunk selects the same pages.  The chunks of a cache head are mapped to one
// XCD so that the second one's page reads hit that XCD's L2.
template <typename MT, int NREP, bool FUSED, bool HCH = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_int8_mfma_kernel(Int8Params a) {
    constexpr int D = 128, NW = 8, NT = 512;
    static_assert(NREP <= 4, "query heads per KV head");
    static_assert(!HCH || FUSED, "head chunks run in the fused kernel");
    constexpr int NSLOT = FUSED ? NW + 1 : NW;      // the fused kernel's extra slot: the partial-page tail
    constexpr int TTOK = FUSED ? kTailMax : 1;
    __shared__ SplitLds<D, NREP, NSLOT> s_split;
    __shared__ WaveLds8 s_wave[NW];
    __shared__ int s_ent[kMaxWgPages];
    __shared__ float s_q[NREP][D];

    const Int4Cache& c = a.c;
    const QueryArgs& q = a.q;
    const int gy = blockIdx.y, GY = gridDim.y, split = blockIdx.x;
    // head chunks: workgroup index i takes group (i % 8) * (G / 8) + i / 8, so
    // consecutive groups (the chunks of one cache head) share an XCD
    const int g = (HCH && gridDim.x == 1 && GY % 8 == 0) ? (gy % 8) * (GY / 8) + gy / 8 : gy;
    const int h = g % c.Hkv, b = (g / c.Hkv) % c.B, l = g / (c.Hkv * c.B);
    const int HC = HCH ? a.sel.head_chunks : 1;
    const int hk = HCH ? h / HC : h;
    const bool chunk_sum = HCH && a.sel.mode == FQ_SELECT_PER_KV_HEAD_SUM;
    const int tid = threadIdx.x, L = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
    const int n16 = L & 15, lg = L >> 4;
    WaveLds8& W = s_wave[w];
    const int S = c.S;

    // q: element tid of the group's heads, two branch-free 16-bit loads (the
    // high one used only for fp32 q), issued before the metadata loads
    // chunk_sum: all 2 NREP heads of the cache head (two elements per
    // thread; rows chunk * NREP .. are this workgroup's own)
    const int q_rows = chunk_sum ? 2 * NREP : NREP;
    const int q_row0 = chunk_sum ? (h - hk * HC) * NREP : 0;
    const int64_t qb = l * q.q_s[0] + b * q.q_s[1] + (int64_t)(chunk_sum ? hk * 2 * NREP : h * NREP) * q.q_s[2];
    const int qi = min(tid, q_rows * D - 1);
    const int qi1 = min(tid + NT, q_rows * D - 1);
    const bool q32 = q.q_dtype == FQ_F32;
    const int esz = q32 ? 4 : 2;
    uint32_t hi_mask = (0u - (uint32_t)q32) & 0xFFFF0000u;
    asm volatile("" : "+s"(hi_mask));
    uint32_t ql, qh, ql1 = 0u, qh1 = 0u;
    {
        const char* qc = (const char*)q.q + (qb + (qi >> 7) * q.q_s[2] + (qi & 127) * q.q_s[3]) * esz;
        ql = *(const uint16_t*)qc;
        qh = *(const uint16_t*)(qc + esz - 2);
        if constexpr (HCH) {
            const char* qc1 = (const char*)q.q + (qb + (qi1 >> 7) * q.q_s[2] + (qi1 & 127) * q.q_s[3]) * esz;
            ql1 = *(const uint16_t*)qc1;
            qh1 = *(const uint16_t*)(qc1 + esz - 2);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    float ret_l = 0.f;
    ScoreRegs<NT> sr;
    ScoreRowRegs<NREP, NT> srow;        // kSelectOnly: the group's precomputed scores
    const bool from_scores = FUSED && a.sel.enabled == kSelectOnly;
    const int score_rows = a.sel.mode == FQ_SELECT_PER_KV_HEAD_SUM ? 1 : NREP;
    // Partial-page tail (tail.in_kernel, split 0 of a group): its <= 64 raw
    // 16-bit K / V rows go to LDS with q.  The loads are unconditional: without
    // a tail the buffer is empty and they read 0.
    __shared__ uint16_t s_tk[TTOK][D], s_tv[TTOK][D];
    __shared__ float s_tp[NREP][TTOK];
    uint4 tkr[2], tvr[2];
    const int tail_T = FUSED && a.tail.in_kernel && split == 0 ? a.tail.len : 0;
    if constexpr (FUSED) {
        if (chunk_sum)      // uniform: the k of the summed row is the cache head's largest retention
            ret_l = wave_max(a.sel.retention[l * q.ret_ls + hk * 2 * NREP + min(L, 2 * NREP - 1)]);
        else
            ret_l = a.sel.retention[l * q.ret_ls + h * NREP + min(L, NREP - 1)];
        const TailArgs& t = a.tail;
        const char* tkb = tail_T > 0 ? (const char*)t.k + 2 * (l * t.ks[0] + b * t.ks[1] + hk * t.ks[2]) : nullptr;
        const char* tvb = tail_T > 0 ? (const char*)t.v + 2 * (l * t.vs[0] + b * t.vs[1] + hk * t.vs[2]) : nullptr;
        const auto rk = make_rsrc(tkb, tail_T > 0 ? 2 * (int64_t)(tail_T - 1) * t.ks[3] + 2 * D : 0);
        const auto rv = make_rsrc(tvb, tail_T > 0 ? 2 * (int64_t)(tail_T - 1) * t.vs[3] + 2 * D : 0);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int i = tid + NT * u, tt = i >> 4, j = i & 15;       // token tt, bytes 16j .. 16j+15
            tkr[u] = ld128(rk, (int)(2 * tt * t.ks[3]) + 16 * j);
            tvr[u] = ld128(rv, (int)(2 * tt * t.vs[3]) + 16 * j);
        }
        if (from_scores)      // per_kv_head_sum with head chunks: the cache head's one summed row
            scores_load<NREP, NT>(srow, a.ws.scores + (int64_t)(chunk_sum ? g - (h - hk * HC) : g) * NREP * c.P,
                                  score_rows, c.P, tid);
        else score_group_load<MT, NT>(sr, c, tid, l, b, hk);
    }
    auto q_value = [&](uint32_t lo, uint32_t hi) {
        const uint32_t u = (lo & ~hi_mask) | ((hi << 16) & hi_mask);
        const float fh = f16_bits_to_f(u), fb = bf16_bits_to_f(u);
        return q32 ? __uint_as_float(u) : (q.q_dtype == FQ_BF16 ? fb : fh);
    };
    const float qv_raw = q_value(ql, qh);

    Int8Rsrc rs;
    rs.k = make_rsrc(c.kp + l * c.kp_s[0] + b * c.kp_s[1] + hk * c.kp_s[2], (int64_t)S * 128);
    rs.v = make_rsrc(c.vp + l * c.vp_s[0] + b * c.vp_s[1] + hk * c.vp_s[2], (int64_t)S * 128);
    rs.vs = make_rsrc((const uint16_t*)c.vsc + l * c.vsc_s[0] + b * c.vsc_s[1] + hk * c.vsc_s[2], (int64_t)S * 2);
    rs.vm = make_rsrc((const uint16_t*)c.vmn + l * c.vmn_s[0] + b * c.vmn_s[1] + hk * c.vmn_s[2], (int64_t)S * 2);
    rs.ks = make_rsrc((const MT*)c.ksc + l * c.ksc_s[0] + b * c.ksc_s[1] + hk * c.ksc_s[2], (int64_t)c.P * 256);
    rs.km = make_rsrc((const MT*)c.kmn + l * c.kmn_s[0] + b * c.kmn_s[1] + hk * c.kmn_s[2], (int64_t)c.P * 256);
    auto issue_half = [&](HalfBuf& bf, int p, int hp) {
        __builtin_amdgcn_sched_barrier(0);
        load_half(bf, rs, p, hp, n16, lg, L);
        __builtin_amdgcn_sched_barrier(0);
    };
    HalfBuf b0, b1;
    bool first_issued = false;

    int e0, e1;
    if constexpr (FUSED) {
        __shared__ float s_qraw[HCH ? 2 * NREP : NREP][D];      // chunk_sum: every head of the cache head
        __shared__ uint32_t s_key[NREP * 64 * kSelC];
        __shared__ BlockSelectLds s_bsel;
        if constexpr (HCH) {
            const float qv1 = q_value(ql1, qh1);
            if (tid < q_rows * D) {
                const int r = (qi >> 7) - q_row0;
                if ((unsigned)r < (unsigned)NREP) s_q[r][qi & 127] = qv_raw * q.qk_scale;
                s_qraw[qi >> 7][qi & 127] = qv_raw;
            }
            if (tid + NT < q_rows * D) {
                const int r = (qi1 >> 7) - q_row0;
                if ((unsigned)r < (unsigned)NREP) s_q[r][qi1 & 127] = qv1 * q.qk_scale;
                s_qraw[qi1 >> 7][qi1 & 127] = qv1;
            }
        } else if (tid < NREP * D) {
            s_q[qi >> 7][qi & 127] = qv_raw * q.qk_scale;
            s_qraw[qi >> 7][qi & 127] = qv_raw;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int i = tid + NT * u;
            *(uint4*)&s_tk[i >> 4][8 * (i & 15)] = tkr[u];
            *(uint4*)&s_tv[i >> 4][8 * (i & 15)] = tvr[u];
        }
        __syncthreads();
        if (from_scores)     // uniform: a scoring launch wrote the group's scores
            scores_to_keys<NREP, NT>(srow, s_key, score_rows, c.P, tid);
        else if (chunk_sum)
            score_group_regs<MT, HCH ? 2 * NREP : NREP, NT, true>(sr, s_qraw, s_key, tid, c.P, 255.0f);
        else if (a.sel.mode == FQ_SELECT_PER_KV_HEAD_SUM)
            score_group_regs<MT, NREP, NT, true>(sr, s_qraw, s_key, tid, c.P, 255.0f);
        else
            score_group_regs<MT, NREP, NT, false>(sr, s_qraw, s_key, tid, c.P, 255.0f);
        const ForcedPages fp = forced_pages(c.P, a.sel.num_sinks, a.sel.window);
        if (S > 0 && split == 0 && w < fp.count) {       // split 0's first entries are the forced pages
            issue_half(b0, fp.page(w), 0);
            first_issued = true;
        }
        __syncthreads();
        const int total = block_select_group<kSelC, NW, NREP>(s_key, c.P, a.sel.mode, ret_l, a.sel.k_max,
                                                              a.sel.num_sinks, a.sel.window, s_ent, s_bsel);
        if (a.sel.mask_out && split == 0)            // uniform: the caller asked for the selection
            block_write_mask<NT, NREP>(s_ent, total, c.P, (uint8_t*)s_key, a.sel.mask_out + (int64_t)g * NREP * c.P,
                                       tid);
        e0 = (int)((int64_t)total * split / a.splits);
        e1 = (int)((int64_t)total * (split + 1) / a.splits);
    } else {
        const int n_sel = a.ws.n_sel[g];
        e0 = (int)((int64_t)n_sel * split / a.splits);
        e1 = (int)((int64_t)n_sel * (split + 1) / a.splits);
        for (int i = tid; i < e1 - e0; i += NT) s_ent[i] = a.ws.entries[(int64_t)g * c.P + e0 + i];
        if (tid < NREP * D) s_q[qi >> 7][qi & 127] = qv_raw * q.qk_scale;
        __syncthreads();
    }
    const int ent_base = FUSED ? e0 : 0;
    const int n_mine = S > 0 && w < e1 - e0 ? (e1 - e0 - w + NW - 1) / NW : 0;   // pages w, w + NW, ...

    // A-operand values of this lane: channels c0 .. c0 + 3, heads r0, r0 + 1
    const int c0 = 4 * (L & 31), r0 = 2 * (L >> 5);
    float qv[2][4];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int j = 0; j < 4; ++j) qv[hh][j] = r0 + hh < NREP ? s_q[min(r0 + hh, NREP - 1)][c0 + j] : 0.f;

    auto entry_of = [&](int k) { return __builtin_amdgcn_readfirstlane(s_ent[ent_base + w + NW * k]); };

    constexpr bool kBound = std::is_same<MT, bf16>::value;
    float m_run[NREP];
#pragma unroll
    for (int r = 0; r < NREP; ++r) m_run[r] = -INFINITY;
    float s_run = kBound ? 0.f : 1.f, inv_s = 1.f;
    float m_lane = 0.f;
    v4f pacc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) pacc[t] = (v4f){0.f, 0.f, 0.f, 0.f};
    float l_acc = 0.f, bias = 0.f;
    float Cr = 0.f, unscale = 0.f;           // the current page's q.K_mn + 128 sum A (head lg), digit scale

    // the INT4 kernel's priority rule for the two waves of a SIMD: the one
    // with more pages left, on a tie the younger, runs at the higher priority
    __shared__ int s_left[NW];
    auto balance = [&](int k) {
        s_left[w] = n_mine - k;
        const int other = __builtin_amdgcn_readfirstlane(s_left[w ^ 4]);
        if (n_mine - k > other || (n_mine - k == other && w >= 4)) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
    };

    auto compute = [&](const HalfBuf& cb, int k, int hp) {
        const int ent = entry_of(k);
        const int p = ent & 0xFFFF, qm = ent >> 16;
        const int tok0 = p * 64 + 32 * hp;
        if (hp == 0) {
            balance(k);
            // ---- the page's q.k A digits, q.K_mn and sum A per head
            const uint32_t sw[2] = {cb.ks.x, cb.ks.y}, mw[2] = {cb.km.x, cb.km.y};
            float Av[2][4], cpart[2] = {0.f, 0.f}, apart[2] = {0.f, 0.f}, amax = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float sf = half_to_f<MT>(sw[j >> 1] >> (16 * (j & 1)));
                const float mf = half_to_f<MT>(mw[j >> 1] >> (16 * (j & 1)));
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    Av[hh][j] = qv[hh][j] * sf;
                    cpart[hh] = fmaf(qv[hh][j], mf, cpart[hh]);
                    apart[hh] += Av[hh][j];
                    amax = fmaxf(amax, fabsf(Av[hh][j]));
                }
            }
            const float sigma = wave_max(amax);
            const float inv = sigma > 0.f ? kQkScale8 * __builtin_amdgcn_rcpf(sigma) : 0.f;
            const int s = c0 >> 6, kg = (c0 >> 4) & 3, bo = c0 & 15;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                if (r0 + hh < NREP) {
                    uint32_t Y[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) Y[j] = (uint32_t)fmaf(Av[hh][j], inv, 8421504.0f);
                    const int row = 4 * (r0 + hh);
                    *(uint32_t*)&W.aqk[s][row][swz8(row, kg)][bo] = byte_of4<2>(Y[0], Y[1], Y[2], Y[3]) ^ kFlip8;
                    *(uint32_t*)&W.aqk[s][row + 1][swz8(row + 1, kg)][bo] = byte_of4<1>(Y[0], Y[1], Y[2], Y[3]) ^ kFlip8;
                    *(uint32_t*)&W.aqk[s][row + 2][swz8(row + 2, kg)][bo] = byte_of4<0>(Y[0], Y[1], Y[2], Y[3]) ^ kFlip8;
                }
                float cs = fmaf(apart[hh], 128.0f, cpart[hh]);       // q.K_mn + 128 sum A over this lane's channels
                cs += __shfl_xor(cs, 16, 64);
                cpart[hh] = row_sum<16>(cs);
            }
            const float x0 = __shfl(cpart[0], (lg >> 1) * 32, 64);
            const float x1 = __shfl(cpart[1], (lg >> 1) * 32, 64);
            Cr = (lg & 1) ? x1 : x0;
            unscale = sigma * (1.0f / kQkScale8);
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        }
        const v4i a0 = *(const v4i*)&W.aqk[0][n16][swz8(n16, lg)][0];
        const v4i a1 = *(const v4i*)&W.aqk[1][n16][swz8(n16, lg)][0];
        // ---- q.k of tiles T = 2 hp, 2 hp + 1
        float lg2[2], mp = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint4 k0 = cb.kt[t][0], k1 = cb.kt[t][1];
            const v4i bk0 = {(int)(k0.x ^ kFlip8), (int)(k0.y ^ kFlip8), (int)(k0.z ^ kFlip8), (int)(k0.w ^ kFlip8)};
            const v4i bk1 = {(int)(k1.x ^ kFlip8), (int)(k1.y ^ kFlip8), (int)(k1.z ^ kFlip8), (int)(k1.w ^ kFlip8)};
            v4i acc = {0, 0, 0, 0};
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bk0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bk1, acc, 0, 0, 0);
            const float f = fmaf((float)acc[0], 65536.f, fmaf((float)acc[1], 256.f, (float)acc[2]));
            const float lgt = fmaf(f, unscale, Cr);
            const bool ok = lg < NREP && ((qm >> lg) & 1) && tok0 + 16 * t + n16 < S;
            lg2[t] = ok ? lgt : -INFINITY;
            mp = fmaxf(mp, lg2[t]);
        }
        // ---- running references
        float vs_t[2], vm_t[2], sp = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            vs_t[t] = half_to_f<MT>(cb.vs[t]);
            vm_t[t] = half_to_f<MT>(cb.vm[t]);
            sp = fmaxf(sp, vs_t[t]);
        }
        mp = row16_max(mp);
        bool grow = false;
        float mp_r[NREP];
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
            mp_r[r] = lane_value(mp, 16 * r);
            grow |= mp_r[r] > m_run[r];
        }
        if constexpr (kBound) {
            sp = lane_value(row16_max(sp), 0);
            grow |= sp > s_run;
        }
        if (grow) {      // wave-uniform
            float am[NREP];
#pragma unroll
            for (int r = 0; r < NREP; ++r) {
                const float mn = fmaxf(mp_r[r], m_run[r]);
                am[r] = mn == m_run[r] ? 1.0f : exp2_fast(m_run[r] - mn);
                m_run[r] = mn;
            }
            float as = 1.0f;
            if constexpr (kBound) {
                const float sn = sp > s_run ? 2.0f * sp : s_run;
                as = sn > 0.f ? s_run / sn : 1.0f;
                s_run = sn;
                inv_s = sn > 0.f ? 1.0f / sn : 0.f;
            }
            float am_lg = am[0], ml = m_run[0];
#pragma unroll
            for (int r = 1; r < NREP; ++r) {
                am_lg = lg == r ? am[r] : am_lg;
                ml = lg == r ? m_run[r] : ml;
            }
            m_lane = ml == -INFINITY ? 0.f : ml;
            l_acc *= am_lg;
            bias *= am_lg;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float f = r < NREP ? am[r] * as : 0.f;
#pragma unroll
                for (int t = 0; t < 8; ++t) pacc[t][r] *= f;
            }
        }
        // ---- p.v A: p * V_scale (/ s_run) in fp16; operand k = 8 kg + 2 ai + jj is
        // token 16 (2 hp + jj) + 4 ai + kg
        float pr[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            pr[t] = exp2_fast(lg2[t] - m_lane);
            l_acc += pr[t];
            bias = fmaf(pr[t], vm_t[t], bias);
        }
        if (lg < NREP) {
            float x0 = pr[0] * vs_t[0], x1 = pr[1] * vs_t[1];
            if constexpr (kBound) { x0 *= inv_s; x1 *= inv_s; }
            const f2v xv = {x0, x1};
            const h2v hv = __builtin_convertvector(xv, h2v);
            const h2v lv = __builtin_convertvector(xv - __builtin_convertvector(hv, f2v), h2v);
            const int kq = n16 & 3, kql = kq ^ 1;      // rows lg (hi) and 4 + lg (lo), swizzled
            *(uint32_t*)&W.apv[lg][kq][4 * (n16 >> 2)] = __builtin_bit_cast(uint32_t, hv);
            *(uint32_t*)&W.apv[4 + lg][kql][4 * (n16 >> 2)] = __builtin_bit_cast(uint32_t, lv);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const v8h ap = *(const v8h*)&W.apv[n16][lg ^ ((n16 >> 2) & 3)][0];
        // ---- p.v B: byte j of the lane's 8 channels for the step's 8 tokens, as fp16 subnormals
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t sel = 0x0C000C00u | ((4u + (j & 3)) << 16) | (uint32_t)(j & 3);
            uint32_t bw[4];
#pragma unroll
            for (int ai = 0; ai < 4; ++ai) {
                const uint32_t t0 = j < 4 ? cb.vw[2 * ai].x : cb.vw[2 * ai].y;
                const uint32_t t1 = j < 4 ? cb.vw[2 * ai + 1].x : cb.vw[2 * ai + 1].y;
                bw[ai] = __builtin_amdgcn_perm(t1, t0, sel);
            }
            const v8h bv = __builtin_bit_cast(v8h, (v4i){(int)bw[0], (int)bw[1], (int)bw[2], (int)bw[3]});
            pacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ap, bv, pacc[j], 0, 0, 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    };

    // Half-page pipeline: step u = 2k + hp; the next half is in flight while
    // one is computed.  Past the end the last half is reloaded, so every path
    // has the same loads in flight.
    {
        s_left[w] = n_mine;
        const int nsteps = 2 * n_mine;
        auto page_of = [&](int u) { return entry_of(min(u, max(nsteps - 1, 0)) >> 1) & 0xFFFF; };
        auto half_of = [&](int u) { return min(u, max(nsteps - 1, 0)) & 1; };
        if (!first_issued) issue_half(b0, page_of(0), 0);
        if constexpr (FUSED) {
            // the partial-page tail's state (the merge's last slot) while the
            // first half page is in flight: its barriers wait on LDS only
            if (tail_T > 0)      // uniform
                tail_state_lds<D, NREP, NT>(s_tk, s_tv, a.tail.dtype == FQ_BF16, tail_T, s_q, s_tp, s_split.m[NW],
                                            s_split.l[NW], s_split.acc[NW]);
        }
        for (int u = 0; u < nsteps; u += 2) {
            issue_half(b1, page_of(u + 1), half_of(u + 1));
            compute(b0, u >> 1, 0);
            issue_half(b0, page_of(u + 2), half_of(u + 2));
            compute(b1, u >> 1, 1);
        }
        __builtin_amdgcn_s_setprio(0);
    }

    // ---- wave state -> LDS (head r in lane group 0 component r; channel 8 n16 + j)
    // the lo rows 4 + r (lane group 1) join the hi rows
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < NREP; ++r) pacc[j][r] += __shfl_xor(pacc[j][r], 16, 64);
    l_acc = row_sum<16>(l_acc);
    bias = row_sum<16>(bias);
    const float pv_unscale = s_run * kSubnormal8;
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
        const float ll = __shfl(l_acc, 16 * r + n16, 64);
        const float bb = __shfl(bias, 16 * r + n16, 64);
        if (lg == 0) {
#pragma unroll
            for (int j = 0; j < 8; ++j) s_split.acc[w][r][8 * n16 + j] = fmaf(pacc[j][r], pv_unscale, bb);
            if (n16 == 0) { s_split.m[w][r] = m_run[r]; s_split.l[w][r] = ll; }
        }
    }
    int nslots = NW;
    if constexpr (FUSED) {
        if (tail_T > 0) nslots = NW + 1;       // the tail state (computed before the page loop) joins the merge
    }
    __syncthreads();
    merge_waves_and_store<D, NREP, false, NSLOT, NT>(s_split, q, a.ws, g, l, b, h, split,
                                                     a.splits > 1 || (a.tail.len > 0 && !a.tail.in_kernel), nslots);
}

template <typename MT, bool FUSED>
hipError_t launch_int8_nrep(const Int8Params& a, dim3 grid, hipStream_t st) {
    switch (a.q.nrep) {
#define FQ_CASE(N)                                                                                      \
    case N:                                                                                             \
        timer_before_launch(st);                                                                        \
        if (FUSED && (N == 3 || N == 4) && a.sel.head_chunks > 1)                                       \
            hipLaunchKernelGGL((attn_int8_mfma_kernel<MT, N, FUSED, FUSED && N >= 3>), grid, dim3(512), 0, \
                               st, a);                                                                  \
        else                                                                                            \
            hipLaunchKernelGGL((attn_int8_mfma_kernel<MT, N, FUSED>), grid, dim3(512), 0, st, a);       \
        timer_after_launch(st);                                                                         \
        if (a.splits > 1 || (a.tail.len > 0 && !a.tail.in_kernel))                                      \
            launch_split_merge<N, false>(a.q, a.ws, a.c.Hkv, a.c.B, grid.y, a.splits,                   \
                                         a.tail.in_kernel ? TailArgs{} : a.tail, st);                    \
        break;
        FQ_CASE(1) FQ_CASE(2) FQ_CASE(3) FQ_CASE(4)
#undef FQ_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool int8_mfma_supported(const Int4Cache& c, const QueryArgs& q, const AttnLaunch& al) {
    if (c.bits != 8 || c.D != 128 || c.page != 64 || c.G != 1 || q.nrep > 4) return false;
    if ((int64_t)al.s_max * kMaxWgPages < al.max_entries) return false;
    // dense rows: 128-byte code rows, per-token V metadata, 128-channel K metadata rows
    if (c.kp_s[3] != 128 || c.vp_s[3] != 128 || c.vsc_s[3] != 1 || c.vmn_s[3] != 1) return false;
    if (c.ksc_s[3] != 128 || c.kmn_s[3] != 128) return false;
    for (int i = 0; i < 3; ++i) {
        if (c.kp_s[i] % 16 || c.vp_s[i] % 16 || c.ksc_s[i] % 8 || c.kmn_s[i] % 8) return false;
    }
    if (((uintptr_t)c.kp | (uintptr_t)c.vp) & 15) return false;
    if (((uintptr_t)c.ksc | (uintptr_t)c.kmn) & 15) return false;
    if (((uintptr_t)c.vsc | (uintptr_t)c.vmn) & 1) return false;
    return true;
}

bool int8_select_in_kernel(const Int4Cache& c, const QueryArgs& q, const AttnLaunch& al) {
    return int8_mfma_supported(c, q, al) && c.P <= 64 * kSelC && al.max_entries <= kMaxWgPages &&
           attention_splits_request() <= 0;
}

hipError_t launch_attn_int8_mfma(const Int4Cache& c, const QueryArgs& q, const Workspace& ws, const AttnLaunch& al,
                                 hipStream_t st, const SelectArgs* sel, const TailArgs* tail) {
    Int8Params a{};
    a.c = c; a.q = q; a.ws = ws;
    if (tail) a.tail = *tail;
    const int groups = c.L * c.B * c.Hkv;
    // one workgroup per group when the groups fill the GPU, else balanced slices
    // (at least 8 pages each) for about one workgroup per CU
    int s = groups >= 192 || al.max_entries <= kFusedSmallPages ? 1 : (256 + groups - 1) / std::max(groups, 1);
    s = std::min(s, (al.max_entries + 7) / 8);
    s = std::max(s, (al.max_entries + kMaxWgPages - 1) / kMaxWgPages);
    a.splits = std::max(1, std::min(s, al.s_max));
    dim3 grid(a.splits, groups);
    const bool fused = sel && sel->enabled;
    if (fused) {
        if (!int8_select_in_kernel(c, q, al)) return hipErrorInvalidValue;
        a.sel = *sel;
        // split 0 of each group attends a 16-bit tail itself (16-byte aligned
        // rows, at least D apart); other tails are attended in the split merge
        a.tail.in_kernel = mfma_tail_in_kernel(a.tail);
        // head chunks: a tail only inside the kernel (the split merge's tail
        // work indexes the cache by the virtual heads)
        if (a.sel.head_chunks > 1 && a.tail.len > 0 && !a.tail.in_kernel) return hipErrorInvalidValue;
    }
    if (c.meta_dtype == FQ_BF16)
        return fused ? launch_int8_nrep<bf16, true>(a, grid, st) : launch_int8_nrep<bf16, false>(a, grid, st);
    return fused ? launch_int8_nrep<f16, true>(a, grid, st) : launch_int8_nrep<f16, false>(a, grid, st);
}

}  // namespace fq
