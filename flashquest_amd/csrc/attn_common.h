// Split-K epilogue shared by the INT4 and turbo decode-attention kernels.
//
// Each lane holds, for NREP query heads, an online-softmax state (m in the
// log2 domain, l, acc for its 8 channels cc*8..cc*8+7) covering the tokens of
// its token row.  finish_split() merges rows (cross-lane) and waves (LDS);
// splits meet in merge_splits_kernel (a separate launch, so no cross-workgroup
// fences are needed).  Outputs use the reference's epilogue: O = acc / l, lse = (m + log2 l) * ln2, and
// O = 0 / lse = -inf for an empty selection (sparse_int4_fwd.py:147-157).
// The split merge is _merge_two_attentions (llama_persistent_patch.py:50-61)
// in the log2 domain.  ROT = true applies the inverse rotation
// O = WHT(O_rot) before the store (sparse_turbo_fwd.py:343-344).
#pragma once

#include "fq_common.h"

namespace fq {

FQ_DEV float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

FQ_DEV void merge_weights(float m_self, float m_other, float& M, float& w_self, float& w_other) {
    M = fmaxf(m_self, m_other);
    w_self = m_self == -INFINITY ? 0.f : exp2_fast(m_self - M);
    w_other = m_other == -INFINITY ? 0.f : exp2_fast(m_other - M);
}

// Walsh-Hadamard entry H[i][j] / sqrt(D) with the Sylvester sign (-1)^popc(i&j).
FQ_DEV float hadamard_sign(int i, int j) { return (__popc(i & j) & 1) ? -1.f : 1.f; }

template <int D, int NREP, int NW = 4>
struct SplitLds {
    float m[NW][NREP], l[NW][NREP];
    float acc[NW][NREP][D];
    float out[NREP][D];
    float L[NREP], M[NREP];
};

// Writes O (vals[r][d] = acc / l, rotated back when ROT) and lse for the NREP
// query heads of KV group (l, b, h).  Must be called by the whole workgroup
// after vals / Ls / Ms are complete in LDS.
template <int D, int NREP, bool ROT, int NT = kThreads>
FQ_DEV void store_outputs(const QueryArgs& q, int l, int b, int h, const float (*vals)[D], const float* Ls,
                          const float* Ms) {
    const int tid = threadIdx.x;
    const float inv = 1.0f / sqrtf((float)D);
    for (int i = tid; i < NREP * D; i += NT) {
        const int r = i / D, d = i % D;
        float o = vals[r][d];
        if constexpr (ROT) {
            o = 0.f;
            for (int k = 0; k < D; ++k) o = fmaf(hadamard_sign(d, k), vals[r][k], o);
            o *= inv;
        }
        const int hq = h * NREP + r;
        store_any(q.out, q.out_dtype, l * q.o_s[0] + b * q.o_s[1] + hq * q.o_s[2] + d * q.o_s[3], o);
    }
    if (q.lse)
        for (int r = tid; r < NREP; r += NT) {
            const int hq = h * NREP + r;
            q.lse[l * q.lse_s[0] + b * q.lse_s[1] + hq * q.lse_s[2]] =
                Ls[r] > 0.f ? (Ms[r] + log2f(Ls[r])) * kLn2 : -INFINITY;
        }
}

// Merges the NW waves' (m, l, acc) states held in s (after a barrier); with one
// split writes O / lse, otherwise stores the workgroup's split partial.
template <int D, int NREP, bool ROT, int NW = 4>
FQ_DEV void merge_waves_and_store(SplitLds<D, NREP, NW>& s, const QueryArgs& q, const Workspace& ws, int g, int l,
                                  int b, int h, int split, int splits) {
    constexpr int NT = 64 * NW;
    const int tid = threadIdx.x;
    const int64_t part = ((int64_t)g * ws.s_max + split) * NREP;
    for (int i = tid; i < NREP * D; i += NT) {
        const int r = i / D, d = i % D;
        float M = -INFINITY, L = 0.f, A = 0.f;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) {
            float Mn, w_s, w_o;
            merge_weights(M, s.m[ww][r], Mn, w_s, w_o);
            L = L * w_s + s.l[ww][r] * w_o;
            A = A * w_s + s.acc[ww][r][d] * w_o;
            M = Mn;
        }
        if (splits == 1) {
            s.out[r][d] = L > 0.f ? A / L : 0.f;
            if (d == 0) { s.L[r] = L; s.M[r] = M; }
        } else {
            ws.part_acc[(part + r) * D + d] = A;
            if (d == 0) {
                ws.part_ml[(part + r) * 2] = M;
                ws.part_ml[(part + r) * 2 + 1] = L;
            }
        }
    }
    if (splits == 1) {
        __syncthreads();
        store_outputs<D, NREP, ROT, NT>(q, l, b, h, s.out, s.L, s.M);
    }
}

// Merges the lanes' row states and the workgroup's waves.  With one split the
// workgroup writes O / lse directly; otherwise it stores its partial
// (m, l, acc) for merge_splits_kernel.
template <int D, int NREP, bool ROT>
FQ_DEV void finish_split(SplitLds<D, NREP>& s, float (&m)[NREP], float (&lsum)[NREP], float (&acc)[NREP][8],
                         bool active, const QueryArgs& q, const Workspace& ws, int g, int l, int b, int h,
                         int split, int splits) {
    constexpr int NCC = D / 8;
    const int lane = lane_id(), w = wave_id();
    const int cc = lane % NCC, row = lane / NCC;
    if (!active) return;     // uniform per workgroup
#pragma unroll
    for (int off = NCC; off < 64; off <<= 1) {
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
            const float mo = __shfl_xor(m[r], off, 64);
            float M, ws_, wo;
            merge_weights(m[r], mo, M, ws_, wo);
            lsum[r] = lsum[r] * ws_ + __shfl_xor(lsum[r], off, 64) * wo;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[r][j] = acc[r][j] * ws_ + __shfl_xor(acc[r][j], off, 64) * wo;
            m[r] = M;
        }
    }
    if (row == 0) {
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
            if (cc == 0) { s.m[w][r] = m[r]; s.l[w][r] = lsum[r]; }
#pragma unroll
            for (int j = 0; j < 8; ++j) s.acc[w][r][cc * 8 + j] = acc[r][j];
        }
    }
    __syncthreads();
    merge_waves_and_store<D, NREP, ROT>(s, q, ws, g, l, b, h, split, splits);
}

// Split merge (the rule of _merge_two_attentions, llama_persistent_patch.py:50-61,
// in the log2 domain): one workgroup per KV group over its used splits.
// pps > 0: group g used ceil(n_sel / pps) splits; pps == 0: all `splits` were used.
// Two parallel phases instead of a serial walk over the splits: wave r reduces
// head r's (m, l) over the splits into per-split weights in LDS (its lanes
// stride over the splits), then every output element sums its splits'
// weighted partials with the loads issued 8 at a time.  Per split the weight is
// exp2(m_s - M) with M the maximum over the splits (0 for an empty split).
constexpr int kMergeMaxSplits = 2048;

template <int D, int NREP, bool ROT>
__global__ __launch_bounds__(kThreads) void merge_splits_kernel(QueryArgs q, Workspace ws, int Hkv, int B,
                                                                int pps, int splits) {
    __shared__ float s_out[NREP][D];
    __shared__ float s_L[NREP], s_M[NREP];
    __shared__ float s_w[NREP][kMergeMaxSplits];
    const int g = blockIdx.x;
    const int h = g % Hkv, b = (g / Hkv) % B, l = g / (Hkv * B);
    const int used = min(pps > 0 ? (ws.n_sel[g] + pps - 1) / pps : splits, kMergeMaxSplits);
    const int64_t base = (int64_t)g * ws.s_max * NREP;
    const int lane = lane_id(), w = wave_id();
    for (int r = w; r < NREP; r += kThreads / 64) {
        float M = -INFINITY;
        for (int sp = lane; sp < used; sp += 64) M = fmaxf(M, ws.part_ml[(base + (int64_t)sp * NREP + r) * 2]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        float Lsum = 0.f;
        for (int sp = lane; sp < used; sp += 64) {
            const int64_t pr = base + (int64_t)sp * NREP + r;
            const float m = ws.part_ml[pr * 2];
            const float wt = m == -INFINITY ? 0.f : exp2_fast(m - M);
            s_w[r][sp] = wt;
            Lsum += wt * ws.part_ml[pr * 2 + 1];
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) Lsum += __shfl_xor(Lsum, off, 64);
        if (lane == 0) { s_L[r] = Lsum; s_M[r] = M; }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < NREP * D; i += kThreads) {
        const int r = i / D, d = i % D;
        float A = 0.f;
        int sp = 0;
        for (; sp + 8 <= used; sp += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = ws.part_acc[(base + (int64_t)(sp + u) * NREP + r) * D + d];
#pragma unroll
            for (int u = 0; u < 8; ++u) A = fmaf(s_w[r][sp + u], v[u], A);
        }
        for (; sp < used; ++sp) A = fmaf(s_w[r][sp], ws.part_acc[(base + (int64_t)sp * NREP + r) * D + d], A);
        s_out[r][d] = s_L[r] > 0.f ? A / s_L[r] : 0.f;
    }
    __syncthreads();
    store_outputs<D, NREP, ROT>(q, l, b, h, s_out, s_L, s_M);
}

}  // namespace fq
