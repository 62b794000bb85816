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

#include <type_traits>

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

// Unnormalised Sylvester Hadamard transform of a 128-vector held by one wave
// (lane holds elements lane and lane + 64): y_i = sum_j (-1)^popc(i & j) x_j,
// by butterflies (a + b, a - b) for h = 1, 2, ..., 64.
FQ_DEV void wave_hadamard128(float& v0, float& v1) {
    const int lane = lane_id();
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) {
        const float y0 = __shfl_xor(v0, h, 64), y1 = __shfl_xor(v1, h, 64);
        v0 = (lane & h) ? y0 - v0 : v0 + y0;
        v1 = (lane & h) ? y1 - v1 : v1 + y1;
    }
    const float a = v0, c = v1;
    v0 = a + c;
    v1 = a - c;
}

// Writes O (vals[r][d] = acc / l, rotated back when ROT) and lse for the NREP
// query heads of KV group (l, b, h).  Must be called by the whole workgroup
// after vals / Ls / Ms are complete in LDS.
template <int D, int NREP, bool ROT, int NT = kThreads>
FQ_DEV void store_outputs(const QueryArgs& q, int l, int b, int h, const float (*vals)[D], const float* Ls,
                          const float* Ms) {
    const int tid = threadIdx.x;
    const float inv = 1.0f / sqrtf((float)D);
    if (D == 128 && (ROT || q.rot)) {       // one wave per head; q.rot: then times the signs, s WHT(O) / sqrt(D)
        const int lane = lane_id();
        const float s0 = q.rot ? q.rot[lane] : 1.f, s1 = q.rot ? q.rot[lane + 64] : 1.f;
        for (int r = wave_id(); r < NREP; r += NT / 64) {
            float v0 = vals[r][lane], v1 = vals[r][lane + 64];
            wave_hadamard128(v0, v1);
            const int64_t ob = l * q.o_s[0] + b * q.o_s[1] + (h * NREP + r) * q.o_s[2];
            store_any(q.out, q.out_dtype, ob + lane * q.o_s[3], v0 * inv * s0);
            store_any(q.out, q.out_dtype, ob + (lane + 64) * q.o_s[3], v1 * inv * s1);
        }
    } else
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

// Merges the NW waves' (m, l, acc) states held in s (after a barrier); writes
// O / lse, or with `partial` (more than one split, or a tail to fold in) stores
// the workgroup's split partial for merge_splits_kernel.
template <int D, int NREP, bool ROT, int NW = 4, int NT = 64 * NW>
FQ_DEV void merge_waves_and_store(SplitLds<D, NREP, NW>& s, const QueryArgs& q, const Workspace& ws, int g, int l,
                                  int b, int h, int split, bool partial, int nslots = NW) {
    const int tid = threadIdx.x;
    const int64_t part = ((int64_t)g * ws.s_max + split) * NREP;
    for (int i = tid; i < NREP * D; i += NT) {
        const int r = i / D, d = i % D;
        float M = -INFINITY, L = 0.f, A = 0.f;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) {
            if (ww >= nslots) break;
            float Mn, w_s, w_o;
            merge_weights(M, s.m[ww][r], Mn, w_s, w_o);
            L = L * w_s + s.l[ww][r] * w_o;
            A = A * w_s + s.acc[ww][r][d] * w_o;
            M = Mn;
        }
        if (!partial) {
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
    if (!partial) {
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
    merge_waves_and_store<D, NREP, ROT>(s, q, ws, g, l, b, h, split, splits > 1);
}

// The dense attention state (log2-domain max m, sum l, acc) of one KV group's
// partial-page tail, for every query head of the group, by the whole
// workgroup (kThreads threads).  TT: the tail's element type (float, bf16 or
// f16), so every load is a plain typed load issued ahead of its use.
template <typename TT> FQ_DEV float tail_elem(const void* p, int64_t i);
template <> FQ_DEV float tail_elem<float>(const void* p, int64_t i) { return ((const float*)p)[i]; }
template <> FQ_DEV float tail_elem<bf16>(const void* p, int64_t i) { return bf16_bits_to_f(((const uint16_t*)p)[i]); }
template <> FQ_DEV float tail_elem<f16>(const void* p, int64_t i) { return f16_bits_to_f(((const uint16_t*)p)[i]); }
// 8 consecutive elements (16-byte aligned for 2-byte types, 32 for fp32)
template <typename TT> FQ_DEV void tail_elem8(const void* p, int64_t i, float (&o)[8]) {
    if constexpr (std::is_same<TT, float>::value) {
        const float4 a = *(const float4*)((const float*)p + i), c = *(const float4*)((const float*)p + i + 4);
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = c.x; o[5] = c.y; o[6] = c.z; o[7] = c.w;
    } else {
        const uint4 a = *(const uint4*)((const uint16_t*)p + i);
        const uint32_t wv[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o[2 * k] = half_to_f<TT>(wv[k]);
            o[2 * k + 1] = half_to_f<TT>(wv[k] >> 16);
        }
    }
}

template <int D, int NREP, typename TT>
FQ_DEV void tail_state(const QueryArgs& q, const TailArgs& tail, int l, int b, int h, float (*s_tq)[D],
                       float (*s_tp)[kTailMax], float* s_tm, float* s_tl) {
    static_assert(D % 16 == 0 && kThreads % D == 0 && D / 16 == 8, "tail layout: 8 channels per logit lane");
    constexpr int NH = kThreads / D;                 // token groups in the p.v phase
    constexpr int KI = kTailMax * 16 / kThreads;     // logit items per thread
    constexpr int VI = kTailMax / NH;                // V tokens per thread
    const int lane = lane_id(), w = wave_id();
    const int T = tail.len;
    const int d = threadIdx.x % D, hf = threadIdx.x / D;
    // every load goes out first: q, the thread's K rows (8 channels each), its V column
    float qv[(NREP * D + kThreads - 1) / kThreads];
#pragma unroll
    for (int u = 0; u * kThreads < NREP * D; ++u) {
        const int i = min(u * kThreads + (int)threadIdx.x, NREP * D - 1);
        qv[u] = load_any(q.q, q.q_dtype, l * q.q_s[0] + b * q.q_s[1] + (h * NREP + i / D) * q.q_s[2] +
                                             (i % D) * q.q_s[3]);
    }
    const int64_t kb = l * tail.ks[0] + b * tail.ks[1] + h * tail.ks[2];
    float kv[KI][8];
#pragma unroll
    for (int u = 0; u < KI; ++u) {
        const int i = u * kThreads + threadIdx.x;
        tail_elem8<TT>(tail.k, kb + min(i >> 4, T - 1) * tail.ks[3] + 8 * (i & 15), kv[u]);
    }
    const int64_t vb = l * tail.vs[0] + b * tail.vs[1] + h * tail.vs[2];
    float vv[VI];
#pragma unroll
    for (int u = 0; u < VI; ++u) vv[u] = tail_elem<TT>(tail.v, vb + min(hf + NH * u, T - 1) * tail.vs[3] + d);
#pragma unroll
    for (int u = 0; u * kThreads < NREP * D; ++u) {
        const int i = u * kThreads + threadIdx.x;
        if (i < NREP * D) s_tq[i / D][i % D] = qv[u] * q.qk_scale;
    }
    __syncthreads();
    // logits: 16 lanes per token, lane j owns channels 8j .. 8j+7
#pragma unroll
    for (int u = 0; u < KI; ++u) {
        const int i = u * kThreads + threadIdx.x;
        const int t = min(i >> 4, T - 1), j = i & 15;
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
            float v = 0.f;
#pragma unroll
            for (int c = 0; c < 8; ++c) v = fmaf(s_tq[r][8 * j + c], kv[u][c], v);
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) v += __shfl_xor(v, off, 64);
            if (j == 0 && i < T * 16) s_tp[r][t] = v;
        }
    }
    __syncthreads();
    for (int r = w; r < NREP; r += kThreads / 64) {
        const float v = lane < T ? s_tp[r][lane] : -INFINITY;
        float m = v;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        const float pe = lane < T ? exp2_fast(v - m) : 0.f;
        float ls = pe;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ls += __shfl_xor(ls, off, 64);
        if (lane < T) s_tp[r][lane] = pe;
        if (lane == 0) { s_tm[r] = m; s_tl[r] = ls; }
    }
    __syncthreads();
    // p.v: thread (channel d, token group hf) sums tokens hf, hf + NH, ... for
    // every head; the NH groups meet in LDS (s_tq, no longer read, takes them)
    float a[NREP];
#pragma unroll
    for (int r = 0; r < NREP; ++r) a[r] = 0.f;
#pragma unroll
    for (int u = 0; u < VI; ++u) {
        if (hf + NH * u < T) {
#pragma unroll
            for (int r = 0; r < NREP; ++r) a[r] = fmaf(s_tp[r][hf + NH * u], vv[u], a[r]);
        }
    }
    if (hf == 0) {
#pragma unroll
        for (int r = 0; r < NREP; ++r) s_tq[r][d] = a[r];
    }
    for (int g2 = 1; g2 < NH; ++g2) {
        __syncthreads();
        if (hf == g2) {
#pragma unroll
            for (int r = 0; r < NREP; ++r) s_tq[r][d] += a[r];
        }
    }
    __syncthreads();
}

// The tail's attention state from LDS, for the fused decode kernel: tk / tv
// hold the tail's T <= kTailMax tokens as raw 16-bit values (bf16 when bf16,
// else fp16), sq the group's queries pre-scaled by sm_scale * log2(e).  All NT
// threads take part; the state goes to (m_out, l_out, acc_out) -- one more slot
// of the workgroup's wave merge.  sp: kTailMax-float scratch per head.
template <int D, int NREP, int NT>
FQ_DEV void tail_state_lds(const uint16_t (*tk)[D], const uint16_t (*tv)[D], bool bf, int T, const float (*sq)[D],
                           float (*sp)[kTailMax], float* m_out, float* l_out, float (*acc_out)[D]) {
    static_assert(D == 128 && NT % D == 0 && NT % 16 == 0, "tail layout");
    constexpr int NH = NT / D;                       // token groups in the p.v phase
    const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
    auto cvt = [&](uint32_t bits) { return bf ? bf16_bits_to_f(bits & 0xFFFFu) : f16_bits_to_f(bits & 0xFFFFu); };
    // logits: 16 lanes per token, lane j owns channels 8j .. 8j+7 (one 16-byte LDS read)
    for (int i0 = 0; i0 < kTailMax * 16; i0 += NT) {
        const int i = i0 + tid;
        const int t = min(i >> 4, kTailMax - 1), j = i & 15;
        const uint4 raw = *(const uint4*)&tk[t][8 * j];
        const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
        float kv[8];
#pragma unroll
        for (int c = 0; c < 4; ++c) { kv[2 * c] = cvt(wv[c]); kv[2 * c + 1] = cvt(wv[c] >> 16); }
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
            float v = 0.f;
#pragma unroll
            for (int c = 0; c < 8; ++c) v = fmaf(sq[r][8 * j + c], kv[c], v);
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) v += __shfl_xor(v, off, 64);
            if (j == 0 && t < T) sp[r][t] = v;
        }
    }
    lds_barrier();
    for (int r = w; r < NREP; r += NT / 64) {
        const float v = lane < T ? sp[r][lane] : -INFINITY;
        float m = v;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        const float pe = lane < T ? exp2_fast(v - m) : 0.f;
        float ls = pe;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ls += __shfl_xor(ls, off, 64);
        if (lane < T) sp[r][lane] = pe;
        if (lane == 0) { m_out[r] = m; l_out[r] = ls; }
    }
    lds_barrier();
    // p.v: thread (channel d, token group hf) over tokens hf, hf + NH, ...; the
    // groups meet in acc_out
    const int d = tid % D, hf = tid / D;
    float a[NREP];
#pragma unroll
    for (int r = 0; r < NREP; ++r) a[r] = 0.f;
    for (int t = hf; t < T; t += NH) {
        const float v = cvt(tv[t][d]);
#pragma unroll
        for (int r = 0; r < NREP; ++r) a[r] = fmaf(sp[r][t], v, a[r]);
    }
    if (hf == 0) {
#pragma unroll
        for (int r = 0; r < NREP; ++r) acc_out[r][d] = a[r];
    }
    for (int g2 = 1; g2 < NH; ++g2) {
        lds_barrier();
        if (hf == g2) {
#pragma unroll
            for (int r = 0; r < NREP; ++r) acc_out[r][d] += a[r];
        }
    }
    lds_barrier();
}

// Split merge (the rule of _merge_two_attentions, llama_persistent_patch.py:50-61,
// in the log2 domain): one workgroup per KV group over its used splits.
// pps > 0: group g used ceil(n_sel / pps) splits; pps == 0: all `splits` were used.
// Two parallel phases instead of a serial walk over the splits: wave r reduces
// head r's (m, l) over the splits into per-split weights in LDS (its lanes
// stride over the splits), then every output element sums its splits'
// weighted partials with the loads issued 8 at a time.  Per split the weight is
// exp2(m_s - M) with M the maximum over the splits (0 for an empty split).
//
// With a tail (the partial page, llama_persistent_patch.py:229-240), the
// workgroup first attends the group's tail tokens densely in fp32
// (_bf16_dense_attn_with_lse, 30-47: q.k * sm_scale, softmax, p.v) and folds
// that state in as one more split: the result is softmax attention over the
// selected pages and the tail together, which is what _merge_two_attentions
// computes from the two parts (up to its bf16 rounding of each part).
constexpr int kMergeMaxSplits = 2048;

template <int D, int NREP, bool ROT>
__global__ __launch_bounds__(kThreads) void merge_splits_kernel(QueryArgs q, Workspace ws, int Hkv, int B,
                                                            int pps, int splits, TailArgs tail) {
    __shared__ float s_out[NREP][D];
    __shared__ float s_L[NREP], s_M[NREP];
    __shared__ float s_w[NREP][kMergeMaxSplits];
    __shared__ float s_tq[NREP][D];          // tail: q * qk_scale, then the tail's acc
    __shared__ float s_tp[NREP][kTailMax];   // tail logits, then probabilities
    __shared__ float s_tm[NREP], s_tl[NREP];
    const int g = blockIdx.x;
    const int h = g % Hkv, b = (g / Hkv) % B, l = g / (Hkv * B);
    const int used = min(pps > 0 ? (ws.n_sel[g] + pps - 1) / pps : splits, kMergeMaxSplits);
    const int64_t base = (int64_t)g * ws.s_max * NREP;
    const int lane = lane_id(), w = wave_id();
    const int T = D == 128 ? tail.len : 0;
    if constexpr (D == 128) {             // only the matrix-core path (D = 128) passes a tail
        if (T > 0) {
            if (tail.dtype == FQ_F32) tail_state<D, NREP, float>(q, tail, l, b, h, s_tq, s_tp, s_tm, s_tl);
            else if (tail.dtype == FQ_BF16) tail_state<D, NREP, bf16>(q, tail, l, b, h, s_tq, s_tp, s_tm, s_tl);
            else tail_state<D, NREP, f16>(q, tail, l, b, h, s_tq, s_tp, s_tm, s_tl);
        }
    }
    for (int r = w; r < NREP; r += kThreads / 64) {
    float M = T > 0 ? s_tm[r] : -INFINITY;
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
    if (lane == 0) {
        if (T > 0) {
            const float wt = exp2_fast(s_tm[r] - M);
            s_tm[r] = wt;                  // the tail's weight from here on
            Lsum += wt * s_tl[r];
        }
        s_L[r] = Lsum;
        s_M[r] = M;
    }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < NREP * D; i += kThreads) {
    const int r = i / D, d = i % D;
    float A = T > 0 ? s_tm[r] * s_tq[r][d] : 0.f;
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

// The same merge for few splits (<= SM) and no tail to fold in, as a latency
// path: one wave per (group, query head), lane d holding channels d and
// d + 64, every split's (m, l) and partial acc loaded in one round, then
// M = max_s m_s, w_s = exp2(m_s - M) (0 for an empty split), L = sum_s w_s l_s,
// O = (sum_s w_s acc_s) / L, splits summed in ascending order.  ROT (or
// q.rot): O rotated back by the wave butterflies, as store_outputs does.
template <bool ROT, int SM>
__global__ __launch_bounds__(64) void merge_splits_wave_kernel(QueryArgs q, Workspace ws, int Hkv, int B,
                                                                int splits) {
    constexpr int D = 128;
    const int g = blockIdx.x, r = blockIdx.y, nrep = q.nrep;
    const int h = g % Hkv, b = (g / Hkv) % B, l = g / (Hkv * B);
    const int lane = threadIdx.x;
    const int64_t base = (int64_t)g * ws.s_max * nrep + r;
    float m[SM], lv[SM], a0[SM], a1[SM];
#pragma unroll
    for (int s = 0; s < SM; ++s) {
        const int64_t pr = base + (int64_t)min(s, splits - 1) * nrep;
        m[s] = ws.part_ml[pr * 2];
        lv[s] = ws.part_ml[pr * 2 + 1];
        a0[s] = ws.part_acc[pr * D + lane];
        a1[s] = ws.part_acc[pr * D + lane + 64];
    }
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < SM; ++s)
        if (s < splits) M = fmaxf(M, m[s]);
    float L = 0.f, A0 = 0.f, A1 = 0.f;
#pragma unroll
    for (int s = 0; s < SM; ++s) {
        if (s < splits) {
            const float w = m[s] == -INFINITY ? 0.f : exp2_fast(m[s] - M);
            L = fmaf(w, lv[s], L);
            A0 = fmaf(w, a0[s], A0);
            A1 = fmaf(w, a1[s], A1);
        }
    }
    float v0 = L > 0.f ? A0 / L : 0.f, v1 = L > 0.f ? A1 / L : 0.f;
    if (ROT || q.rot) {
        const float inv = 1.0f / sqrtf((float)D);
        const float s0 = q.rot ? q.rot[lane] : 1.f, s1 = q.rot ? q.rot[lane + 64] : 1.f;
        wave_hadamard128(v0, v1);
        v0 *= inv * s0;
        v1 *= inv * s1;
    }
    const int hq = h * nrep + r;
    const int64_t ob = l * q.o_s[0] + b * q.o_s[1] + hq * q.o_s[2];
    store_any(q.out, q.out_dtype, ob + lane * q.o_s[3], v0);
    store_any(q.out, q.out_dtype, ob + (lane + 64) * q.o_s[3], v1);
    if (q.lse && lane == 0)
        q.lse[l * q.lse_s[0] + b * q.lse_s[1] + hq * q.lse_s[2]] = L > 0.f ? (M + log2f(L)) * kLn2 : -INFINITY;
}

// The split merge launch of the D = 128 matrix-core paths: the one-round wave
// merge for up to 32 splits without a tail, merge_splits_kernel otherwise.
template <int NREP, bool ROT>
inline void launch_split_merge(const QueryArgs& q, const Workspace& ws, int Hkv, int B, int groups, int splits,
                               const TailArgs& tail, hipStream_t st) {
    if (tail.len == 0 && splits <= 32) {
        const dim3 grid(groups, NREP);
        if (splits <= 8) hipLaunchKernelGGL((merge_splits_wave_kernel<ROT, 8>), grid, dim3(64), 0, st, q, ws, Hkv, B, splits);
        else if (splits <= 16) hipLaunchKernelGGL((merge_splits_wave_kernel<ROT, 16>), grid, dim3(64), 0, st, q, ws, Hkv, B, splits);
        else if (splits <= 24) hipLaunchKernelGGL((merge_splits_wave_kernel<ROT, 24>), grid, dim3(64), 0, st, q, ws, Hkv, B, splits);
        else hipLaunchKernelGGL((merge_splits_wave_kernel<ROT, 32>), grid, dim3(64), 0, st, q, ws, Hkv, B, splits);
        return;
    }
    hipLaunchKernelGGL((merge_splits_kernel<128, NREP, ROT>), dim3(groups), dim3(kThreads), 0, st, q, ws, Hkv, B, 0,
                       splits, tail);
}

}  // namespace fq
