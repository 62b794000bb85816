// Cache-write quantisers, Walsh-Hadamard transform, LSE merge and the dense
// bf16 tail attention (gfx950).  These are the operators on either side of the
// sparse decode kernel in the reference's decode path.
#include "fq_common.h"
#include "turbo_quant.h"

namespace fq {

constexpr float kEps = 1e-6f;                 // kv_quant.py:14
// Reciprocal torch's CUDA true-division uses for "tensor / 15.0"
// (the divisor is a CPU scalar, so the kernel multiplies by fp32(1/15)).
__device__ __constant__ float kInv15 = 1.0f / 15.0f;
__device__ __constant__ float kInv255 = 1.0f / 255.0f;   // the INT8 quantisers' "/ 255.0"

namespace {

// -------------------------------------------------------------------------
// quantize_k_int4 (kv_quant.py:131-171) and, BITS = 8, quantize_k
// (kv_quant.py:18-61: "/ 255.0", codes 0..255 one per byte).  One thread per
// (b, h, page, channel pair).  Scale arithmetic in the input dtype, codes by
// IEEE fp32 division.
// -------------------------------------------------------------------------
struct QuantKParams {
    const void* k; int in_dtype; int64_t k_s[4];
    int B, H, S, D, page, P;
    uint8_t* packed; int64_t p_s[4];
    void* scale; int64_t s_s[4];
    void* mn; int64_t m_s[4];
    int meta_dtype;
};

template <int BITS>
__global__ __launch_bounds__(kThreads) void quant_k_kernel(QuantKParams a) {
    constexpr float kMaxCode = (1 << BITS) - 1;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int half_d = a.D / 2;
    const int64_t total = (int64_t)a.B * a.H * a.P * half_d;
    if (idx >= total) return;
    const int jp = idx % half_d;
    const int p = (idx / half_d) % a.P;
    const int h = (idx / ((int64_t)half_d * a.P)) % a.H;
    const int b = idx / ((int64_t)half_d * a.P * a.H);
    const int64_t base = b * a.k_s[0] + h * a.k_s[1];
    const int t0 = p * a.page, t1 = min(a.S, t0 + a.page);
    float mn[2] = {INFINITY, INFINITY}, mx[2] = {-INFINITY, -INFINITY};
    for (int t = t0; t < t1; ++t) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const float v = load_any(a.k, a.in_dtype, base + t * a.k_s[2] + (2 * jp + u) * a.k_s[3]);
            mn[u] = fminf(mn[u], v);
            mx[u] = fmaxf(mx[u], v);
        }
    }
    float sc[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const float diff = round_to(mx[u] - mn[u], a.in_dtype);
        float s = round_to(diff * (BITS == 8 ? kInv255 : kInv15), a.in_dtype);
        s = round_to(fmaxf(s, kEps), a.in_dtype);
        sc[u] = s;
        const int64_t mo = b * a.s_s[0] + h * a.s_s[1] + p * a.s_s[2] + (2 * jp + u) * a.s_s[3];
        const int64_t mm = b * a.m_s[0] + h * a.m_s[1] + p * a.m_s[2] + (2 * jp + u) * a.m_s[3];
        store_any(a.scale, a.meta_dtype, mo, s);
        store_any(a.mn, a.meta_dtype, mm, mn[u]);
    }
    for (int t = t0; t < t1; ++t) {
        uint32_t byte = 0;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const float v = load_any(a.k, a.in_dtype, base + t * a.k_s[2] + (2 * jp + u) * a.k_s[3]);
            float c = rintf(__fdiv_rn(v - mn[u], sc[u]));
            c = fminf(fmaxf(c, 0.f), kMaxCode);
            if constexpr (BITS == 8)
                a.packed[b * a.p_s[0] + h * a.p_s[1] + t * a.p_s[2] + (2 * jp + u) * a.p_s[3]] = (uint8_t)c;
            byte |= ((uint32_t)c) << (4 * u);
        }
        if constexpr (BITS == 4) a.packed[b * a.p_s[0] + h * a.p_s[1] + t * a.p_s[2] + jp * a.p_s[3]] = (uint8_t)byte;
    }
}

// -------------------------------------------------------------------------
// quantize_v_int4 (kv_quant.py:189-205) and, BITS = 8, quantize_v
// (kv_quant.py:78-89), fp32 arithmetic.  One thread per (b, h, token,
// channel group).
// -------------------------------------------------------------------------
struct QuantVParams {
    const void* v; int in_dtype; int64_t v_s[4];
    int B, H, S, D, group, G;
    uint8_t* packed; int64_t p_s[4];
    void* scale; int64_t s_s[4];
    void* mn; int64_t m_s[4];
    int meta_dtype;
};

template <int BITS>
__global__ __launch_bounds__(kThreads) void quant_v_kernel(QuantVParams a) {
    constexpr float kMaxCode = (1 << BITS) - 1;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.H * a.S * a.G;
    if (idx >= total) return;
    const int gi = idx % a.G;
    const int t = (idx / a.G) % a.S;
    const int h = (idx / ((int64_t)a.G * a.S)) % a.H;
    const int b = idx / ((int64_t)a.G * a.S * a.H);
    const int64_t base = b * a.v_s[0] + h * a.v_s[1] + t * a.v_s[2];
    const int d0 = gi * a.group;
    float mn = INFINITY, mx = -INFINITY;
    for (int d = d0; d < d0 + a.group; ++d) {
        const float v = load_any(a.v, a.in_dtype, base + d * a.v_s[3]);
        mn = fminf(mn, v);
        mx = fmaxf(mx, v);
    }
    const float s = fmaxf((mx - mn) * (BITS == 8 ? kInv255 : kInv15), kEps);
    store_any(a.scale, a.meta_dtype, b * a.s_s[0] + h * a.s_s[1] + t * a.s_s[2] + gi * a.s_s[3], s);
    store_any(a.mn, a.meta_dtype, b * a.m_s[0] + h * a.m_s[1] + t * a.m_s[2] + gi * a.m_s[3], mn);
    uint8_t* prow = a.packed + b * a.p_s[0] + h * a.p_s[1] + t * a.p_s[2];
    for (int d = d0; d < d0 + a.group; d += 2) {
        uint32_t byte = 0;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const float v = load_any(a.v, a.in_dtype, base + (d + u) * a.v_s[3]);
            float c = rintf(__fdiv_rn(v - mn, s));
            c = fminf(fmaxf(c, 0.f), kMaxCode);
            if constexpr (BITS == 8) prow[(d + u) * a.p_s[3]] = (uint8_t)c;
            byte |= ((uint32_t)c) << (4 * u);
        }
        if constexpr (BITS == 4) prow[(d / 2) * a.p_s[3]] = (uint8_t)byte;
    }
}

// The same quantiser with a lane per channel pair (channels 2p, 2p + 1): a
// token's row is read by consecutive lanes (coalesced), the group's min / max
// come from lane shuffles over group / 2 lanes, and each lane writes its two
// codes.  For D in {64, 128} and power-of-two groups (the cache layouts); the
// arithmetic per element is the one-thread kernel's.
template <int BITS>
__global__ __launch_bounds__(kThreads) void quant_v_wave_kernel(QuantVParams a) {
    constexpr float kMaxCode = (1 << BITS) - 1;
    const int64_t p = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int half = a.D / 2;
    const int64_t total = (int64_t)a.B * a.H * a.S * half;
    const bool live = p < total;
    const int64_t pp = live ? p : 0;
    const int pair = pp % half;
    const int64_t tok = pp / half;
    const int t = tok % a.S;
    const int h = (tok / a.S) % a.H;
    const int b = tok / ((int64_t)a.S * a.H);
    const int64_t base = b * a.v_s[0] + h * a.v_s[1] + t * a.v_s[2];
    const int d = 2 * pair;
    const float v0 = load_any(a.v, a.in_dtype, base + d * a.v_s[3]);
    const float v1 = load_any(a.v, a.in_dtype, base + (d + 1) * a.v_s[3]);
    float mn = fminf(v0, v1), mx = fmaxf(v0, v1);
    for (int off = 1; off < a.group / 2; off <<= 1) {   // lanes of one group: aligned, power-of-two span
        mn = fminf(mn, __shfl_xor(mn, off, 64));
        mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    }
    if (!live) return;
    const float s = fmaxf((mx - mn) * (BITS == 8 ? kInv255 : kInv15), kEps);
    const int gi = d / a.group;
    if (d % a.group == 0) {
        store_any(a.scale, a.meta_dtype, b * a.s_s[0] + h * a.s_s[1] + t * a.s_s[2] + gi * a.s_s[3], s);
        store_any(a.mn, a.meta_dtype, b * a.m_s[0] + h * a.m_s[1] + t * a.m_s[2] + gi * a.m_s[3], mn);
    }
    const float c0 = fminf(fmaxf(rintf(__fdiv_rn(v0 - mn, s)), 0.f), kMaxCode);
    const float c1 = fminf(fmaxf(rintf(__fdiv_rn(v1 - mn, s)), 0.f), kMaxCode);
    uint8_t* prow = a.packed + b * a.p_s[0] + h * a.p_s[1] + t * a.p_s[2];
    if constexpr (BITS == 8) {
        prow[d * a.p_s[3]] = (uint8_t)c0;
        prow[(d + 1) * a.p_s[3]] = (uint8_t)c1;
    } else {
        prow[pair * a.p_s[3]] = (uint8_t)((uint32_t)c0 | ((uint32_t)c1 << 4));
    }
}

// -------------------------------------------------------------------------
// WHT along the last axis (wht.py:17-41): stages h = 1, 2, ..., D/2 of
// (a + b, a - b), each rounded to arith_dtype, then * fp32(1/sqrt(D)).
// One thread per row.  Optional sign vector: forward = WHT(s * x),
// inverse = s * WHT(x).
// -------------------------------------------------------------------------
struct WhtParams {
    const void* x; int x_dtype; int64_t x_rs;
    void* out; int out_dtype; int64_t o_rs;
    int N;
    const float* signs; int inverse; int arith;
};

// One wave per row (D = 128: lane l holds elements l and l + 64) or 64 / D
// rows per wave (D <= 64: one element per lane), so loads and stores are
// coalesced.  The butterflies run in the reference's order, h = 1, 2, ..., D/2
// (partners h < 64 apart by a lane shuffle, h = 64 within the lane), each
// sum and difference rounded to the arithmetic dtype as before.
template <int D>
__global__ __launch_bounds__(kThreads) void wht_kernel(WhtParams a) {
    constexpr int E = D > 64 ? 2 : 1;               // elements per lane
    constexpr int RPW = D >= 64 ? 1 : 64 / D;        // rows per wave
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
    const int64_t row = wave * RPW + (D >= 64 ? 0 : lane / D);
    const int e0 = D >= 64 ? lane : lane % D;
    const bool live = row < a.N;
    const int64_t r = live ? row : 0;
    float v[E];
#pragma unroll
    for (int k = 0; k < E; ++k) {
        const int d = e0 + 64 * k;
        float x = load_any(a.x, a.x_dtype, r * a.x_rs + d);
        if (a.signs && !a.inverse) x *= a.signs[d];
        v[k] = x;
    }
#pragma unroll
    for (int h = 1; h < (D < 64 ? D : 64); h <<= 1) {
#pragma unroll
        for (int k = 0; k < E; ++k) {
            const float y = __shfl_xor(v[k], h, 64);
            v[k] = (e0 & h) ? round_to(y - v[k], a.arith) : round_to(v[k] + y, a.arith);
        }
    }
    if constexpr (D == 128) {
        const float x = v[0], y = v[1];
        v[0] = round_to(x + y, a.arith);
        v[1] = round_to(x - y, a.arith);
    }
    const float inv = 1.0f / sqrtf((float)D);
    if (!live) return;
#pragma unroll
    for (int k = 0; k < E; ++k) {
        const int d = e0 + 64 * k;
        float y = round_to(v[k] * inv, a.arith);
        if (a.signs && a.inverse) y *= a.signs[d];
        store_any(a.out, a.out_dtype, r * a.o_rs + d, y);
    }
}

// -------------------------------------------------------------------------
// TurboQuant quantiser (kv_quant.py:327-363, 381-405) for one tensor: WHT in
// the input dtype -> rms (sequential fp32 sum of squares) clamped >= 1e-6 ->
// nearest of 8 codepoints (first on ties) -> bit-split planes.  One thread
// per token.
// -------------------------------------------------------------------------
struct TurboQParams {
    const void* x; int in_dtype; int64_t x_s[4];
    int B, H, S;
    uint8_t* msb; int64_t msb_s[4];
    uint8_t* lsb; int64_t lsb_s[4];
    void* scale; int64_t s_s[4];
};

template <int D>
__global__ __launch_bounds__(kThreads) void turbo_quant_kernel(TurboQParams a) {
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.H * a.S;
    if (idx >= total) return;
    const int t = idx % a.S;
    const int h = (idx / a.S) % a.H;
    const int b = idx / ((int64_t)a.S * a.H);
    float v[D];
    const int64_t base = b * a.x_s[0] + h * a.x_s[1] + t * a.x_s[2];
#pragma unroll
    for (int d = 0; d < D; ++d) v[d] = load_any(a.x, a.in_dtype, base + d * a.x_s[3]);
    turbo_quant_row<D>(v, a.in_dtype, a.msb + b * a.msb_s[0] + h * a.msb_s[1] + t * a.msb_s[2], a.msb_s[3],
                       a.lsb + b * a.lsb_s[0] + h * a.lsb_s[1] + t * a.lsb_s[2], a.lsb_s[3],
                       a.scale, b * a.s_s[0] + h * a.s_s[1] + t * a.s_s[2]);
}

// -------------------------------------------------------------------------
// _merge_two_attentions (llama_persistent_patch.py:50-61): one thread per (n, d).
// -------------------------------------------------------------------------
struct MergeParams {
    const void* oa; const float* la; const void* ob; const float* lb;
    int dtype; int64_t rs_a, rs_b;
    void* out; int64_t rs_o; float* lse_out;
    int N, D;
};

__global__ __launch_bounds__(kThreads) void merge_kernel(MergeParams a) {
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (idx >= (int64_t)a.N * a.D) return;
    const int n = idx / a.D, d = idx % a.D;
    const float la = a.la[n], lb = a.lb[n];
    const float m = fmaxf(la, lb);
    const float wa = expf(la - m), wb = expf(lb - m);
    const float oa = load_any(a.oa, a.dtype, n * a.rs_a + d);
    const float ob = load_any(a.ob, a.dtype, n * a.rs_b + d);
    store_any(a.out, a.dtype, n * a.rs_o + d, (wa * oa + wb * ob) / (wa + wb));
    if (d == 0 && a.lse_out) a.lse_out[n] = m + logf(wa + wb);
}

// -------------------------------------------------------------------------
// _bf16_dense_attn_with_lse (llama_persistent_patch.py:30-47): fp32 softmax
// attention of one decode query over T tail tokens.  One workgroup per
// (b, h_q); thread t owns token t's logit.
// -------------------------------------------------------------------------
struct TailParams {
    const void* q; int64_t q_s[3];
    const void* k; int64_t k_s[4];
    const void* v; int64_t v_s[4];
    int kv_dtype;
    void* out; int64_t o_s[3]; float* lse;
    int B, Hq, Hkv, T, D;
};

__global__ __launch_bounds__(kThreads) void tail_attn_kernel(TailParams a) {
    __shared__ float s_q[256];
    __shared__ float s_p[1024];
    __shared__ float s_red[8];
    const int bh = blockIdx.x;
    const int hq = bh % a.Hq, b = bh / a.Hq;
    const int hk = hq / (a.Hq / a.Hkv);
    const int tid = threadIdx.x;
    for (int d = tid; d < a.D; d += kThreads)
        s_q[d] = load_any(a.q, a.kv_dtype, b * a.q_s[0] + hq * a.q_s[1] + d * a.q_s[2]);
    __syncthreads();
    const float sm = 1.0f / sqrtf((float)a.D);
    float lmax = -INFINITY;
    for (int t = tid; t < a.T; t += kThreads) {
        float dot = 0.f;
        for (int d = 0; d < a.D; ++d)
            dot = fmaf(s_q[d], load_any(a.k, a.kv_dtype, b * a.k_s[0] + hk * a.k_s[1] + t * a.k_s[2] + d * a.k_s[3]), dot);
        s_p[t] = dot * sm;
        lmax = fmaxf(lmax, dot * sm);
    }
    for (int off = 32; off >= 1; off >>= 1) lmax = fmaxf(lmax, __shfl_xor(lmax, off, 64));
    if (lane_id() == 0) s_red[wave_id()] = lmax;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    __syncthreads();
    float lsum = 0.f;
    for (int t = tid; t < a.T; t += kThreads) {
        const float p = expf(s_p[t] - M);
        s_p[t] = p;
        lsum += p;
    }
    for (int off = 32; off >= 1; off >>= 1) lsum += __shfl_xor(lsum, off, 64);
    if (lane_id() == 0) s_red[4 + wave_id()] = lsum;
    __syncthreads();
    const float L = s_red[4] + s_red[5] + s_red[6] + s_red[7];
    for (int d = tid; d < a.D; d += kThreads) {
        float o = 0.f;
        for (int t = 0; t < a.T; ++t)
            o = fmaf(s_p[t], load_any(a.v, a.kv_dtype, b * a.v_s[0] + hk * a.v_s[1] + t * a.v_s[2] + d * a.v_s[3]), o);
        store_any(a.out, FQ_BF16, b * a.o_s[0] + hq * a.o_s[1] + d * a.o_s[2], o / L);
    }
    if (tid == 0 && a.lse) a.lse[b * a.Hq + hq] = M + logf(L);
}

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

}  // namespace

hipError_t launch_quant_k(const void* k, int in_dtype, const int64_t* k_s, int B, int H, int S, int D,
                          int page, uint8_t* packed, const int64_t* p_s, void* scale, const int64_t* s_s,
                          void* mn, const int64_t* m_s, int meta_dtype, hipStream_t st, int bits) {
    QuantKParams a{};
    a.k = k; a.in_dtype = in_dtype; a.B = B; a.H = H; a.S = S; a.D = D; a.page = page;
    a.P = (S + page - 1) / page;
    a.packed = packed; a.scale = scale; a.mn = mn; a.meta_dtype = meta_dtype;
    for (int i = 0; i < 4; ++i) { a.k_s[i] = k_s[i]; a.p_s[i] = p_s[i]; a.s_s[i] = s_s[i]; a.m_s[i] = m_s[i]; }
    const int64_t total = (int64_t)B * H * a.P * (D / 2);
    if (total == 0) return hipSuccess;
    if (bits == 8) hipLaunchKernelGGL(quant_k_kernel<8>, dim3(blocks_for(total)), dim3(kThreads), 0, st, a);
    else hipLaunchKernelGGL(quant_k_kernel<4>, dim3(blocks_for(total)), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_quant_v(const void* v, int in_dtype, const int64_t* v_s, int B, int H, int S, int D,
                          int group, uint8_t* packed, const int64_t* p_s, void* scale, const int64_t* s_s,
                          void* mn, const int64_t* m_s, int meta_dtype, hipStream_t st, int bits) {
    QuantVParams a{};
    a.v = v; a.in_dtype = in_dtype; a.B = B; a.H = H; a.S = S; a.D = D; a.group = group;
    a.G = D / group;
    a.packed = packed; a.scale = scale; a.mn = mn; a.meta_dtype = meta_dtype;
    for (int i = 0; i < 4; ++i) { a.v_s[i] = v_s[i]; a.p_s[i] = p_s[i]; a.s_s[i] = s_s[i]; a.m_s[i] = m_s[i]; }
    const int64_t total = (int64_t)B * H * S * a.G;
    if (total == 0) return hipSuccess;
    const bool pow2 = group >= 2 && (group & (group - 1)) == 0;
    if ((D == 64 || D == 128) && pow2) {
        const int64_t pairs = (int64_t)B * H * S * (D / 2);
        if (bits == 8) hipLaunchKernelGGL(quant_v_wave_kernel<8>, dim3(blocks_for(pairs)), dim3(kThreads), 0, st, a);
        else hipLaunchKernelGGL(quant_v_wave_kernel<4>, dim3(blocks_for(pairs)), dim3(kThreads), 0, st, a);
    } else if (bits == 8) {
        hipLaunchKernelGGL(quant_v_kernel<8>, dim3(blocks_for(total)), dim3(kThreads), 0, st, a);
    } else {
        hipLaunchKernelGGL(quant_v_kernel<4>, dim3(blocks_for(total)), dim3(kThreads), 0, st, a);
    }
    return hipGetLastError();
}

hipError_t launch_wht(const void* x, int x_dtype, int64_t x_rs, void* out, int out_dtype, int64_t o_rs,
                      int N, int D, const float* signs, int inverse, int arith, hipStream_t st) {
    WhtParams a{x, x_dtype, x_rs, out, out_dtype, o_rs, N, signs, inverse, arith};
    if (N == 0) return hipSuccess;
    const int64_t rows_per_wave = D >= 64 ? 1 : 64 / D;
    const int64_t waves = (N + rows_per_wave - 1) / rows_per_wave;
    dim3 grid((unsigned)((waves * 64 + kThreads - 1) / kThreads));
    switch (D) {
        case 8: hipLaunchKernelGGL(wht_kernel<8>, grid, dim3(kThreads), 0, st, a); break;
        case 16: hipLaunchKernelGGL(wht_kernel<16>, grid, dim3(kThreads), 0, st, a); break;
        case 32: hipLaunchKernelGGL(wht_kernel<32>, grid, dim3(kThreads), 0, st, a); break;
        case 64: hipLaunchKernelGGL(wht_kernel<64>, grid, dim3(kThreads), 0, st, a); break;
        case 128: hipLaunchKernelGGL(wht_kernel<128>, grid, dim3(kThreads), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_turbo_quant(const void* x, int in_dtype, const int64_t* x_s, int B, int H, int S, int D,
                              uint8_t* msb, const int64_t* msb_s, uint8_t* lsb, const int64_t* lsb_s,
                              void* scale, const int64_t* s_s, hipStream_t st) {
    TurboQParams a{};
    a.x = x; a.in_dtype = in_dtype; a.B = B; a.H = H; a.S = S;
    a.msb = msb; a.lsb = lsb; a.scale = scale;
    for (int i = 0; i < 4; ++i) { a.x_s[i] = x_s[i]; a.msb_s[i] = msb_s[i]; a.lsb_s[i] = lsb_s[i]; a.s_s[i] = s_s[i]; }
    const int64_t total = (int64_t)B * H * S;
    if (total == 0) return hipSuccess;
    dim3 grid(blocks_for(total));
    if (D == 128) hipLaunchKernelGGL(turbo_quant_kernel<128>, grid, dim3(kThreads), 0, st, a);
    else if (D == 64) hipLaunchKernelGGL(turbo_quant_kernel<64>, grid, dim3(kThreads), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_merge(const void* oa, const float* la, const void* ob, const float* lb, int dtype,
                        int64_t rs_a, int64_t rs_b, void* out, int64_t rs_o, float* lse_out, int N, int D,
                        hipStream_t st) {
    MergeParams a{oa, la, ob, lb, dtype, rs_a, rs_b, out, rs_o, lse_out, N, D};
    if ((int64_t)N * D == 0) return hipSuccess;
    hipLaunchKernelGGL(merge_kernel, dim3(blocks_for((int64_t)N * D)), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_tail(const void* q, const int64_t* q_s, const void* k, const int64_t* k_s, const void* v,
                       const int64_t* v_s, int kv_dtype, void* out, const int64_t* o_s, float* lse, int B,
                       int Hq, int Hkv, int T, int D, hipStream_t st) {
    TailParams a{};
    a.q = q; a.k = k; a.v = v; a.kv_dtype = kv_dtype; a.out = out; a.lse = lse;
    for (int i = 0; i < 3; ++i) { a.q_s[i] = q_s[i]; a.o_s[i] = o_s[i]; }
    for (int i = 0; i < 4; ++i) { a.k_s[i] = k_s[i]; a.v_s[i] = v_s[i]; }
    a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.T = T; a.D = D;
    hipLaunchKernelGGL(tail_attn_kernel, dim3(B * Hq), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace fq
