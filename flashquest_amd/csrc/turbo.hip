// Split-K sparse GQA decode attention over the TurboQuant K3-V3 cache (gfx950).
//
// Reference semantics: src/flashquest/kernel/sparse_turbo_fwd.py:110-251 and
// its wrapper 254-346: Q is rotated by the normalised WHT, each selected
// page's 3-bit indices idx = (msb << 2) | lsb (msb bit i of byte j is channel
// 8j+i, lsb field i of byte j is channel 4j+i; kv_quant.py:253-279) map to the
// 8-level codebook (kv_quant.py:225-229) times the per-token scale, the same
// online softmax as the INT4 kernel runs, and O is rotated back (O = WHT(O_rot)).
// Here the rotations are fused: the prologue rotates Q in LDS, the epilogue
// rotates O before the store.
#include "attn_common.h"

namespace fq {
namespace {

struct TurboParams {
    fq_turbo_cache c;
    QueryArgs q;
    Workspace ws;
    int pps, splits;
};

// codebook value of a 3-bit index: sign from bit 2, magnitude from bits 0-1
// ([-2.1519, -1.3439, -0.7560, -0.2451, 0.2451, 0.7560, 1.3439, 2.1519]).
FQ_DEV float turbo_cb(uint32_t idx) {
    const uint32_t pos = idx & 4u;
    const uint32_t t = pos ? (idx & 3u) : ((idx & 3u) ^ 3u);
    const float m01 = (t & 1u) ? 0.7560f : 0.2451f;
    const float m23 = (t & 1u) ? 2.1519f : 1.3439f;
    const float mag = (t & 2u) ? m23 : m01;
    return pos ? mag : -mag;
}

FQ_DEV void turbo_decode8(uint32_t msb, uint32_t lsb16, float (&out)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = turbo_cb((((msb >> j) & 1u) << 2) | ((lsb16 >> (2 * j)) & 3u));
}

template <int D, int NREP>
__global__ __launch_bounds__(kThreads) void attn_turbo_kernel(TurboParams a) {
    constexpr int NCC = D / 8;
    constexpr int NROW = 64 / NCC;
    constexpr int NW = kThreads / 64;
    __shared__ SplitLds<D, NREP> s_split;
    __shared__ float s_qraw[NREP][D];

    const fq_turbo_cache& c = a.c;
    const QueryArgs& q = a.q;
    const int g = blockIdx.y, split = blockIdx.x;
    const int h = g % c.H_kv, b = (g / c.H_kv) % c.B, l = g / (c.H_kv * c.B);
    const int lane = lane_id(), w = wave_id();
    const int cc = lane % NCC, row = lane / NCC;

    const int n_sel = a.ws.n_sel[g];
    const int e0 = split * a.pps;
    const int e1 = min(n_sel, e0 + a.pps);
    const bool active = e0 < n_sel || a.splits == 1;

    float m[NREP], lsum[NREP], acc[NREP][8];
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
        m[r] = -INFINITY; lsum[r] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[r][j] = 0.f;
    }
    if (active) {
        for (int i = threadIdx.x; i < NREP * D; i += kThreads) {
            const int r = i / D, d = i % D;
            s_qraw[r][d] = load_any(q.q, q.q_dtype, l * q.q_s[0] + b * q.q_s[1] + (h * NREP + r) * q.q_s[2] + d * q.q_s[3]);
        }
    }
    __syncthreads();
    if (active) {
        // q_rot = WHT(q) / sqrt(D), pre-scaled by sm_scale * log2(e)
        float qv[NREP][8];
        const float inv = q.qk_scale / sqrtf((float)D);
#pragma unroll
        for (int r = 0; r < NREP; ++r)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float v = 0.f;
                for (int k = 0; k < D; ++k) v = fmaf(hadamard_sign(cc * 8 + j, k), s_qraw[r][k], v);
                qv[r][j] = v * inv;
            }
        const int64_t bl = (int64_t)l;
        const uint8_t* kmsb = c.k_msb + bl * c.kmsb_strides[0] + b * c.kmsb_strides[1] + h * c.kmsb_strides[2] + cc;
        const uint8_t* klsb = c.k_lsb + bl * c.klsb_strides[0] + b * c.klsb_strides[1] + h * c.klsb_strides[2] + 2 * cc;
        const uint8_t* vmsb = c.v_msb + bl * c.vmsb_strides[0] + b * c.vmsb_strides[1] + h * c.vmsb_strides[2] + cc;
        const uint8_t* vlsb = c.v_lsb + bl * c.vlsb_strides[0] + b * c.vlsb_strides[1] + h * c.vlsb_strides[2] + 2 * cc;
        const uint16_t* kst = (const uint16_t*)c.k_scale + bl * c.kst_strides[0] + b * c.kst_strides[1] + h * c.kst_strides[2];
        const uint16_t* vst = (const uint16_t*)c.v_scale + bl * c.vst_strides[0] + b * c.vst_strides[1] + h * c.vst_strides[2];
        const int* entries = a.ws.entries + (int64_t)g * c.P;

        for (int e = e0 + w; e < e1; e += NW) {
            const int ent = entries[e];
            const int p = ent & 0xFFFF;
            const int qm = ent >> 16;
            const int tok0 = p * c.page_size;
            for (int t0 = 0; t0 < c.page_size; t0 += 4 * NROW) {
                uint32_t km[4], kl[4], vmv[4], vl[4];
                float ks[4], vs[4];
                bool valid[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = t0 + row + NROW * i;
                    const int64_t tok = tok0 + t;
                    valid[i] = t < c.page_size && tok < c.S;
                    km[i] = valid[i] ? kmsb[tok * c.kmsb_strides[3]] : 0u;
                    kl[i] = valid[i] ? *(const uint16_t*)(klsb + tok * c.klsb_strides[3]) : 0u;
                    vmv[i] = valid[i] ? vmsb[tok * c.vmsb_strides[3]] : 0u;
                    vl[i] = valid[i] ? *(const uint16_t*)(vlsb + tok * c.vlsb_strides[3]) : 0u;
                    ks[i] = valid[i] ? bf16_bits_to_f(kst[tok * c.kst_strides[3]]) : 0.f;
                    vs[i] = valid[i] ? bf16_bits_to_f(vst[tok * c.vst_strides[3]]) : 0.f;
                }
                float s[4][NREP];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float kv[8];
                    turbo_decode8(km[i], kl[i], kv);
#pragma unroll
                    for (int r = 0; r < NREP; ++r) {
                        float d = 0.f;
#pragma unroll
                        for (int j = 0; j < 8; ++j) d = fmaf(qv[r][j], kv[j], d);
                        d = row_sum<NCC>(d) * ks[i];
                        s[i][r] = (valid[i] && ((qm >> r) & 1)) ? d : -INFINITY;
                    }
                }
                float vv[4][8];
#pragma unroll
                for (int i = 0; i < 4; ++i) turbo_decode8(vmv[i], vl[i], vv[i]);
#pragma unroll
                for (int r = 0; r < NREP; ++r) {
                    const float mx = fmaxf(fmaxf(s[0][r], s[1][r]), fmaxf(s[2][r], s[3][r]));
                    const float mnew = fmaxf(m[r], mx);
                    if (mnew == -INFINITY) continue;
                    const float alpha = m[r] == -INFINITY ? 0.f : exp2_fast(m[r] - mnew);
                    float psum = 0.f;
                    lsum[r] *= alpha;
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc[r][j] *= alpha;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float pi = s[i][r] == -INFINITY ? 0.f : exp2_fast(s[i][r] - mnew);
                        psum += pi;
                        const float pv = pi * vs[i];
#pragma unroll
                        for (int j = 0; j < 8; ++j) acc[r][j] = fmaf(pv, vv[i][j], acc[r][j]);
                    }
                    lsum[r] += psum;
                    m[r] = mnew;
                }
            }
        }
    }
    finish_split<D, NREP, true>(s_split, m, lsum, acc, active, q, a.ws, g, l, b, h, split, a.splits);
}

template <int D>
hipError_t launch_turbo_nrep(const TurboParams& a, dim3 grid, hipStream_t st) {
    switch (a.q.nrep) {
#define FQ_CASE(N)                                                                                     \
    case N:                                                                                            \
        timer_before_launch(st);                                                                      \
        hipLaunchKernelGGL((attn_turbo_kernel<D, N>), grid, dim3(kThreads), 0, st, a);                \
        timer_after_launch(st);                                                                       \
        if (a.splits > 1)                                                                              \
            hipLaunchKernelGGL((merge_splits_kernel<D, N, true>), dim3(grid.y), dim3(kThreads), 0, st, \
                               a.q, a.ws, a.c.H_kv, a.c.B, a.pps, a.splits, TailArgs{});                                   \
        break;
        FQ_CASE(1) FQ_CASE(2) FQ_CASE(3) FQ_CASE(4) FQ_CASE(5) FQ_CASE(6) FQ_CASE(7) FQ_CASE(8)
#undef FQ_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_turbo(const fq_turbo_cache& c, const QueryArgs& q, const Workspace& ws,
                             const AttnLaunch& al, hipStream_t st) {
    TurboParams a{};
    a.c = c; a.q = q; a.ws = ws; a.pps = al.pages_per_split; a.splits = al.splits;
    dim3 grid(al.splits, c.L * c.B * c.H_kv);
    if (c.D == 128) return launch_turbo_nrep<128>(a, grid, st);
    if (c.D == 64) return launch_turbo_nrep<64>(a, grid, st);
    return hipErrorInvalidValue;
}

}  // namespace fq
