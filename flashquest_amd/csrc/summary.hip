// Quest page scores from the exact page summary of the dequantised INT8 keys
// (gfx950): the scoring of the reference's DuoAttention dispatch
// (src/flashquest/duo/fused_dispatch.py:64-67), i.e.
//   K_bf16 = bf16(code * fp32(K_scale[p]) + fp32(K_mn[p]))     dequantize_k, kv_quant.py:64-75
//   page_min / page_max = channel min / max of K_bf16 over the   compute_page_summary,
//     page's tokens (a partial last page: its valid tokens)       eager/page_summary.py:7-39
//   score[b, h_q, p] = sum_d max(q_d * page_max_d, q_d * page_min_d)   page_scores,
//     in fp32, query head h_q reading KV head h_q / n_rep           eager/criticality.py:7-31
//
// The dequantisation is increasing in the code (K_scale > 0 after the
// quantiser's clamp), and so are the fp32 and bf16 roundings, so the page's
// minimum / maximum key is the dequantised minimum / maximum code: one pass
// over the page's codes finds those, and only 2 * D values are dequantised.
// code * scale is exact in fp32 (8-bit code times an 8- or 11-bit significand),
// so fmaf(code, scale, mn) rounds exactly like the reference's multiply then add.
//
// Layout: one 256-thread workgroup per (page, batch x KV head).  Thread t reads
// dword t % (D/4) (channels 4j .. 4j+3) of the page's tokens t / (D/4),
// + 256/(D/4), ...; the partial extrema meet in LDS.  The score's fp32 order
// (restated by the CPU oracle): lane j < D/4 sums its 4 channels' terms left to
// right, then the lanes combine by a butterfly v += v[lane ^ o] for o = D/8,
// D/16, ..., 1.
#include "fq_common.h"

namespace fq {

namespace {

template <typename MT, int D>
__global__ __launch_bounds__(kThreads) void page_summary_scores_kernel(SummaryArgs a) {
    constexpr int NJ = D / 4;                 // dwords per token row
    constexpr int NR = kThreads / NJ;         // token rows per pass
    __shared__ int s_lo[NR][D], s_hi[NR][D];
    __shared__ float s_flo[D], s_fhi[D];
    const int p = blockIdx.x, bh = blockIdx.y;
    const int b = bh / a.Hkv, h = bh % a.Hkv;
    const int tid = threadIdx.x, j = tid % NJ, rg = tid / NJ;

    int lo[4] = {255, 255, 255, 255}, hi[4] = {0, 0, 0, 0};
    const uint8_t* base = a.codes + b * a.c_s[0] + h * a.c_s[1] + 4 * j;
    const int t0 = p * a.page;
    const int t1 = min(t0 + a.page, a.S);
    for (int t = t0 + rg; t < t1; t += NR) {
        const uint32_t w = *(const uint32_t*)(base + (int64_t)t * a.c_s[2]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int v = (w >> (8 * i)) & 0xFF;
            lo[i] = min(lo[i], v);
            hi[i] = max(hi[i], v);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s_lo[rg][4 * j + i] = lo[i];
        s_hi[rg][4 * j + i] = hi[i];
    }
    __syncthreads();
    if (tid < D) {
        int cl = 255, ch = 0;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            cl = min(cl, s_lo[r][tid]);
            ch = max(ch, s_hi[r][tid]);
        }
        const uint16_t* ksp = (const uint16_t*)a.ks + b * a.ks_s[0] + h * a.ks_s[1] + p * a.ks_s[2] + tid * a.ks_s[3];
        const uint16_t* kmp = (const uint16_t*)a.km + b * a.km_s[0] + h * a.km_s[1] + p * a.km_s[2] + tid * a.km_s[3];
        const float sc = half_to_f<MT>(*ksp), mn = half_to_f<MT>(*kmp);
        const uint16_t blo = f_to_bf16_bits(fmaf((float)cl, sc, mn));
        const uint16_t bhi = f_to_bf16_bits(fmaf((float)ch, sc, mn));
        s_flo[tid] = bf16_bits_to_f(blo);
        s_fhi[tid] = bf16_bits_to_f(bhi);
        if (a.pmin) {
            const int64_t o = b * a.pm_s[0] + h * a.pm_s[1] + p * a.pm_s[2] + tid * a.pm_s[3];
            a.pmin[o] = blo;
            a.pmax[o] = bhi;
        }
    }
    __syncthreads();
    if (tid >= 64) return;
    const int nrep = a.Hq / a.Hkv;
    const int L = tid;
    for (int r = 0; r < nrep; ++r) {
        const int hq = h * nrep + r;
        float acc = 0.f;
        if (L < NJ) {
            const int64_t qo = b * a.q_s[0] + hq * a.q_s[1];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 4 * L + i;
                const float qd = load_any(a.q, a.q_dtype, qo + d * a.q_s[3]);
                const float term = fmaxf(qd * s_fhi[d], qd * s_flo[d]);
                acc = i == 0 ? term : acc + term;
            }
        }
#pragma unroll
        for (int o = NJ / 2; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
        if (L == 0) a.scores[b * a.sc_s[0] + hq * a.sc_s[1] + p * a.sc_s[3]] = acc;
    }
}

// compute_page_summary (eager/page_summary.py:7-39) over any float K: thread
// d of workgroup (page, b x h) takes channel d's minimum and maximum over the
// page's valid tokens, NaN propagating as in torch's min / max; the results
// are elements of K, stored in K's dtype.
__global__ __launch_bounds__(1024) void page_minmax_kernel(PageMinMaxArgs a) {
    const int p = blockIdx.x, bh = blockIdx.y, d = threadIdx.x;
    if (d >= a.D) return;
    const int b = bh / a.H, h = bh % a.H;
    const int64_t base = b * a.k_s[0] + h * a.k_s[1] + d * a.k_s[3];
    const int t0 = p * a.page, t1 = min(t0 + a.page, a.S);
    float lo = INFINITY, hi = -INFINITY;
    for (int t = t0; t < t1; ++t) {
        const float x = load_any(a.k, a.k_dtype, base + (int64_t)t * a.k_s[2]);
        lo = (x < lo || x != x) ? (lo != lo ? lo : x) : lo;
        hi = (x > hi || x != x) ? (hi != hi ? hi : x) : hi;
    }
    const int64_t o = b * a.pm_s[0] + h * a.pm_s[1] + p * a.pm_s[2] + d * a.pm_s[3];
    store_any(a.pmin, a.k_dtype, o, lo);
    store_any(a.pmax, a.k_dtype, o, hi);
}

// Quest scores from page bounds, one wave per (page, b x KV head), for every
// query row of the group (n_rep heads x S_q positions): the bounds go to
// LDS as fp32 (lo / hi, or from the INT8 metadata lo = K_mn, hi = K_mn +
// levels * K_scale in fp32 -- criticality.py:66-67), then each row's
// sum_d max(q_d * hi_d, q_d * lo_d) in the fixed order of the summary kernel
// above (4 channels per lane left to right, then the butterfly).
template <int D>
__global__ __launch_bounds__(64) void quest_scores_kernel(QuestScoreArgs a) {
    constexpr int NJ = D / 4;
    __shared__ float s_lo[D], s_hi[D];
    const int p = blockIdx.x, bh = blockIdx.y, L = threadIdx.x;
    const int b = bh / a.Hkv, h = bh % a.Hkv;
    for (int d = L; d < D; d += 64) {
        const int64_t ol = b * a.lo_s[0] + h * a.lo_s[1] + p * a.lo_s[2] + d * a.lo_s[3];
        const int64_t oh = b * a.hi_s[0] + h * a.hi_s[1] + p * a.hi_s[2] + d * a.hi_s[3];
        const float lo = load_any(a.lo, a.b_dtype, ol);
        const float x = load_any(a.hi, a.b_dtype, oh);
        s_lo[d] = lo;
        s_hi[d] = a.from_meta ? __fadd_rn(lo, __fmul_rn(a.levels, x)) : x;
    }
    __syncthreads();
    const int nrep = a.Hq / a.Hkv;
    for (int r = 0; r < nrep * a.Sq; ++r) {
        const int hq = h * nrep + r / a.Sq, sq = r % a.Sq;
        float acc = 0.f;
        if (L < NJ) {
            const int64_t qo = b * a.q_s[0] + hq * a.q_s[1] + sq * a.q_s[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 4 * L + i;
                const float qd = load_any(a.q, a.q_dtype, qo + d * a.q_s[3]);
                const float term = fmaxf(__fmul_rn(qd, s_hi[d]), __fmul_rn(qd, s_lo[d]));
                acc = i == 0 ? term : acc + term;
            }
        }
#pragma unroll
        for (int o = NJ / 2; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
        if (L == 0) a.scores[b * a.sc_s[0] + hq * a.sc_s[1] + sq * a.sc_s[2] + p * a.sc_s[3]] = acc;
    }
}

}  // namespace

hipError_t launch_page_summary_scores(const SummaryArgs& a, hipStream_t st) {
    dim3 grid(a.P, a.B * a.Hkv);
#define FQ_L(MT, D_) hipLaunchKernelGGL((page_summary_scores_kernel<MT, D_>), grid, dim3(kThreads), 0, st, a)
    if (a.meta_dtype == FQ_BF16) {
        if (a.D == 128) FQ_L(bf16, 128); else FQ_L(bf16, 64);
    } else {
        if (a.D == 128) FQ_L(f16, 128); else FQ_L(f16, 64);
    }
#undef FQ_L
    return hipGetLastError();
}

hipError_t launch_page_minmax(const PageMinMaxArgs& a, hipStream_t st) {
    const int threads = (a.D + 63) / 64 * 64;
    hipLaunchKernelGGL(page_minmax_kernel, dim3(a.P, a.B * a.H), dim3(threads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_quest_scores(const QuestScoreArgs& a, hipStream_t st) {
    dim3 grid(a.P, a.B * a.Hkv);
    if (a.D == 128) hipLaunchKernelGGL((quest_scores_kernel<128>), grid, dim3(64), 0, st, a);
    else hipLaunchKernelGGL((quest_scores_kernel<64>), grid, dim3(64), 0, st, a);
    return hipGetLastError();
}

}  // namespace fq
