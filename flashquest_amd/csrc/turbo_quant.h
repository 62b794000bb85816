// The TurboQuant K3-V3 quantiser of one token row (kv_quant.py:225-279,
// 366-405), shared by the standalone quantiser (quant.hip) and the cache
// append (cache.hip) so both produce the same bits: WHT butterflies
// h = 1, 2, ..., D/2 with every sum and difference rounded to the input dtype,
// times fp32(1/sqrt(D)) rounded likewise, rms = sqrt(mean(x^2)) (sequential
// fp32 sum) clamped to >= 1e-6 and stored as bf16, then the nearest of the 8
// codebook points to x / rms (ties to the lower index), split into the 1-bit
// MSB plane (bit i of byte j = channel 8j + i) and the 2-bit LSB plane
// (field i of byte j = channel 4j + i).
#pragma once

#include "fq_common.h"

namespace fq {

template <int D>
FQ_DEV void turbo_quant_row(float (&v)[D], int in_dtype, uint8_t* mrow, int64_t m_step, uint8_t* lrow,
                            int64_t l_step, void* scale, int64_t scale_off) {
    constexpr float kCodebook[8] = {-2.1519f, -1.3439f, -0.7560f, -0.2451f, 0.2451f, 0.7560f, 1.3439f, 2.1519f};
#pragma unroll
    for (int hh = 1; hh < D; hh <<= 1) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            if ((i & hh) == 0) {
                const float x = v[i], y = v[i + hh];
                v[i] = round_to(x + y, in_dtype);
                v[i + hh] = round_to(x - y, in_dtype);
            }
        }
    }
    const float inv = 1.0f / sqrtf((float)D);
    float ss = 0.f;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        v[d] = round_to(v[d] * inv, in_dtype);
        ss = __fadd_rn(ss, __fmul_rn(v[d], v[d]));
    }
    const float rms = fmaxf(__fsqrt_rn(__fdiv_rn(ss, (float)D)), 1e-6f);
    store_any(scale, FQ_BF16, scale_off, rms);
    uint32_t mbyte = 0, lbyte = 0;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const float x = __fdiv_rn(v[d], rms);
        int best = 0;
        float bd = fabsf(x - kCodebook[0]);
#pragma unroll
        for (int k = 1; k < 8; ++k) {
            const float dd = fabsf(x - kCodebook[k]);
            if (dd < bd) { bd = dd; best = k; }
        }
        mbyte |= (uint32_t)((best >> 2) & 1) << (d % 8);
        lbyte |= (uint32_t)(best & 3) << (2 * (d % 4));
        if (d % 4 == 3) { lrow[(d / 4) * l_step] = (uint8_t)lbyte; lbyte = 0; }
        if (d % 8 == 7) { mrow[(d / 8) * m_step] = (uint8_t)mbyte; mbyte = 0; }
    }
}

}  // namespace fq
