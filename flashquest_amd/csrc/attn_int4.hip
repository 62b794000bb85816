// Split-K sparse GQA decode attention over packed INT4 K/V pages (gfx950).
//
// Reference semantics: src/flashquest/kernel/sparse_int4_fwd.py:23-157 (per
// page: k = code * K_scale[p] + K_mn[p], v = code * V_scale[t] + V_mn[t],
// base-2 online softmax, O = acc / l, lse = (m + log2 l) * ln2, an empty
// selection gives O = 0 and lse = -inf; tokens >= S are masked).
//
// Design: one workgroup per (KV group, split of the group's union page list);
// each of its 4 waves takes every 4th page, so a page's K/V bytes are read
// once for all query heads of the group.  Inside a wave, NCC = D/8 lanes share
// one token (8 channels each, one dword of packed codes) and NROW = 64/NCC
// token rows run side by side, each row with its own online-softmax state.
// Row states merge with cross-lane shuffles, waves through LDS, and splits
// through a workspace: the last workgroup of a group to arrive merges the
// split partials (the same rule as _merge_two_attentions,
// llama_persistent_patch.py:50-61) and writes O and lse.
#include <type_traits>

#include "attn_common.h"

namespace fq {
namespace {

struct AttnParams {
    Int4Cache c;
    QueryArgs q;
    Workspace ws;
    int pps;      // pages (union entries) per split
    int splits;   // gridDim.x
};

// BITS = 8: the INT8 cache of flash_attn_sparse_fwd (sparse_fwd.py:23-157),
// one code byte per channel, the same math with codes 0..255.
template <int D, typename MT, int GV, int NREP, int BITS>
__global__ __launch_bounds__(kThreads) void attn_int4_kernel(AttnParams a) {
    using CodeWord = typename std::conditional<BITS == 8, uint2, uint32_t>::type;     // 8 codes of a lane
    auto code_of = [](const CodeWord& wv, int j) -> float {
        if constexpr (BITS == 8) return (float)(((j < 4 ? wv.x : wv.y) >> (8 * (j & 3))) & 255u);
        else return (float)((wv >> (4 * j)) & 15u);
    };
    constexpr int NCC = D / 8;
    constexpr int NROW = 64 / NCC;
    constexpr int NW = kThreads / 64;
    __shared__ SplitLds<D, NREP> s_split;

    const Int4Cache& c = a.c;
    const QueryArgs& q = a.q;
    const int g = blockIdx.y, split = blockIdx.x;
    const int h = g % c.Hkv, b = (g / c.Hkv) % c.B, l = g / (c.Hkv * c.B);
    const int lane = lane_id(), w = wave_id();
    const int cc = lane % NCC, row = lane / NCC;

    const int n_sel = a.ws.n_sel[g];
    const int e0 = split * a.pps;
    const int e1 = min(n_sel, e0 + a.pps);
    const bool active = e0 < n_sel || a.splits == 1;
    const bool has_tokens = c.S > 0;

    float m[NREP], lsum[NREP], bias[NREP], acc[NREP][8];
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
        m[r] = -INFINITY; lsum[r] = 0.f; bias[r] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[r][j] = 0.f;
    }

    if (active) {
        float qv[NREP][8];
#pragma unroll
        for (int r = 0; r < NREP; ++r)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                qv[r][j] = load_any(q.q, q.q_dtype,
                                    l * q.q_s[0] + b * q.q_s[1] + (h * NREP + r) * q.q_s[2] +
                                        (cc * 8 + j) * q.q_s[3]) * q.qk_scale;

        const uint8_t* kb = c.kp + l * c.kp_s[0] + b * c.kp_s[1] + h * c.kp_s[2] + cc * BITS;
        const uint8_t* vb = c.vp + l * c.vp_s[0] + b * c.vp_s[1] + h * c.vp_s[2] + cc * BITS;
        const MT* ksc = (const MT*)c.ksc + l * c.ksc_s[0] + b * c.ksc_s[1] + h * c.ksc_s[2] + cc * 8;
        const MT* kmn = (const MT*)c.kmn + l * c.kmn_s[0] + b * c.kmn_s[1] + h * c.kmn_s[2] + cc * 8;
        const int gi = GV == 1 ? 0 : (cc * 8) / (D / GV);
        const uint16_t* vsc = (const uint16_t*)c.vsc + l * c.vsc_s[0] + b * c.vsc_s[1] + h * c.vsc_s[2] + gi;
        const uint16_t* vmn = (const uint16_t*)c.vmn + l * c.vmn_s[0] + b * c.vmn_s[1] + h * c.vmn_s[2] + gi;
        const int* entries = a.ws.entries + (int64_t)g * c.P;

        for (int e = e0 + w; has_tokens && e < e1; e += NW) {
            const int ent = entries[e];
            const int p = ent & 0xFFFF;
            const int qm = ent >> 16;
            const uint4 sv = *(const uint4*)(ksc + p * c.ksc_s[3]);
            const uint4 mv = *(const uint4*)(kmn + p * c.kmn_s[3]);
            const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
            const uint32_t mw[4] = {mv.x, mv.y, mv.z, mv.w};
            float sf[8], mf[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sf[2 * j] = half_to_f<MT>(sw[j]);
                sf[2 * j + 1] = half_to_f<MT>(sw[j] >> 16);
                mf[2 * j] = half_to_f<MT>(mw[j]);
                mf[2 * j + 1] = half_to_f<MT>(mw[j] >> 16);
            }
            // q.k = sum_j (q_j s_j) code_j + sum_j q_j mn_j
            float A[NREP][8], Cp[NREP];
#pragma unroll
            for (int r = 0; r < NREP; ++r) {
                float cpart = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    A[r][j] = qv[r][j] * sf[j];
                    cpart = fmaf(qv[r][j], mf[j], cpart);
                }
                Cp[r] = cpart;
            }
            const int tok0 = p * c.page;
            for (int t0 = 0; t0 < c.page; t0 += 16 * NROW) {
                // Issue every load of this block of 16 token rows first: rows past the
                // page or the view are clamped to row S-1 (always in bounds) and masked.
                CodeWord kw[16], vw[16];
                uint16_t vsr[16], vmr[16];
                int vmask = 0;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int t = t0 + row + NROW * i;
                    const int tok = tok0 + t;
                    const bool ok = t < c.page && tok < c.S;
                    vmask |= ok << i;
                    const int64_t tc = ok ? tok : c.S - 1;
                    kw[i] = *(const CodeWord*)(kb + tc * c.kp_s[3]);
                    vw[i] = *(const CodeWord*)(vb + tc * c.vp_s[3]);
                    vsr[i] = vsc[tc * c.vsc_s[3]];
                    vmr[i] = vmn[tc * c.vmn_s[3]];
                }
#pragma unroll
                for (int i0 = 0; i0 < 16; i0 += 4) {
                    float s[4][NREP];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float code[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j) code[j] = code_of(kw[i0 + i], j);
#pragma unroll
                        for (int r = 0; r < NREP; ++r) {
                            float d = Cp[r];
#pragma unroll
                            for (int j = 0; j < 8; ++j) d = fmaf(A[r][j], code[j], d);
                            d = row_sum<NCC>(d);
                            s[i][r] = (((vmask >> (i0 + i)) & 1) && ((qm >> r) & 1)) ? d : -INFINITY;
                        }
                    }
                    float vcode[4][8], vs[4], vm[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        vs[i] = half_to_f<MT>(vsr[i0 + i]);
                        vm[i] = half_to_f<MT>(vmr[i0 + i]);
#pragma unroll
                        for (int j = 0; j < 8; ++j) vcode[i][j] = code_of(vw[i0 + i], j);
                    }
#pragma unroll
                    for (int r = 0; r < NREP; ++r) {
                        const float mx = fmaxf(fmaxf(s[0][r], s[1][r]), fmaxf(s[2][r], s[3][r]));
                        const float mnew = fmaxf(m[r], mx);
                        if (mnew == -INFINITY) continue;
                        const float alpha = m[r] == -INFINITY ? 0.f : exp2_fast(m[r] - mnew);
                        float psum = 0.f;
                        lsum[r] *= alpha;
                        bias[r] *= alpha;
#pragma unroll
                        for (int j = 0; j < 8; ++j) acc[r][j] *= alpha;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float pi = s[i][r] == -INFINITY ? 0.f : exp2_fast(s[i][r] - mnew);
                            psum += pi;
                            const float pv = pi * vs[i];
                            bias[r] = fmaf(pi, vm[i], bias[r]);
#pragma unroll
                            for (int j = 0; j < 8; ++j) acc[r][j] = fmaf(pv, vcode[i][j], acc[r][j]);
                        }
                        lsum[r] += psum;
                        m[r] = mnew;
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < NREP; ++r)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[r][j] += bias[r];
    }
    finish_split<D, NREP, false>(s_split, m, lsum, acc, active, q, a.ws, g, l, b, h, split, a.splits);
}

template <int D, typename MT, int GV, int BITS>
hipError_t launch_nrep(const AttnParams& a, dim3 grid, hipStream_t st) {
    switch (a.q.nrep) {
#define FQ_CASE(N)                                                                                      \
    case N:                                                                                             \
        timer_before_launch(st);                                                                       \
        hipLaunchKernelGGL((attn_int4_kernel<D, MT, GV, N, BITS>), grid, dim3(kThreads), 0, st, a);    \
        timer_after_launch(st);                                                                        \
        if (a.splits > 1)                                                                               \
            hipLaunchKernelGGL((merge_splits_kernel<D, N, false>), dim3(grid.y), dim3(kThreads), 0, st, \
                               a.q, a.ws, a.c.Hkv, a.c.B, a.pps, a.splits, TailArgs{});                                       \
        break;
        FQ_CASE(1) FQ_CASE(2) FQ_CASE(3) FQ_CASE(4) FQ_CASE(5) FQ_CASE(6) FQ_CASE(7) FQ_CASE(8)
#undef FQ_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int D, typename MT>
hipError_t launch_gv(const AttnParams& a, dim3 grid, hipStream_t st) {
    if (a.c.bits == 8) return a.c.G == 1 ? launch_nrep<D, MT, 1, 8>(a, grid, st) : hipErrorInvalidValue;
    if (a.c.G == 1) return launch_nrep<D, MT, 1, 4>(a, grid, st);
    if (a.c.G == D / 32) return launch_nrep<D, MT, D / 32, 4>(a, grid, st);
    return hipErrorInvalidValue;
}

}  // namespace

bool attn_selects_in_kernel(const Int4Cache& c, const QueryArgs& q, const AttnLaunch& al) {
    return c.bits == 8 ? int8_select_in_kernel(c, q, al) : mfma_select_in_kernel(c, q, al);
}

hipError_t launch_attn_int4(const Int4Cache& c, const QueryArgs& q, const Workspace& ws,
                            const AttnLaunch& al, hipStream_t st, const SelectArgs* sel, const TailArgs* tail) {
    if (c.bits == 8 && int8_mfma_supported(c, q, al)) return launch_attn_int8_mfma(c, q, ws, al, st, sel, tail);
    if (mfma_supported(c, q, al)) return launch_attn_int4_mfma(c, q, ws, al, st, sel, tail);
    if ((sel && sel->enabled) || (tail && tail->len > 0)) return hipErrorInvalidValue;
    AttnParams a{};
    a.c = c; a.q = q; a.ws = ws; a.pps = al.pages_per_split; a.splits = al.splits;
    dim3 grid(al.splits, c.L * c.B * c.Hkv);
    if (c.D == 128) {
        return c.meta_dtype == FQ_BF16 ? launch_gv<128, bf16>(a, grid, st) : launch_gv<128, f16>(a, grid, st);
    }
    if (c.D == 64) {
        return c.meta_dtype == FQ_BF16 ? launch_gv<64, bf16>(a, grid, st) : launch_gv<64, f16>(a, grid, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace fq
