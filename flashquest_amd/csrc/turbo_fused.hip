// Sparse GQA decode attention over the TurboQuant K3-V3 cache, one workgroup
// of 8 waves per KV group (gfx950).  Semantics of flash_attn_sparse_turbo_fwd
// (src/flashquest/kernel/sparse_turbo_fwd.py:110-251, wrapper 254-346): Q is
// rotated by the normalised WHT, a token's K / V channel value is
// codebook[(msb << 2) | lsb] * scale[token] (msb bit i of byte j is channel
// 8j + i, lsb field i of byte j is channel 4j + i; kv_quant.py:225-279), base-2
// online softmax, O rotated back.
//
// FUSED: the workgroup also scores the group's pages from the un-rotated K's
// page scale/min (K_scale_raw / K_mn_raw, bf16; criticality.py:128-163) and
// selects them, like the INT4 fused decode (one launch per decode step).
// Otherwise the pages come from the workspace lists and splits of a group
// meet in merge_splits_kernel.
//
// Layout: lane = (c16 = lane & 7: channels 16 c16 .. +15, slot = lane >> 3:
// tokens 8 slot .. +7 of the page).  Per token a lane loads 2 bytes of the MSB
// plane and 4 bytes of the LSB plane (its 16 channels).  Codes decode two
// channels at a time through a 64-entry LDS table: the index is
// (lsb field d0 | lsb field d1 << 2 | msb d0 << 4 | msb d1 << 5) and the entry
// the two fp32 codebook values (one 8-byte LDS read per channel pair).  q.k sums the lane's 16 channels and reduces over the 8 lanes
// of a slot; p.v accumulates the lane's 16 channels over its tokens and reduces
// over the slots once, at the end.
#include "attn_common.h"
#include "fused_common.h"

namespace fq {
namespace {

__device__ __constant__ float kTurboCodebookF[8] = {-2.1519f, -1.3439f, -0.7560f, -0.2451f,
                                                    0.2451f, 0.7560f, 1.3439f, 2.1519f};

struct TurboFusedParams {
    fq_turbo_cache c;
    Int4Cache raw;          // FUSED: ksc / kmn = K_scale_raw / K_mn_raw (bf16), P, D
    QueryArgs q;
    Workspace ws;
    int splits;
    SelectArgs sel;
};

// One page step of a lane: 8 tokens' MSB (16 bits) and LSB (32 bits) words of
// K and V for its 16 channels, and the K and V scale of one token of its slot
// (token 8 slot + c16; the slot's 8 lanes exchange them by shuffles), so
// every scale load is exactly in range on a partial last page.
struct TurboPage {
    uint32_t km[8], kl[8], vm[8], vl[8];
    uint32_t ks, vs;
};

struct TurboRsrc {
    __amdgpu_buffer_rsrc_t km, kl, ks, vm, vl, vs;
    int km_t, kl_t, vm_t, vl_t, ks_t, vs_t;     // token strides in bytes
};

FQ_DEV void load_turbo_page(TurboPage& b, const TurboRsrc& r, int tok0, int c16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int t = tok0 + i;
        b.km[i] = ld16(r.km, t * r.km_t + 2 * c16);
        b.kl[i] = ld32(r.kl, t * r.kl_t + 4 * c16);
    }
    b.ks = ld16(r.ks, (tok0 + c16) * r.ks_t);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int t = tok0 + i;
        b.vm[i] = ld16(r.vm, t * r.vm_t + 2 * c16);
        b.vl[i] = ld32(r.vl, t * r.vl_t + 4 * c16);
    }
    b.vs = ld16(r.vs, (tok0 + c16) * r.vs_t);
}

FQ_DEV uint32_t lut_index(uint32_t lsb, uint32_t msb, int jp) {
    return __builtin_amdgcn_ubfe(lsb, 4 * jp, 4) | (__builtin_amdgcn_ubfe(msb, 2 * jp, 2) << 4);
}
// scale of token i of the lane's slot, held by lane (slot base + i)
FQ_DEV float scale_of(uint32_t s, int lane, int i) {
    return bf16_bits_to_f(__shfl(s, (lane & ~7) | i, 64) & 0xFFFFu);
}

template <int NREP, bool FUSED>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_turbo_fused_kernel(TurboFusedParams a) {
    constexpr int D = 128, NW = 8, NT = 512;
    __shared__ SplitLds<D, NREP, NW> s_split;
    __shared__ int s_ent[kMaxWgPages];
    __shared__ float2 s_lut[64];
    __shared__ float s_qraw[NREP][D];
    __shared__ float s_qrot[NREP][D];

    const fq_turbo_cache& c = a.c;
    const QueryArgs& q = a.q;
    const int g = blockIdx.y, split = blockIdx.x;
    const int h = g % c.H_kv, b = (g / c.H_kv) % c.B, l = g / (c.H_kv * c.B);
    const int tid = threadIdx.x, L = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
    const int c16 = L & 7, slot = L >> 3;
    const int S = c.S;

    // q (raw basis): element tid of the group's NREP heads
    const int64_t qb = l * q.q_s[0] + b * q.q_s[1] + (int64_t)h * NREP * q.q_s[2];
    const int qi = min(tid, NREP * D - 1);
    const float qv_raw = load_any(q.q, q.q_dtype, qb + (qi >> 7) * q.q_s[2] + (qi & 127) * q.q_s[3]);
    float ret_l = 0.f;
    ScoreRegs<NT> sr;
    if constexpr (FUSED) {
        ret_l = a.sel.retention[h * NREP + min(L, NREP - 1)];
        score_group_load<bf16, NT>(sr, a.raw, tid, l, b, h);
    }
    if (tid < 64) {
        const float c0 = kTurboCodebookF[((tid >> 2) & 4) | (tid & 3)];
        const float c1 = kTurboCodebookF[((tid >> 3) & 4) | ((tid >> 2) & 3)];
        s_lut[tid] = make_float2(c0, c1);
    }
    if (tid < NREP * D) s_qraw[qi >> 7][qi & 127] = qv_raw;
    __syncthreads();
    // q_rot = WHT(q) / sqrt(D) (Sylvester order), pre-scaled by sm_scale * log2(e)
    if (tid < NREP * D) {
        const int r = tid >> 7, d = tid & 127;
        float v = 0.f;
        for (int k = 0; k < D; ++k) v = fmaf(hadamard_sign(d, k), s_qraw[r][k], v);
        s_qrot[r][d] = v * (q.qk_scale / sqrtf((float)D));
    }

    // page buffers and the loads of one page (tokens 8 slot .. +7)
    TurboRsrc rs;
    {
        const int64_t bl = l;
        const uint8_t* km = c.k_msb + bl * c.kmsb_strides[0] + b * c.kmsb_strides[1] + h * c.kmsb_strides[2];
        const uint8_t* kl = c.k_lsb + bl * c.klsb_strides[0] + b * c.klsb_strides[1] + h * c.klsb_strides[2];
        const uint8_t* vm = c.v_msb + bl * c.vmsb_strides[0] + b * c.vmsb_strides[1] + h * c.vmsb_strides[2];
        const uint8_t* vl = c.v_lsb + bl * c.vlsb_strides[0] + b * c.vlsb_strides[1] + h * c.vlsb_strides[2];
        const uint16_t* ks = (const uint16_t*)c.k_scale + bl * c.kst_strides[0] + b * c.kst_strides[1] + h * c.kst_strides[2];
        const uint16_t* vs = (const uint16_t*)c.v_scale + bl * c.vst_strides[0] + b * c.vst_strides[1] + h * c.vst_strides[2];
        rs.km_t = (int)c.kmsb_strides[3]; rs.kl_t = (int)c.klsb_strides[3];
        rs.vm_t = (int)c.vmsb_strides[3]; rs.vl_t = (int)c.vlsb_strides[3];
        rs.km = make_rsrc(km, (int64_t)S * rs.km_t);
        rs.kl = make_rsrc(kl, (int64_t)S * rs.kl_t);
        rs.vm = make_rsrc(vm, (int64_t)S * rs.vm_t);
        rs.vl = make_rsrc(vl, (int64_t)S * rs.vl_t);
        rs.ks_t = (int)c.kst_strides[3] * 2; rs.vs_t = (int)c.vst_strides[3] * 2;
        rs.ks = make_rsrc(ks, (int64_t)S * rs.ks_t);
        rs.vs = make_rsrc(vs, (int64_t)S * rs.vs_t);
    }
    auto issue_page = [&](TurboPage& bf, int p) {
        __builtin_amdgcn_sched_barrier(0);
        load_turbo_page(bf, rs, p * 64 + 8 * slot, c16);
        __builtin_amdgcn_sched_barrier(0);
    };
    TurboPage b0, b1;
    bool first_issued = false;

    int e0, e1;
    if constexpr (FUSED) {
        __shared__ uint32_t s_key[NREP * 64 * kSelC];
        __shared__ BlockSelectLds s_bsel;
        if (a.sel.mode == FQ_SELECT_PER_KV_HEAD_SUM) score_group_regs<bf16, NREP, NT, true>(sr, s_qraw, s_key, tid, c.P);
        else score_group_regs<bf16, NREP, NT, false>(sr, s_qraw, s_key, tid, c.P);
        const ForcedPages fp = forced_pages(c.P, a.sel.num_sinks, a.sel.window);
        if (S > 0 && w < fp.count) {
            issue_page(b0, fp.page(w));
            first_issued = true;
        }
        __syncthreads();
        e0 = 0;
        e1 = block_select_group<kSelC, NW, NREP>(s_key, c.P, a.sel.mode, ret_l, a.sel.k_max, a.sel.num_sinks,
                                                 a.sel.window, s_ent, s_bsel);
    } else {
        const int n_sel = a.ws.n_sel[g];
        e0 = (int)((int64_t)n_sel * split / a.splits);
        e1 = (int)((int64_t)n_sel * (split + 1) / a.splits);
        for (int i = tid; i < e1 - e0; i += NT) s_ent[i] = a.ws.entries[(int64_t)g * c.P + e0 + i];
        __syncthreads();
    }
    const int n_mine = S > 0 && w < e1 - e0 ? (e1 - e0 - w + NW - 1) / NW : 0;

    float qv[NREP][16];
#pragma unroll
    for (int r = 0; r < NREP; ++r)
#pragma unroll
        for (int j = 0; j < 16; ++j) qv[r][j] = s_qrot[r][16 * c16 + j];

    float m_run[NREP], l_acc[NREP], acc[NREP][16];
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
        m_run[r] = -INFINITY;
        l_acc[r] = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[r][j] = 0.f;
    }

    auto entry_of = [&](int k) { return __builtin_amdgcn_readfirstlane(s_ent[w + NW * k]); };
    auto compute = [&](const TurboPage& pb, int k) {
        const int ent = entry_of(k);
        const int p = ent & 0xFFFF, qm = ent >> 16;
        const int tok0 = p * 64 + 8 * slot;
        // ---- logits of the lane's 8 tokens (summed over the slot's 8 lanes)
        float s[8][NREP];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float d[NREP];
#pragma unroll
            for (int r = 0; r < NREP; ++r) d[r] = 0.f;
#pragma unroll
            for (int jp = 0; jp < 8; ++jp) {
                const float2 pr = s_lut[lut_index(pb.kl[i], pb.km[i], jp)];
                const float k0 = pr.x, k1 = pr.y;
#pragma unroll
                for (int r = 0; r < NREP; ++r) d[r] = fmaf(qv[r][2 * jp + 1], k1, fmaf(qv[r][2 * jp], k0, d[r]));
            }
            const float ksc = scale_of(pb.ks, L, i);
            const bool tok_ok = tok0 + i < S;
#pragma unroll
            for (int r = 0; r < NREP; ++r) {
                float v = d[r];
                v += __shfl_xor(v, 1, 64);
                v += __shfl_xor(v, 2, 64);
                v += __shfl_xor(v, 4, 64);
                s[i][r] = (tok_ok && ((qm >> r) & 1)) ? v * ksc : -INFINITY;
            }
        }
        // ---- online softmax (wave-uniform maxima per head)
        float vsc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) vsc[i] = scale_of(pb.vs, L, i);
        float pw[8][NREP];
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
            float mx = s[0][r];
#pragma unroll
            for (int i = 1; i < 8; ++i) mx = fmaxf(mx, s[i][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 8, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mn = fmaxf(m_run[r], mx);
            if (mn > m_run[r]) {
                const float al = m_run[r] == -INFINITY ? 0.f : exp2_fast(m_run[r] - mn);
                l_acc[r] *= al;
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[r][j] *= al;
                m_run[r] = mn;
            }
            const float mref = m_run[r] == -INFINITY ? 0.f : m_run[r];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float pe = exp2_fast(s[i][r] - mref);      // exp2(-inf) = 0
                l_acc[r] += pe;
                pw[i][r] = pe * vsc[i];
            }
        }
        // ---- p.v over the lane's 16 channels
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
            for (int jp = 0; jp < 8; ++jp) {
                const float2 pr = s_lut[lut_index(pb.vl[i], pb.vm[i], jp)];
                const float v0 = pr.x, v1 = pr.y;
#pragma unroll
                for (int r = 0; r < NREP; ++r) {
                    acc[r][2 * jp] = fmaf(pw[i][r], v0, acc[r][2 * jp]);
                    acc[r][2 * jp + 1] = fmaf(pw[i][r], v1, acc[r][2 * jp + 1]);
                }
            }
        }
    };

    {
        if (!first_issued) issue_page(b0, n_mine > 0 ? entry_of(0) & 0xFFFF : 0);
        for (int k = 0; k < n_mine; k += 2) {
            issue_page(b1, entry_of(min(k + 1, n_mine - 1)) & 0xFFFF);
            compute(b0, k);
            issue_page(b0, entry_of(min(k + 2, n_mine - 1)) & 0xFFFF);
            if (k + 1 < n_mine) compute(b1, k + 1);
        }
    }

    // ---- wave state -> LDS: l over the slots (the slot's 8 lanes hold the same
    // values), acc over the slots for the lane's 16 channels
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
        float lv = l_acc[r];
        lv += __shfl_xor(lv, 8, 64);
        lv += __shfl_xor(lv, 16, 64);
        lv += __shfl_xor(lv, 32, 64);
        l_acc[r] = lv;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            float v = acc[r][j];
            v += __shfl_xor(v, 8, 64);
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            acc[r][j] = v;
        }
    }
    if (slot == 0) {
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
#pragma unroll
            for (int j = 0; j < 16; ++j) s_split.acc[w][r][16 * c16 + j] = acc[r][j];
            if (c16 == 0) { s_split.m[w][r] = m_run[r]; s_split.l[w][r] = l_acc[r]; }
        }
    }
    __syncthreads();
    merge_waves_and_store<D, NREP, true, NW>(s_split, q, a.ws, g, l, b, h, split, a.splits > 1);
}

template <bool FUSED>
hipError_t launch_turbo_fused_nrep(const TurboFusedParams& a, dim3 grid, hipStream_t st) {
    switch (a.q.nrep) {
#define FQ_CASE(N)                                                                                          \
    case N:                                                                                                 \
        timer_before_launch(st);                                                                            \
        hipLaunchKernelGGL((attn_turbo_fused_kernel<N, FUSED>), grid, dim3(512), 0, st, a);                 \
        timer_after_launch(st);                                                                             \
        if (a.splits > 1)                                                                                   \
            hipLaunchKernelGGL((merge_splits_kernel<128, N, true>), dim3(grid.y), dim3(kThreads), 0, st, a.q, \
                               a.ws, a.c.H_kv, a.c.B, 0, a.splits, TailArgs{});                                         \
        break;
        FQ_CASE(1) FQ_CASE(2) FQ_CASE(3) FQ_CASE(4)
#undef FQ_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool turbo_fused_supported(const fq_turbo_cache& c, const QueryArgs& q) {
    // 4 query heads per KV head would spill registers: the split kernel takes them
    if (c.D != 128 || c.page_size != 64 || q.nrep > 3 || c.P > kMaxWgPages) return false;
    if (c.kmsb_strides[4] != 1 || c.klsb_strides[4] != 1 || c.vmsb_strides[4] != 1 || c.vlsb_strides[4] != 1)
        return false;
    // 2-byte MSB and 4-byte LSB words per lane
    if (c.kmsb_strides[3] % 2 || c.vmsb_strides[3] % 2 || c.klsb_strides[3] % 4 || c.vlsb_strides[3] % 4) return false;
    for (int i = 0; i < 3; ++i) {
        if (c.kmsb_strides[i] % 2 || c.vmsb_strides[i] % 2 || c.klsb_strides[i] % 4 || c.vlsb_strides[i] % 4)
            return false;
    }
    if (((uintptr_t)c.k_msb | (uintptr_t)c.v_msb) & 1) return false;
    if (((uintptr_t)c.k_lsb | (uintptr_t)c.v_lsb) & 3) return false;
    if (((uintptr_t)c.k_scale | (uintptr_t)c.v_scale) & 1) return false;
    return true;
}

// Pages from the workspace lists (splits per group chosen like the INT4
// matrix-core kernel), or, with raw != null and sel, scored and selected in the
// kernel (one workgroup per group).
hipError_t launch_attn_turbo_fused(const fq_turbo_cache& c, const Int4Cache* raw, const QueryArgs& q,
                                   const Workspace& ws, int max_entries, const SelectArgs* sel, hipStream_t st) {
    TurboFusedParams a{};
    a.c = c; a.q = q; a.ws = ws;
    const int groups = c.L * c.B * c.H_kv;
    if (raw && sel && sel->enabled) {
        a.raw = *raw;
        a.sel = *sel;
        a.splits = 1;
        return launch_turbo_fused_nrep<true>(a, dim3(1, groups), st);
    }
    int s = groups >= 192 ? 1 : (512 + groups - 1) / groups;
    s = std::min(s, (max_entries + 7) / 8);
    s = std::max(s, (max_entries + kMaxWgPages - 1) / kMaxWgPages);
    a.splits = std::max(1, std::min(s, ws.s_max));
    return launch_turbo_fused_nrep<false>(a, dim3(a.splits, groups), st);
}

}  // namespace fq
