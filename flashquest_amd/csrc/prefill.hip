// Causal prefill attention over the packed KV cache on the gfx950 matrix cores.
//
// Semantics (S_q > 1 branch of the reference's attention patch,
// src/flashquest/eager/llama_persistent_patch.py:196-201):
//   K_full = cat(dequantize(K codes), K_partial)   (dequantize_k_int4 / dequantize_k,
//   V_full = cat(dequantize(V codes), V_partial)    kv_quant.py:174-186, 208-215, 64-100)
//   O = SDPA(q, K_full, V_full, is_causal=True, enable_gqa=True)
// Each dequantised element is code * scale + mn in fp32 (the product of a code
// and a half-precision scale is exact in fp32, so one FMA rounds the same as
// the reference's multiply then add) rounded to bf16 -- the same bf16 K / V the
// reference feeds SDPA.  Query row i attends keys j <= i + causal_off;
// causal_off = 0 is torch's is_causal (upper-left aligned when S_q < S_kv).
//
// One 8-wave workgroup per (256 GQA-flattened query rows, KV head): row
// m = pos * n_rep + r is query position pos of head kvh * n_rep + r, so every
// K/V tile a workgroup dequantises serves all n_rep heads of the group.  Per
// 64-key tile all 512 threads dequantise K into LDS as [key][channel] bf16 and
// V transposed as [channel][key] bf16 (keys in vt_pos order; the next tile is
// fetched into registers while the current one is computed), then each wave runs
//   S^T = K Q^T     v_mfma_f32_16x16x32_bf16, 4 key blocks x 2 query blocks
//   online softmax  per query column (base 2, fp32), P rounded to bf16
//   O^T += V^T P^T  v_mfma_f32_16x16x32_bf16, 8 channel blocks x 2 query blocks
// Computing the transposed products keeps each lane on one query column, so
// the softmax statistics are per lane and P leaves the S^T accumulator already
// in the layout of the P^T operand (keys 4g..4g+3 and 16+4g..16+4g+3 of a
// 32-key step; V^T is read with the same key order).
//
// That single pass (prefill_attn_kernel) serves short prompts.  Longer ones
// take two: prefill_dequant_kernel writes the attended keys once as dense
// bf16 K and V^T, then prefill_dense_kernel runs the same products over
// 128-key stages that direct-to-LDS buffer loads fill (no staging registers),
// optionally split over key ranges with prefill_merge_kernel combining them.
#include <algorithm>

#include "fq_common.h"

namespace fq {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
// native vectors (not HIP's u32x4 / u32x2 wrapper structs) keep the fetch
// registers out of private memory
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kPD = 128;               // head dim
constexpr int kPW = 8;                 // waves per workgroup
constexpr int kPKT = 64;               // keys per tile
constexpr int kPRW = 32;               // query rows per wave (two 16-column blocks)
constexpr int kPRows = kPW * kPRW;     // query rows per workgroup
constexpr int kKStr = kPD + 8;         // bf16 per K row in LDS (272 B: conflict-free 16-byte reads)
constexpr int kVStr = kPKT + 8;        // bf16 per V^T row in LDS (144 B)
constexpr int kDenseKT = 128;          // keys per LDS stage of the dense (two-pass) source
constexpr float kLazyLog2 = 8.0f;      // dense pass: rescale O only when a maximum grows by > 2^8

struct PrefillParams {
    Int4Cache c;
    TailArgs t;            // bf16 tail rows (the partial page), keys S .. S + t.len - 1
    const void* q; int64_t q_s[3];     // (b, h_q, pos) element strides, channels contiguous
    void* out; int64_t o_s[3];
    uint16_t* kd;          // dense bf16 K   [b][h][S_pad][128]   (two-pass path)
    uint16_t* vtd;         // dense bf16 V^T [b][h][128][S_pad]
    int s_pad;             // keys in the dense arrays, a multiple of 128 (zeros beyond S_kv)
    int kv_splits;         // > 1: workgroups take slices of the key stages and store partials
    float* part;           // [split][b][h][row][128] unnormalised O, then [split][b][h][row][2] (m, l)
    int nrep, Sq, Skv, causal_off;
    float qk_scale;                    // sm_scale * log2(e)
};

template <int META>
FQ_DEV float meta_lo(uint32_t w) {   // low half of a dword of half-precision metadata
    return META == FQ_BF16 ? __uint_as_float(w << 16) : f16_bits_to_f(w & 0xFFFFu);
}
template <int META>
FQ_DEV float meta_hi(uint32_t w) {
    return META == FQ_BF16 ? __uint_as_float(w & 0xFFFF0000u) : f16_bits_to_f(w >> 16);
}
FQ_DEV uint32_t bf16_rne(float f) {    // fp32 -> bf16 bits, round to nearest even (finite inputs)
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
FQ_DEV uint32_t pack_bf16(float lo, float hi) { return bf16_rne(lo) | (bf16_rne(hi) << 16); }

// Key order of V^T rows (LDS and the dense array): inside each 32-key block,
// keys 4g..4g+3 and 16+4g..16+4g+3 sit together at 8g..8g+7 -- the eight keys
// one lane of the p.v operand needs -- so the operand is one 16-byte read.
// Groups of 4 consecutive keys stay consecutive.
FQ_DEV int vt_pos(int k) {
    const int r = k & 31;
    return (k & ~31) + 8 * ((r & 15) >> 2) + 4 * (r >> 4) + (r & 3);
}

// Across the four 16-lane rows of a wave (lanes n, n + 16, n + 32, n + 48):
// v_permlane16_swap / v_permlane32_swap exchange rows in VALU, no LDS trip.
// Both partners of each swap combine the same two values in the same order.
FQ_DEV float rows_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
FQ_DEV float rows_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

// ---- K: one thread = one key x 16 channels --------------------------------
// Raw bytes before dequantisation.
struct KFetch {
    u32x4 c0, c1;          // codes (INT4: c0.xy, INT8: c0) or 16 bf16 tail values
    u32x4 s0, s1, m0, m1;  // 16 half scales / mins
    int kind;              // 0 codes, 1 tail, 2 beyond the keys (zeros)
};

template <int BITS>
FQ_DEV void fetch_k_codes(KFetch& f, const Int4Cache& c, int b, int h, int key, int kc) {
    const uint8_t* row = c.kp + b * c.kp_s[1] + h * c.kp_s[2] + (int64_t)key * c.kp_s[3];
    if (BITS == 4) {
        const u32x2 v = *(const u32x2*)(row + kc / 2);
        f.c0 = u32x4{v.x, v.y, 0u, 0u};
    } else {
        f.c0 = *(const u32x4*)(row + kc);
    }
    const int64_t page = key / c.page;
    const uint16_t* ks = (const uint16_t*)c.ksc + b * c.ksc_s[1] + h * c.ksc_s[2] + page * c.ksc_s[3] + kc;
    const uint16_t* km = (const uint16_t*)c.kmn + b * c.kmn_s[1] + h * c.kmn_s[2] + page * c.kmn_s[3] + kc;
    f.s0 = *(const u32x4*)ks; f.s1 = *(const u32x4*)(ks + 8);
    f.m0 = *(const u32x4*)km; f.m1 = *(const u32x4*)(km + 8);
    f.kind = 0;
}

// `whole`: the tile lies inside the completed pages (no tail or padding keys).
template <int BITS>
FQ_DEV void fetch_k(KFetch& f, const PrefillParams& a, int b, int h, int key, int kc, bool whole) {
    if (whole || key < a.c.S) {
        fetch_k_codes<BITS>(f, a.c, b, h, key, kc);
    } else if (key < a.Skv) {
        f.kind = 1;
        const uint16_t* row = (const uint16_t*)a.t.k + b * a.t.ks[1] + h * a.t.ks[2] + (int64_t)(key - a.c.S) * a.t.ks[3] + kc;
        f.c0 = *(const u32x4*)row; f.c1 = *(const u32x4*)(row + 8);
    } else {
        f.kind = 2;
    }
}

FQ_DEV uint32_t dw(const u32x4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// Dequantise 16 channels: code * scale + mn in fp32 (exact product, one rounding), then bf16.
template <int BITS, int META>
FQ_DEV void dequant_k16(const KFetch& f, u32x4& o0, u32x4& o1) {
    uint32_t out[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
        float c0, c1;
        if (BITS == 4) {
            const uint32_t wd = dw(f.c0, i >> 3);
            const uint32_t lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
            const int by = (i >> 1) & 3;
            c0 = (float)((lo >> (8 * by)) & 0xFFu);
            c1 = (float)((hi >> (8 * by)) & 0xFFu);
        } else {
            const uint32_t wd = dw(f.c0, i >> 2);
            c0 = (float)((wd >> (8 * (i & 3))) & 0xFFu);
            c1 = (float)((wd >> (8 * (i & 3) + 8)) & 0xFFu);
        }
        const uint32_t sw = i < 8 ? dw(f.s0, i >> 1) : dw(f.s1, (i >> 1) - 4);
        const uint32_t mw = i < 8 ? dw(f.m0, i >> 1) : dw(f.m1, (i >> 1) - 4);
        out[i >> 1] = pack_bf16(fmaf(c0, meta_lo<META>(sw), meta_lo<META>(mw)),
                                fmaf(c1, meta_hi<META>(sw), meta_hi<META>(mw)));
    }
    o0 = u32x4{out[0], out[1], out[2], out[3]};
    o1 = u32x4{out[4], out[5], out[6], out[7]};
}

template <int BITS, int META>
FQ_DEV void store_k(const KFetch& f, uint16_t* dst) {
    u32x4 o0 = u32x4{0u, 0u, 0u, 0u}, o1 = o0;
    if (f.kind == 0) dequant_k16<BITS, META>(f, o0, o1);
    else if (f.kind == 1) { o0 = f.c0; o1 = f.c1; }
    *(u32x4*)dst = o0;
    *(u32x4*)(dst + 8) = o1;
}

// ---- V: one thread = 4 keys x 4 channels, stored transposed -----------------
struct VFetch {
    u32x2 raw[4];          // per key: codes (INT4: 16 bits, INT8: 32 bits) or 4 bf16 tail values
    uint32_t sc[4], mn[4]; // per key: half bits of scale / mn
    int kinds;             // 2 bits per key, as KFetch::kind
};

template <int BITS>
FQ_DEV void fetch_v(VFetch& f, const PrefillParams& a, int b, int h, int key0, int vd, bool whole) {
    const Int4Cache& c = a.c;
    const int grp = vd / (kPD / c.G);
    f.kinds = 0;
    const uint8_t* rows = c.vp + b * c.vp_s[1] + h * c.vp_s[2] + (int64_t)key0 * c.vp_s[3] + (BITS == 4 ? vd / 2 : vd);
    const uint16_t* vs = (const uint16_t*)c.vsc + b * c.vsc_s[1] + h * c.vsc_s[2] + (int64_t)key0 * c.vsc_s[3] + grp;
    const uint16_t* vm = (const uint16_t*)c.vmn + b * c.vmn_s[1] + h * c.vmn_s[2] + (int64_t)key0 * c.vmn_s[3] + grp;
    // per-token metadata (one group) of 4 whole keys: one 8-byte load each for
    // scale and min (the 4 keys' values are adjacent)
    if (whole && c.G == 1 && c.vsc_s[3] == 1 && c.vmn_s[3] == 1 && (((uintptr_t)vs | (uintptr_t)vm) & 7) == 0) {
        const u32x2 s4 = *(const u32x2*)vs, m4 = *(const u32x2*)vm;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f.raw[j].x = BITS == 4 ? (uint32_t)*(const uint16_t*)(rows + j * c.vp_s[3])
                                   : *(const uint32_t*)(rows + j * c.vp_s[3]);
            f.sc[j] = ((j < 2 ? s4.x : s4.y) >> (16 * (j & 1))) & 0xFFFFu;
            f.mn[j] = ((j < 2 ? m4.x : m4.y) >> (16 * (j & 1))) & 0xFFFFu;
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int key = key0 + j;
        if (whole || key < c.S) {
            f.raw[j].x = BITS == 4 ? (uint32_t)*(const uint16_t*)(rows + j * c.vp_s[3])
                                   : *(const uint32_t*)(rows + j * c.vp_s[3]);
            f.sc[j] = vs[j * c.vsc_s[3]];
            f.mn[j] = vm[j * c.vmn_s[3]];
        } else if (key < a.Skv) {
            f.kinds |= 1 << (2 * j);
            const uint16_t* row = (const uint16_t*)a.t.v + b * a.t.vs[1] + h * a.t.vs[2] + (int64_t)(key - c.S) * a.t.vs[3] + vd;
            f.raw[j] = *(const u32x2*)row;
        } else {
            f.kinds |= 2 << (2 * j);
        }
    }
}

// v[key][i] as bf16 bits for channels vd + i
template <int BITS, int META>
FQ_DEV void dequant_v44(const VFetch& f, uint32_t (&v)[4][4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int kind = (f.kinds >> (2 * j)) & 3;
        const float sc = meta_lo<META>(f.sc[j]), mn = meta_lo<META>(f.mn[j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t code = BITS == 4 ? (f.raw[j].x >> (4 * i)) & 15u : (f.raw[j].x >> (8 * i)) & 0xFFu;
            const uint32_t tail = ((i < 2 ? f.raw[j].x : f.raw[j].y) >> (16 * (i & 1))) & 0xFFFFu;
            v[j][i] = kind == 0 ? bf16_rne(fmaf((float)code, sc, mn)) : (kind == 1 ? tail : 0u);
        }
    }
}

template <int BITS, int META>
FQ_DEV void store_v(const VFetch& f, uint16_t* dst /* V^T row vd, column key0 */, int row_stride) {
    uint32_t v[4][4];
    dequant_v44<BITS, META>(f, v);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *(u32x2*)(dst + i * row_stride) = u32x2{v[0][i] | (v[1][i] << 16), v[2][i] | (v[3][i] << 16)};
}

// ---- dense bf16 source (two-pass path) --------------------------------------

// The first pass: dequantise the cache and the tail once into dense bf16 K and
// V^T (keys padded with zeros to a multiple of 64).  One 512-thread block per
// (64-key tile, b, h); V goes through LDS to be written transposed.
template <int BITS, int META>
__global__ __launch_bounds__(512) void prefill_dequant_kernel(PrefillParams a) {
    __shared__ __attribute__((aligned(16))) uint16_t s_v[kPD * kVStr];
    __shared__ u32x4 s_kmeta[2][16];        // the tile's K page scale / min (one page per tile)
    const int tid = threadIdx.x;
    const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int key0 = tile * kPKT;
    const bool whole = key0 + kPKT <= a.c.S;
    const int kk = tid >> 3, kc = (tid & 7) * 16;
    const int vk = (tid & 15) * 4, vd = (tid >> 4) * 4;
    // A tile inside the completed pages with one page per tile: its 64 keys
    // share one row of K scale / min, loaded once into LDS instead of by every
    // thread (uniform per block)
    const bool one_page = whole && a.c.page % kPKT == 0;
    KFetch kf;
    VFetch vf;
    if (one_page) {
        const Int4Cache& c = a.c;
        const uint8_t* row = c.kp + b * c.kp_s[1] + h * c.kp_s[2] + (int64_t)(key0 + kk) * c.kp_s[3];
        if (BITS == 4) {
            const u32x2 v = *(const u32x2*)(row + kc / 2);
            kf.c0 = u32x4{v.x, v.y, 0u, 0u};
        } else {
            kf.c0 = *(const u32x4*)(row + kc);
        }
        kf.kind = 0;
        if (tid < 32) {
            const bool sc = tid < 16;
            const int64_t page = key0 / c.page;
            const uint16_t* src = sc ? (const uint16_t*)c.ksc + b * c.ksc_s[1] + h * c.ksc_s[2] + page * c.ksc_s[3]
                                     : (const uint16_t*)c.kmn + b * c.kmn_s[1] + h * c.kmn_s[2] + page * c.kmn_s[3];
            s_kmeta[tid >> 4][tid & 15] = *(const u32x4*)(src + 8 * (tid & 15));
        }
    } else {
        fetch_k<BITS>(kf, a, b, h, key0 + kk, kc, whole);
    }
    fetch_v<BITS>(vf, a, b, h, key0 + vk, vd, whole);
    if (one_page) {
        __syncthreads();
        kf.s0 = s_kmeta[0][kc / 8]; kf.s1 = s_kmeta[0][kc / 8 + 1];
        kf.m0 = s_kmeta[1][kc / 8]; kf.m1 = s_kmeta[1][kc / 8 + 1];
    }
    const int64_t bh = (int64_t)b * a.c.Hkv + h;
    store_k<BITS, META>(kf, a.kd + (bh * a.s_pad + key0 + kk) * kPD + kc);
    store_v<BITS, META>(vf, &s_v[vd * kVStr + vt_pos(vk)], kVStr);
    __syncthreads();
    const int d = tid >> 2, q = (tid & 3) * 16;
    uint16_t* dst = a.vtd + (bh * kPD + d) * a.s_pad + key0 + q;
    *(u32x4*)dst = *(const u32x4*)&s_v[d * kVStr + q];
    *(u32x4*)(dst + 8) = *(const u32x4*)&s_v[d * kVStr + q + 8];
}

// S^T (64 keys x 32 query columns of this wave) = K Q^T for one LDS K tile.
// k-step outer: eight independent accumulators between dependent MFMAs.
FQ_DEV void qk_tile(const uint16_t* sk, const v8bf (&qf)[2][4], v4f (&s)[2][4], int n, int g) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        s[0][kb] = v4f{0.f, 0.f, 0.f, 0.f};
        s[1][kb] = v4f{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const v8bf ak = *(const v8bf*)(sk + (kb * 16 + n) * kKStr + 32 * ks + 8 * g);
            s[0][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, qf[0][ks], s[0][kb], 0, 0, 0);
            s[1][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, qf[1][ks], s[1][kb], 0, 0, 0);
        }
}

// Online softmax of one S^T tile in three steps (mask, running max, exp and
// pack P as the bf16 P^T operand), then O^T += V^T P^T from the LDS V^T tile.
FQ_DEV void mask_tile(v4f (&s)[2][4], const int (&qpos)[2], int key0, int causal_off, int Skv, int g) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int lim = min(qpos[qb] + causal_off, Skv - 1) - key0 - 4 * g;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int cc = 0; cc < 4; ++cc)
                if (kb * 16 + cc > lim) s[qb][kb][cc] = -INFINITY;
    }
}

// New running max per query column; returns whether it moved for any lane's column.
FQ_DEV bool tile_max(const v4f (&s)[2][4], float (&m_run)[2], float (&m_use)[2], float (&alpha)[2], float qk_scale) {
    bool moved = false;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        float mx = fmaxf(fmaxf(s[qb][0][0], s[qb][0][1]), fmaxf(s[qb][0][2], s[qb][0][3]));
#pragma unroll
        for (int kb = 1; kb < 4; ++kb)
            mx = fmaxf(mx, fmaxf(fmaxf(s[qb][kb][0], s[qb][kb][1]), fmaxf(s[qb][kb][2], s[qb][kb][3])));
        mx = rows_max(mx);
        const float m_new = fmaxf(m_run[qb], mx * qk_scale);
        m_use[qb] = m_new == -INFINITY ? 0.f : m_new;
        alpha[qb] = __builtin_amdgcn_exp2f(m_run[qb] - m_use[qb]);
        moved |= m_new != m_run[qb];
        m_run[qb] = m_new;
    }
    return moved;
}

FQ_DEV void tile_exp(const v4f (&s)[2][4], const float (&m_use)[2], const float (&alpha)[2], float (&l_run)[2],
                     v8bf (&pb)[2][2], float qk_scale) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        float sum = 0.f;
        float p[4][4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                p[kb][cc] = __builtin_amdgcn_exp2f(fmaf(s[qb][kb][cc], qk_scale, -m_use[qb]));
                sum += p[kb][cc];
            }
        l_run[qb] = fmaf(l_run[qb], alpha[qb], sum);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                pb[qb][j][cc] = (__bf16)p[2 * j][cc];
                pb[qb][j][4 + cc] = (__bf16)p[2 * j + 1][cc];
            }
    }
}

FQ_DEV void tile_pv(v4f (&o)[2][8], const v8bf (&pb)[2][2], const uint16_t* sv, int vstr, int n, int g) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const v8bf av = *(const v8bf*)(sv + (db * 16 + n) * vstr + 32 * j + 8 * g);   // keys in vt_pos order
            o[0][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb[0][j], o[0][db], 0, 0, 0);
            o[1][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb[1][j], o[1][db], 0, 0, 0);
        }
}

FQ_DEV void softmax_pv(v4f (&s)[2][4], v4f (&o)[2][8], float (&m_run)[2], float (&l_run)[2], const uint16_t* sv,
                       int vstr, const int (&qpos)[2], int key0, int pmin, int causal_off, int Skv, float qk_scale, int n,
                       int g) {
    if (key0 + kPKT - 1 > pmin + causal_off || key0 + kPKT > Skv) mask_tile(s, qpos, key0, causal_off, Skv, g);
    float m_use[2], alpha[2];
    const bool moved = tile_max(s, m_run, m_use, alpha, qk_scale);
    v8bf pb[2][2];
    tile_exp(s, m_use, alpha, l_run, pb, qk_scale);
    if (__builtin_amdgcn_ballot_w64(moved)) {   // the running max moved for some column
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int db = 0; db < 8; ++db) o[qb][db] *= alpha[qb];
    }
    tile_pv(o, pb, sv, vstr, n, g);
}

// ---- TurboQuant source: dequantise the rotated codes and rotate back ---------
// dequantize_k_turbo / dequantize_v_turbo (kv_quant.py:366-420): index
// idx = (msb bit << 2) | lsb field (msb byte j bit i = channel 8j + i, lsb
// byte j field i = channel 4j + i), value = codebook[idx] * fp32(scale), then
// the normalised WHT (wht.py:17-41: stages h = 1, 2, ..., 64 of (a + b, a - b)
// in fp32, then times fp32(1 / sqrt(128))), then bf16.
struct TurboPrefill {
    const uint8_t* k_msb; int64_t kmsb_s[3];   // (b, h, token) byte strides
    const uint8_t* k_lsb; int64_t klsb_s[3];
    const uint16_t* k_sc; int64_t ksc_s[3];     // bf16 per-token scale
    const uint8_t* v_msb; int64_t vmsb_s[3];
    const uint8_t* v_lsb; int64_t vlsb_s[3];
    const uint16_t* v_sc; int64_t vsc_s[3];
};

FQ_DEV float turbo_value(uint32_t idx) {   // kv_quant.py:225-229
    const uint32_t pos = idx & 4u;
    const uint32_t t = pos ? (idx & 3u) : ((idx & 3u) ^ 3u);
    const float m01 = (t & 1u) ? 0.7560f : 0.2451f;
    const float m23 = (t & 1u) ? 2.1519f : 1.3439f;
    const float mag = (t & 2u) ? m23 : m01;
    return pos ? mag : -mag;
}

// One wave per token: lane l holds channels l and l + 64.
FQ_DEV void turbo_token(const uint8_t* msb, const uint8_t* lsb, const uint16_t* sc, int lane, float& v0, float& v1) {
    const float scale = bf16_bits_to_f(*sc);
    const uint32_t m0 = msb[lane >> 3], m1 = msb[(lane + 64) >> 3];
    const uint32_t l0 = lsb[lane >> 2], l1 = lsb[(lane + 64) >> 2];
    v0 = turbo_value((((m0 >> (lane & 7)) & 1u) << 2) | ((l0 >> (2 * (lane & 3))) & 3u)) * scale;
    v1 = turbo_value((((m1 >> (lane & 7)) & 1u) << 2) | ((l1 >> (2 * (lane & 3))) & 3u)) * scale;
#pragma unroll
    for (int hh = 1; hh < 64; hh <<= 1) {
        const float y0 = __shfl_xor(v0, hh, 64), y1 = __shfl_xor(v1, hh, 64);
        v0 = (lane & hh) ? y0 - v0 : v0 + y0;
        v1 = (lane & hh) ? y1 - v1 : v1 + y1;
    }
    const float x = v0, y = v1;
    const float inv = 1.0f / sqrtf(128.0f);
    v0 = (x + y) * inv;
    v1 = (x - y) * inv;
}

// The first pass for the TurboQuant cache: dense bf16 K and V^T of the
// attended keys (tail rows copied, zeros beyond S_kv).  One 512-thread block
// per (64-key tile, b, h), one wave per token, V through LDS to be written
// transposed.
__global__ __launch_bounds__(512) void prefill_dequant_turbo_kernel(PrefillParams a, TurboPrefill tq) {
    __shared__ __attribute__((aligned(16))) uint16_t s_v[kPD * kVStr];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int key0 = blockIdx.x * kPKT, h = blockIdx.y, b = blockIdx.z;
    const int64_t bh = (int64_t)b * a.c.Hkv + h;
    for (int j = w; j < kPKT; j += kPW) {
        const int key = key0 + j;
        float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
        uint32_t kb0, kb1, vb0, vb1;
        if (key < a.c.S) {
            turbo_token(tq.k_msb + b * tq.kmsb_s[0] + h * tq.kmsb_s[1] + (int64_t)key * tq.kmsb_s[2],
                        tq.k_lsb + b * tq.klsb_s[0] + h * tq.klsb_s[1] + (int64_t)key * tq.klsb_s[2],
                        tq.k_sc + b * tq.ksc_s[0] + h * tq.ksc_s[1] + (int64_t)key * tq.ksc_s[2], lane, k0, k1);
            turbo_token(tq.v_msb + b * tq.vmsb_s[0] + h * tq.vmsb_s[1] + (int64_t)key * tq.vmsb_s[2],
                        tq.v_lsb + b * tq.vlsb_s[0] + h * tq.vlsb_s[1] + (int64_t)key * tq.vlsb_s[2],
                        tq.v_sc + b * tq.vsc_s[0] + h * tq.vsc_s[1] + (int64_t)key * tq.vsc_s[2], lane, v0, v1);
            kb0 = bf16_rne(k0); kb1 = bf16_rne(k1); vb0 = bf16_rne(v0); vb1 = bf16_rne(v1);
        } else if (key < a.Skv) {
            const uint16_t* kr = (const uint16_t*)a.t.k + b * a.t.ks[1] + h * a.t.ks[2] + (int64_t)(key - a.c.S) * a.t.ks[3];
            const uint16_t* vr = (const uint16_t*)a.t.v + b * a.t.vs[1] + h * a.t.vs[2] + (int64_t)(key - a.c.S) * a.t.vs[3];
            kb0 = kr[lane]; kb1 = kr[lane + 64]; vb0 = vr[lane]; vb1 = vr[lane + 64];
        } else {
            kb0 = kb1 = vb0 = vb1 = 0u;
        }
        uint16_t* krow = a.kd + (bh * a.s_pad + key) * kPD;
        krow[lane] = (uint16_t)kb0;
        krow[lane + 64] = (uint16_t)kb1;
        s_v[lane * kVStr + vt_pos(j)] = (uint16_t)vb0;
        s_v[(lane + 64) * kVStr + vt_pos(j)] = (uint16_t)vb1;
    }
    __syncthreads();
    const int tid = threadIdx.x;
    const int d = tid >> 2, q = (tid & 3) * 16;
    uint16_t* dst = a.vtd + (bh * kPD + d) * a.s_pad + key0 + q;
    *(u32x4*)dst = *(const u32x4*)&s_v[d * kVStr + q];
    *(u32x4*)(dst + 8) = *(const u32x4*)&s_v[d * kVStr + q + 8];
}

template <int SRC>
FQ_DEV void prefill_fetch(const PrefillParams& a, KFetch& kf, VFetch& vf, int key0, int b, int h, int kk, int kc, int vk,
                          int vd) {
    const bool whole = key0 + kPKT <= a.c.S;
    fetch_k<SRC>(kf, a, b, h, key0 + kk, kc, whole);
    fetch_v<SRC>(vf, a, b, h, key0 + vk, vd, whole);
}

template <int SRC>
FQ_DEV void prefill_stage(const PrefillParams& a, const KFetch& kf, const VFetch& vf, uint16_t* sk, uint16_t* sv, int kk,
                          int kc, int vd, int vk) {
    if (a.c.meta_dtype == FQ_BF16) {
        store_k<SRC, FQ_BF16>(kf, sk + kk * kKStr + kc);
        store_v<SRC, FQ_BF16>(vf, sv + vd * kVStr + vt_pos(vk), kVStr);
    } else {
        store_k<SRC, FQ_F16>(kf, sk + kk * kKStr + kc);
        store_v<SRC, FQ_F16>(vf, sv + vd * kVStr + vt_pos(vk), kVStr);
    }
}

template <int SRC, int META>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_attn_kernel(PrefillParams a) {
    constexpr int ST = kPKT;       // keys per LDS stage, double-buffered
    constexpr int VSTR = kVStr;    // bf16 per V^T row (row stride = 4 banks mod 64: conflict-free reads)
    __shared__ __attribute__((aligned(16))) uint16_t s_k[2][ST * kKStr];
    __shared__ __attribute__((aligned(16))) uint16_t s_v[2][kPD * VSTR];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const Int4Cache& c = a.c;
    // KV head in the low bits of the block index: consecutive blocks go to
    // different XCDs, so with H_kv * B a multiple of 8 each XCD's L2 holds the
    // K/V of its own heads.  Row blocks run last-first (the longest first).
    const int HB = c.Hkv * c.B;
    const int nblk = gridDim.x / HB;
    const int hb = blockIdx.x % HB;
    const int rb = nblk - 1 - (int)(blockIdx.x / HB);
    const int h = hb % c.Hkv, b = hb / c.Hkv;
    const int Mtot = a.Sq * a.nrep;
    const int m0 = rb * kPRows;
    const int last_wg = (min(m0 + kPRows, Mtot) - 1) / a.nrep;
    const int nt = (min(a.Skv, last_wg + a.causal_off + 1) + ST - 1) / ST;   // >= 1: key 0 is attended

    const int mw0 = m0 + w * kPRW;
    const bool wave_on = mw0 < Mtot;
    const int pmin = min(mw0, Mtot - 1) / a.nrep;
    const int pmax = (min(mw0 + kPRW, Mtot) - 1) / a.nrep;
    const int limit_w = min(a.Skv, pmax + a.causal_off + 1);

    // this lane's two query columns: B operands of q.k (channels 32 ks + 8 g .. + 8)
    int qpos[2];
    bool qok[2];
    v8bf qf[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int m = mw0 + qb * 16 + n;
        qok[qb] = m < Mtot;
        const int mm = qok[qb] ? m : (wave_on ? mw0 : 0);
        qpos[qb] = qok[qb] ? mm / a.nrep : pmin;
        const int hq = h * a.nrep + mm % a.nrep;
        const uint16_t* qrow = (const uint16_t*)a.q + b * a.q_s[0] + hq * a.q_s[1] + (int64_t)(mm / a.nrep) * a.q_s[2];
        // unconditional loads (an idle wave reads a valid row it never uses):
        // no branch leaves these loads pending at the tile loop
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qf[qb][ks] = *(const v8bf*)(qrow + 32 * ks + 8 * g);
    }

    v4f o[2][8];
    float m_run[2], l_run[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        m_run[qb] = -INFINITY; l_run[qb] = 0.f;
#pragma unroll
        for (int db = 0; db < 8; ++db) o[qb][db] = v4f{0.f, 0.f, 0.f, 0.f};
    }

    const int kk = tid >> 3, kc = (tid & 7) * 16;         // K loader: one key, 16 channels
    const int vk = (tid & 15) * 4, vd = (tid >> 4) * 4;   // V loader: 4 keys, 4 channels

    KFetch kf;
    VFetch vf;
    prefill_fetch<SRC>(a, kf, vf, 0, b, h, kk, kc, vk, vd);
    prefill_stage<SRC>(a, kf, vf, s_k[0], s_v[0], kk, kc, vd, vk);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): prologue loads (Q included) land before the loop
    __syncthreads();
    for (int t = 0; t < nt; ++t) {
        const int cur = t & 1;
        const int key0 = t * ST;
        if (t + 1 < nt) prefill_fetch<SRC>(a, kf, vf, key0 + ST, b, h, kk, kc, vk, vd);
        __builtin_amdgcn_sched_barrier(0);
        if (wave_on && key0 < limit_w) {
            v4f s[2][4];
            qk_tile(s_k[cur], qf, s, n, g);
            softmax_pv(s, o, m_run, l_run, s_v[cur], VSTR, qpos, key0, pmin, a.causal_off, a.Skv, a.qk_scale, n, g);
        }
        // the dequantising LDS writes of the next tile after this tile's math
        __builtin_amdgcn_sched_barrier(0);
        if (t + 1 < nt) prefill_stage<SRC>(a, kf, vf, s_k[cur ^ 1], s_v[cur ^ 1], kk, kc, vd, vk);
        __syncthreads();
    }

    if (!wave_on) return;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const float l = rows_sum(l_run[qb]);
        if (!qok[qb]) continue;
        const float inv = 1.0f / l;
        const int m = mw0 + qb * 16 + n;
        const int hq = h * a.nrep + m % a.nrep;
        uint16_t* orow = (uint16_t*)a.out + b * a.o_s[0] + hq * a.o_s[1] + (int64_t)(m / a.nrep) * a.o_s[2];
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const v4f r = o[qb][db] * inv;
            *(u32x2*)(orow + db * 16 + 4 * g) = u32x2{pack_bf16(r[0], r[1]), pack_bf16(r[2], r[3])};
        }
    }
}

// ---- the two-pass path's attention: LDS filled by direct-to-LDS loads -------
// A stage is 128 keys of the dense source: K as [key][16 chunks of 8
// channels], V^T as [channel][16 chunks of 8 keys].  Chunk c of row r sits in
// slot c ^ (r & 15), so the 16 rows of an MFMA operand read (lanes n = 0..15,
// one chunk each) hit 16 distinct slots, and one direct-to-LDS load of a wave
// fills 4 whole rows (1 KB; lane L lands in slot L & 15 of row L >> 4) from
// the matching global chunks.  No staging registers and no LDS stores: stage
// t + 1 streams into the other buffer while stage t is computed.  Each wave
// owns QB blocks of 16 query columns, so every K / V^T operand read from LDS
// feeds QB matrix instructions.
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Buffer descriptor words (base, stride 0, num_records, the flags word of a raw
// buffer) for dma16_to_lds; p is wave-uniform.
FQ_DEV i32x4 dma_rsrc(const void* p, int num_records) {
    const uint64_t v = (uint64_t)p;
    return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)v),
                 __builtin_amdgcn_readfirstlane((int)((uint32_t)(v >> 32) & 0xFFFFu)), num_records, 0x00020000};
}
// Lane L loads 16 bytes at (voff + soff) of the buffer into LDS at dst + 16 L
// (buffer_load_dwordx4 ... lds, the LDS address in m0).  dst and soff are
// wave-uniform.  The load counts in vmcnt like any buffer load.
FQ_DEV void dma16_to_lds(i32x4 rsrc, const uint16_t* dst, int voff, int soff) {
    const int lds = __builtin_amdgcn_readfirstlane((int)(size_t)(lds_ptr_t)dst);
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :: "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds) : "memory");
}

template <int QB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_dense_kernel(PrefillParams a) {
    constexpr int ST = kDenseKT;
    constexpr int RW = 16 * QB, RWG = kPW * RW;
    __shared__ __attribute__((aligned(1024))) uint16_t s_k[2][ST * kPD];
    __shared__ __attribute__((aligned(1024))) uint16_t s_v[2][kPD * ST];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const Int4Cache& c = a.c;
    // KV head in the low bits of the block index (each XCD's L2 keeps its
    // heads' K / V); row blocks run last-first (the longest first)
    const int HB = c.Hkv * c.B;
    const int KS = a.kv_splits > 1 ? a.kv_splits : 1;
    const int nblk = gridDim.x / (HB * KS);
    const int hb = blockIdx.x % HB;
    const int rb = nblk - 1 - (int)((blockIdx.x / HB) % nblk);
    const int split = (int)(blockIdx.x / (HB * nblk));
    const int h = hb % c.Hkv, b = hb / c.Hkv;
    const int Mtot = a.Sq * a.nrep;
    const int m0 = rb * RWG;
    const int last_wg = (min(m0 + RWG, Mtot) - 1) / a.nrep;
    const int nt_all = (min(a.Skv, last_wg + a.causal_off + 1) + ST - 1) / ST;
    const int per = (nt_all + KS - 1) / KS;
    const int t_begin = min(nt_all, split * per);
    const int nt = min(nt_all, t_begin + per);

    const int mw0 = m0 + w * RW;
    const bool wave_on = mw0 < Mtot;
    const int pmin = min(mw0, Mtot - 1) / a.nrep;

    int qpos[QB];
    bool qok[QB];
    v8bf qf[QB][4];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int m = mw0 + qb * 16 + n;
        qok[qb] = m < Mtot;
        const int mm = qok[qb] ? m : (wave_on ? mw0 : 0);
        qpos[qb] = qok[qb] ? mm / a.nrep : pmin;
        const int hq = h * a.nrep + mm % a.nrep;
        const uint16_t* qrow = (const uint16_t*)a.q + b * a.q_s[0] + hq * a.q_s[1] + (int64_t)(mm / a.nrep) * a.q_s[2];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qf[qb][ks] = *(const v8bf*)(qrow + 32 * ks + 8 * g);
    }

    // o[qb][0..7]: O^T of the 128 channels; o[qb][8]: a block of ones times P^T,
    // i.e. sum p (the softmax denominator) of this lane's column in every row
    v4f o[QB][9];
    float m_run[QB];      // the reference maximum the exponents are taken against (log2 domain)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        m_run[qb] = -INFINITY;
#pragma unroll
        for (int db = 0; db < 9; ++db) o[qb][db] = v4f{0.f, 0.f, 0.f, 0.f};
    }
    v8bf ones;
#pragma unroll
    for (int i = 0; i < 8; ++i) ones[i] = (__bf16)1.0f;

    // wave w fills rows 16 w .. 16 w + 15 of both tiles, 4 rows per load: a
    // stage's uniform base address plus per-lane byte offsets fixed for the kernel
    const int64_t bh = (int64_t)b * c.Hkv + h;
    const int64_t dense_bytes = (int64_t)a.s_pad * kPD * 2;      // one (b, h) slice of K or of V^T
    const int nrec = __builtin_amdgcn_readfirstlane((int)min(dense_bytes, (int64_t)INT32_MAX));
    const int wu = __builtin_amdgcn_readfirstlane(w);
    const int lrow = lane >> 4, slot = lane & 15;
    int koff[4], voff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 16 * wu + 4 * j + lrow, ch = slot ^ ((4 * j + lrow) & 15);
        koff[j] = (r * kPD + ch * 8) * 2;
        voff[j] = (r * a.s_pad + ch * 8) * 2;
    }
    // The stage loads are issued as inline assembly: the compiler does not see
    // their LDS writes, so it adds no waits of its own before the LDS reads of
    // the other buffers while they are in flight (it cannot tell a load issued
    // in the previous iteration from the buffer read in this one).  The loop
    // orders them itself with the vmcnt waits and barriers below.
    const i32x4 krw = dma_rsrc(a.kd + bh * a.s_pad * kPD, nrec), vrw = dma_rsrc(a.vtd + bh * kPD * a.s_pad, nrec);
    auto issue_k = [&](int buf, int key0_) {
        const int key0 = __builtin_amdgcn_readfirstlane(key0_);
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16_to_lds(krw, s_k[buf] + (16 * wu + 4 * j) * kPD, koff[j], key0 * kPD * 2);
    };
    auto issue_v = [&](int buf, int key0_) {
        const int key0 = __builtin_amdgcn_readfirstlane(key0_);
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16_to_lds(vrw, s_v[buf] + (16 * wu + 4 * j) * ST, voff[j], key0 * 2);
    };

    // S^T = K Q^T for one 64-key sub-tile (sk: its first key row; row & 15 = n)
    auto qk = [&](const uint16_t* sk, v4f (&s)[QB][4]) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) s[qb][kb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const v8bf ak = *(const v8bf*)(sk + (kb * 16 + n) * kPD + (((4 * ks + g) ^ n) * 8));
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
                    s[qb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, qf[qb][ks], s[qb][kb], 0, 0, 0);
            }
    };
    // causal / length mask of a sub-tile starting at key k0 (only near the diagonal or the end)
    auto diag_mask = [&](int k0, v4f (&s)[QB][4]) {
        if (k0 + kPKT - 1 > pmin + a.causal_off || k0 + kPKT > a.Skv) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const int lim = min(qpos[qb] + a.causal_off, a.Skv - 1) - k0 - 4 * g;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc)
                        if (kb * 16 + cc > lim) s[qb][kb][cc] = -INFINITY;
            }
        }
    };
    // per-column maxima (log2 domain); true where one exceeds the reference by
    // more than 2^kLazyLog2: the reference then moves (raise_ref).  Until it
    // does, p <= 2^kLazyLog2 (exact in fp32, relative bf16 rounding unchanged)
    // and O and its denominator need no rescale.
    auto tile_max = [&](const v4f (&s)[QB][4], float (&mx)[QB]) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            float t4[4];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                t4[kb] = fmaxf(fmaxf(s[qb][kb][0], s[qb][kb][1]), fmaxf(s[qb][kb][2], s[qb][kb][3]));
            mx[qb] = rows_max(fmaxf(fmaxf(t4[0], t4[1]), fmaxf(t4[2], t4[3]))) * a.qk_scale;
        }
    };
    auto moved = [&](const float (&mx)[QB]) {
        bool mv = false;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) mv |= mx[qb] > m_run[qb] + kLazyLog2;
        return mv;
    };
    auto raise_ref = [&](const float (&mx)[QB]) {      // wave-uniform: new references for every column
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const float m_new = fmaxf(m_run[qb], mx[qb]);
            const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - (m_new == -INFINITY ? 0.f : m_new));
            m_run[qb] = m_new;
#pragma unroll
            for (int db = 0; db < 9; ++db) o[qb][db] *= alpha;
        }
    };
    // P = exp2(s * qk_scale - reference) as the bf16 P^T operands
    auto exp_p = [&](const v4f (&s)[QB][4], v8bf (&pb)[QB][2]) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const float m_use = m_run[qb] == -INFINITY ? 0.f : m_run[qb];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    pb[qb][j][cc] = (__bf16)__builtin_amdgcn_exp2f(fmaf(s[qb][2 * j][cc], a.qk_scale, -m_use));
                    pb[qb][j][4 + cc] = (__bf16)__builtin_amdgcn_exp2f(fmaf(s[qb][2 * j + 1][cc], a.qk_scale, -m_use));
                }
        }
    };
    // O^T += V^T P^T (channel rows db * 16 + n, key chunks 8 sub + 4 j + g, vt_pos
    // order) and the denominator block ones * P^T
    auto pv = [&](const uint16_t* sv, int sub, const v8bf (&pb)[QB][2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                const v8bf av = *(const v8bf*)(sv + (db * 16 + n) * ST + (((8 * sub + 4 * j + g) ^ n) * 8));
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
                    o[qb][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb[qb][j], o[qb][db], 0, 0, 0);
            }
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
                o[qb][8] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[qb][j], o[qb][8], 0, 0, 0);
        }
    };

    // Stage t sits in buffer (t - t_begin) & 1.  The loop is pipelined across
    // stages so that every phase pairs matrix work with vector work:
    //   q.k of sub-tile 0 (stage t)        | exp of sub-tile 1 (stage t - 1)
    //   p.v of sub-tile 1 (stage t - 1)    | maximum of sub-tile 0
    //   -- barrier: V(t - 1) is free, V(t) has landed; V(t + 1) is issued --
    //   q.k of sub-tile 1                  | exp of sub-tile 0
    //   p.v of sub-tile 0                  | maximum of sub-tile 1
    // O accumulates the sub-tiles in key order.  Every wave computes
    // every sub-tile of the workgroup's stages (a wave with no rows computes
    // none): the causal / length mask zeroes the keys past a wave's rows (exact
    // zeros added to O and its denominator).
    // K(t + 1) is issued at the top of iteration t, V(t + 1) after the middle
    // barrier; the waits count the 4 loads per wave issued after the ones needed.
    if (t_begin < nt) {
        issue_k(0, t_begin * ST);
        issue_v(0, t_begin * ST);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the first stage and Q have landed
    __syncthreads();
    v4f s1p[QB][4];       // sub-tile 1 scores of the previous stage
    for (int t = t_begin; t < nt; ++t) {
        const int cur = (t - t_begin) & 1;
        const int key0 = t * ST;
        const bool more = t + 1 < nt;
        // the other K buffer was last read before the previous iteration's end barrier
        if (more) issue_k(cur ^ 1, key0 + ST);
        v4f s0[QB][4];
        float mx0[QB];
        if (wave_on && t > t_begin) {
            v8bf pp[QB][2];
            exp_p(s1p, pp);
            qk(s_k[cur], s0);
            diag_mask(key0, s0);
            tile_max(s0, mx0);
            pv(s_v[cur ^ 1], 1, pp);
        } else if (wave_on) {
            qk(s_k[cur], s0);
            diag_mask(key0, s0);
            tile_max(s0, mx0);
        }
        if (more) __builtin_amdgcn_s_waitcnt(0x0F74);   // vmcnt(4): V(t) is in LDS (K(t + 1) may be in flight)
        else __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
        if (more) issue_v(cur ^ 1, key0 + ST);
        if (wave_on) {
            if (__builtin_amdgcn_ballot_w64(moved(mx0))) raise_ref(mx0);
            v8bf p0[QB][2];
            float mx1[QB];
            exp_p(s0, p0);
            qk(s_k[cur] + kPKT * kPD, s1p);
            diag_mask(key0 + kPKT, s1p);
            tile_max(s1p, mx1);
            pv(s_v[cur], 0, p0);
            if (__builtin_amdgcn_ballot_w64(moved(mx1))) raise_ref(mx1);
        }
        if (more) __builtin_amdgcn_s_waitcnt(0x0F74);   // vmcnt(4): K(t + 1) is in LDS (V(t + 1) may be in flight)
        else __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
    }
    if (wave_on && t_begin < nt) {   // the last stage's sub-tile 1 (its V buffer is not reloaded)
        v8bf pp[QB][2];
        exp_p(s1p, pp);
        pv(s_v[(nt - 1 - t_begin) & 1], 1, pp);
    }

    if (!wave_on) return;
    if (KS > 1) {   // unnormalised partial + (m, l) per row for prefill_merge_kernel
        const int64_t rows = (int64_t)c.B * c.Hkv * Mtot;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const float l = o[qb][8][0];
            if (!qok[qb]) continue;
            const int64_t row = ((int64_t)split * c.B * c.Hkv + hb) * Mtot + mw0 + qb * 16 + n;
            float* prow = a.part + row * kPD;
#pragma unroll
            for (int db = 0; db < 8; ++db) *(v4f*)(prow + db * 16 + 4 * g) = o[qb][db];
            if (g == 0) {
                float* ml = a.part + (int64_t)KS * rows * kPD + row * 2;
                ml[0] = m_run[qb];
                ml[1] = l;
            }
        }
        return;
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const float l = o[qb][8][0];
        if (!qok[qb]) continue;
        const float inv = 1.0f / l;
        const int m = mw0 + qb * 16 + n;
        const int hq = h * a.nrep + m % a.nrep;
        uint16_t* orow = (uint16_t*)a.out + b * a.o_s[0] + hq * a.o_s[1] + (int64_t)(m / a.nrep) * a.o_s[2];
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const v4f r = o[qb][db] * inv;
            *(u32x2*)(orow + db * 16 + 4 * g) = u32x2{pack_bf16(r[0], r[1]), pack_bf16(r[2], r[3])};
        }
    }
}

}  // namespace

// Combines the key-range partials of the split path: per row (b, h, m)
// M = max m_i, L = sum 2^(m_i - M) l_i, O = sum 2^(m_i - M) O_i / L, in split
// order; one wave per row, lane = two channels.  The splits go in batches of
// 8 whose loads are all issued before any is used; the running maximum moves
// once per batch (earlier sums are rescaled by 2^(M_old - M_new)).
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillParams a) {
    constexpr int kBatch = 8;
    const int64_t rows = (int64_t)a.c.B * a.c.Hkv * a.Sq * a.nrep;
    const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 6;
    if (row >= rows) return;
    const int lane = threadIdx.x & 63;
    const int KS = a.kv_splits;
    const float* ml = a.part + (int64_t)KS * rows * kPD;
    float M = -INFINITY, L = 0.f, o0 = 0.f, o1 = 0.f;
    for (int sp0 = 0; sp0 < KS; sp0 += kBatch) {
        float m[kBatch], l[kBatch];
        float2 po[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int64_t sp = min(sp0 + u, KS - 1);
            m[u] = ml[(sp * rows + row) * 2];
            l[u] = ml[(sp * rows + row) * 2 + 1];
            po[u] = *(const float2*)(a.part + (sp * rows + row) * kPD + 2 * lane);
        }
        float Mb = M;
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (sp0 + u < KS) Mb = fmaxf(Mb, m[u]);
        if (Mb == -INFINITY) continue;          // nothing attended yet
        const float r = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - Mb);
        L *= r; o0 *= r; o1 *= r;
        M = Mb;
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            if (sp0 + u >= KS) break;
            const float wt = m[u] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[u] - M);
            L = fmaf(wt, l[u], L);
            o0 = fmaf(wt, po[u].x, o0);
            o1 = fmaf(wt, po[u].y, o1);
        }
    }
    const int Mtot = a.Sq * a.nrep;
    const int mi = (int)(row % Mtot);
    const int hb = (int)(row / Mtot);
    const int h = hb % a.c.Hkv, b = hb / a.c.Hkv;
    const int hq = h * a.nrep + mi % a.nrep;
    uint16_t* orow = (uint16_t*)a.out + b * a.o_s[0] + hq * a.o_s[1] + (int64_t)(mi / a.nrep) * a.o_s[2];
    const float inv = 1.0f / L;
    *(uint32_t*)(orow + 2 * lane) = pack_bf16(o0 * inv, o1 * inv);
}

// The keys any query can attend: min(S_kv, S_q + causal_off).
int64_t prefill_keys_needed(int Skv, int Sq, int causal_off) { return std::min<int64_t>(Skv, (int64_t)Sq + causal_off); }

int64_t prefill_row_blocks(int Sq, int nrep) { return ((int64_t)Sq * nrep + kPRows - 1) / kPRows; }

constexpr int kDenseQB = 2;                       // 16-column query blocks per wave, dense path
constexpr int kDenseRows = kPW * 16 * kDenseQB;   // query rows per dense workgroup
int64_t dense_row_blocks(int Sq, int nrep) { return ((int64_t)Sq * nrep + kDenseRows - 1) / kDenseRows; }

// The fused path (each workgroup dequantises the K/V tiles it attends) only
// for one row block per KV head over at most 1024 keys; otherwise the
// two-pass path (dequantise the needed keys once, in parallel, into dense
// bf16 K and V^T, then attend plain bf16 tiles) is faster.
// Key-range splits of the dense path: when the row blocks leave most CUs idle
// (few query rows over many keys, e.g. a chunk with causal_off = S_kv - S_q),
// workgroups take slices of at least 4 key stages and a merge launch combines
// their partials.
// Between 128 and 256 workgroups (one round on 256 CUs with some idle), the
// split count k <= 8 with the fewest rounds per unit of work,
// ceil(wgs k / 256) / k, evens the rounds out (192 workgroups: 4 splits, 3
// full rounds of a quarter of the work each).
int prefill_kv_splits(int64_t nblk, int64_t heads, int64_t keys) {
    const int64_t wgs = nblk * heads;
    const int64_t stages = (keys + kDenseKT - 1) / kDenseKT;
    if (stages < 8) return 1;
    if (wgs < 128) return (int)std::max<int64_t>(1, std::min<int64_t>((256 + wgs - 1) / wgs, stages / 4));
    if (wgs >= 256) return 1;
    int best = 1;
    double best_cost = 1.0;                  // rounds per unit of work with k = 1: one round
    for (int k = 2; k <= 8 && stages / k >= 4; ++k) {
        const double cost = (double)((wgs * k + 255) / 256) / k;
        if (cost < best_cost - 1e-9) { best = k; best_cost = cost; }
    }
    return best;
}

// Dense K / V^T of the attended keys, then (with key-range splits) the partials.
size_t prefill_dense_bytes(int Hkv, int B, int Skv, int Sq, int nrep, int causal_off) {
    const int64_t keys = prefill_keys_needed(Skv, Sq, causal_off);
    const int64_t s_pad = (keys + kDenseKT - 1) / kDenseKT * kDenseKT;
    size_t n = (size_t)(2 * s_pad * kPD * 2) * Hkv * B;
    const int ks = prefill_kv_splits(dense_row_blocks(Sq, nrep), (int64_t)Hkv * B, keys);
    if (ks > 1) n += (size_t)ks * B * Hkv * Sq * nrep * (kPD + 2) * sizeof(float);
    return n;
}

size_t prefill_workspace_bytes(const Int4Cache& c, int Skv, int Sq, int nrep, int causal_off) {
    const int64_t keys = prefill_keys_needed(Skv, Sq, causal_off);
    if (prefill_row_blocks(Sq, nrep) == 1 && keys <= 1024) return 0;
    return prefill_dense_bytes(c.Hkv, c.B, Skv, Sq, nrep, causal_off);
}

// The attention launch of the dense path (a.kd / a.vtd / a.s_pad set), with
// key-range splits and their merge when the row blocks are few.
hipError_t launch_dense_attn(PrefillParams& a, int Sq, int nrep, hipStream_t st) {
    const int64_t nblk = dense_row_blocks(Sq, nrep);
    const int64_t heads = (int64_t)a.c.Hkv * a.c.B;
    const int ks = prefill_kv_splits(nblk, heads, prefill_keys_needed(a.Skv, Sq, a.causal_off));
    a.kv_splits = ks;
    a.part = ks > 1 ? (float*)(a.vtd + (int64_t)a.s_pad * kPD * heads) : nullptr;
    timer_before_launch(st);
    hipLaunchKernelGGL((prefill_dense_kernel<kDenseQB>), dim3((unsigned)(nblk * heads * ks)), dim3(512), 0, st, a);
    timer_after_launch(st);
    if (ks > 1) {
        const int64_t rows = heads * Sq * nrep;
        hipLaunchKernelGGL(prefill_merge_kernel, dim3((unsigned)((rows * 64 + 255) / 256)), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

// Launch the prefill.  The caller has checked shapes, strides and alignment
// (capi.cpp: fq_prefill_int4 / fq_prefill_int8) and provides a workspace of
// prefill_workspace_bytes (the dense K and V^T of the two-pass path).
hipError_t launch_prefill(const Int4Cache& c, const TailArgs& t, const void* q, const int64_t* q_s, void* out,
                          const int64_t* o_s, int nrep, int Sq, int causal_off, float qk_scale, void* ws,
                          hipStream_t st) {
    PrefillParams a{};
    a.c = c;
    a.t = t;
    a.q = q; a.out = out;
    for (int i = 0; i < 3; ++i) { a.q_s[i] = q_s[i]; a.o_s[i] = o_s[i]; }
    a.nrep = nrep; a.Sq = Sq; a.Skv = c.S + t.len; a.causal_off = causal_off; a.qk_scale = qk_scale;
    const int64_t nblk = prefill_row_blocks(Sq, nrep);
    const dim3 grid((unsigned)(nblk * c.Hkv * c.B));
    const bool bf = c.meta_dtype == FQ_BF16;
    if (prefill_workspace_bytes(c, a.Skv, Sq, nrep, causal_off) > 0) {
        a.s_pad = (int)((prefill_keys_needed(a.Skv, Sq, causal_off) + kDenseKT - 1) / kDenseKT * kDenseKT);
        a.kd = (uint16_t*)ws;
        a.vtd = a.kd + (int64_t)a.s_pad * kPD * c.Hkv * c.B;
        const dim3 dgrid(a.s_pad / kPKT, c.Hkv, c.B);
        if (c.bits == 8) {
            if (bf) hipLaunchKernelGGL((prefill_dequant_kernel<8, FQ_BF16>), dgrid, dim3(512), 0, st, a);
            else hipLaunchKernelGGL((prefill_dequant_kernel<8, FQ_F16>), dgrid, dim3(512), 0, st, a);
        } else {
            if (bf) hipLaunchKernelGGL((prefill_dequant_kernel<4, FQ_BF16>), dgrid, dim3(512), 0, st, a);
            else hipLaunchKernelGGL((prefill_dequant_kernel<4, FQ_F16>), dgrid, dim3(512), 0, st, a);
        }
        return launch_dense_attn(a, Sq, nrep, st);
    }
    timer_before_launch(st);
    if (c.bits == 8) hipLaunchKernelGGL((prefill_attn_kernel<8, FQ_BF16>), grid, dim3(512), 0, st, a);
    else hipLaunchKernelGGL((prefill_attn_kernel<4, FQ_BF16>), grid, dim3(512), 0, st, a);
    timer_after_launch(st);
    return hipGetLastError();
}

size_t prefill_turbo_workspace_bytes(int Hkv, int B, int Skv, int Sq, int nrep, int causal_off) {
    return prefill_dense_bytes(Hkv, B, Skv, Sq, nrep, causal_off);
}

// Prefill over the TurboQuant cache: always the two-pass path (the first pass
// dequantises and rotates back every attended key).
hipError_t launch_prefill_turbo(const fq_turbo_cache& tc, const TailArgs& t, const void* q, const int64_t* q_s,
                                void* out, const int64_t* o_s, int nrep, int Sq, int causal_off, float qk_scale,
                                void* ws, hipStream_t st) {
    PrefillParams a{};
    a.c.B = tc.B; a.c.Hkv = tc.H_kv; a.c.S = tc.S; a.c.D = tc.D; a.c.page = tc.page_size; a.c.G = 1;
    a.c.meta_dtype = FQ_BF16;
    a.t = t;
    a.q = q; a.out = out;
    for (int i = 0; i < 3; ++i) { a.q_s[i] = q_s[i]; a.o_s[i] = o_s[i]; }
    a.nrep = nrep; a.Sq = Sq; a.Skv = tc.S + t.len; a.causal_off = causal_off; a.qk_scale = qk_scale;
    a.s_pad = (int)((prefill_keys_needed(a.Skv, Sq, causal_off) + kDenseKT - 1) / kDenseKT * kDenseKT);
    a.kd = (uint16_t*)ws;
    a.vtd = a.kd + (int64_t)a.s_pad * kPD * tc.H_kv * tc.B;
    TurboPrefill tp{};
    tp.k_msb = tc.k_msb; tp.k_lsb = tc.k_lsb; tp.k_sc = (const uint16_t*)tc.k_scale;
    tp.v_msb = tc.v_msb; tp.v_lsb = tc.v_lsb; tp.v_sc = (const uint16_t*)tc.v_scale;
    for (int i = 0; i < 3; ++i) {   // layer 0: (l, b, h, token) -> (b, h, token)
        tp.kmsb_s[i] = tc.kmsb_strides[i + 1]; tp.klsb_s[i] = tc.klsb_strides[i + 1];
        tp.ksc_s[i] = tc.kst_strides[i + 1];
        tp.vmsb_s[i] = tc.vmsb_strides[i + 1]; tp.vlsb_s[i] = tc.vlsb_strides[i + 1];
        tp.vsc_s[i] = tc.vst_strides[i + 1];
    }
    hipLaunchKernelGGL(prefill_dequant_turbo_kernel, dim3(a.s_pad / kPKT, tc.H_kv, tc.B), dim3(512), 0, st, a, tp);
    return launch_dense_attn(a, Sq, nrep, st);
}

}  // namespace fq
