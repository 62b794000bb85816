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
// Layout: the page loop runs on the matrix cores (attn_turbo_fused_kernel
// below); the wave merge, the inverse rotation of O and the split merge are
// the INT4 kernels' (attn_common.h).
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

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f2v __attribute__((ext_vector_type(2)));

// Everything one page step of a lane reads (lane = (n16 = lane & 15, lg = lane >> 4)):
//   q.k (B operand: token 16T + n16, channels 32 lg .. 32 lg + 31):
//     km[T]: K MSB dword (channel 32 lg + c at bit c), kl[T]: K LSB 8 bytes
//     (channel 32 lg + c at bits 2c, 2c + 1), ks[T]: K scale of the token;
//   p.v (B operand: channels 8 n16 .. 8 n16 + 7 of token 16 T + 4 ai + lg):
//     vm[4T + ai]: V MSB byte, vl[4T + ai]: V LSB half; vs[T]: V scale of token 16T + n16.
struct TurboPage {
    uint32_t km[4];
    uint2 kl[4];
    uint32_t ks[4], vs[4];
    uint32_t vm[16], vl[16];
};

struct TurboRsrc {
    __amdgpu_buffer_rsrc_t km, kl, ks, vm, vl, vs;
    int km_t, kl_t, vm_t, vl_t, ks_t, vs_t;     // token strides in bytes
};

FQ_DEV uint32_t ld8(__amdgpu_buffer_rsrc_t r, int off) { return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0); }

// Per-lane offsets of the page loads (page 0).  Token rows are dense (16-byte
// MSB, 32-byte LSB rows, 2-byte scales), so every other offset of a page is
// an immediate and a page costs one add per plane.
struct TurboLaneOff {
    int km, kl, ks, vm, vl, vs;
};

FQ_DEV void load_turbo_page(TurboPage& b, const TurboRsrc& r, const TurboLaneOff& o, int p) {
    const int km = o.km + p * 64 * 16, kl = o.kl + p * 64 * 32, ks = o.ks + p * 64 * 2;
    const int vm = o.vm + p * 64 * 16, vl = o.vl + p * 64 * 32, vs = o.vs + p * 64 * 2;
#pragma unroll
    for (int T = 0; T < 4; ++T) {
        b.km[T] = ld32(r.km, km + 16 * T * 16);
        b.kl[T] = ld64(r.kl, kl + 16 * T * 32);
        b.ks[T] = ld16(r.ks, ks + 16 * T * 2);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int t = 16 * (i >> 2) + 4 * (i & 3);
        b.vm[i] = ld8(r.vm, vm + t * 16);
        b.vl[i] = ld16(r.vl, vl + t * 32);
    }
#pragma unroll
    for (int T = 0; T < 4; ++T) b.vs[T] = ld16(r.vs, vs + 16 * T * 2);
}

// Both fp16 parts (hi = fp16(x), lo = fp16(x - hi)) of a float.
FQ_DEV void split_f16(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// Sparse decode attention over the TurboQuant cache on the matrix cores.
//
// q.k (v_mfma_f32_16x16x32_f16, 16 tokens x 32 channels per step): A rows
// 4r + {0, 1} hold query head r's fp16 hi / lo parts (q = hi + lo to fp32
// precision), B the codebook values of 8 channels of a token, once as fp16 hi
// and once as fp16 lo parts, looked up two channels at a time from a 64-entry
// LDS table (index lsb d0 | lsb d1 << 2 | msb d0 << 4 | msb d1 << 5); the fp32
// sum of the four products is q . codebook to fp32 precision.  Logit = that
// times the token's K scale (q is pre-scaled by sm_scale * log2 e / sqrt(D)
// after the rotation).
//
// p.v (v_mfma_f32_16x16x32_f16, 32 tokens x 16 channels per step): A = p *
// V_scale / s_run (s_run a running bound of the V scales) as fp16 hi parts in
// rows r (query heads) and lo parts in rows 4 + r; B = the codebook values
// built in registers, byte permutes assembling each token's 3-bit code and
// looking it up in 8-entry tables with v_perm: once their fp16 hi parts, once
// their fp16 lo parts (two matrix instructions per tile and step into one
// accumulator).  Rows r then hold A_hi (c_hi + c_lo), rows 4 + r A_lo (c_hi +
// c_lo), added at the end: each product p * V_scale * codebook to 2^-22
// relative, fp32-level like the reference's fp32 p * v.  Column n16 of
// channel tile j is channel 8 n16 + j.
//
// HCH (FUSED only): head chunks, sel.head_chunks virtual KV heads per cache KV
// head (virtual head h = cache head hk * HC + chunk, NREP query heads each; q,
// outputs and retention follow h, the cache pages and raw metadata hk).
// per_kv_head_sum then scores the summed query of all 2 NREP heads of the
// cache head, so every chunk selects the same pages; the chunks of a cache
// head are mapped to one XCD.
template <int NREP, bool FUSED, bool HCH = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_turbo_fused_kernel(TurboFusedParams a) {
    constexpr int D = 128, NW = 8, NT = 512;
    static_assert(NREP <= 4, "query heads per KV head");
    static_assert(!HCH || FUSED, "head chunks run in the fused kernel");
    __shared__ SplitLds<D, NREP, NW> s_split;
    __shared__ int s_ent[kMaxWgPages];
    // q.k codebook table: entry e (lsb byte of 4 channels | their msb nibble << 8)
    // holds the fp16 hi parts of the 4 channels' codebook values, then the lo parts
    __shared__ uint4 s_lut[4096];
    __shared__ float s_qraw[HCH ? 2 * NREP : NREP][D];      // chunk_sum: every head of the cache head
    __shared__ float s_qrot[NREP][D];
    __shared__ uint8_t s_apv[NW][2][16][4][16];     // p.v A operands per wave: [step][row][k-group, swizzled][16 bytes]

    const fq_turbo_cache& c = a.c;
    const QueryArgs& q = a.q;
    const int gy = blockIdx.y, GY = gridDim.y, split = blockIdx.x;
    const int g = (HCH && gridDim.x == 1 && GY % 8 == 0) ? (gy % 8) * (GY / 8) + gy / 8 : gy;
    const int h = g % c.H_kv, b = (g / c.H_kv) % c.B, l = g / (c.H_kv * c.B);
    const int HC = HCH ? a.sel.head_chunks : 1;
    const int hk = HCH ? h / HC : h;
    const bool chunk_sum = HCH && a.sel.mode == FQ_SELECT_PER_KV_HEAD_SUM;
    const int tid = threadIdx.x, L = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
    const int n16 = L & 15, lg = L >> 4;
    const int S = c.S;

    // q (raw basis): element tid of the group's NREP heads.  Branch-free (two
    // 16-bit loads, the high one masked off for 16-bit q types), so the
    // metadata loads below go out before the first wait.
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
    ScoreRowRegs<NREP, NT> srow;        // kSelectOnly: the group's scores from the scoring launch
    const bool from_scores = FUSED && a.sel.enabled == kSelectOnly;
    const int score_rows = a.sel.mode == FQ_SELECT_PER_KV_HEAD_SUM ? 1 : NREP;
    if constexpr (FUSED) {
        if (chunk_sum)      // uniform: the k of the summed row is the cache head's largest retention
            ret_l = wave_max(a.sel.retention[l * q.ret_ls + hk * 2 * NREP + min(L, 2 * NREP - 1)]);
        else
            ret_l = a.sel.retention[l * q.ret_ls + h * NREP + min(L, NREP - 1)];
        if (from_scores)      // per_kv_head_sum with head chunks: the cache head's one summed row
            scores_load<NREP, NT>(srow, a.ws.scores + (int64_t)(chunk_sum ? g - (h - hk * HC) : g) * NREP * c.P,
                                  score_rows, c.P, tid);
        else score_group_load<bf16, NT>(sr, a.raw, tid, l, b, hk);
    }
    auto q_value = [&](uint32_t lo, uint32_t hi) {
        const uint32_t u = (lo & ~hi_mask) | ((hi << 16) & hi_mask);
        const float fh = f16_bits_to_f(u), fb = bf16_bits_to_f(u);
        return q32 ? __uint_as_float(u) : (q.q_dtype == FQ_BF16 ? fb : fh);
    };
    const float qv_raw = q_value(ql, qh);
    {
        // byte tables of the codebook's fp16 parts for v_perm: [part][low / high byte][codes 0-3 / 4-7]
        uint32_t tb[2][2][2] = {};
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            _Float16 hi, lo;
            split_f16(kTurboCodebookF[v], hi, lo);
            const uint32_t bh = __builtin_bit_cast(uint16_t, hi), bl = __builtin_bit_cast(uint16_t, lo);
            tb[0][0][v >> 2] |= (bh & 0xFFu) << (8 * (v & 3));
            tb[0][1][v >> 2] |= (bh >> 8) << (8 * (v & 3));
            tb[1][0][v >> 2] |= (bl & 0xFFu) << (8 * (v & 3));
            tb[1][1][v >> 2] |= (bl >> 8) << (8 * (v & 3));
        }
        for (int e = tid; e < 4096; e += NT) {
            // byte i of sel: code of channel i = msb bit i << 2 | lsb field i
            const uint32_t lf = (e & 3) | ((e & 0xC) << 6) | ((e & 0x30) << 12) | ((e & 0xC0) << 18);
            const uint32_t mf = ((e >> 8) & 1) | (((e >> 9) & 1) << 8) | (((e >> 10) & 1) << 16) | (((e >> 11) & 1) << 24);
            const uint32_t sel = lf | (mf << 2);
            uint32_t o[4];
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                const uint32_t lo8 = __builtin_amdgcn_perm(tb[part][0][1], tb[part][0][0], sel);
                const uint32_t hi8 = __builtin_amdgcn_perm(tb[part][1][1], tb[part][1][0], sel);
                o[2 * part] = __builtin_amdgcn_perm(hi8, lo8, 0x05010400u);
                o[2 * part + 1] = __builtin_amdgcn_perm(hi8, lo8, 0x07030602u);
            }
            s_lut[e] = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
    if constexpr (HCH) {
        if (tid < q_rows * D) s_qraw[qi >> 7][qi & 127] = qv_raw;
        if (tid + NT < q_rows * D) s_qraw[qi1 >> 7][qi1 & 127] = q_value(ql1, qh1);
    } else if (tid < NREP * D) {
        s_qraw[qi >> 7][qi & 127] = qv_raw;
    }
    __syncthreads();
    // q_rot = WHT(q) / sqrt(D) (Sylvester order), pre-scaled by sm_scale * log2(e);
    // wave r rotates head r (row q_row0 + r of s_qraw)
    if (w < NREP) {
        float v0 = s_qraw[q_row0 + w][L], v1 = s_qraw[q_row0 + w][L + 64];
        wave_hadamard128(v0, v1);
        const float sc = q.qk_scale / sqrtf((float)D);
        s_qrot[w][L] = v0 * sc;
        s_qrot[w][L + 64] = v1 * sc;
    }

    TurboRsrc rs;
    {
        const int64_t bl = l;
        const uint8_t* km = c.k_msb + bl * c.kmsb_strides[0] + b * c.kmsb_strides[1] + hk * c.kmsb_strides[2];
        const uint8_t* kl = c.k_lsb + bl * c.klsb_strides[0] + b * c.klsb_strides[1] + hk * c.klsb_strides[2];
        const uint8_t* vm = c.v_msb + bl * c.vmsb_strides[0] + b * c.vmsb_strides[1] + hk * c.vmsb_strides[2];
        const uint8_t* vl = c.v_lsb + bl * c.vlsb_strides[0] + b * c.vlsb_strides[1] + hk * c.vlsb_strides[2];
        const uint16_t* ks = (const uint16_t*)c.k_scale + bl * c.kst_strides[0] + b * c.kst_strides[1] + hk * c.kst_strides[2];
        const uint16_t* vs = (const uint16_t*)c.v_scale + bl * c.vst_strides[0] + b * c.vst_strides[1] + hk * c.vst_strides[2];
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
    TurboLaneOff loff;
    loff.km = n16 * 16 + 4 * lg;
    loff.kl = n16 * 32 + 8 * lg;
    loff.ks = n16 * 2;
    loff.vm = lg * 16 + n16;
    loff.vl = lg * 32 + 2 * n16;
    loff.vs = n16 * 2;
    auto issue_page = [&](TurboPage& bf, int p) {
        __builtin_amdgcn_sched_barrier(0);
        load_turbo_page(bf, rs, loff, p);
        __builtin_amdgcn_sched_barrier(0);
    };
    TurboPage b0, b1;
    bool first_issued = false;

    int e0, e1, ent_base = 0;          // this split's entries are s_ent[ent_base ..]
    if constexpr (FUSED) {
        // scores (this workgroup's own, or the scoring launch's), then the
        // selection; every split of a group selects the same list and takes
        // the balanced slice [e0, e1) of it
        __shared__ uint32_t s_key[NREP * 64 * kSelC];
        __shared__ BlockSelectLds s_bsel;
        if (from_scores) scores_to_keys<NREP, NT>(srow, s_key, score_rows, c.P, tid);
        else if (chunk_sum) score_group_regs<bf16, HCH ? 2 * NREP : NREP, NT, true>(sr, s_qraw, s_key, tid, c.P);
        else if (a.sel.mode == FQ_SELECT_PER_KV_HEAD_SUM) score_group_regs<bf16, NREP, NT, true>(sr, s_qraw, s_key, tid, c.P);
        else score_group_regs<bf16, NREP, NT, false>(sr, s_qraw, s_key, tid, c.P);
        const ForcedPages fp = forced_pages(c.P, a.sel.num_sinks, a.sel.window);
        if (S > 0 && split == 0 && w < fp.count) {   // split 0's first entries are the forced pages
            issue_page(b0, fp.page(w));
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
        ent_base = e0;
    } else {
        const int n_sel = a.ws.n_sel[g];
        e0 = (int)((int64_t)n_sel * split / a.splits);
        e1 = (int)((int64_t)n_sel * (split + 1) / a.splits);
        for (int i = tid; i < e1 - e0; i += NT) s_ent[i] = a.ws.entries[(int64_t)g * c.P + e0 + i];
        __syncthreads();
    }
    const int n_mine = S > 0 && w < e1 - e0 ? (e1 - e0 - w + NW - 1) / NW : 0;

    // q.k A operands: row n16 = 4 r + part (part 0: hi, 1: lo, 2-3: zero); k-group
    // lg of step kk = channels 32 lg + 4 kk .. + 3 against their codebook hi
    // parts (k 0-3), then the same channels against the lo parts (k 4-7)
    v8h aqk[8];
    {
        const int r = n16 >> 2, part = n16 & 3;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float x = r < NREP ? s_qrot[min(r, NREP - 1)][32 * lg + 4 * kk + i] : 0.f;
                _Float16 hi, lo;
                split_f16(x, hi, lo);
                const _Float16 v = part == 0 ? hi : (part == 1 ? lo : (_Float16)0.f);
                aqk[kk][i] = v;
                aqk[kk][i + 4] = v;
            }
        }
    }
    // the codebook's fp16 hi / lo parts as byte tables for v_perm:
    // [part][low / high byte][codes 0-3 / 4-7]
    uint32_t tbv[2][2][2] = {};
#pragma unroll
    for (int v = 0; v < 8; ++v) {
        _Float16 hi, lo;
        split_f16(kTurboCodebookF[v], hi, lo);
        const uint32_t bh = __builtin_bit_cast(uint16_t, hi), bl = __builtin_bit_cast(uint16_t, lo);
        tbv[0][0][v >> 2] |= (bh & 0xFFu) << (8 * (v & 3));
        tbv[0][1][v >> 2] |= (bh >> 8) << (8 * (v & 3));
        tbv[1][0][v >> 2] |= (bl & 0xFFu) << (8 * (v & 3));
        tbv[1][1][v >> 2] |= (bl >> 8) << (8 * (v & 3));
    }

    auto entry_of = [&](int k) { return __builtin_amdgcn_readfirstlane(s_ent[ent_base + w + NW * k]); };

    float m_run[NREP];
#pragma unroll
    for (int r = 0; r < NREP; ++r) m_run[r] = -INFINITY;
    float s_run = 0.f, inv_s = 1.f;          // running bound of V scales (p * V_scale / s_run <= 1/2)
    float m_lane = 0.f;                      // m_run[lg], or 0 while head lg has no logit yet
    v4f pacc[8];                             // [channel tile]: component r = head r
#pragma unroll
    for (int t = 0; t < 8; ++t) pacc[t] = (v4f){0.f, 0.f, 0.f, 0.f};
    float l_acc = 0.f;
    auto& W = s_apv[w];

    // the idle partner-wave priority rule of the INT4 fused decode: two waves
    // share a SIMD; the one with more pages left (on a tie the younger) takes
    // the higher priority
    __shared__ int s_left[NW];
    auto balance = [&](int k) {
        s_left[w] = n_mine - k;
        const int other = __builtin_amdgcn_readfirstlane(s_left[w ^ 4]);
        if (n_mine - k > other || (n_mine - k == other && w >= 4)) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
    };

    auto compute = [&](const TurboPage& pb, int k) {
        balance(k);
        const int ent = entry_of(k);
        const int p = ent & 0xFFFF, qm = ent >> 16;
        const int tok0 = p * 64;
        // ---- q.k: the four 16-token tiles' accumulation chains interleaved
        // (k-step outer), so four independent matrix instructions are in flight;
        // each tile still accumulates its k-steps in order
        float lg4[4], mp = -INFINITY;
        v4f acc[4];
#pragma unroll
        for (int T = 0; T < 4; ++T) acc[T] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            // the k-step's four table reads go out together, then its four
            // matrix instructions (one read in flight at a time otherwise)
            uint4 e[4];
#pragma unroll
            for (int T = 0; T < 4; ++T) {
                // table entry of channels 32 lg + 4 kk .. + 3: their LSB byte, MSB nibble
                const uint32_t lw = (kk >> 2) ? pb.kl[T].y : pb.kl[T].x;
                const int lsh = 8 * (kk & 3) - 4, msh = 4 * kk - 12;      // entry * 16, in bytes
                const uint32_t a_l = (lsh >= 0 ? lw >> lsh : lw << -lsh) & 0xFF0u;
                const uint32_t a_m = (msh >= 0 ? pb.km[T] >> msh : pb.km[T] << -msh) & 0xF000u;
                e[T] = *(const uint4*)((const char*)s_lut + (a_l | a_m));
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);     // 4 LDS reads
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);     // then 4 matrix instructions
#pragma unroll
            for (int T = 0; T < 4; ++T) {
                const v8h B = __builtin_bit_cast(v8h, (v4i){(int)e[T].x, (int)e[T].y, (int)e[T].z, (int)e[T].w});
                acc[T] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aqk[kk], B, acc[T], 0, 0, 0);
            }
        }
#pragma unroll
        for (int T = 0; T < 4; ++T) {
            const float lgt = (acc[T][0] + acc[T][1]) * bf16_bits_to_f(pb.ks[T] & 0xFFFFu);
            const bool ok = lg < NREP && ((qm >> lg) & 1) && tok0 + 16 * T + n16 < S;
            lg4[T] = ok ? lgt : -INFINITY;
            mp = fmaxf(mp, lg4[T]);
        }
        // ---- page maxima, running references
        float vs_t[4], sp = 0.f;
#pragma unroll
        for (int T = 0; T < 4; ++T) {
            vs_t[T] = bf16_bits_to_f(pb.vs[T] & 0xFFFFu);
            sp = fmaxf(sp, vs_t[T]);
        }
        mp = row16_max(mp);
        sp = lane_value(row16_max(sp), 0);
        bool grow = sp > s_run;
        float mp_r[NREP];
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
            mp_r[r] = lane_value(mp, 16 * r);
            grow |= mp_r[r] > m_run[r];
        }
        if (grow) {      // wave-uniform
            float am[NREP];
#pragma unroll
            for (int r = 0; r < NREP; ++r) {
                const float mn = fmaxf(mp_r[r], m_run[r]);
                am[r] = mn == m_run[r] ? 1.0f : exp2_fast(m_run[r] - mn);
                m_run[r] = mn;
            }
            const float sn = sp > s_run ? 2.0f * sp : s_run;
            const float as = sn > 0.f ? s_run / sn : 1.0f;
            s_run = sn;
            inv_s = sn > 0.f ? 1.0f / sn : 0.f;
            float am_lg = am[0], ml = m_run[0];
#pragma unroll
            for (int r = 1; r < NREP; ++r) {
                am_lg = lg == r ? am[r] : am_lg;
                ml = lg == r ? m_run[r] : ml;
            }
            m_lane = ml == -INFINITY ? 0.f : ml;
            l_acc *= am_lg;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float f = r < NREP ? am[r] * as : 0.f;
#pragma unroll
                for (int t = 0; t < 8; ++t) pacc[t][r] *= f;
            }
        }
        // ---- p.v A: p * V_scale / s_run (fp16); operand k = 8 kg + 2 ai + jj of
        // step s is token 16 (2s + jj) + 4 ai + kg
        float pr[4];
#pragma unroll
        for (int T = 0; T < 4; ++T) {
            pr[T] = exp2_fast(lg4[T] - m_lane);
            l_acc += pr[T];
        }
        if (lg < NREP) {       // rows lg (hi parts) and 4 + lg (lo parts), k-groups swizzled by row
            const int kq = n16 & 3;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const f2v xv = {pr[2 * st] * vs_t[2 * st] * inv_s, pr[2 * st + 1] * vs_t[2 * st + 1] * inv_s};
                const h2v hv = __builtin_convertvector(xv, h2v);
                const h2v lv = __builtin_convertvector(xv - __builtin_convertvector(hv, f2v), h2v);
                *(uint32_t*)&W[st][lg][kq][4 * (n16 >> 2)] = __builtin_bit_cast(uint32_t, hv);
                *(uint32_t*)&W[st][4 + lg][kq ^ 1][4 * (n16 >> 2)] = __builtin_bit_cast(uint32_t, lv);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const int kr = lg ^ ((n16 >> 2) & 3);
        const v8h ap0 = *(const v8h*)&W[0][n16][kr][0];
        const v8h ap1 = *(const v8h*)&W[1][n16][kr][0];
        // ---- p.v B: codes of channel 8 n16 + j for the step's 8 tokens, 4 at a time
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            // per half hh: operand k = 4 hh + kk is token i = 4 (2 st + (kk & 1)) + 2 hh + (kk >> 1);
            // m4: the 4 tokens' MSB bytes, ll / lh: their LSB fields of channels 0-3 / 4-7
            uint32_t m4[2], ll[2], lh[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int i0 = 8 * st + 2 * hh, i1 = i0 + 4, i2 = i0 + 1, i3 = i0 + 5;
                m4[hh] = pb.vm[i0] | (pb.vm[i1] << 8) | (pb.vm[i2] << 16) | (pb.vm[i3] << 24);
                const uint32_t x01 = __builtin_amdgcn_perm(pb.vl[i1], pb.vl[i0], 0x05010400u);
                const uint32_t x23 = __builtin_amdgcn_perm(pb.vl[i3], pb.vl[i2], 0x05010400u);
                ll[hh] = __builtin_amdgcn_perm(x23, x01, 0x05040100u);
                lh[hh] = __builtin_amdgcn_perm(x23, x01, 0x07060302u);
            }
            const v8h a = st ? ap1 : ap0;
            v8h bl_prev;        // tile j - 1's lo-part operand: its matrix instruction follows tile j's
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                uint32_t bw[4], bwl[4];       // channel tile j: codebook hi / lo parts
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const uint32_t lx = j < 4 ? ll[hh] : lh[hh];
                    // byte k: msb bit j of token k at bit 2, its lsb field j below
                    const uint32_t mj = j >= 2 ? m4[hh] >> (j - 2) : m4[hh] << (2 - j);
                    const uint32_t sel = (mj & 0x04040404u) | ((lx >> (2 * (j & 3))) & 0x03030303u);
                    const uint32_t lo = __builtin_amdgcn_perm(tbv[0][0][1], tbv[0][0][0], sel);
                    const uint32_t hi = __builtin_amdgcn_perm(tbv[0][1][1], tbv[0][1][0], sel);
                    bw[2 * hh] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
                    bw[2 * hh + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
                    const uint32_t llo = __builtin_amdgcn_perm(tbv[1][0][1], tbv[1][0][0], sel);
                    const uint32_t lhi = __builtin_amdgcn_perm(tbv[1][1][1], tbv[1][1][0], sel);
                    bwl[2 * hh] = __builtin_amdgcn_perm(lhi, llo, 0x05010400u);
                    bwl[2 * hh + 1] = __builtin_amdgcn_perm(lhi, llo, 0x07030602u);
                }
                const v8h bv = __builtin_bit_cast(v8h, (v4i){(int)bw[0], (int)bw[1], (int)bw[2], (int)bw[3]});
                const v8h bl = __builtin_bit_cast(v8h, (v4i){(int)bwl[0], (int)bwl[1], (int)bwl[2], (int)bwl[3]});
                pacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bv, pacc[j], 0, 0, 0);
                if (j > 0) pacc[j - 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl_prev, pacc[j - 1], 0, 0, 0);
                bl_prev = bl;
            }
            pacc[7] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl_prev, pacc[7], 0, 0, 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    };

    {
        s_left[w] = n_mine;
        if (!first_issued) issue_page(b0, n_mine > 0 ? entry_of(0) & 0xFFFF : 0);
        for (int k = 0; k < n_mine; k += 2) {
            issue_page(b1, entry_of(min(k + 1, n_mine - 1)) & 0xFFFF);
            compute(b0, k);
            issue_page(b0, entry_of(min(k + 2, n_mine - 1)) & 0xFFFF);
            if (k + 1 < n_mine) compute(b1, k + 1);
        }
        __builtin_amdgcn_s_setprio(0);
    }

    // ---- wave state -> LDS: head r's sums in lane group r (over the 16 token
    // columns); outputs of channel 8 n16 + j in lane group 0, component r, plus
    // the lo rows 4 + r in lane group 1
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < NREP; ++r) pacc[j][r] += __shfl_xor(pacc[j][r], 16, 64);
    l_acc = row_sum<16>(l_acc);
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
        const float ll = __shfl(l_acc, 16 * r + n16, 64);
        if (lg == 0) {
#pragma unroll
            for (int j = 0; j < 8; ++j) s_split.acc[w][r][8 * n16 + j] = pacc[j][r] * s_run;
            if (n16 == 0) { s_split.m[w][r] = m_run[r]; s_split.l[w][r] = ll; }
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
        if (FUSED && (N == 3 || N == 4) && a.sel.head_chunks > 1)                                           \
            hipLaunchKernelGGL((attn_turbo_fused_kernel<N, FUSED, FUSED && N >= 3>), grid, dim3(512), 0, st, a); \
        else                                                                                                \
            hipLaunchKernelGGL((attn_turbo_fused_kernel<N, FUSED>), grid, dim3(512), 0, st, a);             \
        timer_after_launch(st);                                                                             \
        if (a.splits > 1)                                                                                   \
            launch_split_merge<N, true>(a.q, a.ws, a.c.H_kv, a.c.B, grid.y, a.splits, TailArgs{}, st);         \
        break;
        FQ_CASE(1) FQ_CASE(2) FQ_CASE(3) FQ_CASE(4)
#undef FQ_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool turbo_fused_supported(const fq_turbo_cache& c, const QueryArgs& q) {
    if (c.D != 128 || c.page_size != 64 || q.nrep > 4 || c.P > kMaxWgPages) return false;
    if (c.kmsb_strides[4] != 1 || c.klsb_strides[4] != 1 || c.vmsb_strides[4] != 1 || c.vlsb_strides[4] != 1)
        return false;
    // dense token rows (16-byte MSB, 32-byte LSB rows, 2-byte scales); K: 4-byte
    // MSB and 8-byte LSB words per lane; V: 2-byte LSB words
    if (c.kmsb_strides[3] != 16 || c.klsb_strides[3] != 32 || c.vmsb_strides[3] != 16 || c.vlsb_strides[3] != 32)
        return false;
    if (c.kst_strides[3] != 1 || c.vst_strides[3] != 1) return false;
    for (int i = 0; i < 3; ++i) {
        if (c.kmsb_strides[i] % 4 || c.klsb_strides[i] % 4 || c.vlsb_strides[i] % 2) return false;
    }
    if ((uintptr_t)c.k_msb & 3) return false;
    if (((uintptr_t)c.k_lsb & 3) || ((uintptr_t)c.v_lsb & 1)) return false;
    if (((uintptr_t)c.k_scale | (uintptr_t)c.v_scale) & 1) return false;
    return true;
}

// Pages from the workspace lists (splits per group chosen like the INT4
// matrix-core kernel); with sel = kScoreSelect and raw, scored and selected in
// the kernel (one workgroup per group); with sel = kSelectOnly, selected in the
// kernel from the scores a scoring launch left in the workspace, each group
// split over workgroups like the INT4 kernel's split steps.
hipError_t launch_attn_turbo_fused(const fq_turbo_cache& c, const Int4Cache* raw, const QueryArgs& q,
                                   const Workspace& ws, int max_entries, const SelectArgs* sel, hipStream_t st) {
    TurboFusedParams a{};
    a.c = c; a.q = q; a.ws = ws;
    const int groups = c.L * c.B * c.H_kv;
    if (sel && sel->enabled == kScoreSelect && raw) {
        a.raw = *raw;
        a.sel = *sel;
        a.splits = 1;
        return launch_turbo_fused_nrep<true>(a, dim3(1, groups), st);
    }
    if (sel && sel->enabled == kSelectOnly) {
        if (c.P > 64 * kSelC) return hipErrorInvalidValue;
        a.sel = *sel;
        int s = (256 + groups - 1) / std::max(groups, 1);
        s = std::min(s, (max_entries + 7) / 8);
        a.splits = std::max(1, std::min(s, ws.s_max));
        return launch_turbo_fused_nrep<true>(a, dim3(a.splits, groups), st);
    }
    int s = groups >= 192 ? 1 : (512 + groups - 1) / groups;
    s = std::min(s, (max_entries + 7) / 8);
    s = std::max(s, (max_entries + kMaxWgPages - 1) / kMaxWgPages);
    a.splits = std::max(1, std::min(s, ws.s_max));
    return launch_turbo_fused_nrep<false>(a, dim3(a.splits, groups), st);
}

}  // namespace fq
