// Split-K sparse GQA decode attention over packed INT4 pages on the gfx950
// matrix cores.  Same semantics as attn_int4.hip
// (src/flashquest/kernel/sparse_int4_fwd.py:23-157); specialised for
// head_dim 128, 64-token pages and up to 4 query heads per KV head.
//
// Why MFMA on a memory-bound GEMV: with 3 query heads per KV head every INT4
// code feeds 3 multiply-adds for q.k and 3 for p.v, which is more fp32 VALU
// work per byte than the CU can issue at HBM speed.  The codes go to the matrix
// core unchanged apart from a nibble mask:
//   q.k : v_mfma_i32_16x16x64_i8.  A = q_d * K_scale[p,d] as an exact 24-bit
//         fixed-point number per page (3 balanced int8 digits in rows
//         4r+digit, r = query head), B = the codes; plus sum_d q_d * K_mn[p,d].
//         int32 accumulation is exact, so the only rounding is 2^-23 of max|A|.
//   p.v : v_mfma_f32_16x16x32_f16.  A = p_t * V_scale[t,g] (rows 4g+r, g = V
//         channel group) split into fp16 parts hi = fp16(A), lo = fp16(A - hi)
//         (per-token V metadata: lo in the free rows 4 + r of the same operand,
//         added at the end; grouped: a second operand), both multiplied by the same B = the codes as fp16 subnormals (bits =
//         code, value = code * 2^-24, exact) into one fp32 accumulator; plus
//         sum_t p_t * V_mn[t,g] on the VALU.  hi + lo equals the fp32 A to
//         2^-22 relative (the lo part's own fp16 rounding), so the products
//         carry fp32-level precision like the reference's fp32 p * v.
//
// Single pass per page: each wave owns every 4th page of its workgroup's
// split, loads a page (K, V, metadata) one page ahead of the one it computes,
// and accumulates against a running softmax maximum m[r] (log2 domain),
// rescaling when a page raises it.  With bf16 metadata A is also divided by a
// running V-scale bound sigma[g] so that it stays in fp16 range.  The wave
// states merge like the VALU kernel's, and splits meet in merge_splits_kernel.
#include <algorithm>
#include <type_traits>

#include "attn_common.h"
#include "fused_common.h"

namespace fq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float f2v __attribute__((ext_vector_type(2)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

constexpr float kQkScale = 8323071.0f;      // 2^23 - 2^16 - 1: |X| <= this keeps 3 balanced digits in int8
constexpr float kSubnormal = 16777216.0f;   // 2^24: fp16 subnormal with bits c has value c * 2^-24

struct MfmaParams {
    Int4Cache c;
    QueryArgs q;
    Workspace ws;
    int splits;
    SelectArgs sel;         // sel.enabled: every workgroup scores and selects its group's pages itself
    TailArgs tail;          // tail.len > 0: the tail is attended (in_kernel: by the fused kernel, else the split merge)
};

// A operands of one wave: [k-step][row][k-group, XOR-swizzled][16 bytes].
// The k-group of row R is stored at position kg ^ ((R >> 2) & 3), which makes
// the 16-byte operand reads (row = lane & 15, k-group = lane >> 4) conflict-free.
struct WaveLds {
    uint8_t aqk[2][16][4][16];      // q.k: int8 digits, rows 4r + digit
    uint8_t apv[2][16][4][16];      // p.v: fp16 hi parts, rows 4g + r (8 halves per k-group)
    uint8_t apl[2][16][4][16];      // p.v: fp16 lo parts, same layout
};
FQ_DEV int swz(int row, int kg) { return kg ^ ((row >> 2) & 3); }

FQ_DEV uint32_t lo_nib(uint32_t w) { return w & 0x0F0F0F0Fu; }
FQ_DEV uint32_t hi_nib(uint32_t w) { return (w >> 4) & 0x0F0F0F0Fu; }

// Balanced base-256 digits: Y = X + 128 * (1 + 256 + ...) >= 0, and digit i of X
// is byte i of Y minus 128 (as int8: byte ^ 0x80), so sum_i 256^i (b_i - 128) = X.
// byte_i(y0..y3): byte i of four values packed into one dword (byte 0 from y0).
template <int I>
FQ_DEV uint32_t byte_i(uint32_t y0, uint32_t y1, uint32_t y2, uint32_t y3) {
    constexpr uint32_t lo = 0x0C0C0000u | ((4u + I) << 8) | I;          // y0.bI, y1.bI, 0, 0
    constexpr uint32_t hi = ((4u + I) << 24) | ((uint32_t)I << 16) | 0x0C0Cu;  // 0, 0, y2.bI, y3.bI
    return __builtin_amdgcn_perm(y1, y0, lo) | __builtin_amdgcn_perm(y3, y2, hi);
}
constexpr uint32_t kDigitFlip = 0x80808080u;

FQ_DEV void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// Raw V metadata of one token: G halves (G = 4: 8 bytes, G = 1: 2 bytes).
struct VMetaRaw { uint2 v; };

template <typename MT, int G>
FQ_DEV void unpack_vmeta(const VMetaRaw& r, float (&out)[G]) {
    out[0] = half_to_f<MT>(r.v.x);
    if constexpr (G == 4) {
        out[1] = half_to_f<MT>(r.v.x >> 16);
        out[2] = half_to_f<MT>(r.v.y);
        out[3] = half_to_f<MT>(r.v.y >> 16);
    }
}

// Page data is read with buffer loads.  Each tensor slice (l, b, h) gets one
// buffer resource whose size is the slice's S tokens, so rows past S of a
// partial last page read as zero instead of faulting; every per-lane offset is
// (lane part) + (page part) + an immediate, the same for every page.
struct SliceRsrc {
    __amdgpu_buffer_rsrc_t k, v, vs, vm, ks, km;
};

// Raw V metadata of tokens 16T + n16 (T = 0..3); off = byte offset of token n16.
template <int G>
FQ_DEV void load_vmeta(VMetaRaw (&m)[4], __amdgpu_buffer_rsrc_t r, int off) {
#pragma unroll
    for (int T = 0; T < 4; ++T) {
        if constexpr (G == 4) m[T].v = ld64(r, off + T * 16 * 8);
        else m[T].v = make_uint2(ld16(r, off + T * 16 * 2), 0u);
    }
}

// Everything one page step reads.
struct PageBuf {
    uint4 kt[4];            // K codes: token 16T + n16, bytes 16*lg .. +15
    uint4 sv, mv;           // K scale / min: channels ch_base .. +7
    uint32_t vw[16];        // V codes: token 16*(j&3) + 4*(j>>2) + lg, channels 8*n16 .. +7
    VMetaRaw vs[4], vm[4];  // V scale / min of tokens 16T + n16
};

// koff: (token n16, byte 16*lg); voff: (token lg, byte 4*n16); moff: token n16's V
// metadata; soff: K scale / min channel ch_base.  All include the page part.
template <int G>
FQ_DEV void load_page(PageBuf& b, const SliceRsrc& r, int koff, int voff, int moff, int soff) {
#pragma unroll
    for (int T = 0; T < 4; ++T) b.kt[T] = ld128(r.k, koff + T * 16 * 64);
    b.sv = ld128(r.ks, soff);
    b.mv = ld128(r.km, soff);
#pragma unroll
    for (int j = 0; j < 16; ++j) b.vw[j] = ld32(r.v, voff + (16 * (j & 3) + 4 * (j >> 2)) * 64);
    load_vmeta<G>(b.vs, r.vs, moff);
    load_vmeta<G>(b.vm, r.vm, moff);
}

// NW waves per workgroup (4, or 8 when one workgroup takes a whole KV group).
// FUSED (8 waves only): the workgroup scores and selects its group's pages
// itself (a.sel) and attends split `split` of the list; otherwise the pages
// come from the workspace lists.
//
// HCH (FUSED only): head chunks, sel.head_chunks virtual KV heads per cache
// KV head (a separate instantiation, so the other kernels are unchanged).
template <typename MT, int G, int NREP, int NW, bool FUSED, bool HCH = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_int4_mfma_kernel(MfmaParams a) {
    static_assert(!FUSED || NW == 8, "in-kernel selection runs in the 8-wave kernel");
    static_assert(!HCH || FUSED, "head chunks run in the fused kernel");
    constexpr int D = 128;
    constexpr int NT = 64 * NW;
    constexpr int NSLOT = FUSED ? NW + 1 : NW;      // the fused kernel's extra slot: the partial-page tail
    constexpr int TTOK = FUSED ? kTailMax : 1;
    __shared__ SplitLds<D, NREP, NSLOT> s_split;
    __shared__ WaveLds s_wave[NW];
    __shared__ int s_ent[kMaxWgPages];

    const Int4Cache& c = a.c;
    const QueryArgs& q = a.q;
    // the group of this workgroup: workgroups go to the XCDs round-robin by
    // index, so index i takes group (i % 8) * (G / 8) + i / 8, giving every
    // XCD a mix of KV heads and layers instead of one KV head of every layer
    const int gy = blockIdx.y, GY = gridDim.y;
    const int g = (gridDim.x == 1 && GY % 8 == 0) ? (gy % 8) * (GY / 8) + gy / 8 : gy;
    const int split = blockIdx.x;
    const int h = g % c.Hkv, b = (g / c.Hkv) % c.B, l = g / (c.Hkv * c.B);
    // Head chunks (FUSED, sel.head_chunks = HC > 1): the launch sees HC
    // virtual KV heads per KV head of the cache, each with NREP of its query
    // heads (virtual head h = cache head hk * HC + chunk); q, the outputs and
    // the retention follow h, the cache pages follow hk.  per_kv_head_sum
    // (chunk_sum) then scores the summed query of all HC * NREP heads of the
    // cache head, so every chunk selects the same pages.
    const int HC = HCH ? a.sel.head_chunks : 1;
    const int hk = HCH ? h / HC : h;
    const bool chunk_sum = HCH && a.sel.mode == FQ_SELECT_PER_KV_HEAD_SUM;
    const int L = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
    const int n16 = L & 15, lg = L >> 4;
    WaveLds& W = s_wave[w];
    const int S = c.S;

    // Prologue: q (as prescaled fp32) and this split's page entries go to LDS.
    // Every load is unconditional (clamped index), so all are in flight before
    // the first wait.  The entries either come from the workspace (written by a
    // selection kernel) or, with sel.enabled, the workgroup scores its group's
    // pages and wave 0 selects them.
    constexpr int kEntPer = kMaxWgPages / NT;
    static_assert(kMaxWgPages % NT == 0 && NREP * D <= 2 * NT, "prologue sizes");
    static_assert(!FUSED || 2 * NREP * D <= 2 * NT, "chunk_sum prologue sizes");
    __shared__ float s_q[NREP][D];
    const int tid = threadIdx.x;
    // chunk_sum: the prologue loads all 2 NREP heads of the cache head (rows
    // chunk * NREP .. are this workgroup's own)
    const int q_rows = chunk_sum ? 2 * NREP : NREP;
    const int q_row0 = chunk_sum ? (h - hk * HC) * NREP : 0;
    const int64_t qb = l * q.q_s[0] + b * q.q_s[1] + (int64_t)(chunk_sum ? hk * 2 * NREP : h * NREP) * q.q_s[2];
    const int i0 = min(tid, q_rows * D - 1), i1 = min(tid + NT, q_rows * D - 1);
    // q (raw bits) and the retention go out first, then, in the fused decode,
    // the group's K metadata loads for scoring: loads complete in order, so q
    // can be used while the metadata is still in flight.
    // Branch-free, so the compiler can count the loads still in flight: two
    // 16-bit loads per element, both always used (the high one re-reads the
    // low one for 16-bit q types and is masked off).
    const bool q32 = q.q_dtype == FQ_F32;
    const int esz = q32 ? 4 : 2;
    uint32_t hi_mask = (0u - (uint32_t)q32) & 0xFFFF0000u;
    asm volatile("" : "+s"(hi_mask));       // opaque: both loads stay unconditional
    uint32_t l0, h0, l1, h1;
    {
        const char* qc = (const char*)q.q;
        const int64_t o0 = (qb + (i0 >> 7) * q.q_s[2] + (i0 & 127) * q.q_s[3]) * esz;
        const int64_t o1 = (qb + (i1 >> 7) * q.q_s[2] + (i1 & 127) * q.q_s[3]) * esz;
        l0 = *(const uint16_t*)(qc + o0);
        h0 = *(const uint16_t*)(qc + o0 + esz - 2);
        l1 = *(const uint16_t*)(qc + o1);
        h1 = *(const uint16_t*)(qc + o1 + esz - 2);
    }
    // Scoring's q in registers: channels 8 * (tid & 15) .. + 7 of every query
    // head of the group, one 16-byte load per head, so that each wave scores
    // its pages as its own loads land, with no barrier on the other waves' q.
    // Needs 16-bit q with unit channel stride and 16-byte aligned rows; other
    // layouts (q_fast false: an empty buffer, the loads read 0) go through LDS.
    uint4 qsr[NREP];
    const bool q_fast = FUSED && !chunk_sum && !q32 && !q.rot && q.q_s[3] == 1 && (q.q_s[2] & 7) == 0 &&
                        (((uintptr_t)q.q + 2 * (uint64_t)qb) & 15) == 0;
    if constexpr (FUSED) {
        const auto rq = make_rsrc((const char*)q.q + 2 * qb, q_fast ? 2 * ((int64_t)(NREP - 1) * q.q_s[2] + D) : 0);
#pragma unroll
        for (int r = 0; r < NREP; ++r) qsr[r] = ld128(rq, (int)(2 * (r * q.q_s[2] + 8 * (tid & 15))));
    }
    // Rotation signs (rotated decode), loaded with q: loads complete in
    // order, so one issued after the metadata loads would wait for all of them
    // and the scoring could not overlap the metadata's arrival.
    uint32_t rsg0 = 0u, rsg1 = 0u;
    if constexpr (FUSED) {
        const auto rr = make_rsrc(q.rot, q.rot && D == 128 ? 4 * D : 0);
        rsg0 = ld32(rr, 4 * L);
        rsg1 = ld32(rr, 4 * (L + 64));
    }
    __builtin_amdgcn_sched_barrier(0);      // q's loads go out before the metadata loads
    // retention of query head L of the group (lanes past NREP repeat the last)
    float ret_l = 0.f;
    ScoreRegs<NT> sr;
    ScoreRowRegs<NREP, NT> srow;        // kSelectOnly: the group's precomputed scores
    const bool from_scores = FUSED && a.sel.enabled == kSelectOnly;
    const int score_rows = a.sel.mode == FQ_SELECT_PER_KV_HEAD_SUM ? 1 : NREP;
    // Partial-page tail (fused kernel, tail.in_kernel): its <= 64 raw 16-bit
    // K / V rows go to LDS with q, before scoring needs the metadata.  The
    // loads are unconditional: without a tail the buffer is empty and they read 0.
    __shared__ uint16_t s_tk[TTOK][D], s_tv[TTOK][D];
    __shared__ float s_tp[NREP][TTOK];
    uint4 tkr[2], tvr[2];
    const int tail_T = FUSED && a.tail.in_kernel && split == 0 ? a.tail.len : 0;   // split 0 of a group attends it
    if constexpr (FUSED) {
        if (chunk_sum)      // uniform: the k of the summed row is the cache head's largest retention
            ret_l = wave_max(a.sel.retention[l * q.ret_ls + hk * 2 * NREP + min(L, 2 * NREP - 1)]);
        else
            ret_l = a.sel.retention[l * q.ret_ls + h * NREP + min(L, NREP - 1)];
        const TailArgs& t = a.tail;
        const char* tkb = tail_T > 0 ? (const char*)t.k + 2 * (l * t.ks[0] + b * t.ks[1] + hk * t.ks[2]) : nullptr;
        const char* tvb = tail_T > 0 ? (const char*)t.v + 2 * (l * t.vs[0] + b * t.vs[1] + hk * t.vs[2]) : nullptr;
        const auto rk = make_rsrc(tkb, tail_T > 0 ? 2 * (int64_t)(tail_T - 1) * t.ks[3] + 2 * D : 0);
        const auto rv = make_rsrc(tvb, tail_T > 0 ? 2 * (int64_t)(tail_T - 1) * t.vs[3] + 2 * D : 0);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int i = tid + NT * u, tt = i >> 4, j = i & 15;       // token tt, bytes 16j .. 16j+15
            tkr[u] = ld128(rk, (int)(2 * tt * t.ks[3]) + 16 * j);
            tvr[u] = ld128(rv, (int)(2 * tt * t.vs[3]) + 16 * j);
        }
        if (from_scores)      // per_kv_head_sum with head chunks: the cache head's one summed row
            scores_load<NREP, NT>(srow, a.ws.scores + (int64_t)(chunk_sum ? g - (h - hk * HC) : g) * NREP * c.P,
                                  score_rows, c.P, tid);
        else score_group_load<MT, NT>(sr, c, tid, l, b, hk);
    }
    const bool qbf = q.q_dtype == FQ_BF16;
    auto q_float = [&](uint32_t u) {
        const float fh = f16_bits_to_f(u), fb = bf16_bits_to_f(u);
        return q32 ? __uint_as_float(u) : (qbf ? fb : fh);
    };
    const float v0 = q_float((l0 & ~hi_mask) | ((h0 << 16) & hi_mask));
    const float v1 = q_float((l1 & ~hi_mask) | ((h1 << 16) & hi_mask));

    const uint8_t* kb = c.kp + l * c.kp_s[0] + b * c.kp_s[1] + hk * c.kp_s[2];
    const uint8_t* vb = c.vp + l * c.vp_s[0] + b * c.vp_s[1] + hk * c.vp_s[2];
    const MT* ksc = (const MT*)c.ksc + l * c.ksc_s[0] + b * c.ksc_s[1] + hk * c.ksc_s[2];
    const MT* kmn = (const MT*)c.kmn + l * c.kmn_s[0] + b * c.kmn_s[1] + hk * c.kmn_s[2];
    const uint16_t* vsc = (const uint16_t*)c.vsc + l * c.vsc_s[0] + b * c.vsc_s[1] + hk * c.vsc_s[2];
    const uint16_t* vmn = (const uint16_t*)c.vmn + l * c.vmn_s[0] + b * c.vmn_s[1] + hk * c.vmn_s[2];

    // A-operand slot of this lane for the q.k digits: k-step qs_s, k-group qs_kg,
    // operand dword qs_jd; channels ch_base + 2b + par (b = 0..3); heads r0, r0+1.
    const int Dq = L & 31, qs_s = Dq >> 4, qs_kg = (Dq >> 2) & 3, qs_jd = Dq & 3;
    const int ch_base = 32 * qs_kg + 16 * qs_s + 8 * (qs_jd >> 1);
    const int par = qs_jd & 1;
    const int r0 = 2 * (L >> 5);

    SliceRsrc rs;
    rs.k = make_rsrc(kb, (int64_t)S * 64);
    rs.v = make_rsrc(vb, (int64_t)S * 64);
    rs.vs = make_rsrc(vsc, (int64_t)S * G * 2);
    rs.vm = make_rsrc(vmn, (int64_t)S * G * 2);
    rs.ks = make_rsrc(ksc, (int64_t)c.P * D * 2);
    rs.km = make_rsrc(kmn, (int64_t)c.P * D * 2);
    const int koff0 = n16 * 64 + 16 * lg, voff0 = lg * 64 + 4 * n16, moff0 = n16 * G * 2, soff0 = ch_base * 2;
    auto issue_page = [&](PageBuf& bf, int p) {
        // keep the scheduler from moving compute work in front of the loads
        __builtin_amdgcn_sched_barrier(0);
        load_page<G>(bf, rs, koff0 + p * 4096, voff0 + p * 4096, moff0 + p * 64 * G * 2, soff0 + p * D * 2);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Page buffers: one page in flight ahead of the one being computed.
    PageBuf b0, b1;
    bool first_issued = false;       // b0 already holds this wave's first page

    int e0, e1, ent_base = 0;          // this split's entries are s_ent[ent_base ..]
    if constexpr (FUSED) {
        // Fused decode: score every page of the group from its K metadata
        // (the arithmetic of score_kernel), keep the scores in LDS, select.
        // The forced pages (always selected, first in the entry list) are
        // loaded while the selection runs.
        __shared__ float s_qraw[HCH ? 2 * NREP : NREP][D];      // chunk_sum: every head of the cache head
        __shared__ uint32_t s_key[NREP * 64 * kSelC];
        __shared__ BlockSelectLds s_bsel;
        e0 = 0;
        {
            if (tid < q_rows * D) {
                if constexpr (HCH) {
                    const int r = (i0 >> 7) - q_row0;
                    if ((unsigned)r < (unsigned)NREP) s_q[r][i0 & 127] = v0 * q.qk_scale;
                } else {
                    s_q[i0 >> 7][i0 & 127] = v0 * q.qk_scale;
                }
                s_qraw[i0 >> 7][i0 & 127] = v0;
            }
            if (tid + NT < q_rows * D) {
                if constexpr (HCH) {
                    const int r = (i1 >> 7) - q_row0;
                    if ((unsigned)r < (unsigned)NREP) s_q[r][i1 & 127] = v1 * q.qk_scale;
                } else {
                    s_q[i1 >> 7][i1 & 127] = v1 * q.qk_scale;
                }
                s_qraw[i1 >> 7][i1 & 127] = v1;
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int i = tid + NT * u;
                *(uint4*)&s_tk[i >> 4][8 * (i & 15)] = tkr[u];
                *(uint4*)&s_tv[i >> 4][8 * (i & 15)] = tvr[u];
            }
            const bool sum = a.sel.mode == FQ_SELECT_PER_KV_HEAD_SUM;
            if (from_scores) {     // uniform: a scoring launch wrote the group's scores (never with q.rot)
                scores_to_keys<NREP, NT>(srow, s_key, score_rows, c.P, tid);
            } else if (q_fast) {      // uniform
                float qin[NREP][8];
#pragma unroll
                for (int r = 0; r < NREP; ++r) {
                    const uint32_t wv[4] = {qsr[r].x, qsr[r].y, qsr[r].z, qsr[r].w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        qin[r][2 * j] = qbf ? bf16_bits_to_f(wv[j] & 0xFFFFu) : f16_bits_to_f(wv[j] & 0xFFFFu);
                        qin[r][2 * j + 1] = qbf ? bf16_bits_to_f(wv[j] >> 16) : f16_bits_to_f(wv[j] >> 16);
                    }
                }
                if (sum) score_group_regs_q<MT, NREP, NT, true>(sr, qin, s_key, tid, c.P);
                else score_group_regs_q<MT, NREP, NT, false>(sr, qin, s_key, tid, c.P);
            } else {
                __syncthreads();
                if (q.rot) {       // uniform: wave r rotates head r, q -> WHT(s q) / sqrt(D), in fp32
                    if (w < NREP) {
                        float x0 = s_qraw[w][L] * __uint_as_float(rsg0), x1 = s_qraw[w][L + 64] * __uint_as_float(rsg1);
                        wave_hadamard128(x0, x1);
                        const float inv = 1.0f / sqrtf((float)D);
                        x0 *= inv;
                        x1 *= inv;
                        s_qraw[w][L] = x0;
                        s_qraw[w][L + 64] = x1;
                        s_q[w][L] = x0 * q.qk_scale;
                        s_q[w][L + 64] = x1 * q.qk_scale;
                    }
                    __syncthreads();
                }
                if constexpr (HCH) {
                    if (chunk_sum) score_group_sum_lds<MT, 2 * NREP, NT>(sr, s_qraw, s_key, tid, c.P);
                    else score_group_regs<MT, NREP, NT, false>(sr, s_qraw, s_key, tid, c.P);
                } else if (sum) score_group_regs<MT, NREP, NT, true>(sr, s_qraw, s_key, tid, c.P);
                else score_group_regs<MT, NREP, NT, false>(sr, s_qraw, s_key, tid, c.P);
            }
            const ForcedPages fp = forced_pages(c.P, a.sel.num_sinks, a.sel.window);
            if (S > 0 && split == 0 && w < fp.count) {       // split 0's first entries are the forced pages
                issue_page(b0, fp.page(w));
                first_issued = true;
            }
            lds_barrier();      // the keys; the forced pages stay in flight through the selection
            // every split of the group selects the same list; split s takes
            // the balanced slice [e0, e1) of it
            const int total = block_select_group<kSelC, NW, NREP>(s_key, c.P, a.sel.mode, ret_l, a.sel.k_max,
                                                                  a.sel.num_sinks, a.sel.window, s_ent, s_bsel);
            if (a.sel.mask_out && split == 0)        // uniform: the caller asked for the selection
                block_write_mask<NT, NREP>(s_ent, total, c.P, (uint8_t*)s_key,
                                           a.sel.mask_out + (int64_t)g * NREP * c.P, tid);
            e0 = (int)((int64_t)total * split / a.splits);
            e1 = (int)((int64_t)total * (split + 1) / a.splits);
            ent_base = e0;
        }
    } else {
        const int n_sel = a.ws.n_sel[g];
        e0 = (int)((int64_t)n_sel * split / a.splits);           // balanced split: entries [e0, e1)
        e1 = (int)((int64_t)n_sel * (split + 1) / a.splits);
        int ent[kEntPer];
#pragma unroll
        for (int u = 0; u < kEntPer; ++u) ent[u] = a.ws.entries[(int64_t)g * c.P + min(e0 + tid + u * NT, c.P - 1)];
#pragma unroll
        for (int u = 0; u < kEntPer; ++u)
            if (tid + u * NT < e1 - e0) s_ent[tid + u * NT] = ent[u];
        if (tid < NREP * D) s_q[i0 >> 7][i0 & 127] = v0 * q.qk_scale;
        if (tid + NT < NREP * D) s_q[i1 >> 7][i1 & 127] = v1 * q.qk_scale;
        __syncthreads();
    }
    // Wave w takes entries w, w + NW, ... (a fixed assignment, so the fp32
    // accumulation order, and the result, do not depend on timing).
    const int n_mine = S > 0 && w < e1 - e0 ? (e1 - e0 - w + NW - 1) / NW : 0;   // pages w, w + NW, ...

    float qv[2][4];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) qv[hh][bb] = r0 + hh < NREP ? s_q[min(r0 + hh, NREP - 1)][ch_base + 2 * bb + par] : 0.f;

    // k: this wave's k-th page (entry w + NW * k); callers clamp k to the last
    // page, so every step issues the same loads and the waits match on every path
    auto entry_of = [&](int k) { return __builtin_amdgcn_readfirstlane(s_ent[ent_base + w + NW * k]); };
    // past the wave's last page: kNoPage (loads out of range, no memory traffic)
    auto issue = [&](PageBuf& bf, int k) { issue_page(bf, k < n_mine ? entry_of(k) & 0xFFFF : kNoPage); };

    // running references (wave-uniform) and accumulators.  With fp16 metadata
    // p * V_scale <= 65504 needs no bound; bf16 metadata is divided by s_run.
    constexpr bool kBound = std::is_same<MT, bf16>::value;
    float m_run[NREP], s_run[G], inv_s[G];
#pragma unroll
    for (int r = 0; r < NREP; ++r) m_run[r] = -INFINITY;
#pragma unroll
    for (int gv = 0; gv < G; ++gv) { s_run[gv] = kBound ? 0.f : 1.f; inv_s[gv] = 1.f; }
    float m_lane = 0.f;                      // m_run[lg], or 0 while head lg has no logit yet
    v4f pacc[8];                             // [tile]: component r = head, lane group lg = V group
#pragma unroll
    for (int t = 0; t < 8; ++t) pacc[t] = (v4f){0.f, 0.f, 0.f, 0.f};
    float l_acc = 0.f, bias[G];              // head lg: sum p, sum p * V_mn[g] over this lane's tokens
#pragma unroll
    for (int gv = 0; gv < G; ++gv) bias[gv] = 0.f;

    // With 8 waves two share a SIMD (waves w and w ^ 4) and the issue arbiter
    // favours the older one, which would leave the younger wave's pages to
    // run alone at the end.  Each wave publishes its remaining page count and
    // takes the higher priority while it has more left than its partner, or as
    // many and it is the younger of the two (with the older one winning ties,
    // the pair ended one page apart: ~0.9 us of a config-1 step).  The
    // priority changes only timing, never which wave computes which page.
    __shared__ int s_left[NW];
    auto balance = [&](int k) {
        if constexpr (NW == 8) {
            s_left[w] = n_mine - k;
            const int other = __builtin_amdgcn_readfirstlane(s_left[w ^ 4]);
            if (n_mine - k > other || (n_mine - k == other && w >= 4)) __builtin_amdgcn_s_setprio(1);
            else __builtin_amdgcn_s_setprio(0);
        }
    };
    auto compute = [&](const PageBuf& cb, int k) {
        balance(k);
        const int ent = entry_of(k);
        const int p = ent & 0xFFFF, qm = ent >> 16;
        const int tok0 = p * 64;

        // ---- q.k: digits of q * K_scale, then 2 MFMAs per 16-token tile
        const uint32_t sw[4] = {cb.sv.x, cb.sv.y, cb.sv.z, cb.sv.w};
        const uint32_t mw[4] = {cb.mv.x, cb.mv.y, cb.mv.z, cb.mv.w};
        float A[2][4], cpart[2] = {0.f, 0.f}, amax = 0.f;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
            const float sf = half_to_f<MT>(par ? sw[bb] >> 16 : sw[bb]);
            const float mf = half_to_f<MT>(par ? mw[bb] >> 16 : mw[bb]);
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                A[hh][bb] = qv[hh][bb] * sf;
                cpart[hh] = fmaf(qv[hh][bb], mf, cpart[hh]);
                amax = fmaxf(amax, fabsf(A[hh][bb]));
            }
        }
        const float sigma = wave_max(amax);
        const float inv = sigma > 0.f ? kQkScale * __builtin_amdgcn_rcpf(sigma) : 0.f;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            if (r0 + hh < NREP) {
                // Y = round(A * inv) + 0x808080, rounded by the fp32 add itself
                uint32_t Y[4];
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) Y[bb] = (uint32_t)fmaf(A[hh][bb], inv, 8421504.0f);
                const int row = 4 * (r0 + hh);
                uint32_t* dst = (uint32_t*)&W.aqk[qs_s][row][swz(row, qs_kg)][4 * qs_jd];
                dst[0] = byte_i<2>(Y[0], Y[1], Y[2], Y[3]) ^ kDigitFlip;           // row 4r: weight 65536
                dst[64 / 4] = byte_i<1>(Y[0], Y[1], Y[2], Y[3]) ^ kDigitFlip;      // row 4r+1: 256
                dst[128 / 4] = byte_i<0>(Y[0], Y[1], Y[2], Y[3]) ^ kDigitFlip;     // row 4r+2: 1
            }
            float cs = cpart[hh];            // sum over the 32 lanes of this half (heads r0 + hh)
            cs += __shfl_xor(cs, 16, 64);
            cpart[hh] = row_sum<16>(cs);
        }
        // C for head lg lives in half lg >> 1, index lg & 1
        const float c0 = __shfl(cpart[0], (lg >> 1) * 32, 64);
        const float c1 = __shfl(cpart[1], (lg >> 1) * 32, 64);
        const float Cr = (lg & 1) ? c1 : c0;
        const float unscale = sigma * (1.0f / kQkScale);
        wave_lds_fence();
        const v4i a0 = *(const v4i*)&W.aqk[0][n16][swz(n16, lg)][0];
        const v4i a1 = *(const v4i*)&W.aqk[1][n16][swz(n16, lg)][0];
        float lg4[4], mp = -INFINITY;
#pragma unroll
        for (int T = 0; T < 4; ++T) {
            const uint4 kt = cb.kt[T];
            const v4i b0 = {(int)lo_nib(kt.x), (int)hi_nib(kt.x), (int)lo_nib(kt.y), (int)hi_nib(kt.y)};
            const v4i b1 = {(int)lo_nib(kt.z), (int)hi_nib(kt.z), (int)lo_nib(kt.w), (int)hi_nib(kt.w)};
            v4i acc = {0, 0, 0, 0};
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc, 0, 0, 0);
            const float f = fmaf((float)acc[0], 65536.f, fmaf((float)acc[1], 256.f, (float)acc[2]));
            const float lgt = fmaf(f, unscale, Cr);
            const bool ok = lg < NREP && ((qm >> lg) & 1) && tok0 + 16 * T + n16 < S;
            lg4[T] = ok ? lgt : -INFINITY;
            mp = fmaxf(mp, lg4[T]);
        }

        // ---- page maxima: logits per head (row lg), V scale per group (row lg reduces group lg)
        float vs_t[4][G], vm_t[4][G];
#pragma unroll
        for (int T = 0; T < 4; ++T) {
            unpack_vmeta<MT, G>(cb.vs[T], vs_t[T]);
            unpack_vmeta<MT, G>(cb.vm[T], vm_t[T]);
        }
        mp = row16_max(mp);
        bool grow = false;
        float mp_r[NREP], sp_g[G];
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
            mp_r[r] = lane_value(mp, 16 * r);
            grow |= mp_r[r] > m_run[r];
        }
        if constexpr (kBound) {
            float sp = 0.f;
#pragma unroll
            for (int T = 0; T < 4; ++T) {
                float v = vs_t[T][0];
#pragma unroll
                for (int gv = 1; gv < G; ++gv) v = lg == gv ? vs_t[T][gv] : v;
                sp = fmaxf(sp, v);
            }
            sp = row16_max(sp);
#pragma unroll
            for (int gv = 0; gv < G; ++gv) {
                sp_g[gv] = lane_value(sp, 16 * gv);
                grow |= sp_g[gv] > s_run[gv];
            }
        }
        if (grow) {      // wave-uniform: raise the references, rescale what is accumulated
            float am[NREP], as[G];
#pragma unroll
            for (int r = 0; r < NREP; ++r) {
                const float mn = fmaxf(mp_r[r], m_run[r]);
                am[r] = mn == m_run[r] ? 1.0f : exp2_fast(m_run[r] - mn);
                m_run[r] = mn;
            }
#pragma unroll
            for (int gv = 0; gv < G; ++gv) {
                as[gv] = 1.0f;
                if constexpr (kBound) {
                    // A = p * V_scale / s_run <= 1/2: bound set with a factor-2 headroom
                    const float sn = sp_g[gv] > s_run[gv] ? 2.0f * sp_g[gv] : s_run[gv];
                    as[gv] = sn > 0.f ? s_run[gv] / sn : 1.0f;
                    s_run[gv] = sn;
                    inv_s[gv] = sn > 0.f ? 1.0f / sn : 0.f;
                }
            }
            float a_lg = as[0], am_lg = am[0];
            float ml = m_run[0];
#pragma unroll
            for (int gv = 1; gv < G; ++gv) a_lg = lg == gv ? as[gv] : a_lg;
#pragma unroll
            for (int r = 1; r < NREP; ++r) {
                am_lg = lg == r ? am[r] : am_lg;
                ml = lg == r ? m_run[r] : ml;
            }
            m_lane = ml == -INFINITY ? 0.f : ml;
            l_acc *= am_lg;
#pragma unroll
            for (int gv = 0; gv < G; ++gv) bias[gv] *= am_lg;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float f = r < NREP ? am[r] * a_lg : 0.f;
#pragma unroll
                for (int t = 0; t < 8; ++t) pacc[t][r] *= f;
            }
        }

        // ---- p.v: A = p * V_scale (/ s_run) as fp16 hi + lo, 2 steps of 32 tokens x 8 tiles
        float pr[4];
#pragma unroll
        for (int T = 0; T < 4; ++T) {
            pr[T] = exp2_fast(lg4[T] - m_lane);      // exp2(-inf) = 0 for masked tokens
            l_acc += pr[T];
        }
        // Operand k = 8*kg + 2*ai + jj of step s carries token 16*(2s + jj) + 4*ai + kg
        // (the order of the V dwords below): token 16T + n16 is step T>>1, kg = n16&3,
        // half 2*(n16>>2) + (T&1) -> one dword per (group, step) from each lane.
#pragma unroll
        for (int gv = 0; gv < G; ++gv) {
            float a4[4];
#pragma unroll
            for (int T = 0; T < 4; ++T) {
                a4[T] = pr[T] * vs_t[T][gv];
                if constexpr (kBound) a4[T] *= inv_s[gv];
                bias[gv] = fmaf(pr[T], vm_t[T][gv], bias[gv]);
            }
            if (lg < NREP) {
                const int row = 4 * gv + lg;
                const int q = swz(row, n16 & 3);
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const f2v av = {a4[2 * st], a4[2 * st + 1]};
                    const h2v hv = __builtin_convertvector(av, h2v);
                    const h2v lv = __builtin_convertvector(av - __builtin_convertvector(hv, f2v), h2v);
                    *(uint32_t*)&W.apv[st][row][q][4 * (n16 >> 2)] = __builtin_bit_cast(uint32_t, hv);
                    if constexpr (G == 1)        // rows 4..7 are free: lo in row 4 + r, same operand
                        *(uint32_t*)&W.apv[st][row + 4][swz(row + 4, n16 & 3)][4 * (n16 >> 2)] =
                            __builtin_bit_cast(uint32_t, lv);
                    else
                        *(uint32_t*)&W.apl[st][row][q][4 * (n16 >> 2)] = __builtin_bit_cast(uint32_t, lv);
                }
            }
        }
        wave_lds_fence();
        const v8h ap0 = *(const v8h*)&W.apv[0][n16][swz(n16, lg)][0];
        const v8h ap1 = *(const v8h*)&W.apv[1][n16][swz(n16, lg)][0];
        v8h al0 = {}, al1 = {};          // used with G != 1 only
        if constexpr (G != 1) {
            al0 = *(const v8h*)&W.apl[0][n16][swz(n16, lg)][0];
            al1 = *(const v8h*)&W.apl[1][n16][swz(n16, lg)][0];
        }
        // B: nibbles of the V dwords, two tokens per dword as fp16 subnormal bit patterns
        uint32_t nl[16], nh[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            nl[j] = lo_nib(cb.vw[j]);
            nh[j] = hi_nib(cb.vw[j]);
        }
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            // bytes [cc of token j0, 0, cc of token j1, 0]
            const uint32_t sel = 0x0C000C00u | ((4u + cc) << 16) | (uint32_t)cc;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                uint32_t bl[4], bh[4];
#pragma unroll
                for (int ai = 0; ai < 4; ++ai) {
                    const int j0 = 4 * ai + 2 * st;
                    bl[ai] = __builtin_amdgcn_perm(nl[j0 + 1], nl[j0], sel);
                    bh[ai] = __builtin_amdgcn_perm(nh[j0 + 1], nh[j0], sel);
                }
                const v8h blo = __builtin_bit_cast(v8h, (v4i){(int)bl[0], (int)bl[1], (int)bl[2], (int)bl[3]});
                const v8h bhi = __builtin_bit_cast(v8h, (v4i){(int)bh[0], (int)bh[1], (int)bh[2], (int)bh[3]});
                const v8h a = st ? ap1 : ap0, al = st ? al1 : al0;
                pacc[2 * cc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, blo, pacc[2 * cc], 0, 0, 0);
                pacc[2 * cc + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bhi, pacc[2 * cc + 1], 0, 0, 0);
                if constexpr (G != 1) {
                    pacc[2 * cc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, blo, pacc[2 * cc], 0, 0, 0);
                    pacc[2 * cc + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bhi, pacc[2 * cc + 1], 0, 0, 0);
                }
            }
        }
        wave_lds_fence();
    };

    // One page in flight ahead of the one being computed.
    {
        // issued unconditionally (past the wave's last page they read nothing),
        // so every path into the loop has the same loads in flight
        if constexpr (NW == 8) s_left[w] = n_mine;
        if (!first_issued) issue(b0, 0);
        if constexpr (FUSED) {
            // The partial-page tail's attention state (the merge's last slot),
            // while each wave's first page is in flight: its barriers wait on
            // LDS only
            if (tail_T > 0)      // uniform
                tail_state_lds<D, NREP, NT>(s_tk, s_tv, a.tail.dtype == FQ_BF16, tail_T, s_q, s_tp, s_split.m[NW],
                                            s_split.l[NW], s_split.acc[NW]);
        }
        for (int k = 0; k < n_mine; k += 2) {
            issue(b1, k + 1);
            compute(b0, k);
            issue(b0, k + 2);
            if (k + 1 < n_mine) compute(b1, k + 1);
        }
        __builtin_amdgcn_s_setprio(0);
    }

    // ------------------------------------------------ wave state -> LDS
    if constexpr (G == 1) {     // the lo rows 4 + r (lane group 1) join the hi rows
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int r = 0; r < NREP; ++r) pacc[t][r] += __shfl_xor(pacc[t][r], 16, 64);
    }
    l_acc = row_sum<16>(l_acc);
#pragma unroll
    for (int gv = 0; gv < G; ++gv) bias[gv] = row_sum<16>(bias[gv]);
    const int ug = G == 1 ? 0 : (n16 >> 2);      // channel group of this lane's columns
    float bsel = bias[0], ssel = s_run[0];
#pragma unroll
    for (int gv = 1; gv < G; ++gv) {
        if (ug == gv) { bsel = bias[gv]; ssel = s_run[gv]; }
    }
    const float pv_unscale = ssel * kSubnormal;
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
        const int src = 16 * r + n16;
        const float ll = __shfl(l_acc, src, 64);
        const float bb = __shfl(bsel, src, 64);
        if (lg == ug) {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                s_split.acc[w][r][8 * n16 + t] = fmaf(pacc[t][r], pv_unscale, bb);
            }
            if (n16 == 0) { s_split.m[w][r] = m_run[r]; s_split.l[w][r] = ll; }
        }
    }
    int nslots = NW;
    if constexpr (FUSED) {
        if (tail_T > 0) nslots = NW + 1;       // the tail state (computed before the page loop) joins the merge
    }
    __syncthreads();
    merge_waves_and_store<D, NREP, false, NSLOT, NT>(s_split, q, a.ws, g, l, b, h, split,
                                                     a.splits > 1 || (a.tail.len > 0 && !a.tail.in_kernel), nslots);
}

template <typename MT, int G, int NW, bool FUSED>
hipError_t launch_mfma_nrep(const MfmaParams& a, dim3 grid, hipStream_t st) {
    switch (a.q.nrep) {
#define FQ_CASE(N)                                                                                     \
    case N:                                                                                            \
        timer_before_launch(st);                                                                       \
        if (FUSED && (N == 3 || N == 4) && a.sel.head_chunks > 1)                                      \
            hipLaunchKernelGGL((attn_int4_mfma_kernel<MT, G, N, NW, FUSED, FUSED && N >= 3>), grid,       \
                               dim3(64 * NW), 0, st, a);                                               \
        else                                                                                           \
            hipLaunchKernelGGL((attn_int4_mfma_kernel<MT, G, N, NW, FUSED>), grid, dim3(64 * NW), 0, st, a); \
        timer_after_launch(st);                                                                        \
        if (a.splits > 1 || (a.tail.len > 0 && !a.tail.in_kernel))                                     \
            launch_split_merge<N, false>(a.q, a.ws, a.c.Hkv, a.c.B, grid.y, a.splits,                  \
                                         a.tail.in_kernel ? TailArgs{} : a.tail, st);                   \
        break;
        FQ_CASE(1) FQ_CASE(2) FQ_CASE(3) FQ_CASE(4)
#undef FQ_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Work split.  With enough KV groups to cover most CUs, one workgroup of 8
// waves takes a whole group (no split partials, no merge launch).  Otherwise
// workgroups of 4 waves take balanced slices: enough to keep every CU busy in
// one pass (two resident per CU), at least 8 pages per slice.  `request` > 0
// pins the slices per group (4-wave workgroups).
struct MfmaSplit { int splits, waves; };
MfmaSplit mfma_splits(int groups, int max_entries, int s_max, int request) {
    constexpr int kResident = 2 * 256;
    if (request <= 0 && groups >= 192 && max_entries <= kMaxWgPages) return {1, 8};
    int s = request > 0 ? request : kResident / (groups > 0 ? groups : 1);
    if (request <= 0) s = std::min(s, (max_entries + 7) / 8);
    s = std::max(s, (max_entries + kMaxWgPages - 1) / kMaxWgPages);
    s = std::max(s, 1);
    return {std::min(s, s_max), 4};
}

// The fused decode: one workgroup of 8 waves per KV group when the groups
// fill the GPU; otherwise every group is split over enough workgroups for one
// per CU, each scoring and selecting the group's pages itself (the same list
// in every split) and attending a balanced slice of it, at least 8 pages.
int fused_splits(int groups, int max_entries, int s_max) {
    if (groups >= 192 || max_entries <= kFusedSmallPages) return 1;
    int s = (256 + groups - 1) / std::max(groups, 1);
    s = std::min(s, (max_entries + 7) / 8);
    return std::max(1, std::min(s, s_max));
}

}  // namespace

bool mfma_supported(const Int4Cache& c, const QueryArgs& q, const AttnLaunch& al) {
    if (c.D != 128 || c.page != 64 || q.nrep > 4 || c.bits == 8) return false;
    if (c.G != 1 && c.G != 4) return false;
    if ((int64_t)al.s_max * kMaxWgPages < al.max_entries) return false;
    // contiguous 64-byte rows of codes, G-element rows of V metadata, 128-element
    // rows of K metadata; 16-byte aligned code rows and 8-byte aligned metadata
    if (c.kp_s[3] != 64 || c.vp_s[3] != 64 || c.vsc_s[3] != c.G || c.vmn_s[3] != c.G) return false;
    if (c.ksc_s[3] != 128 || c.kmn_s[3] != 128) return false;
    if (c.kp_s[2] % 16 || c.kp_s[1] % 16 || c.kp_s[0] % 16 || ((uintptr_t)c.kp & 15)) return false;
    if (c.vp_s[2] % 16 || c.vp_s[1] % 16 || c.vp_s[0] % 16 || ((uintptr_t)c.vp & 15)) return false;
    if (c.ksc_s[2] % 8 || c.ksc_s[1] % 8 || c.ksc_s[0] % 8 || ((uintptr_t)c.ksc & 15)) return false;
    if (c.kmn_s[2] % 8 || c.kmn_s[1] % 8 || c.kmn_s[0] % 8 || ((uintptr_t)c.kmn & 15)) return false;
    if (c.G == 4 && (c.vsc_s[2] % 4 || c.vmn_s[2] % 4 || c.vsc_s[1] % 4 || c.vmn_s[1] % 4 || c.vsc_s[0] % 4 ||
                     c.vmn_s[0] % 4 || ((uintptr_t)c.vsc & 7) || ((uintptr_t)c.vmn & 7)))
        return false;
    return true;
}

bool mfma_select_in_kernel(const Int4Cache& c, const QueryArgs& q, const AttnLaunch& al) {
    return mfma_supported(c, q, al) && c.P <= 64 * kSelC && al.max_entries <= kMaxWgPages &&
           attention_splits_request() <= 0;
}

bool mfma_tail_in_kernel(const TailArgs& t) {
    const bool t16 = t.dtype == FQ_BF16 || t.dtype == FQ_F16;
    auto al16 = [](const int64_t* s) { return s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0 && s[3] % 8 == 0; };
    return t.len > 0 && t16 && al16(t.ks) && al16(t.vs) && t.ks[3] >= 128 && t.vs[3] >= 128 &&
           ((uintptr_t)t.k & 15) == 0 && ((uintptr_t)t.v & 15) == 0 &&
           2 * (int64_t)t.len * std::max(t.ks[3], t.vs[3]) < INT32_MAX;
}

hipError_t launch_attn_int4_mfma(const Int4Cache& c, const QueryArgs& q, const Workspace& ws, const AttnLaunch& al,
                                 hipStream_t st, const SelectArgs* sel, const TailArgs* tail) {
    MfmaParams a{};
    a.c = c; a.q = q; a.ws = ws;
    if (tail) a.tail = *tail;
    const int groups = c.L * c.B * c.Hkv;
    const MfmaSplit sp = mfma_splits(groups, al.max_entries, al.s_max, attention_splits_request());
    a.splits = sp.splits;
    if (sel && sel->enabled) {
        if (!mfma_select_in_kernel(c, q, al)) return hipErrorInvalidValue;
        a.sel = *sel;
        a.splits = fused_splits(groups, al.max_entries, al.s_max);
        // the kernel attends a 16-bit tail itself (16-byte aligned rows, at
        // least D apart): with one workgroup per group no merge launch follows,
        // with several, split 0 folds it into its partial and the merge has no
        // tail work left
        a.tail.in_kernel = mfma_tail_in_kernel(a.tail);
        // head chunks: a tail only inside the kernel (the split merge's tail
        // work indexes the cache by the virtual heads)
        if (a.sel.head_chunks > 1 && a.tail.len > 0 && !a.tail.in_kernel) return hipErrorInvalidValue;
    }
    dim3 grid(a.splits, groups);
#define FQ_W(MT_, G_)                                                                       \
    (a.sel.enabled ? launch_mfma_nrep<MT_, G_, 8, true>(a, grid, st)                        \
                   : sp.waves == 8 ? launch_mfma_nrep<MT_, G_, 8, false>(a, grid, st)       \
                                   : launch_mfma_nrep<MT_, G_, 4, false>(a, grid, st))
    if (c.meta_dtype == FQ_BF16) return c.G == 4 ? FQ_W(bf16, 4) : FQ_W(bf16, 1);
    return c.G == 4 ? FQ_W(f16, 4) : FQ_W(f16, 1);
#undef FQ_W
}

}  // namespace fq
