// Shared device helpers and kernel parameter blocks for libfq_hip (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_hip.h"

#define FQ_DEV __device__ __forceinline__

namespace fq {

constexpr int kThreads = 256;      // 4 wave64 per workgroup
constexpr int kMaxPages = 8192;    // 512k tokens at 64 tokens / page
// A page index past every cache slice (kMaxPages pages): page loads issued
// past a wave's last page use it, so their buffer loads fall outside the
// slice's range and return zeros without a memory access.
constexpr int kNoPage = 0x7FFF;
// A decode step whose lists hold at most this many pages per KV group runs as
// one launch with one workgroup per group (it scores, selects and attends
// itself: a few pages per wave) even when the groups do not fill the GPU;
// longer lists split each group over workgroups behind a scoring launch.
constexpr int kFusedSmallPages = 40;
constexpr int kMaxRows = 16;       // query rows per KV group in scoring (n_rep * S_q)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------- dtypes --
struct bf16 { uint16_t v; };
struct f16 { uint16_t v; };

FQ_DEV float bf16_bits_to_f(uint32_t b) { return __uint_as_float(b << 16); }
FQ_DEV float f16_bits_to_f(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}
template <typename T> FQ_DEV float half_to_f(uint32_t bits);
template <> FQ_DEV float half_to_f<bf16>(uint32_t b) { return bf16_bits_to_f(b & 0xFFFFu); }
template <> FQ_DEV float half_to_f<f16>(uint32_t b) { return f16_bits_to_f(b & 0xFFFFu); }

FQ_DEV uint16_t f_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;   // NaN
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
FQ_DEV uint16_t f_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
// Round an fp32 value to the given half dtype and back (torch "opmath" rounding).
FQ_DEV float round_to(float f, int dtype) {
    if (dtype == FQ_BF16) return bf16_bits_to_f(f_to_bf16_bits(f));
    if (dtype == FQ_F16) return f16_bits_to_f(f_to_f16_bits(f));
    return f;
}

FQ_DEV float load_any(const void* p, int dtype, int64_t idx) {
    if (dtype == FQ_F32) return ((const float*)p)[idx];
    uint32_t b = ((const uint16_t*)p)[idx];
    return dtype == FQ_BF16 ? bf16_bits_to_f(b) : f16_bits_to_f(b);
}
FQ_DEV void store_any(void* p, int dtype, int64_t idx, float v) {
    if (dtype == FQ_F32) { ((float*)p)[idx] = v; return; }
    ((uint16_t*)p)[idx] = dtype == FQ_BF16 ? f_to_bf16_bits(v) : f_to_f16_bits(v);
}

// Monotone fp32 -> u32 key: larger float -> larger key; -0 == +0; NaN largest.
FQ_DEV uint32_t sortable_key(float f) {
    if (f != f) return 0xFFC00000u;   // every NaN -> the key of +NaN (above +inf)
    if (f == 0.0f) f = 0.0f;
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---------------------------------------------------------- wave helpers --
FQ_DEV int lane_id() { return threadIdx.x & 63; }
FQ_DEV int wave_id() { return threadIdx.x >> 6; }
FQ_DEV uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// DPP moves inside a row of 16 lanes.  Every lane of the row ends with a
// bit-identical sum: each step adds a value to its partner's value (fp32 add
// is commutative), so partners always agree.
template <int CTRL> FQ_DEV float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i -> 7 - i within each 8
constexpr int kDppMirror = 0x140;      // lane i -> 15 - i within each 16

// All-reduce (sum) across groups of NL consecutive lanes (NL = 8 or 16).
template <int NL> FQ_DEV float row_sum(float v) {
    if constexpr (NL == 16) v += dpp<kDppMirror>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    return v;
}

// ------------------------------------------------------- block helpers ----
// A workgroup barrier for data exchanged through LDS only: it waits for this
// wave's LDS operations, not for its global loads, which stay in flight
// (__syncthreads also waits for those).
FQ_DEV void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Ordered compaction over [0, n): calls write(i, rank) for every i with
// flag(i), rank = number of flagged j < i.  Returns the flagged count.
// Must be called by all kThreads threads; s_tmp needs 5 ints of LDS.
template <typename Flag, typename Write>
FQ_DEV int block_compact(int n, Flag flag, Write write, int* s_tmp) {
    const int tid = threadIdx.x, w = wave_id();
    int running = 0;
    for (int base = 0; base < n; base += kThreads) {
        const int i = base + tid;
        const bool f = i < n && flag(i);
        const uint64_t bal = __ballot(f);
        if (lane_id() == 0) s_tmp[w] = __popcll(bal);
        __syncthreads();
        int off = running;
        for (int j = 0; j < w; ++j) off += s_tmp[j];
        if (f) write(i, off + (int)lanes_below(bal));
        running += s_tmp[0] + s_tmp[1] + s_tmp[2] + s_tmp[3];
        __syncthreads();
    }
    return running;
}

// Radix select of the k-th largest key among keys[0..n) (LDS), 1 <= k <= n.
// Returns the threshold key T; *take_eq = how many keys equal to T belong to
// the top k (ties are then resolved by lower index).  s_hist: 256 ints,
// s_tmp: 4 ints of LDS.
FQ_DEV uint32_t block_radix_select(const uint32_t* keys, int n, int k, int* s_hist,
                                   int* s_tmp, int* take_eq) {
    const int tid = threadIdx.x;
    uint32_t prefix = 0, pmask = 0;
    int krem = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += kThreads) s_hist[i] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += kThreads) {
            const uint32_t u = keys[i];
            if ((u & pmask) == prefix) atomicAdd(&s_hist[(u >> shift) & 255u], 1);
        }
        __syncthreads();
        if (tid < 64) {
            const int c0 = s_hist[4 * tid], c1 = s_hist[4 * tid + 1];
            const int c2 = s_hist[4 * tid + 2], c3 = s_hist[4 * tid + 3];
            const int s = c0 + c1 + c2 + c3;
            int suf = s;   // inclusive suffix sum over lanes >= tid
            for (int off = 1; off < 64; off <<= 1) {
                const int o = __shfl_down(suf, off, 64);
                if (tid + off < 64) suf += o;
            }
            const int above = suf - s;   // keys in bins > 4*tid+3
            if (above < krem && krem <= suf) {
                int cum = above, digit = 4 * tid + 3;
                const int cs[4] = {c0, c1, c2, c3};
                for (int j = 3; j >= 0; --j) {
                    if (cum + cs[j] >= krem) { digit = 4 * tid + j; break; }
                    cum += cs[j];
                }
                s_tmp[0] = digit;
                s_tmp[1] = krem - cum;
            }
        }
        __syncthreads();
        prefix |= (uint32_t)s_tmp[0] << shift;
        pmask |= 0xFFu << shift;
        krem = s_tmp[1];
        __syncthreads();
    }
    *take_eq = krem;
    return prefix;
}

// ------------------------------------------------------ kernel params -----
// All strides are in elements of the pointed-to type.
struct Int4Cache {
    const uint8_t* kp; int64_t kp_s[4];   // l, b, h, s  (channel-byte stride 1)
    const uint8_t* vp; int64_t vp_s[4];
    const void* ksc;   int64_t ksc_s[4];  // l, b, h, p  (channel stride 1)
    const void* kmn;   int64_t kmn_s[4];
    const void* vsc;   int64_t vsc_s[4];  // l, b, h, s  (group stride 1)
    const void* vmn;   int64_t vmn_s[4];
    int L, B, Hkv, S, P, D, page, G;
    int meta_dtype;                       // FQ_BF16 / FQ_F16
    int bits;                             // code width: 4 (two codes per byte) or 8 (one byte per code); 0 = 4
};

struct QueryArgs {
    const void* q; int q_dtype; int64_t q_s[4];    // l, b, h_q, d
    void* out; int out_dtype; int64_t o_s[4];
    float* lse; int64_t lse_s[3];
    int Hq, nrep;
    float qk_scale;                                 // sm_scale * log2(e)
    int64_t ret_ls;                                 // retention (L, H_q): layer stride (0: one row for all layers)
    const float* rot;                               // (D,) signs s: q -> WHT(s q) / sqrt(D), O -> s WHT(O) / sqrt(D); or null
};

// Workspace regions (device pointers) for one decode / attention call.
// Dense attention over the partial-page tail (bf16 / fp16 / fp32 K and V,
// (l, b, h, t) element strides, channels contiguous), folded into the split
// merge.  len == 0: no tail.
constexpr int kTailMax = 64;
struct TailArgs {
    const void* k; int64_t ks[4];
    const void* v; int64_t vs[4];
    int dtype, len;
    int in_kernel;      // the fused decode kernel attends the tail (2-byte dtype, 16-byte aligned rows)
};

struct Workspace {
    int* n_sel;           // [G]   union-list length
    int* entries;         // [G][P] page | qmask << 16, ascending page order
    float* scores;        // [G][rows][P]
    float* part_ml;       // [G][S_max][nrep][2]
    float* part_acc;      // [G][S_max][nrep][D]
    int s_max;
};

// Page-selection arguments for an attention kernel that selects its own pages
// (fused decode): retention per query head, forced pages, k_max, policy.
// enabled: 0 = pages from the workspace lists, kScoreSelect = the attention
// kernel scores and selects the pages itself (one launch per decode step).
constexpr int kScoreSelect = 2;
constexpr int kSelectOnly = 1;        // the attention kernel selects from scores a scoring launch wrote to the workspace
struct SelectArgs {
    const float* retention;
    int num_sinks, window, k_max, mode;
    int enabled;
    uint8_t* mask_out;      // fused kernels: the selection as (L, B, H_q, P) bool rows, or null
    int head_chunks;        // INT4 fused kernel: virtual KV heads per cache KV head (0 or 1: none)
};

struct AttnLaunch {
    int pages_per_split;
    int splits;
    int max_entries;      // bound on any group's union-list length
    int s_max;            // split partials the workspace holds per group
};

// Host-side helpers implemented in capi.cpp.
// Kernel timer hooks around an attention kernel launch (no-ops unless armed).
void timer_before_launch(hipStream_t st);
void timer_after_launch(hipStream_t st);
// fq_set_attention_splits value (0 = automatic).
int attention_splits_request();
// Host helpers of the C ABI (capi.cpp), shared with the measurement library:
// error reporting (fq_last_error), HIP status mapping and cache descriptor checks.
int fail(int code, const char* fmt, ...);
int hip_status(hipError_t e, const char* what);
int check_cache(const fq_int4_cache* c, Int4Cache* out, int bits = 4, bool allow_empty = false);
size_t workspace_bytes(int G, int P, int rows, int nrep, int D);
Workspace carve_workspace(void* base, int G, int P, int rows, int nrep, int D);
AttnLaunch choose_split(int G, int max_entries, int s_max);

// Launchers (return hipError_t of the launch).
// Scores into the user buffer and/or ws->scores; with ws, also the per-group
// selection (union lists, n_sel, optional mask_out).
hipError_t launch_score(const Int4Cache& c, const QueryArgs& q, int S_q, const int64_t* q4_s,
                        float* scores, const int64_t* sc4_s, const Workspace* ws, int select_mode,
                        const float* retention, int num_sinks, int window, int k_max,
                        uint8_t* mask_out, hipStream_t st, bool select_groups = true);
hipError_t launch_select_rows(const float* scores, const int64_t* sc_s, int B, int H, int S_q, int P,
                              const float* retention, int num_sinks, int window, int k_max,
                              uint8_t* mask, const int64_t* m_s, hipStream_t st);
hipError_t launch_compact_ids(const uint8_t* mask, const int64_t* m_s, int B, int H, int S_q, int P,
                              int bucket, int32_t* ids, hipStream_t st);
hipError_t launch_read_step(const Int4Cache& c, const Workspace& ws, unsigned* sink, hipStream_t st);
hipError_t launch_read_stream(const void* p, int64_t bytes, unsigned* sink, hipStream_t st);
hipError_t launch_union_from_mask(const uint8_t* mask, const int64_t* m_s, int L, int B, int Hkv,
                                  int nrep, int P, const Workspace& ws, hipStream_t st);
hipError_t launch_union_from_ids(const int32_t* ids, const int64_t* id_s, int bucket, int L, int B,
                                 int Hkv, int nrep, int P, const Workspace& ws, hipStream_t st);
// sel (may be null): the kernel scores and selects the pages itself; only valid
// when attn_selects_in_kernel() says so for the same arguments.
hipError_t launch_attn_int4(const Int4Cache& c, const QueryArgs& q, const Workspace& ws,
                            const AttnLaunch& al, hipStream_t st, const SelectArgs* sel = nullptr,
                            const TailArgs* tail = nullptr);
// Page-tile INT4 quantisers (cache.hip): eligibility of a layout, whole-tensor
// quantisation, and the cache append of update_quantized.
bool page_quant_k_ok(int D, int page, int in_dtype, const void* k, const int64_t* k_s, const uint8_t* packed,
                     const int64_t* p_s, const void* scale, const int64_t* s_s, const void* mn, const int64_t* m_s);
bool page_quant_v_ok(int D, int group, int in_dtype, const void* v, const int64_t* v_s, const uint8_t* packed,
                     const int64_t* p_s, const int64_t* s_s, const int64_t* m_s);
hipError_t launch_quant_k_pages(const void* k, int in_dtype, const int64_t* k_s, int B, int H, int S, int D,
                                uint8_t* packed, const int64_t* p_s, void* scale, const int64_t* s_s, void* mn,
                                const int64_t* m_s, int meta_dtype, hipStream_t st);
hipError_t launch_quant_v_pages(const void* v, int in_dtype, const int64_t* v_s, int B, int H, int S, int D,
                                int group, uint8_t* packed, const int64_t* p_s, void* scale, const int64_t* s_s,
                                void* mn, const int64_t* m_s, int meta_dtype, hipStream_t st);
hipError_t launch_kv_append(const Int4Cache& c, int layer, void* kpart, const int64_t* kpart_s, void* vpart,
                            const int64_t* vpart_s, int part_dtype, const void* knew, const int64_t* kn_s,
                            const void* vnew, const int64_t* vn_s, int seen, int S_new, int bits, hipStream_t st);
hipError_t launch_turbo_append(const fq_turbo_cache& tc, const Int4Cache& raw, int layer, void* kpart,
                               const int64_t* kpart_s, void* vpart, const int64_t* vpart_s, int part_dtype,
                               const void* knew, const int64_t* kn_s, const void* vnew, const int64_t* vn_s, int seen,
                               int S_new, hipStream_t st);
// Fused-layout TurboQuant attention (turbo_fused.hip): D = 128, 64-token pages,
// <= 3 query heads per KV head.  raw + sel: score and select in the kernel.
bool turbo_fused_supported(const fq_turbo_cache& c, const QueryArgs& q);
hipError_t launch_attn_turbo_fused(const fq_turbo_cache& c, const Int4Cache* raw, const QueryArgs& q,
                                   const Workspace& ws, int max_entries, const SelectArgs* sel, hipStream_t st);
bool attn_selects_in_kernel(const Int4Cache& c, const QueryArgs& q, const AttnLaunch& al);
// INT8 cache on the matrix cores (attn_int8_mfma.hip): D = 128, 64-token pages,
// per-token V metadata, dense rows, <= 4 query heads per KV head.
bool int8_mfma_supported(const Int4Cache& c, const QueryArgs& q, const AttnLaunch& al);
bool int8_select_in_kernel(const Int4Cache& c, const QueryArgs& q, const AttnLaunch& al);
hipError_t launch_attn_int8_mfma(const Int4Cache& c, const QueryArgs& q, const Workspace& ws, const AttnLaunch& al,
                                 hipStream_t st, const SelectArgs* sel, const TailArgs* tail = nullptr);
bool mfma_supported(const Int4Cache& c, const QueryArgs& q, const AttnLaunch& al);
bool mfma_select_in_kernel(const Int4Cache& c, const QueryArgs& q, const AttnLaunch& al);
// The fused INT4 kernel attends a 16-bit partial-page tail itself (16-byte
// aligned rows at least D apart).
bool mfma_tail_in_kernel(const TailArgs& t);
// Page summary scores over the INT8 cache (summary.hip).
struct SummaryArgs {
    const uint8_t* codes; int64_t c_s[4];          // (B, H_kv, S, D) bytes
    const void* ks; int64_t ks_s[4];               // (B, H_kv, P, D) elements
    const void* km; int64_t km_s[4];
    int meta_dtype;
    const void* q; int q_dtype; int64_t q_s[4];    // (B, H_q, 1, D)
    float* scores; int64_t sc_s[4];                // (B, H_q, 1, P)
    uint16_t* pmin; uint16_t* pmax; int64_t pm_s[4];   // optional bf16 summaries (B, H_kv, P, D)
    int B, Hq, Hkv, S, P, D, page;
};

hipError_t launch_page_summary_scores(const SummaryArgs& a, hipStream_t st);
// compute_page_summary over any float K, and Quest scores from page bounds
// (summary.hip).
struct PageMinMaxArgs {
    const void* k; int k_dtype; int64_t k_s[4];        // (B, H, S, D)
    void* pmin; void* pmax; int64_t pm_s[4];           // (B, H, P, D), K's dtype
    int B, H, S, P, D, page;
};
hipError_t launch_page_minmax(const PageMinMaxArgs& a, hipStream_t st);
struct QuestScoreArgs {
    const void* q; int q_dtype; int64_t q_s[4];        // (B, H_q, S_q, D)
    const void* lo; const void* hi; int b_dtype; int64_t lo_s[4], hi_s[4];   // (B, H_kv, P, D)
    bool from_meta;                                    // lo = K_mn, hi = K_mn + levels * K_scale (hi = K_scale)
    float levels;
    float* scores; int64_t sc_s[4];                    // (B, H_q, S_q, P)
    int B, Hq, Sq, Hkv, P, D;
};
hipError_t launch_quest_scores(const QuestScoreArgs& a, hipStream_t st);
hipError_t launch_attn_int4_mfma(const Int4Cache& c, const QueryArgs& q, const Workspace& ws,
                                 const AttnLaunch& al, hipStream_t st, const SelectArgs* sel,
                                 const TailArgs* tail = nullptr);

}  // namespace fq
