/*
 * fq_hip.h — C ABI of the MI355X (gfx950) sparse INT4 / turbo decode-attention
 * library (libfq_hip.so).
 *
 * Every entry point takes raw device pointers, int64 element strides, plain
 * sizes and an explicit hipStream_t; nothing allocates device memory (callers
 * pass a workspace sized by fq_workspace_bytes) and nothing synchronises.
 * Every function returns an fq_status; fq_last_error() returns a message for
 * the calling thread's most recent failure.
 *
 * The reference (Dialovos/flashquest) is Python + Triton with no FFI; each
 * entry below replaces one Python operator of its decode path, cited as
 * path:line relative to the reference root.  A caller maps tensors to
 * (pointer, strides) exactly as the reference's Triton launch does
 * (src/flashquest/kernel/sparse_int4_fwd.py:221-244).
 *
 * Layout contract (matches the reference's persistent caches,
 * src/flashquest/cache/persistent_int4.py:46-59):
 *   K_packed, V_packed : (L, B, H_kv, S, D/2) u8, byte k = code[2k] | code[2k+1] << 4
 *   K_scale, K_mn      : (L, B, H_kv, P, D)    bf16 or fp16, per page and channel
 *   V_scale, V_mn      : (L, B, H_kv, S, G)    bf16 or fp16, per token (G = 1, the
 *                        reference) or per token and 32-channel group (G = D/32)
 * The innermost axis of every cache tensor must have stride 1; the packed
 * rows must be 4-byte aligned.  L (layers) is an extra batch axis: the
 * reference calls the operators once per layer (L = 1, layer stride 0).
 */
#ifndef FQ_HIP_H
#define FQ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* fq_stream_t; /* == hipStream_t */

/* Status codes.  The Python layer maps them to the reference's exception
 * types (sparse_int4_fwd.py:187-204, selection.py:92-101, 147-150). */
enum fq_status {
    FQ_OK = 0,
    FQ_ERR_INVALID = 1,     /* bad shape / stride / argument  -> ValueError / AssertionError */
    FQ_ERR_UNSUPPORTED = 2, /* shape or dtype outside the kernels -> NotImplementedError   */
    FQ_ERR_HIP = 3,         /* HIP runtime error (launch failure)  -> RuntimeError          */
    FQ_ERR_WORKSPACE = 4    /* workspace missing or too small      -> RuntimeError          */
};

enum fq_dtype { FQ_BF16 = 0, FQ_F16 = 1, FQ_F32 = 2 };

/* Page selection policy for the fused decode entry.
 * FQ_SELECT_PER_Q_HEAD: top-k per query head (selection.py:103-117), the
 *   reference's behaviour; the kernel reads the union over the GQA group.
 * FQ_SELECT_PER_KV_HEAD_SUM: one top-k per KV head over the fp32 sum of the
 *   group's query-head scores, applied to every query head of the group. */
enum fq_select_mode { FQ_SELECT_PER_Q_HEAD = 0, FQ_SELECT_PER_KV_HEAD_SUM = 1 };

/* Packed INT4 cache view (see the layout contract above). */
typedef struct fq_int4_cache {
    const uint8_t* k_packed; int64_t k_strides[5];
    const uint8_t* v_packed; int64_t v_strides[5];
    const void* k_scale;     int64_t ks_strides[5];
    const void* k_mn;        int64_t km_strides[5];
    const void* v_scale;     int64_t vs_strides[5];
    const void* v_mn;        int64_t vm_strides[5];
    int32_t meta_dtype;      /* FQ_BF16 or FQ_F16 */
    int32_t L, B, H_kv;
    int32_t S;               /* tokens in the view (completed_len); tokens >= S are masked */
    int32_t P;               /* pages (K_scale.shape[-2]) */
    int32_t D;               /* head dim: 64 or 128 */
    int32_t page_size;       /* tokens per page, multiple of 4 (reference default 64) */
    int32_t v_groups;        /* G: 1 (reference) or D/32 */
} fq_int4_cache;

/* INT8 cache view (cache/persistent_int8.py get_views): the same descriptor
 * with one code byte per channel -- k_packed / v_packed hold K_uint8 / V_uint8
 * (L, B, H_kv, S, D) -- K scale/min per (page, channel) and V scale/min per
 * token (v_groups = 1).  Code strides are multiples of 8 bytes. */
typedef fq_int4_cache fq_int8_cache;

/* Decode query and outputs: Q (L, B, H_q, D), O (L, B, H_q, D), lse (L, B, H_q). */
typedef struct fq_query {
    const void* q;   int32_t q_dtype;   int64_t q_strides[4];
    void* out;       int32_t out_dtype; int64_t o_strides[4];
    float* lse;      int64_t lse_strides[3];  /* may be NULL (return_lse=False) */
    int32_t H_q;
    float sm_scale;  /* <= 0 selects 1/sqrt(D) (sparse_int4_fwd.py:206-207) */
    /* Decode entries that select pages: the retention array is (H_q,) for
     * every layer (0), or (L, H_q) with this layer stride (H_q or more), e.g.
     * a DuoAttention head pattern per layer (llama_persistent_patch.py:214-220). */
    int64_t retention_layer_stride;
    /* Rotated decode (benchmark config 3: a cache quantised in the basis
     * x -> WHT(s x) / sqrt(128)): with a device fp32 (128,) sign vector s, the
     * single-launch INT4 decode rotates q the same way (fp32 butterflies, then
     * times fp32(1/sqrt(128))) before scoring and attention, and writes
     * O = s WHT(O_rot) / sqrt(128).  NULL: no rotation.  Other entry points,
     * and decode calls that take the split path, return FQ_ERR_UNSUPPORTED. */
    const float* rotation_signs;
} fq_query;

/* TurboQuant K3-V3 cache (persistent_turbo.py:55-73):
 * msb (L,B,H_kv,S,D/8), lsb (L,B,H_kv,S,D/4) u8; per-token scale (L,B,H_kv,S,1) bf16. */
typedef struct fq_turbo_cache {
    const uint8_t* k_msb; int64_t kmsb_strides[5];
    const uint8_t* k_lsb; int64_t klsb_strides[5];
    const void* k_scale;  int64_t kst_strides[5];
    const uint8_t* v_msb; int64_t vmsb_strides[5];
    const uint8_t* v_lsb; int64_t vlsb_strides[5];
    const void* v_scale;  int64_t vst_strides[5];
    int32_t L, B, H_kv, S, P, D, page_size;
} fq_turbo_cache;

/* The partial-page tail of one decode step (PersistentInt4KVCache.K_partial /
 * V_partial views, persistent_int4.py:56-57): K and V (L, B, H_kv, T, D) with
 * T = len <= 64 tokens, any float dtype (bf16 in the reference). */
typedef struct fq_tail {
    const void* k; int64_t k_strides[5];
    const void* v; int64_t v_strides[5];
    int32_t dtype, len, D;
} fq_tail;

const char* fq_last_error(void);
int fq_abi_version(void);

/* Kernel timing (no counterpart in the reference; used by bench.py).  After
 * fq_kernel_timer_start(n), each of the next n sparse-attention kernel launches
 * (INT4 or turbo, not the split merge) made from this host thread is bracketed by
 * a pair of HIP events on its stream.  fq_kernel_timer_stop waits for them and
 * returns the summed kernel time and the number of timed launches.  Not for use
 * under HIP graph capture. */
int fq_kernel_timer_start(int32_t max_launches);
int fq_kernel_timer_stop(float* total_ms, int32_t* launches);

/* Split-count override for the matrix-core INT4 attention kernel (no
 * counterpart in the reference; for tests and tuning).  0 restores the
 * automatic choice; n > 0 asks for n workgroups per KV group, raised if a split
 * would exceed the kernel's page limit and lowered to the workspace capacity.
 * Process-wide. */
int fq_set_attention_splits(int32_t splits);

/* Bytes of workspace the attention / decode entries need for this cache and
 * H_q (page lists, scores and split partials; no initialisation needed).
 * Calls that share a workspace must be ordered (same stream). */
size_t fq_workspace_bytes(const fq_int4_cache* cache, int32_t H_q);

/* page_scores_int4_fast (src/flashquest/eager/criticality.py:128-163).
 * Q (B, H_q, S_q, D) any dtype; meta (B, H_kv, P, D); scores (B, H_q, S_q, P) fp32.
 * fp32 arithmetic in a fixed order (products rounded, no FMA). */
int fq_page_scores_int4(const void* q, int32_t q_dtype, const int64_t q_strides[4],
                        const void* k_scale, const int64_t ks_strides[4],
                        const void* k_mn, const int64_t km_strides[4], int32_t meta_dtype,
                        float* scores, const int64_t sc_strides[4],
                        int32_t B, int32_t H_q, int32_t S_q, int32_t H_kv, int32_t P, int32_t D,
                        fq_stream_t stream);

/* select_pages_vectorized (src/flashquest/eager/selection.py:65-126).
 * scores (B, H, S_q, P) fp32; retention: device fp32 (H,); k_max: the
 * reference's min(k_max_static, P), or -1 when k_max_static is None.
 * mask (B, H, S_q, P) u8 (0/1, torch.bool storage).  Ties go to the lower page. */
int fq_select_pages(const float* scores, const int64_t sc_strides[4],
                    int32_t B, int32_t H, int32_t S_q, int32_t P,
                    const float* retention, int32_t num_sinks, int32_t window_pages, int32_t k_max,
                    uint8_t* mask, const int64_t mask_strides[4], fq_stream_t stream);

/* build_compact_selection (src/flashquest/eager/selection.py:129-164).
 * mask (B, H, S_q, P) u8 -> ids (B, H, S_q, bucket_max) int32 contiguous:
 * selected ids in descending order, then -1. */
int fq_compact_ids(const uint8_t* mask, const int64_t mask_strides[4],
                   int32_t B, int32_t H, int32_t S_q, int32_t P, int32_t bucket_max,
                   int32_t* ids, fq_stream_t stream);

/* flash_attn_sparse_int4_fwd (src/flashquest/kernel/sparse_int4_fwd.py:160-248).
 * mask (L, B, H_q, P) u8.  Writes O and (if non-NULL) lse; an empty
 * selection gives O = 0, lse = -inf. */
int fq_sparse_int4_fwd_mask(const fq_int4_cache* cache, const fq_query* query,
                            const uint8_t* mask, const int64_t mask_strides[4],
                            void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* flash_attn_sparse_int4_fwd_compact (src/flashquest/kernel/sparse_int4_fwd_compact.py:153-244).
 * ids (L, B, H_q, bucket) int32; -1 (and any id outside [0, P)) is skipped. */
int fq_sparse_int4_fwd_ids(const fq_int4_cache* cache, const fq_query* query,
                           const int32_t* ids, const int64_t id_strides[4], int32_t bucket,
                           void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* One fused decode step over L layers: score (criticality.py:128-163) ->
 * select (selection.py:65-126) -> sparse attention (sparse_int4_fwd.py:23-157),
 * i.e. the completed-page part of llama_persistent_patch.py:220-234.
 * retention: device fp32 (H_q,).  scores_out (L,B,rows,P) fp32 and
 * mask_out (L,B,H_q,P) u8 are optional (NULL) diagnostics. */
int fq_quest_decode_int4(const fq_int4_cache* cache, const fq_query* query,
                         const float* retention, int32_t num_sinks, int32_t window_pages,
                         int32_t k_max, int32_t select_mode,
                         float* scores_out, uint8_t* mask_out,
                         void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* fq_quest_decode_int4 for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Same arguments and results without the
 * workspace: the split-path lists and partials live in a static device array
 * of FQ_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends), whose
 * address is looked up on the first call on each device (the current device).
 * Allocates nothing.  A step whose workspace (fq_workspace_bytes) exceeds the
 * array returns FQ_ERR_UNSUPPORTED before touching any pointer.  All calls on
 * one GPU share the array: calls that overlap on one GPU (different streams,
 * or host threads) race and must be serialised by the caller.  Nothing in the
 * array needs clearing: every region a call reads it writes first. */
#define FQ_NOALLOC_SCRATCH_BYTES (64u << 20)
int fq_quest_decode_int4_noalloc(const fq_int4_cache* cache, const fq_query* query,
                                 const float* retention, int32_t num_sinks, int32_t window_pages,
                                 int32_t k_max, int32_t select_mode,
                                 float* scores_out, uint8_t* mask_out, fq_stream_t stream);

/* The two halves of fq_quest_decode_int4, for callers that time or overlap
 * them separately; call both with the same cache, query, retention, k_max,
 * num_sinks, window_pages, select_mode and workspace.  fq_quest_select_int4
 * leaves the page scores (and, where the attention kernel cannot select for
 * itself, the per-KV-group page lists) in the workspace; fq_quest_attend_int4
 * selects from the scores inside the attention kernel when it takes a whole KV
 * group per workgroup, and otherwise consumes the lists. */
int fq_quest_select_int4(const fq_int4_cache* cache, const fq_query* query,
                         const float* retention, int32_t num_sinks, int32_t window_pages,
                         int32_t k_max, int32_t select_mode,
                         float* scores_out, uint8_t* mask_out,
                         void* workspace, size_t workspace_bytes, fq_stream_t stream);
int fq_quest_attend_int4(const fq_int4_cache* cache, const fq_query* query,
                         const float* retention, int32_t num_sinks, int32_t window_pages,
                         int32_t k_max, int32_t select_mode,
                         void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* PersistentInt4KVCache.update_quantized (src/flashquest/cache/persistent_int4.py:69-132)
 * for one layer of the preallocated cache described by `cache` (S = max_seq_len,
 * P = max_pages, page_size 64): the pages that the append of S_new tokens
 * completes are quantised from (the layer's partial tail, the new tokens) into
 * K_packed / K_scale / K_mn / V_packed / V_scale / V_mn, then the remaining
 * tokens are staged in the tail.  Partial tails (L, B, H_kv, page_size, D) and
 * K_new / V_new (B, H_kv, S_new, D) share one dtype (bf16 or fp16), with
 * contiguous 16-byte aligned rows.  `seen` is the layer's token count before
 * the append; the caller advances it.  Codes and metadata are those of
 * fq_quantize_k_int4 / fq_quantize_v_int4 on the concatenated stream. */
int fq_int4_cache_append(const fq_int4_cache* cache, int32_t layer,
                         void* k_partial, const int64_t kpart_strides[5],
                         void* v_partial, const int64_t vpart_strides[5], int32_t partial_dtype,
                         const void* k_new, const int64_t kn_strides[4],
                         const void* v_new, const int64_t vn_strides[4],
                         int32_t seen, int32_t S_new, fq_stream_t stream);

/* PersistentInt8KVCache.update_quantized (src/flashquest/cache/persistent_int8.py:72-135)
 * for one layer, with the arguments of fq_int4_cache_append over the INT8
 * descriptor (codes one byte per channel, v_groups = 1): completed pages get
 * fq_quantize_k_int8 / fq_quantize_v_int8's codes and metadata, the remaining
 * tokens go to the tail and the tail rows after them are zeroed, as the
 * reference's cache does. */
int fq_int8_cache_append(const fq_int8_cache* cache, int32_t layer,
                         void* k_partial, const int64_t kpart_strides[5],
                         void* v_partial, const int64_t vpart_strides[5], int32_t partial_dtype,
                         const void* k_new, const int64_t kn_strides[4],
                         const void* v_new, const int64_t vn_strides[4],
                         int32_t seen, int32_t S_new, fq_stream_t stream);

/* PersistentTurboKVCache.update_quantized (src/flashquest/cache/persistent_turbo.py:83-147)
 * for one layer of the preallocated TurboQuant cache (`cache`: the full
 * planes and per-token scales, S = max_seq_len, P = max_pages), plus the
 * un-rotated K's bf16 page scale/min K_scale_raw / K_mn_raw (L, B, H_kv, P, D).
 * Completed pages: the page metadata of fq_quantize_k_int4 (no codes) and the
 * planes and scales of fq_quantize_turbo for K and V, bit-identical to
 * quantising the whole stream; the remaining tokens go to the tail. */
int fq_turbo_cache_append(const fq_turbo_cache* cache, void* k_scale_raw, const int64_t ksr_strides[5],
                          void* k_mn_raw, const int64_t kmr_strides[5], int32_t layer,
                          void* k_partial, const int64_t kpart_strides[5],
                          void* v_partial, const int64_t vpart_strides[5], int32_t partial_dtype,
                          const void* k_new, const int64_t kn_strides[4],
                          const void* v_new, const int64_t vn_strides[4],
                          int32_t seen, int32_t S_new, fq_stream_t stream);

/* The whole decode branch of the reference's attention patch for a step with
 * a partial page (llama_persistent_patch.py:202-240): score, select and
 * attend the completed pages, attend the tail densely
 * (_bf16_dense_attn_with_lse, 30-47, sm_scale of the query) and merge
 * (_merge_two_attentions, 50-61) -- as softmax attention over the selected
 * pages and the tail together, the tail attended inside the split-merge
 * launch.  O and lse (if given) are those of the merged attention.  A NULL or
 * empty tail is fq_quest_decode_int4 without scores_out / mask_out.
 * FQ_ERR_UNSUPPORTED for shapes the matrix-core attention kernel does not take
 * (the caller then runs the three operators). */
int fq_quest_decode_int4_tail(const fq_int4_cache* cache, const fq_query* query, const fq_tail* tail,
                              const float* retention, int32_t num_sinks, int32_t window_pages,
                              int32_t k_max, int32_t select_mode,
                              void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* fq_quest_decode_int8 with the bf16 / fp16 partial-page tail attended and
 * merged in the same step (no reference counterpart; the reference's decode
 * branch runs the sparse INT8 attention, _bf16_dense_attn_with_lse and
 * _merge_two_attentions, llama_persistent_patch.py:202-245).  Returns
 * FQ_ERR_UNSUPPORTED for shapes the matrix-core INT8 kernel does not take
 * (the caller then runs the three operators). */
int fq_quest_decode_int8_tail(const fq_int8_cache* cache, const fq_query* query, const fq_tail* tail,
                              const float* retention, int32_t num_sinks, int32_t window_pages,
                              int32_t k_max, int32_t select_mode,
                              void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* Whether fq_quest_attend_int4 scores and selects the pages inside its one
 * attention kernel for these arguments (1; fq_quest_select_int4 then launches
 * nothing unless scores_out or mask_out is given) or consumes page lists left
 * by fq_quest_select_int4 (0).  Negative: an FQ_ERR_* code for invalid
 * arguments.  No reference counterpart: it tells a caller (the benchmark) which
 * kernels one decode step runs. */
int fq_quest_fused_int4(const fq_int4_cache* cache, const fq_query* query,
                        int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode);
/* The same for fq_quest_decode_int8 over the INT8 cache: 1 when the step is one
 * attention launch that scores and selects its own pages.  No reference
 * counterpart. */
int fq_quest_fused_int8(const fq_int8_cache* cache, const fq_query* query,
                        int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode);

/* _merge_two_attentions (src/flashquest/eager/llama_persistent_patch.py:50-61).
 * O_a/O_b/out (N, D) rows with row strides; lse (N,) fp32.  out dtype = O_a dtype. */
int fq_merge_attn(const void* o_a, const float* lse_a, const void* o_b, const float* lse_b,
                  int32_t dtype, int64_t o_row_stride_a, int64_t o_row_stride_b,
                  void* out, int64_t out_row_stride, float* lse_out,
                  int32_t N, int32_t D, fq_stream_t stream);

/* _bf16_dense_attn_with_lse (src/flashquest/eager/llama_persistent_patch.py:30-47).
 * Q (B,H_q,D), K/V (B,H_kv,T,D) bf16 (T <= 1024); out (B,H_q,D) bf16, lse fp32. */
int fq_dense_tail_attn(const void* q, const int64_t q_strides[3],
                       const void* k, const int64_t k_strides[4],
                       const void* v, const int64_t v_strides[4], int32_t kv_dtype,
                       void* out, const int64_t o_strides[3], float* lse,
                       int32_t B, int32_t H_q, int32_t H_kv, int32_t T, int32_t D,
                       fq_stream_t stream);

/* quantize_k_int4 (src/flashquest/kernel/kv_quant.py:131-171): K (B,H,S,D) of
 * dtype in_dtype -> packed (B,H,S,D/2), scale/mn (B,H,P,D) of meta_dtype.
 * Scale arithmetic in the input dtype, codes by fp32 IEEE division,
 * round-half-even, clamp 0..15 (bit-exact with the reference). */
int fq_quantize_k_int4(const void* k, int32_t in_dtype, const int64_t k_strides[4],
                       int32_t B, int32_t H, int32_t S, int32_t D, int32_t page_size,
                       uint8_t* packed, const int64_t p_strides[4],
                       void* scale, const int64_t s_strides[4],
                       void* mn, const int64_t m_strides[4], int32_t meta_dtype,
                       fq_stream_t stream);

/* quantize_v_int4 (src/flashquest/kernel/kv_quant.py:189-205): per token (and
 * per `group` channels; group = D reproduces the reference), fp32 arithmetic. */
int fq_quantize_v_int4(const void* v, int32_t in_dtype, const int64_t v_strides[4],
                       int32_t B, int32_t H, int32_t S, int32_t D, int32_t group,
                       uint8_t* packed, const int64_t p_strides[4],
                       void* scale, const int64_t s_strides[4],
                       void* mn, const int64_t m_strides[4], int32_t meta_dtype,
                       fq_stream_t stream);

/* wht_along_head_dim (src/flashquest/kernel/wht.py:17-41) over N rows of D
 * (power of two <= 256).  signs (D,) fp32 or NULL: out = WHT(signs * x) when
 * inverse == 0, out = signs * WHT(x) when inverse != 0.  arith_dtype rounds
 * every butterfly stage like the reference's tensor dtype (FQ_F32 = exact fp32). */
int fq_wht(const void* x, int32_t x_dtype, int64_t x_row_stride,
           void* out, int32_t out_dtype, int64_t out_row_stride,
           int32_t N, int32_t D, const float* signs, int32_t inverse, int32_t arith_dtype,
           fq_stream_t stream);

/* quantize_k_turbo / quantize_v_turbo (kv_quant.py:327-363, 381-405) for one
 * tensor X (B,H,S,D) bf16: msb (B,H,S,D/8), lsb (B,H,S,D/4), scale (B,H,S,1) bf16. */
int fq_quantize_turbo(const void* x, int32_t in_dtype, const int64_t x_strides[4],
                      int32_t B, int32_t H, int32_t S, int32_t D,
                      uint8_t* msb, const int64_t msb_strides[4],
                      uint8_t* lsb, const int64_t lsb_strides[4],
                      void* scale, const int64_t s_strides[4], fq_stream_t stream);

/* flash_attn_sparse_turbo_fwd (src/flashquest/kernel/sparse_turbo_fwd.py:254-346):
 * Q in the raw basis; the kernel rotates Q, attends over the selected pages of
 * the rotated K3-V3 cache and rotates O back.  mask (L,B,H_q,P) u8. */
int fq_sparse_turbo_fwd_mask(const fq_turbo_cache* cache, const fq_query* query,
                             const uint8_t* mask, const int64_t mask_strides[4],
                             void* workspace, size_t workspace_bytes, fq_stream_t stream);

size_t fq_turbo_workspace_bytes(const fq_turbo_cache* cache, int32_t H_q);

/* The reference's TurboQuant decode branch for completed pages
 * (llama_persistent_patch.py:152-160 with the selection of 196-245):
 * page scores from the un-rotated K's page scale/min (K_scale_raw / K_mn_raw,
 * (L, B, H_kv, P, D) bf16; criticality.py:128-163), top-k selection
 * (selection.py:65-126, or one selection per KV head from the summed group
 * scores with FQ_SELECT_PER_KV_HEAD_SUM), then flash_attn_sparse_turbo_fwd
 * (sparse_turbo_fwd.py:254-346) over the selected pages, for every
 * (layer, batch, KV head) at once.  With enough KV groups to fill the GPU,
 * D = 128, 64-token pages and mask_out NULL this is one kernel launch.
 * mask_out (optional): the (L*B, H_q, P) selection, as fq_quest_select_int4. */
int fq_quest_decode_turbo(const fq_turbo_cache* cache,
                          const void* k_scale_raw, const int64_t ksr_strides[5],
                          const void* k_mn_raw, const int64_t kmr_strides[5],
                          const fq_query* query, const float* retention,
                          int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode,
                          uint8_t* mask_out, void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* Whether fq_quest_decode_turbo selects the pages inside its matrix-core
 * attention kernel for these arguments (1: one launch with enough KV groups,
 * else a scoring launch and the attention; with 6 or 8 query heads per KV
 * head included) or not (0; the caller may then attend a KV group's query
 * heads in chunks).  Negative: an FQ_ERR_* code.  No reference counterpart:
 * it tells a caller which kernels one decode step runs. */
int fq_quest_fused_turbo(const fq_turbo_cache* cache, const fq_query* query);

/* The selection half of fq_quest_decode_turbo (the page scores and
 * select_pages_vectorized of llama_persistent_patch.py:196-245 on the raw K
 * metadata), same arguments; with mask_out it writes the (L*B, H_q, P)
 * selection and runs no attention.  Callers that attend a KV group's query
 * heads in several calls use it to select once from all of the group's heads. */
int fq_quest_select_turbo(const fq_turbo_cache* cache,
                          const void* k_scale_raw, const int64_t ksr_strides[5],
                          const void* k_mn_raw, const int64_t kmr_strides[5],
                          const fq_query* query, const float* retention,
                          int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode,
                          uint8_t* mask_out, void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* ---- INT8 family (kv_bits = 8, the reference dispatcher's default) ---- */

/* Workspace for the INT8 entry points (same sizing as fq_workspace_bytes). */
size_t fq_int8_workspace_bytes(const fq_int8_cache* cache, int32_t H_q);

/* Replaces page_scores_int8_fast (criticality.py:77-125): score = Q.K_mn +
 * 255 * relu(Q).K_scale, fp32 in this library's fixed order; same arguments
 * as fq_page_scores_int4. */
int fq_page_scores_int8(const void* q, int32_t q_dtype, const int64_t q_strides[4],
                        const void* k_scale, const int64_t ks_strides[4],
                        const void* k_mn, const int64_t km_strides[4], int32_t meta_dtype,
                        float* scores, const int64_t sc_strides[4],
                        int32_t B, int32_t H_q, int32_t S_q, int32_t H_kv, int32_t P, int32_t D,
                        fq_stream_t stream);

/* Replaces the scoring of quest_duo_fused_sdpa (duo/fused_dispatch.py:64-67):
 * dequantize_k (kernel/kv_quant.py:64-75, bf16 keys) -> compute_page_summary
 * (eager/page_summary.py:7-39, per page and channel the min / max key over
 * the page's valid tokens) -> page_scores (eager/criticality.py:7-31,
 * sum_d max(q_d * max_d, q_d * min_d) in fp32, GQA broadcast).  Decode
 * queries (B, H_q, 1, D); INT8 codes (B, H_kv, S, D) with a contiguous channel
 * axis and 4-byte aligned token rows; K scale / min (B, H_kv, P, D) in
 * meta_dtype, P = ceil(S / page_size); scores (B, H_q, 1, P).  page_min /
 * page_max (bf16, strides pm_strides, (B, H_kv, P, D)): the summaries, or
 * both NULL.  fp32 order: per 4 channels left to right, then a butterfly over
 * the D/4 partial sums. */
int fq_page_scores_int8_summary(const void* q, int32_t q_dtype, const int64_t q_strides[4],
                                const uint8_t* k_codes, const int64_t kc_strides[4],
                                const void* k_scale, const int64_t ks_strides[4],
                                const void* k_mn, const int64_t km_strides[4], int32_t meta_dtype,
                                uint16_t* page_min, uint16_t* page_max, const int64_t pm_strides[4],
                                float* scores, const int64_t sc_strides[4],
                                int32_t B, int32_t H_q, int32_t H_kv, int32_t S, int32_t P, int32_t D,
                                int32_t page_size, fq_stream_t stream);

/* Replaces compute_page_summary (eager/page_summary.py:7-39): per page and
 * channel the minimum and maximum of K (B, H, S, D; bf16, fp16 or fp32, any
 * strides) over the page's valid tokens (a partial last page: its tokens),
 * NaN propagating; page_min / page_max (B, H, ceil(S / page_size), D) in K's
 * dtype. */
int fq_page_summary(const void* k, int32_t k_dtype, const int64_t k_strides[4], int32_t B, int32_t H,
                    int32_t S, int32_t D, int32_t page_size, void* page_min, void* page_max,
                    const int64_t pm_strides[4], fq_stream_t stream);

/* Replaces page_scores (eager/criticality.py:7-31): scores (B, H_q, S_q, P)
 * fp32 = sum_d max(q_d * max_d, q_d * min_d) for queries (B, H_q, S_q, D) and
 * page bounds (B, H_kv, P, D) in bound_dtype, query head h reading bound row
 * h / (H_q / H_kv) (H_kv = H_q: the reference's one row per head).  fp32
 * order as fq_page_scores_int8_summary.  D in (64, 128). */
int fq_page_scores_quest(const void* q, int32_t q_dtype, const int64_t q_strides[4],
                         const void* page_min, const int64_t pmin_strides[4],
                         const void* page_max, const int64_t pmax_strides[4], int32_t bound_dtype,
                         float* scores, const int64_t sc_strides[4],
                         int32_t B, int32_t H_q, int32_t S_q, int32_t H_kv, int32_t P, int32_t D,
                         fq_stream_t stream);

/* Replaces page_scores_int8 (eager/criticality.py:34-74): the same scores
 * with the bounds taken from the INT8 page metadata as the reference forms
 * them, min = fp32(K_mn), max = fp32(K_mn) + 255 * fp32(K_scale) (fp32
 * multiply, then add).  Arguments as fq_page_scores_int8. */
int fq_page_scores_int8_bound(const void* q, int32_t q_dtype, const int64_t q_strides[4],
                              const void* k_scale, const int64_t ks_strides[4],
                              const void* k_mn, const int64_t km_strides[4], int32_t meta_dtype,
                              float* scores, const int64_t sc_strides[4],
                              int32_t B, int32_t H_q, int32_t S_q, int32_t H_kv, int32_t P, int32_t D,
                              fq_stream_t stream);

/* Replaces flash_attn_sparse_fwd (kernel/sparse_fwd.py:160-228, kernel
 * 23-157): sparse GQA decode attention over the INT8 cache for a boolean page
 * mask (L*B, H_q, P) (strides as fq_sparse_int4_fwd_mask). */
int fq_sparse_int8_fwd_mask(const fq_int8_cache* cache, const fq_query* query,
                            const uint8_t* mask, const int64_t mask_strides[4],
                            void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* The INT8 decode step of llama_persistent_patch.py:143-160 with the selection
 * of 196-245 (page_scores_int8_fast, select_pages_vectorized,
 * flash_attn_sparse_fwd) for every (layer, batch, KV head) at once; arguments
 * as fq_quest_decode_int4. */
int fq_quest_decode_int8(const fq_int8_cache* cache, const fq_query* query, const float* retention,
                         int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode,
                         float* scores_out, uint8_t* mask_out, void* workspace, size_t workspace_bytes,
                         fq_stream_t stream);

/* The selection half of fq_quest_decode_int8 (page_scores_int8_fast and
 * select_pages_vectorized of llama_persistent_patch.py:143-160, 196-245),
 * as fq_quest_select_int4 for the INT8 cache: with mask_out it always writes
 * the (L*B, H_q, P) selection.  Callers that attend a KV group's query heads
 * in several calls use it to select once from all of the group's heads. */
int fq_quest_select_int8(const fq_int8_cache* cache, const fq_query* query, const float* retention,
                         int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode,
                         float* scores_out, uint8_t* mask_out, void* workspace, size_t workspace_bytes,
                         fq_stream_t stream);

/* Replace quantize_k / quantize_v (kernel/kv_quant.py:43-61, 78-89): uint8
 * codes, K scale/min per (page, channel) with the arithmetic in the input
 * dtype ("/ 255.0"), V per token in fp32; metadata written as meta_dtype. */
int fq_quantize_k_int8(const void* k, int32_t in_dtype, const int64_t k_strides[4],
                       int32_t B, int32_t H, int32_t S, int32_t D, int32_t page_size,
                       uint8_t* codes, const int64_t c_strides[4],
                       void* scale, const int64_t s_strides[4],
                       void* mn, const int64_t m_strides[4], int32_t meta_dtype,
                       fq_stream_t stream);
int fq_quantize_v_int8(const void* v, int32_t in_dtype, const int64_t v_strides[4],
                       int32_t B, int32_t H, int32_t S, int32_t D,
                       uint8_t* codes, const int64_t c_strides[4],
                       void* scale, const int64_t s_strides[4],
                       void* mn, const int64_t m_strides[4], int32_t meta_dtype,
                       fq_stream_t stream);

/* Prefill query and output of fq_prefill_int4 / fq_prefill_int8:
 * Q, O (B, H_q, S_q, D) bf16, element strides, channels contiguous. */
typedef struct fq_prefill {
    const void* q; int64_t q_strides[4];
    void* out;     int64_t o_strides[4];
    int32_t H_q, S_q;
    int32_t causal_offset; /* query i attends keys j <= i + causal_offset (>= 0); 0 = torch is_causal */
    float sm_scale;        /* <= 0 selects 1/sqrt(D) */
    int32_t D;             /* head_dim of Q and O: must equal the cache's */
} fq_prefill;

/* The S_q > 1 (prefill) branch of the reference's attention patch,
 * src/flashquest/eager/llama_persistent_patch.py:196-201:
 *   SDPA(q, cat(dequantize_k_int4(cache), K_partial),
 *           cat(dequantize_v_int4(cache), V_partial), is_causal=True, enable_gqa=True)
 * with dequantize_k_int4 / dequantize_v_int4 of kernel/kv_quant.py:174-186,
 * 208-215, fused: the packed codes are dequantised to bf16 tile by tile in the
 * attention kernel.  cache: one layer (L == 1), S completed tokens (S may be 0),
 * D == 128; tail: the bf16 partial-page rows (len >= 0, any length), keys S..
 * S + len - 1.  FQ_ERR_UNSUPPORTED for layouts the kernel does not take. */
int fq_prefill_int4(const fq_int4_cache* cache, const fq_tail* tail, const fq_prefill* query,
                    void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* The same over the INT8 cache (llama_persistent_patch.py:143-150:
 * dequantize_k / dequantize_v, kernel/kv_quant.py:64-100). */
int fq_prefill_int8(const fq_int8_cache* cache, const fq_tail* tail, const fq_prefill* query,
                    void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* The prefill branch over the TurboQuant cache (llama_persistent_patch.py:
 * 93-102, 196-201: dequantize_k_turbo / dequantize_v_turbo, kernel/kv_quant.py:
 * 366-420, i.e. codebook * scale, inverse WHT, bf16; then causal SDPA over
 * cat(dequantised, K_partial / V_partial)).  cache: one layer (L == 1),
 * D == 128, S completed tokens (may be 0).  Always needs the workspace of
 * fq_prefill_turbo_workspace_bytes (dense bf16 K and V^T of the attended keys). */
int fq_prefill_turbo(const fq_turbo_cache* cache, const fq_tail* tail, const fq_prefill* query,
                     void* workspace, size_t workspace_bytes, fq_stream_t stream);
/* No reference counterpart: workspace bytes of fq_prefill_turbo (0 for invalid arguments). */
size_t fq_prefill_turbo_workspace_bytes(const fq_turbo_cache* cache, const fq_tail* tail, const fq_prefill* query);

/* Workspace bytes fq_prefill_int4 (bits 4) / fq_prefill_int8 (bits 8) needs for
 * these arguments: 0 when the attention kernel dequantises its own K/V tiles
 * (at most 256 / n_rep query rows over at most 1024 attended keys), else room
 * for the dense bf16 K and V^T of the two-pass path (the attended keys
 * dequantised once, 2 * 2 * 128 B per key and KV head, keys rounded up to 128).  0 also for invalid
 * arguments (the call then reports the error).  No reference counterpart. */
size_t fq_prefill_workspace_bytes(const fq_int4_cache* cache, const fq_tail* tail, const fq_prefill* query,
                                  int32_t bits);

#ifdef __cplusplus
}
#endif
#endif /* FQ_HIP_H */
