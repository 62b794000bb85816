// C ABI of libfq_hip: argument validation, workspace carving and launches.
// Declarations and reference citations: include/fq_hip.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "fq_common.h"

namespace fq {
hipError_t launch_quant_k(const void* k, int in_dtype, const int64_t* k_s, int B, int H, int S, int D,
                          int page, uint8_t* packed, const int64_t* p_s, void* scale, const int64_t* s_s,
                          void* mn, const int64_t* m_s, int meta_dtype, hipStream_t st, int bits = 4);
hipError_t launch_quant_v(const void* v, int in_dtype, const int64_t* v_s, int B, int H, int S, int D,
                          int group, uint8_t* packed, const int64_t* p_s, void* scale, const int64_t* s_s,
                          void* mn, const int64_t* m_s, int meta_dtype, hipStream_t st, int bits = 4);
hipError_t launch_wht(const void* x, int x_dtype, int64_t x_rs, void* out, int out_dtype, int64_t o_rs,
                      int N, int D, const float* signs, int inverse, int arith, hipStream_t st);
hipError_t launch_turbo_quant(const void* x, int in_dtype, const int64_t* x_s, int B, int H, int S, int D,
                              uint8_t* msb, const int64_t* msb_s, uint8_t* lsb, const int64_t* lsb_s,
                              void* scale, const int64_t* s_s, hipStream_t st);
hipError_t launch_merge(const void* oa, const float* la, const void* ob, const float* lb, int dtype,
                        int64_t rs_a, int64_t rs_b, void* out, int64_t rs_o, float* lse_out, int N, int D,
                        hipStream_t st);
hipError_t launch_tail(const void* q, const int64_t* q_s, const void* k, const int64_t* k_s, const void* v,
                       const int64_t* v_s, int kv_dtype, void* out, const int64_t* o_s, float* lse, int B,
                       int Hq, int Hkv, int T, int D, hipStream_t st);
hipError_t launch_attn_turbo(const fq_turbo_cache& c, const QueryArgs& q, const Workspace& ws,
                             const AttnLaunch& al, hipStream_t st);
hipError_t launch_prefill(const Int4Cache& c, const TailArgs& t, const void* q, const int64_t* q_s, void* out,
                          const int64_t* o_s, int nrep, int Sq, int causal_off, float qk_scale, void* ws,
                          hipStream_t st);
size_t prefill_workspace_bytes(const Int4Cache& c, int Skv, int Sq, int nrep, int causal_off);
size_t prefill_turbo_workspace_bytes(int Hkv, int B, int Skv, int Sq, int nrep, int causal_off);
hipError_t launch_prefill_turbo(const fq_turbo_cache& tc, const TailArgs& t, const void* q, const int64_t* q_s,
                                void* out, const int64_t* o_s, int nrep, int Sq, int causal_off, float qk_scale,
                                void* ws, hipStream_t st);

static thread_local std::string g_err;

// Armed by fq_kernel_timer_start: event pairs recorded around attention kernels.
struct KernelTimer {
    std::vector<hipEvent_t> start, stop;
    int used = 0;
    bool armed = false;
};
static thread_local KernelTimer g_timer;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return FQ_OK;
    return fail(FQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static int s_max_for(int P) { return (P + 3) / 4; }

size_t workspace_bytes(int G, int P, int rows, int nrep, int D) {
    const size_t sm = (size_t)s_max_for(P);
    size_t n = 0;
    n += align256(sizeof(int) * G);                     // n_sel
    n += align256(sizeof(int) * (size_t)G * P);         // entries
    n += align256(sizeof(float) * (size_t)G * rows * P);
    n += align256(sizeof(float) * (size_t)G * sm * nrep * 2);
    n += align256(sizeof(float) * (size_t)G * sm * nrep * D);
    return n;
}

Workspace carve_workspace(void* base, int G, int P, int rows, int nrep, int D) {
    Workspace w{};
    char* p = (char*)base;
    const size_t sm = (size_t)s_max_for(P);
    w.n_sel = (int*)p;        p += align256(sizeof(int) * G);
    w.entries = (int*)p;      p += align256(sizeof(int) * (size_t)G * P);
    w.scores = (float*)p;     p += align256(sizeof(float) * (size_t)G * rows * P);
    w.part_ml = (float*)p;    p += align256(sizeof(float) * (size_t)G * sm * nrep * 2);
    w.part_acc = (float*)p;
    w.s_max = (int)sm;
    return w;
}

AttnLaunch choose_split(int G, int max_entries, int s_max) {
    AttnLaunch al{};
    if (max_entries < 1) max_entries = 1;
    // aim for ~1536 workgroups in flight (6 per CU on 256 CUs), >= 1 page per wave
    const long target = 1536;
    long pps = ((long)G * max_entries + 4 * target - 1) / (4 * target) * 4;
    if (pps < 4) pps = 4;
    if (pps > 32) pps = 32;          // <= 8 pages per wave (the MFMA kernel keeps their logits in LDS)
    long splits = (max_entries + pps - 1) / pps;
    if (splits > s_max) {
        pps = ((max_entries + s_max - 1) / s_max + 3) / 4 * 4;
        splits = (max_entries + pps - 1) / pps;
    }
    al.pages_per_split = (int)pps;
    al.splits = (int)(splits < 1 ? 1 : splits);
    al.max_entries = max_entries;
    al.s_max = s_max;
    return al;
}

static bool is_half(int dt) { return dt == FQ_BF16 || dt == FQ_F16; }
static bool is_float_dtype(int dt) { return dt == FQ_BF16 || dt == FQ_F16 || dt == FQ_F32; }

// 16-byte aligned base and rows: every stride but the innermost, in bytes.
static bool rows_aligned16(const void* p, const int64_t* strides, int n_outer, int esize) {
    if ((uintptr_t)p & 15) return false;
    for (int i = 0; i < n_outer; ++i)
        if ((strides[i] * esize) % 16) return false;
    return true;
}

// bits = 4: packed INT4 (two codes per byte); bits = 8: one code byte per
// channel (the INT8 cache of flash_attn_sparse_fwd), V metadata per token.
int check_cache(const fq_int4_cache* c, Int4Cache* out, int bits, bool allow_empty) {
    if (!c) return fail(FQ_ERR_INVALID, "cache descriptor is NULL");
    if (c->D != 64 && c->D != 128) return fail(FQ_ERR_UNSUPPORTED, "head_dim=%d not in (64, 128)", c->D);
    if (!is_half(c->meta_dtype)) return fail(FQ_ERR_UNSUPPORTED, "metadata dtype must be bf16 or fp16");
    if (c->L < 1 || c->B < 1 || c->H_kv < 1) return fail(FQ_ERR_INVALID, "empty L/B/H_kv");
    if (allow_empty && c->S == 0) {   // no completed pages: nothing of the cache is read
        Int4Cache& o = *out;
        o = Int4Cache{};
        o.L = c->L; o.B = c->B; o.Hkv = c->H_kv; o.D = c->D; o.page = c->page_size > 0 ? c->page_size : 1;
        o.G = 1; o.meta_dtype = c->meta_dtype; o.bits = bits;
        return FQ_OK;
    }
    if (c->P < 1 || c->P > kMaxPages) return fail(FQ_ERR_UNSUPPORTED, "pages=%d outside [1, %d]", c->P, kMaxPages);
    if (c->page_size < 1 || c->page_size > 4096) return fail(FQ_ERR_INVALID, "page_size=%d", c->page_size);
    if (c->S < 0) return fail(FQ_ERR_INVALID, "negative S");
    if (c->v_groups != 1 && c->v_groups != c->D / 32)
        return fail(FQ_ERR_UNSUPPORTED, "V groups=%d must be 1 or D/32", c->v_groups);
    if (bits == 8 && c->v_groups != 1) return fail(FQ_ERR_UNSUPPORTED, "INT8 V metadata is per token (v_groups=1)");
    if (!c->k_packed || !c->v_packed || !c->k_scale || !c->k_mn || !c->v_scale || !c->v_mn)
        return fail(FQ_ERR_INVALID, "NULL cache tensor");
    for (int i = 0; i < 4; ++i) {
        if (c->k_strides[i] % bits || c->v_strides[i] % bits)
            return fail(FQ_ERR_UNSUPPORTED, "K/V code strides must be multiples of %d bytes", bits);
        if (c->ks_strides[i] % 8 || c->km_strides[i] % 8)
            return fail(FQ_ERR_UNSUPPORTED, "K metadata strides must be multiples of 8 elements");
    }
    if (c->k_strides[4] != 1 || c->v_strides[4] != 1 || c->ks_strides[4] != 1 || c->km_strides[4] != 1 ||
        c->vs_strides[4] != 1 || c->vm_strides[4] != 1)
        return fail(FQ_ERR_UNSUPPORTED, "innermost cache axis must be contiguous");
    if (((uintptr_t)c->k_packed | (uintptr_t)c->v_packed) & (bits - 1))
        return fail(FQ_ERR_UNSUPPORTED, "K/V codes must be %d-byte aligned", bits);
    if (((uintptr_t)c->k_scale | (uintptr_t)c->k_mn) & 15)
        return fail(FQ_ERR_UNSUPPORTED, "K metadata must be 16-byte aligned");
    Int4Cache& o = *out;
    o.kp = c->k_packed; o.vp = c->v_packed; o.ksc = c->k_scale; o.kmn = c->k_mn;
    o.vsc = c->v_scale; o.vmn = c->v_mn;
    for (int i = 0; i < 4; ++i) {
        o.kp_s[i] = c->k_strides[i]; o.vp_s[i] = c->v_strides[i];
        o.ksc_s[i] = c->ks_strides[i]; o.kmn_s[i] = c->km_strides[i];
        o.vsc_s[i] = c->vs_strides[i]; o.vmn_s[i] = c->vm_strides[i];
    }
    o.L = c->L; o.B = c->B; o.Hkv = c->H_kv; o.S = c->S; o.P = c->P; o.D = c->D;
    o.page = c->page_size; o.G = c->v_groups; o.meta_dtype = c->meta_dtype; o.bits = bits;
    return FQ_OK;
}

static int check_query(const fq_query* q, int D, int Hkv, QueryArgs* out) {
    if (!q || !q->q || !q->out) return fail(FQ_ERR_INVALID, "query/output is NULL");
    if (!is_float_dtype(q->q_dtype) || !is_float_dtype(q->out_dtype))
        return fail(FQ_ERR_INVALID, "query/output dtype must be bf16, fp16 or fp32");
    if (q->H_q < 1 || q->H_q % Hkv) return fail(FQ_ERR_INVALID, "H_q=%d must be divisible by H_kv=%d", q->H_q, Hkv);
    const int nrep = q->H_q / Hkv;
    if (nrep > 8)    // the selection keeps one bit per query head of a group
        return fail(FQ_ERR_UNSUPPORTED, "GQA ratio %d above 8", nrep);
    QueryArgs& o = *out;
    o.q = q->q; o.q_dtype = q->q_dtype; o.out = q->out; o.out_dtype = q->out_dtype; o.lse = q->lse;
    for (int i = 0; i < 4; ++i) { o.q_s[i] = q->q_strides[i]; o.o_s[i] = q->o_strides[i]; }
    for (int i = 0; i < 3; ++i) o.lse_s[i] = q->lse_strides[i];
    o.Hq = q->H_q; o.nrep = nrep;
    if (q->retention_layer_stride < 0 || (q->retention_layer_stride > 0 && q->retention_layer_stride < q->H_q))
        return fail(FQ_ERR_INVALID, "retention layer stride %lld must be 0 or at least H_q=%d",
                    (long long)q->retention_layer_stride, q->H_q);
    o.ret_ls = q->retention_layer_stride;
    o.rot = q->rotation_signs;
    if (o.rot && D != 128) return fail(FQ_ERR_UNSUPPORTED, "the rotated decode takes head_dim 128");
    const float sm = q->sm_scale > 0.f ? q->sm_scale : 1.0f / sqrtf((float)D);
    o.qk_scale = sm * kLog2e;
    return FQ_OK;
}

static std::atomic<int> g_split_request{0};
// code width for fq_page_scores_int4's scoring constant (set by fq_page_scores_int8 for its call)
static thread_local int g_score_bits = 4;
int attention_splits_request() { return g_split_request.load(std::memory_order_relaxed); }

void timer_before_launch(hipStream_t st) {
    KernelTimer& t = g_timer;
    if (t.armed && t.used < (int)t.start.size()) (void)hipEventRecord(t.start[t.used], st);
}
void timer_after_launch(hipStream_t st) {
    KernelTimer& t = g_timer;
    if (t.armed && t.used < (int)t.stop.size()) (void)hipEventRecord(t.stop[t.used++], st);
}

}  // namespace fq

using namespace fq;

// Scratch of fq_quest_decode_int4_noalloc: one array per GPU (each device holds
// its own copy at its own address), held until the process ends.  Its host-side
// name is only a stand-in: kernels get the device address that
// hipGetSymbolAddress returns, looked up once per device and kept here.
static __device__ __align__(256) unsigned char scratch[FQ_NOALLOC_SCRATCH_BYTES];
static constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices];

static int noalloc_scratch(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxScratchDevices) return fail(FQ_ERR_UNSUPPORTED, "device %d: scratch table holds %d devices", dev, kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
        if (!p || ((uintptr_t)p & 255)) return fail(FQ_ERR_HIP, "scratch address %p is not 256-byte aligned", p);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return FQ_OK;
}

extern "C" {

int fq_set_attention_splits(int32_t splits) {
    if (splits < 0) return fail(FQ_ERR_INVALID, "splits must be >= 0");
    g_split_request.store(splits, std::memory_order_relaxed);
    return FQ_OK;
}

int fq_kernel_timer_start(int32_t max_launches) {
    KernelTimer& t = g_timer;
    if (max_launches < 1) return fail(FQ_ERR_INVALID, "max_launches must be positive");
    while ((int)t.start.size() < max_launches) {
        hipEvent_t a, b;
        if (hipEventCreate(&a) != hipSuccess) return fail(FQ_ERR_HIP, "hipEventCreate failed");
        if (hipEventCreate(&b) != hipSuccess) { (void)hipEventDestroy(a); return fail(FQ_ERR_HIP, "hipEventCreate failed"); }
        t.start.push_back(a);
        t.stop.push_back(b);
    }
    t.used = 0;
    t.armed = true;
    return FQ_OK;
}

int fq_kernel_timer_stop(float* total_ms, int32_t* launches) {
    KernelTimer& t = g_timer;
    if (!t.armed) return fail(FQ_ERR_INVALID, "kernel timer not started");
    t.armed = false;
    float sum = 0.f;
    for (int i = 0; i < t.used; ++i) {
        if (hipEventSynchronize(t.stop[i]) != hipSuccess) return fail(FQ_ERR_HIP, "hipEventSynchronize failed");
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, t.start[i], t.stop[i]) != hipSuccess) return fail(FQ_ERR_HIP, "hipEventElapsedTime failed");
        sum += ms;
    }
    if (total_ms) *total_ms = sum;
    if (launches) *launches = t.used;
    return FQ_OK;
}

const char* fq_last_error(void) { return g_err.c_str(); }
int fq_abi_version(void) { return 1; }

size_t fq_workspace_bytes(const fq_int4_cache* cache, int32_t H_q) {
    if (!cache || cache->H_kv < 1 || H_q % cache->H_kv) return 0;
    const int G = cache->L * cache->B * cache->H_kv;
    const int nrep = H_q / cache->H_kv;
    return workspace_bytes(G, cache->P, nrep, nrep, cache->D);
}

int fq_page_scores_int4(const void* q, int32_t q_dtype, const int64_t q_strides[4], const void* k_scale,
                        const int64_t ks_strides[4], const void* k_mn, const int64_t km_strides[4],
                        int32_t meta_dtype, float* scores, const int64_t sc_strides[4], int32_t B,
                        int32_t H_q, int32_t S_q, int32_t H_kv, int32_t P, int32_t D, fq_stream_t stream) {
    if (H_kv < 1 || H_q % H_kv) return fail(FQ_ERR_INVALID, "H_q=%d must be divisible by H_kv=%d", H_q, H_kv);
    if (D != 64 && D != 128) return fail(FQ_ERR_UNSUPPORTED, "head_dim=%d not in (64, 128)", D);
    if (!is_half(meta_dtype) || !is_float_dtype(q_dtype)) return fail(FQ_ERR_UNSUPPORTED, "dtype");
    if (P > kMaxPages) return fail(FQ_ERR_UNSUPPORTED, "pages=%d > %d", P, kMaxPages);
    if ((H_q / H_kv) * S_q > kMaxRows) return fail(FQ_ERR_UNSUPPORTED, "n_rep * S_q > %d", kMaxRows);
    if (B == 0 || P == 0 || S_q == 0) return FQ_OK;
    if (ks_strides[3] != 1 || km_strides[3] != 1 || ks_strides[2] % 8 || km_strides[2] % 8 ||
        ks_strides[1] % 8 || km_strides[1] % 8 || ks_strides[0] % 8 || km_strides[0] % 8 ||
        (((uintptr_t)k_scale | (uintptr_t)k_mn) & 15))
        return fail(FQ_ERR_UNSUPPORTED, "K metadata must be 16-byte aligned with a contiguous channel axis");
    Int4Cache c{};
    c.ksc = k_scale; c.kmn = k_mn;
    c.ksc_s[0] = 0; c.kmn_s[0] = 0;
    for (int i = 0; i < 3; ++i) { c.ksc_s[i + 1] = ks_strides[i]; c.kmn_s[i + 1] = km_strides[i]; }
    c.L = 1; c.B = B; c.Hkv = H_kv; c.P = P; c.D = D; c.meta_dtype = meta_dtype; c.bits = g_score_bits;
    QueryArgs qa{};
    qa.q = q; qa.q_dtype = q_dtype; qa.q_s[0] = 0; qa.Hq = H_q; qa.nrep = H_q / H_kv;
    return hip_status(launch_score(c, qa, S_q, q_strides, scores, sc_strides, nullptr, 0, nullptr, 0, 0, -1,
                                   nullptr, (hipStream_t)stream),
                      "page scores");
}

int fq_select_pages(const float* scores, const int64_t sc_strides[4], int32_t B, int32_t H, int32_t S_q,
                    int32_t P, const float* retention, int32_t num_sinks, int32_t window_pages, int32_t k_max,
                    uint8_t* mask, const int64_t mask_strides[4], fq_stream_t stream) {
    if (P > kMaxPages) return fail(FQ_ERR_UNSUPPORTED, "pages=%d > %d", P, kMaxPages);
    if (!retention) return fail(FQ_ERR_INVALID, "retention is NULL");
    if (B * H * S_q == 0 || P == 0) return FQ_OK;
    return hip_status(launch_select_rows(scores, sc_strides, B, H, S_q, P, retention, num_sinks < 0 ? 0 : num_sinks,
                                         window_pages < 0 ? 0 : window_pages, k_max, mask, mask_strides,
                                         (hipStream_t)stream),
                      "select pages");
}

int fq_compact_ids(const uint8_t* mask, const int64_t mask_strides[4], int32_t B, int32_t H, int32_t S_q,
                   int32_t P, int32_t bucket_max, int32_t* ids, fq_stream_t stream) {
    if (bucket_max < 1) return fail(FQ_ERR_INVALID, "BUCKET_MAX must be >= 1, got %d", bucket_max);
    if (B * H * S_q == 0) return FQ_OK;
    return hip_status(launch_compact_ids(mask, mask_strides, B, H, S_q, P, bucket_max, ids, (hipStream_t)stream),
                      "compact ids");
}

static int attn_common(const fq_int4_cache* cache, const fq_query* query, void* workspace,
                       size_t workspace_bytes_, Int4Cache* c, QueryArgs* q, Workspace* ws, int bits = 4) {
    int st = check_cache(cache, c, bits);
    if (st) return st;
    st = check_query(query, c->D, c->Hkv, q);
    if (st) return st;
    if (((uintptr_t)q->q) & 1) return fail(FQ_ERR_UNSUPPORTED, "query must be 2-byte aligned");
    if (q->rot && bits == 8) return fail(FQ_ERR_UNSUPPORTED, "the rotated decode is INT4 only");
    const int G = c->L * c->B * c->Hkv;
    const size_t need = workspace_bytes(G, c->P, q->nrep, q->nrep, c->D);
    if (!workspace || workspace_bytes_ < need)
        return fail(FQ_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, workspace_bytes_);
    if ((uintptr_t)workspace & 255) return fail(FQ_ERR_WORKSPACE, "workspace must be 256-byte aligned");
    *ws = carve_workspace(workspace, G, c->P, q->nrep, q->nrep, c->D);
    return FQ_OK;
}

static int sparse_fwd_mask(const fq_int4_cache* cache, const fq_query* query, const uint8_t* mask,
                           const int64_t mask_strides[4], void* workspace, size_t workspace_bytes_,
                           fq_stream_t stream, int bits) {
    Int4Cache c{};
    QueryArgs q{};
    Workspace ws{};
    int st = attn_common(cache, query, workspace, workspace_bytes_, &c, &q, &ws, bits);
    if (st) return st;
    if (!mask) return fail(FQ_ERR_INVALID, "selection mask is NULL");
    if (q.rot) return fail(FQ_ERR_UNSUPPORTED, "rotation is a decode-step option (fq_quest_decode_int4)");
    hipStream_t s = (hipStream_t)stream;
    st = hip_status(launch_union_from_mask(mask, mask_strides, c.L, c.B, c.Hkv, q.nrep, c.P, ws, s), "page union");
    if (st) return st;
    const AttnLaunch al = choose_split(c.L * c.B * c.Hkv, c.P, ws.s_max);
    return hip_status(launch_attn_int4(c, q, ws, al, s), bits == 8 ? "sparse int8 attention" : "sparse int4 attention");
}

int fq_sparse_int4_fwd_mask(const fq_int4_cache* cache, const fq_query* query, const uint8_t* mask,
                            const int64_t mask_strides[4], void* workspace, size_t workspace_bytes_,
                            fq_stream_t stream) {
    return sparse_fwd_mask(cache, query, mask, mask_strides, workspace, workspace_bytes_, stream, 4);
}

int fq_sparse_int8_fwd_mask(const fq_int8_cache* cache, const fq_query* query, const uint8_t* mask,
                            const int64_t mask_strides[4], void* workspace, size_t workspace_bytes_,
                            fq_stream_t stream) {
    return sparse_fwd_mask(cache, query, mask, mask_strides, workspace, workspace_bytes_, stream, 8);
}

int fq_sparse_int4_fwd_ids(const fq_int4_cache* cache, const fq_query* query, const int32_t* ids,
                           const int64_t id_strides[4], int32_t bucket, void* workspace, size_t workspace_bytes_,
                           fq_stream_t stream) {
    Int4Cache c{};
    QueryArgs q{};
    Workspace ws{};
    int st = attn_common(cache, query, workspace, workspace_bytes_, &c, &q, &ws);
    if (st) return st;
    if (!ids || bucket < 1) return fail(FQ_ERR_INVALID, "page id list is NULL or empty");
    if (q.rot) return fail(FQ_ERR_UNSUPPORTED, "rotation is a decode-step option (fq_quest_decode_int4)");
    hipStream_t s = (hipStream_t)stream;
    st = hip_status(launch_union_from_ids(ids, id_strides, bucket, c.L, c.B, c.Hkv, q.nrep, c.P, ws, s),
                    "page union");
    if (st) return st;
    long bound = (long)q.nrep * bucket;
    if (bound > c.P) bound = c.P;
    const AttnLaunch al = choose_split(c.L * c.B * c.Hkv, (int)bound, ws.s_max);
    return hip_status(launch_attn_int4(c, q, ws, al, s), "sparse int4 attention");
}

static int quest_bound(const Int4Cache& c, const QueryArgs& q, int num_sinks, int window_pages, int k_max,
                       int select_mode) {
    long bound = c.P;
    if (k_max >= 0) {
        const long per = (long)k_max + num_sinks + window_pages;
        bound = select_mode == FQ_SELECT_PER_Q_HEAD ? per * q.nrep : per;
        if (bound > c.P) bound = c.P;
    }
    return (int)bound;
}

// The fused decode's attention kernel scores and selects its own pages when it
// takes a whole KV group per workgroup; fq_quest_select_int4 then launches
// nothing unless the caller asks for the scores or the mask.
static int mfma_head_chunks(Int4Cache& c, QueryArgs& q, int num_sinks, int window_pages, int k_max, int select_mode,
                            int s_max, const TailArgs* tail);

static bool decode_selects_in_attention(const Int4Cache& c, const QueryArgs& q, int num_sinks, int window_pages,
                                        int k_max, int select_mode, const Workspace& ws) {
    const AttnLaunch al = choose_split(c.L * c.B * c.Hkv, quest_bound(c, q, num_sinks, window_pages, k_max,
                                                                      select_mode), ws.s_max);
    return attn_selects_in_kernel(c, q, al);
}

// Decode steps that split KV groups over several workgroups (too few groups
// to fill the GPU) score each group once in a scoring launch over all CUs; the
// attention workgroups then select from those scores (kSelectOnly) instead of
// each re-scoring the group's pages.  INT4 and INT8, unrotated.
static bool attend_from_scores(const Int4Cache& c, const QueryArgs& q, int bound) {
    return c.L * c.B * c.Hkv < 192 && !q.rot && bound > kFusedSmallPages;
}

// 6 or 8 query heads per KV head on the INT4 / INT8 matrix-core decode,
// whose workgroups take at most 4: when the attention kernel selects for
// itself, every KV head of the cache becomes 2 virtual KV heads of 3 or 4
// query heads, each its own workgroup(s), all reading the same cache head
// (the kernel maps them back; per_kv_head_sum selects from the summed query
// of all the head's queries in each, so every chunk takes the same pages).
// Split steps select from the scores of a scoring launch over the real KV
// heads.  Rewrites c / q to the virtual heads and returns the chunk count,
// or 1 with c / q untouched.
static int mfma_head_chunks(Int4Cache& c, QueryArgs& q, int num_sinks, int window_pages, int k_max, int select_mode,
                            int s_max, const TailArgs* tail) {
    if ((c.bits != 4 && c.bits != 8) || q.rot || (q.nrep != 6 && q.nrep != 8)) return 1;
    if (tail && tail->len > 0 && !mfma_tail_in_kernel(*tail)) return 1;
    Int4Cache c2 = c;
    QueryArgs q2 = q;
    c2.Hkv *= 2;
    q2.nrep /= 2;
    const int bound = quest_bound(c2, q2, num_sinks, window_pages, k_max, select_mode);
    const AttnLaunch al = choose_split(c2.L * c2.B * c2.Hkv, bound, s_max);
    if (!attn_selects_in_kernel(c2, q2, al)) return 1;
    c = c2;
    q = q2;
    return 2;
}

static int quest_select(const fq_int4_cache* cache, const fq_query* query, const float* retention,
                        int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode,
                        float* scores_out, uint8_t* mask_out, void* workspace, size_t workspace_bytes_,
                        fq_stream_t stream, int bits, bool mask_from_attention = false) {
    Int4Cache c{};
    QueryArgs q{};
    Workspace ws{};
    int st = attn_common(cache, query, workspace, workspace_bytes_, &c, &q, &ws, bits);
    if (st) return st;
    if (!retention) return fail(FQ_ERR_INVALID, "retention is NULL");
    if (select_mode != FQ_SELECT_PER_Q_HEAD && select_mode != FQ_SELECT_PER_KV_HEAD_SUM)
        return fail(FQ_ERR_INVALID, "select_mode=%d", select_mode);
    if (num_sinks < 0) num_sinks = 0;
    if (window_pages < 0) window_pages = 0;
    if (k_max > c.P) k_max = c.P;
    const int64_t q4[4] = {q.q_s[1], q.q_s[2], 0, q.q_s[3]};
    int64_t sc4[4] = {(int64_t)q.Hq * c.P, c.P, c.P, 1};   // (L*B, H_q, 1, P) contiguous
    float* sc_user = (scores_out && select_mode == FQ_SELECT_PER_Q_HEAD) ? scores_out : nullptr;
    // the fused attention kernel selects for itself (and, when the whole step
    // is one call, writes the mask too); vc / vq: the heads it runs (virtual
    // heads with 6 or 8 query heads per KV head), the scoring launch takes the
    // real ones
    Int4Cache vc = c;
    QueryArgs vq = q;
    mfma_head_chunks(vc, vq, num_sinks, window_pages, k_max, select_mode, ws.s_max, nullptr);
    if ((!mask_out || mask_from_attention) && !sc_user &&
        decode_selects_in_attention(vc, vq, num_sinks, window_pages, k_max, select_mode, ws)) {
        if (!attend_from_scores(vc, vq, quest_bound(vc, vq, num_sinks, window_pages, k_max, select_mode)))
            return FQ_OK;      // the attention kernel scores too
        return hip_status(launch_score(c, q, 1, q4, nullptr, sc4, &ws, select_mode, retention, num_sinks,
                                       window_pages, k_max, nullptr, (hipStream_t)stream, false),
                          "page scores");
    }
    if (q.rot)
        return fail(FQ_ERR_UNSUPPORTED, "the rotated decode runs as the single-launch kernel only (enough KV groups to "
                                        "fill the GPU, no score output)");
    return hip_status(launch_score(c, q, 1, q4, sc_user, sc4, &ws, select_mode, retention, num_sinks, window_pages,
                                   k_max, mask_out, (hipStream_t)stream),
                      "score+select");
}

int fq_quest_select_int4(const fq_int4_cache* cache, const fq_query* query, const float* retention,
                         int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode,
                         float* scores_out, uint8_t* mask_out, void* workspace, size_t workspace_bytes_,
                         fq_stream_t stream) {
    return quest_select(cache, query, retention, num_sinks, window_pages, k_max, select_mode, scores_out, mask_out,
                        workspace, workspace_bytes_, stream, 4);
}

static int quest_attend(const fq_int4_cache* cache, const fq_query* query, const float* retention, int32_t num_sinks,
                        int32_t window_pages, int32_t k_max, int32_t select_mode, const TailArgs* tail,
                        void* workspace, size_t workspace_bytes_, fq_stream_t stream, int bits = 4,
                        uint8_t* mask_out = nullptr) {
    Int4Cache c{};
    QueryArgs q{};
    Workspace ws{};
    int st = attn_common(cache, query, workspace, workspace_bytes_, &c, &q, &ws, bits);
    if (st) return st;
    if (!retention) return fail(FQ_ERR_INVALID, "retention is NULL");
    if (num_sinks < 0) num_sinks = 0;
    if (window_pages < 0) window_pages = 0;
    if (k_max > c.P) k_max = c.P;
    const int chunks = mfma_head_chunks(c, q, num_sinks, window_pages, k_max, select_mode, ws.s_max, tail);
    const AttnLaunch al = choose_split(c.L * c.B * c.Hkv, quest_bound(c, q, num_sinks, window_pages, k_max,
                                                                      select_mode), ws.s_max);
    if (tail && tail->len > 0 && !(bits == 8 ? int8_mfma_supported(c, q, al) : mfma_supported(c, q, al)))
        return fail(FQ_ERR_UNSUPPORTED, "the fused tail needs the matrix-core attention layout");
    SelectArgs sel{};
    if (q.rot && !attn_selects_in_kernel(c, q, al))
        return fail(FQ_ERR_UNSUPPORTED, "the rotated decode runs as the single-launch kernel only");
    if (attn_selects_in_kernel(c, q, al)) {
        sel.retention = retention; sel.num_sinks = num_sinks; sel.window = window_pages;
        sel.k_max = k_max; sel.mode = select_mode; sel.mask_out = mask_out;
        sel.enabled = attend_from_scores(c, q, al.max_entries) ? kSelectOnly : kScoreSelect;
        sel.head_chunks = chunks;
    }
    return hip_status(launch_attn_int4(c, q, ws, al, (hipStream_t)stream, &sel, tail),
                      bits == 8 ? "sparse int8 attention" : "sparse int4 attention");
}

int fq_quest_attend_int4(const fq_int4_cache* cache, const fq_query* query, const float* retention,
                         int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode,
                         void* workspace, size_t workspace_bytes_, fq_stream_t stream) {
    return quest_attend(cache, query, retention, num_sinks, window_pages, k_max, select_mode, nullptr, workspace,
                        workspace_bytes_, stream);
}

// The partial-page tail of a decode step: validated here, attended by the
// attention launch (inside the kernel or in the split merge).
static int check_tail(const fq_tail* tail, const fq_int4_cache* cache, TailArgs& t) {
    t = TailArgs{};
    if (!tail || tail->len <= 0) return FQ_OK;
    if (tail->len > kTailMax) return fail(FQ_ERR_UNSUPPORTED, "tail of %d tokens (at most %d)", tail->len, kTailMax);
    if (!tail->k || !tail->v) return fail(FQ_ERR_INVALID, "tail K/V is NULL");
    if (!is_float_dtype(tail->dtype)) return fail(FQ_ERR_INVALID, "tail dtype");
    if (tail->k_strides[4] != 1 || tail->v_strides[4] != 1)
        return fail(FQ_ERR_UNSUPPORTED, "tail channel axis must be contiguous");
    if (cache && cache->D != tail->D) return fail(FQ_ERR_INVALID, "tail head_dim %d != cache head_dim %d", tail->D, cache->D);
    t.k = tail->k; t.v = tail->v; t.dtype = tail->dtype; t.len = tail->len;
    for (int i = 0; i < 4; ++i) { t.ks[i] = tail->k_strides[i]; t.vs[i] = tail->v_strides[i]; }
    return FQ_OK;
}

static int decode_with_tail(const fq_int4_cache* cache, const fq_query* query, const fq_tail* tail,
                            const float* retention, int32_t num_sinks, int32_t window_pages, int32_t k_max,
                            int32_t select_mode, void* workspace, size_t workspace_bytes_, fq_stream_t stream,
                            int bits) {
    TailArgs t{};
    int st = check_tail(tail, cache, t);
    if (st) return st;
    st = quest_select(cache, query, retention, num_sinks, window_pages, k_max, select_mode, nullptr, nullptr,
                      workspace, workspace_bytes_, stream, bits);
    if (st) return st;
    return quest_attend(cache, query, retention, num_sinks, window_pages, k_max, select_mode, t.len > 0 ? &t : nullptr,
                        workspace, workspace_bytes_, stream, bits);
}

int fq_quest_decode_int4_tail(const fq_int4_cache* cache, const fq_query* query, const fq_tail* tail,
                              const float* retention, int32_t num_sinks, int32_t window_pages, int32_t k_max,
                              int32_t select_mode, void* workspace, size_t workspace_bytes_, fq_stream_t stream) {
    return decode_with_tail(cache, query, tail, retention, num_sinks, window_pages, k_max, select_mode, workspace,
                            workspace_bytes_, stream, 4);
}

int fq_quest_decode_int8_tail(const fq_int8_cache* cache, const fq_query* query, const fq_tail* tail,
                              const float* retention, int32_t num_sinks, int32_t window_pages, int32_t k_max,
                              int32_t select_mode, void* workspace, size_t workspace_bytes_, fq_stream_t stream) {
    return decode_with_tail(cache, query, tail, retention, num_sinks, window_pages, k_max, select_mode, workspace,
                            workspace_bytes_, stream, 8);
}

static int quest_fused(const fq_int4_cache* cache, const fq_query* query, int32_t num_sinks, int32_t window_pages,
                       int32_t k_max, int32_t select_mode, int bits) {
    Int4Cache c{};
    QueryArgs q{};
    int st = check_cache(cache, &c, bits);
    if (st) return -st;
    st = check_query(query, c.D, c.Hkv, &q);
    if (st) return -st;
    if (select_mode != FQ_SELECT_PER_Q_HEAD && select_mode != FQ_SELECT_PER_KV_HEAD_SUM)
        return -fail(FQ_ERR_INVALID, "select_mode=%d", select_mode);
    if (num_sinks < 0) num_sinks = 0;
    if (window_pages < 0) window_pages = 0;
    if (k_max > c.P) k_max = c.P;
    mfma_head_chunks(c, q, num_sinks, window_pages, k_max, select_mode, s_max_for(c.P), nullptr);
    const AttnLaunch al = choose_split(c.L * c.B * c.Hkv, quest_bound(c, q, num_sinks, window_pages, k_max, select_mode),
                                       s_max_for(c.P));
    return attn_selects_in_kernel(c, q, al) ? 1 : 0;
}

int fq_quest_fused_int4(const fq_int4_cache* cache, const fq_query* query, int32_t num_sinks, int32_t window_pages,
                        int32_t k_max, int32_t select_mode) {
    return quest_fused(cache, query, num_sinks, window_pages, k_max, select_mode, 4);
}

int fq_quest_fused_int8(const fq_int8_cache* cache, const fq_query* query, int32_t num_sinks, int32_t window_pages,
                        int32_t k_max, int32_t select_mode) {
    return quest_fused(cache, query, num_sinks, window_pages, k_max, select_mode, 8);
}

int fq_quest_decode_int4(const fq_int4_cache* cache, const fq_query* query, const float* retention,
                         int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode,
                         float* scores_out, uint8_t* mask_out, void* workspace, size_t workspace_bytes_,
                         fq_stream_t stream) {
    int st = quest_select(cache, query, retention, num_sinks, window_pages, k_max, select_mode, scores_out, mask_out,
                          workspace, workspace_bytes_, stream, 4, true);
    if (st) return st;
    return quest_attend(cache, query, retention, num_sinks, window_pages, k_max, select_mode, nullptr, workspace,
                        workspace_bytes_, stream, 4, mask_out);
}

int fq_quest_decode_int8(const fq_int8_cache* cache, const fq_query* query, const float* retention,
                         int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode,
                         float* scores_out, uint8_t* mask_out, void* workspace, size_t workspace_bytes_,
                         fq_stream_t stream) {
    int st = quest_select(cache, query, retention, num_sinks, window_pages, k_max, select_mode, scores_out, mask_out,
                          workspace, workspace_bytes_, stream, 8, true);
    if (st) return st;
    return quest_attend(cache, query, retention, num_sinks, window_pages, k_max, select_mode, nullptr, workspace,
                        workspace_bytes_, stream, 8, mask_out);
}

int fq_quest_select_int8(const fq_int8_cache* cache, const fq_query* query, const float* retention,
                         int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode,
                         float* scores_out, uint8_t* mask_out, void* workspace, size_t workspace_bytes_,
                         fq_stream_t stream) {
    return quest_select(cache, query, retention, num_sinks, window_pages, k_max, select_mode, scores_out, mask_out,
                        workspace, workspace_bytes_, stream, 8);
}

size_t fq_int8_workspace_bytes(const fq_int8_cache* cache, int32_t H_q) { return fq_workspace_bytes(cache, H_q); }

int fq_page_scores_int8(const void* q, int32_t q_dtype, const int64_t q_strides[4], const void* k_scale,
                        const int64_t ks_strides[4], const void* k_mn, const int64_t km_strides[4],
                        int32_t meta_dtype, float* scores, const int64_t sc_strides[4], int32_t B,
                        int32_t H_q, int32_t S_q, int32_t H_kv, int32_t P, int32_t D, fq_stream_t stream) {
    g_score_bits = 8;
    const int st = fq_page_scores_int4(q, q_dtype, q_strides, k_scale, ks_strides, k_mn, km_strides, meta_dtype,
                                       scores, sc_strides, B, H_q, S_q, H_kv, P, D, stream);
    g_score_bits = 4;
    return st;
}

int fq_page_scores_int8_summary(const void* q, int32_t q_dtype, const int64_t q_strides[4], const uint8_t* k_codes,
                                const int64_t kc_strides[4], const void* k_scale, const int64_t ks_strides[4],
                                const void* k_mn, const int64_t km_strides[4], int32_t meta_dtype,
                                uint16_t* page_min, uint16_t* page_max, const int64_t pm_strides[4], float* scores,
                                const int64_t sc_strides[4], int32_t B, int32_t H_q, int32_t H_kv, int32_t S,
                                int32_t P, int32_t D, int32_t page_size, fq_stream_t stream) {
    if (H_kv < 1 || H_q % H_kv) return fail(FQ_ERR_INVALID, "H_q=%d must be divisible by H_kv=%d", H_q, H_kv);
    if (D != 64 && D != 128) return fail(FQ_ERR_UNSUPPORTED, "head_dim=%d not in (64, 128)", D);
    if (!is_half(meta_dtype) || !is_float_dtype(q_dtype)) return fail(FQ_ERR_UNSUPPORTED, "dtype");
    if (!q || !k_codes || !k_scale || !k_mn || !scores) return fail(FQ_ERR_INVALID, "NULL tensor");
    if ((page_min == nullptr) != (page_max == nullptr)) return fail(FQ_ERR_INVALID, "page_min / page_max: both or neither");
    if (page_size < 1) return fail(FQ_ERR_INVALID, "page_size must be >= 1");
    if (S < 0 || P != (S + page_size - 1) / page_size)
        return fail(FQ_ERR_INVALID, "pages=%d != ceil(S=%d / page_size=%d)", P, S, page_size);
    if (kc_strides[3] != 1 || kc_strides[2] % 4 || kc_strides[1] % 4 || kc_strides[0] % 4 || ((uintptr_t)k_codes & 3))
        return fail(FQ_ERR_UNSUPPORTED, "K codes need a contiguous channel axis and 4-byte aligned token rows");
    if (B == 0 || P == 0) return FQ_OK;
    if ((int64_t)B * H_kv > 65535) return fail(FQ_ERR_UNSUPPORTED, "batch x KV heads > 65535");
    SummaryArgs a{};
    a.codes = k_codes; a.ks = k_scale; a.km = k_mn; a.meta_dtype = meta_dtype;
    a.q = q; a.q_dtype = q_dtype; a.scores = scores; a.pmin = page_min; a.pmax = page_max;
    for (int i = 0; i < 4; ++i) {
        a.c_s[i] = kc_strides[i]; a.ks_s[i] = ks_strides[i]; a.km_s[i] = km_strides[i];
        a.q_s[i] = q_strides[i]; a.sc_s[i] = sc_strides[i]; a.pm_s[i] = page_min ? pm_strides[i] : 0;
    }
    a.B = B; a.Hq = H_q; a.Hkv = H_kv; a.S = S; a.P = P; a.D = D; a.page = page_size;
    return hip_status(launch_page_summary_scores(a, (hipStream_t)stream), "page summary scores");
}

int fq_page_summary(const void* k, int32_t k_dtype, const int64_t k_strides[4], int32_t B, int32_t H, int32_t S,
                    int32_t D, int32_t page_size, void* page_min, void* page_max, const int64_t pm_strides[4],
                    fq_stream_t stream) {
    if (!is_float_dtype(k_dtype)) return fail(FQ_ERR_INVALID, "K dtype must be bf16, fp16 or fp32");
    if (page_size < 1) return fail(FQ_ERR_INVALID, "page_size must be >= 1");
    if (D < 1 || D > 1024) return fail(FQ_ERR_UNSUPPORTED, "head_dim=%d not in [1, 1024]", D);
    if (B < 0 || H < 0 || S < 0) return fail(FQ_ERR_INVALID, "negative size");
    const int P = (S + page_size - 1) / page_size;
    if ((int64_t)B * H * P == 0) return FQ_OK;
    if (!k || !page_min || !page_max) return fail(FQ_ERR_INVALID, "NULL tensor");
    if ((int64_t)B * H > 65535) return fail(FQ_ERR_UNSUPPORTED, "batch x heads > 65535");
    PageMinMaxArgs a{};
    a.k = k; a.k_dtype = k_dtype; a.pmin = page_min; a.pmax = page_max;
    for (int i = 0; i < 4; ++i) { a.k_s[i] = k_strides[i]; a.pm_s[i] = pm_strides[i]; }
    a.B = B; a.H = H; a.S = S; a.P = P; a.D = D; a.page = page_size;
    return hip_status(launch_page_minmax(a, (hipStream_t)stream), "page summary");
}

static int quest_scores(const void* q, int32_t q_dtype, const int64_t q_strides[4], const void* lo,
                        const int64_t lo_strides[4], const void* hi, const int64_t hi_strides[4], int32_t b_dtype,
                        bool from_meta, float levels, float* scores, const int64_t sc_strides[4], int32_t B,
                        int32_t H_q, int32_t S_q, int32_t H_kv, int32_t P, int32_t D, fq_stream_t stream) {
    if (H_kv < 1 || H_q % H_kv) return fail(FQ_ERR_INVALID, "H_q=%d must be divisible by H_kv=%d", H_q, H_kv);
    if (D != 64 && D != 128) return fail(FQ_ERR_UNSUPPORTED, "head_dim=%d not in (64, 128)", D);
    if (!is_float_dtype(q_dtype) || !is_float_dtype(b_dtype)) return fail(FQ_ERR_INVALID, "dtype");
    if (B < 0 || S_q < 0 || P < 0) return fail(FQ_ERR_INVALID, "negative size");
    if ((int64_t)B * P * S_q == 0) return FQ_OK;
    if (!q || !lo || !hi || !scores) return fail(FQ_ERR_INVALID, "NULL tensor");
    if ((int64_t)B * H_kv > 65535) return fail(FQ_ERR_UNSUPPORTED, "batch x KV heads > 65535");
    QuestScoreArgs a{};
    a.q = q; a.q_dtype = q_dtype; a.lo = lo; a.hi = hi; a.b_dtype = b_dtype; a.from_meta = from_meta;
    a.levels = levels; a.scores = scores;
    for (int i = 0; i < 4; ++i) {
        a.q_s[i] = q_strides[i]; a.lo_s[i] = lo_strides[i]; a.hi_s[i] = hi_strides[i]; a.sc_s[i] = sc_strides[i];
    }
    a.B = B; a.Hq = H_q; a.Sq = S_q; a.Hkv = H_kv; a.P = P; a.D = D;
    return hip_status(launch_quest_scores(a, (hipStream_t)stream), "quest page scores");
}

int fq_page_scores_quest(const void* q, int32_t q_dtype, const int64_t q_strides[4], const void* page_min,
                         const int64_t pmin_strides[4], const void* page_max, const int64_t pmax_strides[4],
                         int32_t bound_dtype, float* scores, const int64_t sc_strides[4], int32_t B, int32_t H_q,
                         int32_t S_q, int32_t H_kv, int32_t P, int32_t D, fq_stream_t stream) {
    return quest_scores(q, q_dtype, q_strides, page_min, pmin_strides, page_max, pmax_strides, bound_dtype, false, 0.f,
                        scores, sc_strides, B, H_q, S_q, H_kv, P, D, stream);
}

int fq_page_scores_int8_bound(const void* q, int32_t q_dtype, const int64_t q_strides[4], const void* k_scale,
                              const int64_t ks_strides[4], const void* k_mn, const int64_t km_strides[4],
                              int32_t meta_dtype, float* scores, const int64_t sc_strides[4], int32_t B, int32_t H_q,
                              int32_t S_q, int32_t H_kv, int32_t P, int32_t D, fq_stream_t stream) {
    if (!is_half(meta_dtype)) return fail(FQ_ERR_INVALID, "metadata dtype must be bf16 or fp16");
    return quest_scores(q, q_dtype, q_strides, k_mn, km_strides, k_scale, ks_strides, meta_dtype, true, 255.0f,
                        scores, sc_strides, B, H_q, S_q, H_kv, P, D, stream);
}

int fq_quantize_k_int8(const void* k, int32_t in_dtype, const int64_t k_strides[4], int32_t B, int32_t H,
                       int32_t S, int32_t D, int32_t page_size, uint8_t* codes, const int64_t c_strides[4],
                       void* scale, const int64_t s_strides[4], void* mn, const int64_t m_strides[4],
                       int32_t meta_dtype, fq_stream_t stream) {
    if (D % 2) return fail(FQ_ERR_INVALID, "quantize_k requires even head_dim; got %d", D);
    if (page_size < 1) return fail(FQ_ERR_INVALID, "page_size must be >= 1");
    if (!is_float_dtype(in_dtype) || !is_half(meta_dtype)) return fail(FQ_ERR_INVALID, "dtype");
    return hip_status(launch_quant_k(k, in_dtype, k_strides, B, H, S, D, page_size, codes, c_strides, scale,
                                     s_strides, mn, m_strides, meta_dtype, (hipStream_t)stream, 8),
                      "quantize k int8");
}

int fq_quantize_v_int8(const void* v, int32_t in_dtype, const int64_t v_strides[4], int32_t B, int32_t H,
                       int32_t S, int32_t D, uint8_t* codes, const int64_t c_strides[4], void* scale,
                       const int64_t s_strides[4], void* mn, const int64_t m_strides[4], int32_t meta_dtype,
                       fq_stream_t stream) {
    if (D % 2) return fail(FQ_ERR_INVALID, "quantize_v requires even head_dim; got %d", D);
    if (!is_float_dtype(in_dtype) || !is_half(meta_dtype)) return fail(FQ_ERR_INVALID, "dtype");
    return hip_status(launch_quant_v(v, in_dtype, v_strides, B, H, S, D, D, codes, c_strides, scale, s_strides, mn,
                                     m_strides, meta_dtype, (hipStream_t)stream, 8),
                      "quantize v int8");
}

int fq_merge_attn(const void* o_a, const float* lse_a, const void* o_b, const float* lse_b, int32_t dtype,
                  int64_t o_row_stride_a, int64_t o_row_stride_b, void* out, int64_t out_row_stride,
                  float* lse_out, int32_t N, int32_t D, fq_stream_t stream) {
    if (!is_float_dtype(dtype)) return fail(FQ_ERR_INVALID, "dtype");
    return hip_status(launch_merge(o_a, lse_a, o_b, lse_b, dtype, o_row_stride_a, o_row_stride_b, out,
                                   out_row_stride, lse_out, N, D, (hipStream_t)stream),
                      "merge");
}

int fq_dense_tail_attn(const void* q, const int64_t q_strides[3], const void* k, const int64_t k_strides[4],
                       const void* v, const int64_t v_strides[4], int32_t kv_dtype, void* out,
                       const int64_t o_strides[3], float* lse, int32_t B, int32_t H_q, int32_t H_kv, int32_t T,
                       int32_t D, fq_stream_t stream) {
    if (T < 1 || T > 1024) return fail(FQ_ERR_UNSUPPORTED, "tail length %d outside [1, 1024]", T);
    if (D > 256) return fail(FQ_ERR_UNSUPPORTED, "head_dim %d > 256", D);
    if (H_kv < 1 || H_q % H_kv) return fail(FQ_ERR_INVALID, "H_q must be divisible by H_kv");
    if (!is_float_dtype(kv_dtype)) return fail(FQ_ERR_INVALID, "dtype");
    if (B * H_q == 0) return FQ_OK;
    return hip_status(launch_tail(q, q_strides, k, k_strides, v, v_strides, kv_dtype, out, o_strides, lse, B, H_q,
                                  H_kv, T, D, (hipStream_t)stream),
                      "tail attention");
}

int fq_quantize_k_int4(const void* k, int32_t in_dtype, const int64_t k_strides[4], int32_t B, int32_t H,
                       int32_t S, int32_t D, int32_t page_size, uint8_t* packed, const int64_t p_strides[4],
                       void* scale, const int64_t s_strides[4], void* mn, const int64_t m_strides[4],
                       int32_t meta_dtype, fq_stream_t stream) {
    if (D % 2) return fail(FQ_ERR_INVALID, "quantize_k_int4 requires even head_dim; got %d", D);
    if (page_size < 1) return fail(FQ_ERR_INVALID, "page_size must be >= 1");
    if (!is_float_dtype(in_dtype) || !is_half(meta_dtype)) return fail(FQ_ERR_INVALID, "dtype");
    if (page_quant_k_ok(D, page_size, in_dtype, k, k_strides, packed, p_strides, scale, s_strides, mn, m_strides))
        return hip_status(launch_quant_k_pages(k, in_dtype, k_strides, B, H, S, D, packed, p_strides, scale, s_strides,
                                               mn, m_strides, meta_dtype, (hipStream_t)stream),
                          "quantize k");
    return hip_status(launch_quant_k(k, in_dtype, k_strides, B, H, S, D, page_size, packed, p_strides, scale,
                                     s_strides, mn, m_strides, meta_dtype, (hipStream_t)stream),
                      "quantize k");
}

int fq_quantize_v_int4(const void* v, int32_t in_dtype, const int64_t v_strides[4], int32_t B, int32_t H,
                       int32_t S, int32_t D, int32_t group, uint8_t* packed, const int64_t p_strides[4],
                       void* scale, const int64_t s_strides[4], void* mn, const int64_t m_strides[4],
                       int32_t meta_dtype, fq_stream_t stream) {
    if (D % 2) return fail(FQ_ERR_INVALID, "quantize_v_int4 requires even head_dim; got %d", D);
    if (group < 2 || group % 2 || D % group) return fail(FQ_ERR_INVALID, "bad V group %d for D=%d", group, D);
    if (!is_float_dtype(in_dtype) || !is_half(meta_dtype)) return fail(FQ_ERR_INVALID, "dtype");
    if (page_quant_v_ok(D, group, in_dtype, v, v_strides, packed, p_strides, s_strides, m_strides))
        return hip_status(launch_quant_v_pages(v, in_dtype, v_strides, B, H, S, D, group, packed, p_strides, scale,
                                               s_strides, mn, m_strides, meta_dtype, (hipStream_t)stream),
                          "quantize v");
    return hip_status(launch_quant_v(v, in_dtype, v_strides, B, H, S, D, group, packed, p_strides, scale,
                                     s_strides, mn, m_strides, meta_dtype, (hipStream_t)stream),
                      "quantize v");
}

// Checks shared by the three cache appends: bounds of the append, the tail
// dtype, 16-byte aligned contiguous rows of the tails and the new tokens.
static int check_append(int L, int S, int P, int page, int layer, void* k_partial, const int64_t kpart_strides[5],
                        void* v_partial, const int64_t vpart_strides[5], int32_t partial_dtype, const void* k_new,
                        const int64_t kn_strides[4], const void* v_new, const int64_t vn_strides[4], int32_t seen,
                        int32_t S_new) {
    if (layer < 0 || layer >= L) return fail(FQ_ERR_INVALID, "layer %d is not one of the cache's %d layers", layer, L);
    if (seen < 0 || S_new < 0) return fail(FQ_ERR_INVALID, "negative token count (seen %d, new %d)", seen, S_new);
    if ((int64_t)seen + S_new > S)
        return fail(FQ_ERR_INVALID, "%lld tokens do not fit the cache's %d token slots", (long long)seen + S_new, S);
    if (page != 64) return fail(FQ_ERR_UNSUPPORTED, "page_size=%d (the append kernel takes 64)", page);
    if ((int64_t)(seen + S_new + page - 1) / page > P) return fail(FQ_ERR_INVALID, "page metadata holds %d pages", P);
    if (partial_dtype != FQ_BF16 && partial_dtype != FQ_F16)
        return fail(FQ_ERR_UNSUPPORTED, "partial tail dtype must be bf16 or fp16");
    if (!k_partial || !v_partial || (!k_new && S_new) || (!v_new && S_new)) return fail(FQ_ERR_INVALID, "NULL tensor");
    if (!rows_aligned16(k_partial, kpart_strides, 4, 2) || !rows_aligned16(v_partial, vpart_strides, 4, 2) ||
        kpart_strides[4] != 1 || vpart_strides[4] != 1)
        return fail(FQ_ERR_UNSUPPORTED, "partial tails need 16-byte aligned contiguous rows");
    if (S_new > 0 && (!rows_aligned16(k_new, kn_strides, 3, 2) || !rows_aligned16(v_new, vn_strides, 3, 2) ||
                      kn_strides[3] != 1 || vn_strides[3] != 1))
        return fail(FQ_ERR_UNSUPPORTED, "new K/V need 16-byte aligned contiguous rows");
    return FQ_OK;
}

static int kv_cache_append(const fq_int4_cache* cache, int bits, int32_t layer, void* k_partial,
                           const int64_t kpart_strides[5], void* v_partial, const int64_t vpart_strides[5],
                           int32_t partial_dtype, const void* k_new, const int64_t kn_strides[4], const void* v_new,
                           const int64_t vn_strides[4], int32_t seen, int32_t S_new, fq_stream_t stream) {
    Int4Cache c{};
    int st = check_cache(cache, &c, bits);
    if (st) return st;
    st = check_append(c.L, c.S, c.P, c.page, layer, k_partial, kpart_strides, v_partial, vpart_strides, partial_dtype,
                      k_new, kn_strides, v_new, vn_strides, seen, S_new);
    if (st) return st;
    if (c.D != 64 && c.D != 128) return fail(FQ_ERR_UNSUPPORTED, "head_dim=%d (the append kernel takes 64, 128)", c.D);
    if (((uintptr_t)c.vsc | (uintptr_t)c.vmn) & 1) return fail(FQ_ERR_UNSUPPORTED, "V metadata must be 2-byte aligned");
    return hip_status(launch_kv_append(c, layer, k_partial, kpart_strides, v_partial, vpart_strides, partial_dtype,
                                       k_new, kn_strides, v_new, vn_strides, seen, S_new, bits, (hipStream_t)stream),
                      bits == 8 ? "int8 cache append" : "int4 cache append");
}

int fq_int4_cache_append(const fq_int4_cache* cache, int32_t layer, void* k_partial, const int64_t kpart_strides[5],
                         void* v_partial, const int64_t vpart_strides[5], int32_t partial_dtype, const void* k_new,
                         const int64_t kn_strides[4], const void* v_new, const int64_t vn_strides[4], int32_t seen,
                         int32_t S_new, fq_stream_t stream) {
    return kv_cache_append(cache, 4, layer, k_partial, kpart_strides, v_partial, vpart_strides, partial_dtype, k_new,
                           kn_strides, v_new, vn_strides, seen, S_new, stream);
}

int fq_int8_cache_append(const fq_int8_cache* cache, int32_t layer, void* k_partial, const int64_t kpart_strides[5],
                         void* v_partial, const int64_t vpart_strides[5], int32_t partial_dtype, const void* k_new,
                         const int64_t kn_strides[4], const void* v_new, const int64_t vn_strides[4], int32_t seen,
                         int32_t S_new, fq_stream_t stream) {
    if (cache && cache->v_groups != 1) return fail(FQ_ERR_UNSUPPORTED, "INT8 V metadata is per token (v_groups=1)");
    return kv_cache_append(cache, 8, layer, k_partial, kpart_strides, v_partial, vpart_strides, partial_dtype, k_new,
                           kn_strides, v_new, vn_strides, seen, S_new, stream);
}

int fq_turbo_cache_append(const fq_turbo_cache* cache, void* k_scale_raw, const int64_t ksr_strides[5],
                          void* k_mn_raw, const int64_t kmr_strides[5], int32_t layer, void* k_partial,
                          const int64_t kpart_strides[5], void* v_partial, const int64_t vpart_strides[5],
                          int32_t partial_dtype, const void* k_new, const int64_t kn_strides[4], const void* v_new,
                          const int64_t vn_strides[4], int32_t seen, int32_t S_new, fq_stream_t stream) {
    if (!cache) return fail(FQ_ERR_INVALID, "cache descriptor is NULL");
    const fq_turbo_cache& tc = *cache;
    if (tc.D != 64 && tc.D != 128) return fail(FQ_ERR_UNSUPPORTED, "head_dim=%d (the append kernel takes 64, 128)", tc.D);
    if (tc.L < 1 || tc.B < 1 || tc.H_kv < 1) return fail(FQ_ERR_INVALID, "empty L/B/H_kv");
    int st = check_append(tc.L, tc.S, tc.P, tc.page_size, layer, k_partial, kpart_strides, v_partial, vpart_strides,
                          partial_dtype, k_new, kn_strides, v_new, vn_strides, seen, S_new);
    if (st) return st;
    if (!tc.k_msb || !tc.k_lsb || !tc.k_scale || !tc.v_msb || !tc.v_lsb || !tc.v_scale || !k_scale_raw || !k_mn_raw)
        return fail(FQ_ERR_INVALID, "NULL cache tensor");
    if (tc.kmsb_strides[4] != 1 || tc.klsb_strides[4] != 1 || tc.vmsb_strides[4] != 1 || tc.vlsb_strides[4] != 1)
        return fail(FQ_ERR_UNSUPPORTED, "code planes need contiguous rows");
    if (((uintptr_t)tc.k_scale | (uintptr_t)tc.v_scale) & 1) return fail(FQ_ERR_UNSUPPORTED, "scales must be 2-byte aligned");
    if (ksr_strides[4] != 1 || kmr_strides[4] != 1 || !rows_aligned16(k_scale_raw, ksr_strides, 4, 2) ||
        !rows_aligned16(k_mn_raw, kmr_strides, 4, 2))
        return fail(FQ_ERR_UNSUPPORTED, "raw K page metadata needs 16-byte aligned contiguous rows");
    Int4Cache raw{};
    raw.ksc = k_scale_raw; raw.kmn = k_mn_raw;
    for (int i = 0; i < 4; ++i) { raw.ksc_s[i] = ksr_strides[i]; raw.kmn_s[i] = kmr_strides[i]; }
    return hip_status(launch_turbo_append(tc, raw, layer, k_partial, kpart_strides, v_partial, vpart_strides,
                                          partial_dtype, k_new, kn_strides, v_new, vn_strides, seen, S_new,
                                          (hipStream_t)stream),
                      "turbo cache append");
}

int fq_wht(const void* x, int32_t x_dtype, int64_t x_row_stride, void* out, int32_t out_dtype,
           int64_t out_row_stride, int32_t N, int32_t D, const float* signs, int32_t inverse, int32_t arith_dtype,
           fq_stream_t stream) {
    if (D < 8 || D > 128 || (D & (D - 1)))
        return fail(FQ_ERR_INVALID, "head_dim must be a positive power of 2 in [8, 128], got %d", D);
    if (!is_float_dtype(x_dtype) || !is_float_dtype(out_dtype) || !is_float_dtype(arith_dtype))
        return fail(FQ_ERR_INVALID, "dtype");
    return hip_status(launch_wht(x, x_dtype, x_row_stride, out, out_dtype, out_row_stride, N, D, signs, inverse,
                                 arith_dtype, (hipStream_t)stream),
                      "wht");
}

int fq_quantize_turbo(const void* x, int32_t in_dtype, const int64_t x_strides[4], int32_t B, int32_t H,
                      int32_t S, int32_t D, uint8_t* msb, const int64_t msb_strides[4], uint8_t* lsb,
                      const int64_t lsb_strides[4], void* scale, const int64_t s_strides[4], fq_stream_t stream) {
    if (D != 64 && D != 128) return fail(FQ_ERR_UNSUPPORTED, "head_dim=%d not in (64, 128)", D);
    if (!is_float_dtype(in_dtype)) return fail(FQ_ERR_INVALID, "dtype");
    return hip_status(launch_turbo_quant(x, in_dtype, x_strides, B, H, S, D, msb, msb_strides, lsb, lsb_strides,
                                         scale, s_strides, (hipStream_t)stream),
                      "quantize turbo");
}

// The TurboQuant cache descriptor as the decode entries read it: head_dim,
// page count, contiguous plane rows, tensors present once the cache holds
// tokens, and per-token fp16/bf16 scales on 2-byte boundaries.
static int check_turbo_cache(const fq_turbo_cache* c) {
    if (!c) return fail(FQ_ERR_INVALID, "cache descriptor is NULL");
    if (c->D != 64 && c->D != 128) return fail(FQ_ERR_UNSUPPORTED, "head_dim=%d not in (64, 128)", c->D);
    if (c->L < 1 || c->B < 1 || c->H_kv < 1) return fail(FQ_ERR_INVALID, "empty L/B/H_kv");
    if (c->P < 1 || c->P > kMaxPages) return fail(FQ_ERR_UNSUPPORTED, "pages=%d", c->P);
    if (c->page_size < 1) return fail(FQ_ERR_INVALID, "page_size");
    // the raw K metadata beside the descriptor is read for every page: a page
    // count past the planes' tokens names rows the caller never wrote
    if ((int64_t)c->P > ((int64_t)c->S + c->page_size - 1) / c->page_size)
        return fail(FQ_ERR_INVALID, "pages=%d but the planes hold %lld tokens of page_size %d", c->P,
                    (long long)c->S, c->page_size);
    if (!c->k_msb || !c->k_lsb || !c->k_scale || !c->v_msb || !c->v_lsb || !c->v_scale)
        return fail(FQ_ERR_INVALID, "NULL cache tensor");
    if (c->kmsb_strides[4] != 1 || c->klsb_strides[4] != 1 || c->vmsb_strides[4] != 1 || c->vlsb_strides[4] != 1)
        return fail(FQ_ERR_UNSUPPORTED, "innermost turbo plane axis must be contiguous");
    if (((uintptr_t)c->k_scale | (uintptr_t)c->v_scale) & 1)
        return fail(FQ_ERR_UNSUPPORTED, "scales must be 2-byte aligned");
    return FQ_OK;
}

size_t fq_turbo_workspace_bytes(const fq_turbo_cache* cache, int32_t H_q) {
    if (!cache || cache->H_kv < 1 || H_q % cache->H_kv) return 0;
    const int G = cache->L * cache->B * cache->H_kv;
    const int nrep = H_q / cache->H_kv;
    return workspace_bytes(G, cache->P, nrep, nrep, cache->D);
}

int fq_sparse_turbo_fwd_mask(const fq_turbo_cache* cache, const fq_query* query, const uint8_t* mask,
                             const int64_t mask_strides[4], void* workspace, size_t workspace_bytes_,
                             fq_stream_t stream) {
    int st = check_turbo_cache(cache);
    if (st) return st;
    QueryArgs q{};
    st = check_query(query, cache->D, cache->H_kv, &q);
    if (st) return st;
    if (q.rot) return fail(FQ_ERR_UNSUPPORTED, "the rotated decode is INT4 only");
    const int G = cache->L * cache->B * cache->H_kv;
    const size_t need = workspace_bytes(G, cache->P, q.nrep, q.nrep, cache->D);
    if (!workspace || workspace_bytes_ < need)
        return fail(FQ_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, workspace_bytes_);
    Workspace ws = carve_workspace(workspace, G, cache->P, q.nrep, q.nrep, cache->D);
    hipStream_t s = (hipStream_t)stream;
    st = hip_status(launch_union_from_mask(mask, mask_strides, cache->L, cache->B, cache->H_kv, q.nrep, cache->P,
                                           ws, s),
                    "page union");
    if (st) return st;
    if (turbo_fused_supported(*cache, q))
        return hip_status(launch_attn_turbo_fused(*cache, nullptr, q, ws, cache->P, nullptr, s), "sparse turbo attention");
    const AttnLaunch al = choose_split(G, cache->P, ws.s_max);
    return hip_status(launch_attn_turbo(*cache, q, ws, al, s), "sparse turbo attention");
}

// The TurboQuant step (select_only false) or its selection half alone (true:
// scores and the selection, mask_out written when given, no attention).
// 6 or 8 query heads per KV head on the matrix-core TurboQuant kernel (at
// most 4 per workgroup): every KV head as two virtual KV heads of 3 or 4
// query heads, like the INT4 / INT8 decode.  Whether that layout applies.
static bool turbo_head_chunks(const fq_turbo_cache& cache, const QueryArgs& q) {
    if (q.rot || (q.nrep != 6 && q.nrep != 8) || cache.P > 64 * 8 || attention_splits_request() > 0) return false;
    fq_turbo_cache vc = cache;
    vc.H_kv *= 2;
    QueryArgs vq = q;
    vq.nrep /= 2;
    return turbo_fused_supported(vc, vq);
}

// Whether the TurboQuant decode is one launch that scores and selects its own
// pages: 0 no, 1 yes, 2 yes with head chunks.
static int turbo_one_launch(const fq_turbo_cache& cache, const QueryArgs& q) {
    const int G = cache.L * cache.B * cache.H_kv;
    if (q.rot || cache.P > 64 * 8 || attention_splits_request() > 0) return 0;      // in-kernel selection: 512 pages
    if (turbo_fused_supported(cache, q)) return G >= 192 ? 1 : 0;
    return 2 * G >= 192 && turbo_head_chunks(cache, q) ? 2 : 0;
}

static int quest_turbo(const fq_turbo_cache* cache, const void* k_scale_raw, const int64_t ksr_strides[5],
                       const void* k_mn_raw, const int64_t kmr_strides[5], const fq_query* query,
                       const float* retention, int32_t num_sinks, int32_t window_pages, int32_t k_max,
                       int32_t select_mode, uint8_t* mask_out, void* workspace, size_t workspace_bytes_,
                       fq_stream_t stream, bool select_only) {
    int st = check_turbo_cache(cache);
    if (st) return st;
    if (!retention) return fail(FQ_ERR_INVALID, "retention is NULL");
    if (select_mode != FQ_SELECT_PER_Q_HEAD && select_mode != FQ_SELECT_PER_KV_HEAD_SUM)
        return fail(FQ_ERR_INVALID, "select_mode=%d", select_mode);
    QueryArgs q{};
    st = check_query(query, cache->D, cache->H_kv, &q);
    if (st) return st;
    if (q.rot) return fail(FQ_ERR_UNSUPPORTED, "the rotated decode is INT4 only");
    if (((uintptr_t)q.q) & 1) return fail(FQ_ERR_UNSUPPORTED, "query must be 2-byte aligned");
    // the raw page metadata as an INT4 cache descriptor (scoring reads only K scale/min)
    if (!k_scale_raw || !k_mn_raw) return fail(FQ_ERR_INVALID, "NULL raw K metadata");
    if (ksr_strides[4] != 1 || kmr_strides[4] != 1) return fail(FQ_ERR_UNSUPPORTED, "raw K metadata channel axis must be contiguous");
    for (int i = 0; i < 4; ++i)
        if (ksr_strides[i] % 8 || kmr_strides[i] % 8)
            return fail(FQ_ERR_UNSUPPORTED, "raw K metadata strides must be multiples of 8 elements");
    if (((uintptr_t)k_scale_raw | (uintptr_t)k_mn_raw) & 15)
        return fail(FQ_ERR_UNSUPPORTED, "raw K metadata must be 16-byte aligned");
    Int4Cache c{};
    c.ksc = k_scale_raw; c.kmn = k_mn_raw;
    for (int i = 0; i < 4; ++i) { c.ksc_s[i] = ksr_strides[i]; c.kmn_s[i] = kmr_strides[i]; }
    c.L = cache->L; c.B = cache->B; c.Hkv = cache->H_kv; c.S = cache->S; c.P = cache->P; c.D = cache->D;
    c.page = cache->page_size; c.G = 1; c.meta_dtype = FQ_BF16;
    const int G = c.L * c.B * c.Hkv;
    const size_t need = workspace_bytes(G, c.P, q.nrep, q.nrep, c.D);
    if (!workspace || workspace_bytes_ < need)
        return fail(FQ_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, workspace_bytes_);
    if ((uintptr_t)workspace & 255) return fail(FQ_ERR_WORKSPACE, "workspace must be 256-byte aligned");
    Workspace ws = carve_workspace(workspace, G, c.P, q.nrep, q.nrep, c.D);
    if (num_sinks < 0) num_sinks = 0;
    if (window_pages < 0) window_pages = 0;
    if (k_max > c.P) k_max = c.P;
    hipStream_t s = (hipStream_t)stream;
    const int bound = quest_bound(c, q, num_sinks, window_pages, k_max, select_mode);
    const bool fusable = turbo_fused_supported(*cache, q);
    const int one = select_only ? 0 : turbo_one_launch(*cache, q);
    if (one) {
        SelectArgs sel{};
        sel.retention = retention; sel.num_sinks = num_sinks; sel.window = window_pages;
        sel.k_max = k_max; sel.mode = select_mode; sel.enabled = kScoreSelect; sel.mask_out = mask_out;
        if (one == 1) return hip_status(launch_attn_turbo_fused(*cache, &c, q, ws, bound, &sel, s), "quest turbo decode");
        fq_turbo_cache vc = *cache;      // head chunks: the virtual KV heads
        vc.H_kv *= 2;
        QueryArgs vq = q;
        vq.nrep /= 2;
        Int4Cache vr = c;
        vr.Hkv *= 2;
        sel.head_chunks = 2;
        return hip_status(launch_attn_turbo_fused(vc, &vr, vq, ws, quest_bound(vr, vq, num_sinks, window_pages, k_max,
                                                                                select_mode),
                                                  &sel, s),
                          "quest turbo decode");
    }
    const int64_t q4[4] = {q.q_s[1], q.q_s[2], 0, q.q_s[3]};
    int64_t sc4[4] = {(int64_t)q.Hq * c.P, c.P, c.P, 1};
    const bool chunks = !select_only && !fusable && turbo_head_chunks(*cache, q);
    if (!select_only && (fusable || chunks) && c.P <= 64 * 8 && attention_splits_request() <= 0) {
        // few groups (a single layer's step): the scoring launch writes the
        // scores of the real KV heads, the attention workgroups of each group
        // (virtual heads with 6 or 8 query heads per KV head) select from them
        st = hip_status(launch_score(c, q, 1, q4, nullptr, sc4, &ws, select_mode, retention, num_sinks, window_pages,
                                     k_max, nullptr, s, false),
                        "page scores");
        if (st) return st;
        SelectArgs sel{};
        sel.retention = retention; sel.num_sinks = num_sinks; sel.window = window_pages;
        sel.k_max = k_max; sel.mode = select_mode; sel.enabled = kSelectOnly; sel.mask_out = mask_out;
        if (!chunks) return hip_status(launch_attn_turbo_fused(*cache, nullptr, q, ws, bound, &sel, s), "quest turbo decode");
        fq_turbo_cache vc = *cache;
        vc.H_kv *= 2;
        QueryArgs vq = q;
        vq.nrep /= 2;
        Int4Cache vr = c;
        vr.Hkv *= 2;
        sel.head_chunks = 2;
        return hip_status(launch_attn_turbo_fused(vc, nullptr, vq, ws,
                                                  quest_bound(vr, vq, num_sinks, window_pages, k_max, select_mode), &sel,
                                                  s),
                          "quest turbo decode");
    }
    st = hip_status(launch_score(c, q, 1, q4, nullptr, sc4, &ws, select_mode, retention, num_sinks, window_pages,
                                 k_max, mask_out, s),
                    "score+select");
    if (st || select_only) return st;
    if (fusable) return hip_status(launch_attn_turbo_fused(*cache, nullptr, q, ws, bound, nullptr, s), "quest turbo decode");
    const AttnLaunch al = choose_split(G, bound, ws.s_max);
    return hip_status(launch_attn_turbo(*cache, q, ws, al, s), "quest turbo decode");
}

int fq_quest_fused_turbo(const fq_turbo_cache* cache, const fq_query* query) {
    int st = check_turbo_cache(cache);
    if (st) return -st;
    QueryArgs q{};
    st = check_query(query, cache->D, cache->H_kv, &q);
    if (st) return -st;
    return turbo_one_launch(*cache, q) || turbo_head_chunks(*cache, q) ? 1 : 0;
}

int fq_quest_decode_turbo(const fq_turbo_cache* cache, const void* k_scale_raw, const int64_t ksr_strides[5],
                          const void* k_mn_raw, const int64_t kmr_strides[5], const fq_query* query,
                          const float* retention, int32_t num_sinks, int32_t window_pages, int32_t k_max,
                          int32_t select_mode, uint8_t* mask_out, void* workspace, size_t workspace_bytes_,
                          fq_stream_t stream) {
    return quest_turbo(cache, k_scale_raw, ksr_strides, k_mn_raw, kmr_strides, query, retention, num_sinks,
                       window_pages, k_max, select_mode, mask_out, workspace, workspace_bytes_, stream, false);
}

int fq_quest_select_turbo(const fq_turbo_cache* cache, const void* k_scale_raw, const int64_t ksr_strides[5],
                          const void* k_mn_raw, const int64_t kmr_strides[5], const fq_query* query,
                          const float* retention, int32_t num_sinks, int32_t window_pages, int32_t k_max,
                          int32_t select_mode, uint8_t* mask_out, void* workspace, size_t workspace_bytes_,
                          fq_stream_t stream) {
    return quest_turbo(cache, k_scale_raw, ksr_strides, k_mn_raw, kmr_strides, query, retention, num_sinks,
                       window_pages, k_max, select_mode, mask_out, workspace, workspace_bytes_, stream, true);
}

static bool aligned(const void* p, int bytes) { return ((uintptr_t)p & (uintptr_t)(bytes - 1)) == 0; }

// Validates a prefill call; on success fills c, t and the needed workspace size.
static int prefill_check_tail_query(const fq_tail* tail, const fq_prefill* q, int D, int Hkv, int B, int S,
                                    TailArgs& t) {
    t = TailArgs{};
    if (tail && tail->len > 0) {
        if (!tail->k || !tail->v) return fail(FQ_ERR_INVALID, "tail K/V is NULL");
        if (tail->dtype != FQ_BF16) return fail(FQ_ERR_UNSUPPORTED, "prefill tail must be bf16");
        if (tail->D != D) return fail(FQ_ERR_INVALID, "tail head_dim %d != cache head_dim %d", tail->D, D);
        if (tail->k_strides[4] != 1 || tail->v_strides[4] != 1)
            return fail(FQ_ERR_UNSUPPORTED, "tail channel axis must be contiguous");
        for (int i = 1; i < 4; ++i)
            if (tail->k_strides[i] % 8 || tail->v_strides[i] % 4)
                return fail(FQ_ERR_UNSUPPORTED, "tail row strides must be multiples of 8 (K) / 4 (V) elements");
        if (!aligned(tail->k, 16) || !aligned(tail->v, 8)) return fail(FQ_ERR_UNSUPPORTED, "tail K/V alignment");
        t.k = tail->k; t.v = tail->v; t.dtype = tail->dtype; t.len = tail->len;
        for (int i = 0; i < 4; ++i) { t.ks[i] = tail->k_strides[i]; t.vs[i] = tail->v_strides[i]; }
    }
    if (!q || !q->q || !q->out) return fail(FQ_ERR_INVALID, "query/output is NULL");
    if (q->D != D) return fail(FQ_ERR_INVALID, "query head_dim %d != cache head_dim %d", q->D, D);
    if (q->H_q < 1 || q->H_q % Hkv) return fail(FQ_ERR_INVALID, "H_q=%d must be divisible by H_kv=%d", q->H_q, Hkv);
    if (q->S_q < 1) return fail(FQ_ERR_INVALID, "S_q=%d", q->S_q);
    if (q->causal_offset < 0) return fail(FQ_ERR_INVALID, "causal_offset=%d must be >= 0", q->causal_offset);
    if ((int64_t)S + t.len < 1) return fail(FQ_ERR_INVALID, "no keys (S + tail = 0)");
    if (q->q_strides[3] != 1 || q->o_strides[3] != 1) return fail(FQ_ERR_UNSUPPORTED, "Q/O channels must be contiguous");
    for (int i = 0; i < 3; ++i)
        if (q->q_strides[i] % 8 || q->o_strides[i] % 4)
            return fail(FQ_ERR_UNSUPPORTED, "Q / O strides must be multiples of 8 / 4 elements");
    if (!aligned(q->q, 16) || !aligned(q->out, 8)) return fail(FQ_ERR_UNSUPPORTED, "Q/O alignment");
    const int64_t rows = (int64_t)q->S_q * (q->H_q / Hkv);
    if ((rows + 255) / 256 * Hkv * B > 0x7FFFFFFF) return fail(FQ_ERR_UNSUPPORTED, "grid too large");
    // the dense pass addresses one head's bf16 K (or V^T) with 32-bit byte offsets
    if (((int64_t)S + t.len + 128) * D * 2 > 0x7FFFFFFF)
        return fail(FQ_ERR_UNSUPPORTED, "prefill over %lld keys exceeds one call's 2 GiB per-head K range",
                    (long long)S + t.len);
    return FQ_OK;
}

static int prefill_check(const fq_int4_cache* cache, const fq_tail* tail, const fq_prefill* q, int bits, Int4Cache& c,
                         TailArgs& t, size_t* ws_bytes) {
    int st = check_cache(cache, &c, bits, true);
    if (st) return st;
    if (c.L != 1) return fail(FQ_ERR_INVALID, "prefill takes one layer's cache view (L=%d)", c.L);
    if (c.D != 128) return fail(FQ_ERR_UNSUPPORTED, "prefill head_dim=%d (128 only)", c.D);
    if (c.S > 0) {
        if ((int64_t)c.P * c.page < c.S) return fail(FQ_ERR_INVALID, "%d pages of %d tokens < S=%d", c.P, c.page, c.S);
        const int kal = bits == 4 ? 8 : 16;   // one thread loads 16 channels of codes
        for (int i = 0; i < 4; ++i)
            if (c.kp_s[i] % kal) return fail(FQ_ERR_UNSUPPORTED, "K code strides must be multiples of %d bytes", kal);
        if (!aligned(c.kp, kal)) return fail(FQ_ERR_UNSUPPORTED, "K codes must be %d-byte aligned", kal);
    }
    st = prefill_check_tail_query(tail, q, c.D, c.Hkv, c.B, c.S, t);
    if (st) return st;
    *ws_bytes = prefill_workspace_bytes(c, c.S + t.len, q->S_q, q->H_q / c.Hkv, q->causal_offset);
    return FQ_OK;
}

static int prefill(const fq_int4_cache* cache, const fq_tail* tail, const fq_prefill* q, void* workspace,
                   size_t workspace_bytes_, fq_stream_t stream, int bits) {
    Int4Cache c{};
    TailArgs t{};
    size_t need = 0;
    int st = prefill_check(cache, tail, q, bits, c, t, &need);
    if (st) return st;
    if (need > 0 && (!workspace || workspace_bytes_ < need))
        return fail(FQ_ERR_WORKSPACE, "prefill workspace of %zu bytes needed (got %zu)", need, workspace_bytes_);
    if (need > 0 && !aligned(workspace, 16)) return fail(FQ_ERR_INVALID, "workspace must be 16-byte aligned");
    const float sm = q->sm_scale > 0.f ? q->sm_scale : 1.0f / sqrtf((float)c.D);
    return hip_status(launch_prefill(c, t, q->q, q->q_strides, q->out, q->o_strides, q->H_q / c.Hkv, q->S_q,
                                     q->causal_offset, sm * kLog2e, workspace, (hipStream_t)stream),
                      "prefill attention launch");
}

size_t fq_prefill_workspace_bytes(const fq_int4_cache* cache, const fq_tail* tail, const fq_prefill* query,
                                  int32_t bits) {
    Int4Cache c{};
    TailArgs t{};
    size_t need = 0;
    if (bits != 4 && bits != 8) return 0;
    if (prefill_check(cache, tail, query, bits, c, t, &need)) return 0;
    return need;
}

static int prefill_turbo_check(const fq_turbo_cache* c, const fq_tail* tail, const fq_prefill* q, TailArgs& t,
                               size_t* ws_bytes) {
    if (!c) return fail(FQ_ERR_INVALID, "cache descriptor is NULL");
    if (c->L != 1) return fail(FQ_ERR_INVALID, "prefill takes one layer's cache view (L=%d)", c->L);
    if (c->D != 128) return fail(FQ_ERR_UNSUPPORTED, "prefill head_dim=%d (128 only)", c->D);
    if (c->B < 1 || c->H_kv < 1 || c->S < 0) return fail(FQ_ERR_INVALID, "empty B/H_kv or negative S");
    if (c->S > 0) {
        if (!c->k_msb || !c->k_lsb || !c->k_scale || !c->v_msb || !c->v_lsb || !c->v_scale)
            return fail(FQ_ERR_INVALID, "NULL cache tensor");
        if (c->kmsb_strides[4] != 1 || c->klsb_strides[4] != 1 || c->vmsb_strides[4] != 1 || c->vlsb_strides[4] != 1)
            return fail(FQ_ERR_UNSUPPORTED, "innermost plane axis must be contiguous");
        if (((uintptr_t)c->k_scale | (uintptr_t)c->v_scale) & 1)
            return fail(FQ_ERR_UNSUPPORTED, "scales must be 2-byte aligned");
    }
    int st = prefill_check_tail_query(tail, q, c->D, c->H_kv, c->B, c->S, t);
    if (st) return st;
    *ws_bytes = prefill_turbo_workspace_bytes(c->H_kv, c->B, c->S + t.len, q->S_q, q->H_q / c->H_kv, q->causal_offset);
    return FQ_OK;
}

size_t fq_prefill_turbo_workspace_bytes(const fq_turbo_cache* cache, const fq_tail* tail, const fq_prefill* query) {
    TailArgs t{};
    size_t need = 0;
    if (prefill_turbo_check(cache, tail, query, t, &need)) return 0;
    return need;
}

int fq_prefill_turbo(const fq_turbo_cache* cache, const fq_tail* tail, const fq_prefill* q, void* workspace,
                     size_t workspace_bytes_, fq_stream_t stream) {
    TailArgs t{};
    size_t need = 0;
    int st = prefill_turbo_check(cache, tail, q, t, &need);
    if (st) return st;
    if (!workspace || workspace_bytes_ < need)
        return fail(FQ_ERR_WORKSPACE, "prefill workspace of %zu bytes needed (got %zu)", need, workspace_bytes_);
    if (!aligned(workspace, 16)) return fail(FQ_ERR_INVALID, "workspace must be 16-byte aligned");
    const float sm = q->sm_scale > 0.f ? q->sm_scale : 1.0f / sqrtf((float)cache->D);
    return hip_status(launch_prefill_turbo(*cache, t, q->q, q->q_strides, q->out, q->o_strides, q->H_q / cache->H_kv,
                                           q->S_q, q->causal_offset, sm * kLog2e, workspace, (hipStream_t)stream),
                      "turbo prefill launch");
}

int fq_prefill_int4(const fq_int4_cache* cache, const fq_tail* tail, const fq_prefill* query, void* workspace,
                    size_t workspace_bytes, fq_stream_t stream) {
    return prefill(cache, tail, query, workspace, workspace_bytes, stream, 4);
}

int fq_prefill_int8(const fq_int8_cache* cache, const fq_tail* tail, const fq_prefill* query, void* workspace,
                    size_t workspace_bytes, fq_stream_t stream) {
    return prefill(cache, tail, query, workspace, workspace_bytes, stream, 8);
}

int fq_quest_decode_int4_noalloc(const fq_int4_cache* cache, const fq_query* query, const float* retention,
                                 int32_t num_sinks, int32_t window_pages, int32_t k_max, int32_t select_mode,
                                 float* scores_out, uint8_t* mask_out, fq_stream_t stream) {
    if (!cache || !query) return fail(FQ_ERR_INVALID, "cache or query descriptor is NULL");
    const size_t need = fq_workspace_bytes(cache, query->H_q);
    if (need == 0) return fail(FQ_ERR_INVALID, "H_q=%d must be a positive multiple of H_kv=%d", query->H_q, cache->H_kv);
    if (need > (size_t)FQ_NOALLOC_SCRATCH_BYTES)
        return fail(FQ_ERR_UNSUPPORTED,
                    "fq_quest_decode_int4_noalloc: this step needs %zu bytes of scratch, the static buffer holds %zu "
                    "(call fq_quest_decode_int4 with a workspace)", need, (size_t)FQ_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    const int st = noalloc_scratch(&ws);
    if (st) return st;
    return fq_quest_decode_int4(cache, query, retention, num_sinks, window_pages, k_max, select_mode, scores_out,
                                mask_out, ws, (size_t)FQ_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
