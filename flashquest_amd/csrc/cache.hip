// Cache writes on page completion: INT4 quantisation of whole 64-token pages
// straight from their two sources (the bf16 partial-page tail and the newly
// appended tokens), and the tail staging copy.  Reference semantics:
// src/flashquest/cache/persistent_int4.py:69-132 (update_quantized) with the
// quantisers of src/flashquest/kernel/kv_quant.py:131-205.
//
// One workgroup of 256 threads per (page, batch * head).  Thread t owns 8
// channels (c8 = t % (D/8)) of tokens r, r + RPP, ... (r = t / (D/8)): every
// load is 16 contiguous bytes and the D/8 threads of a token read one
// contiguous row.  K: per-channel min/max over the page (lane shuffles, then
// LDS across the 4 waves), scale arithmetic in the input dtype, codes by IEEE
// fp32 division (the same operations as quant_k_kernel).  V: per-token,
// per-group min/max over the group's lanes, fp32 arithmetic (as
// quant_v_kernel).  Codes are stored 4 bytes (8 channels) per thread and token.
#include "fq_common.h"
#include "turbo_quant.h"

namespace fq {

constexpr float kCacheEps = 1e-6f;                      // kv_quant.py:14
__device__ __constant__ float kCacheInv15 = 1.0f / 15.0f;
__device__ __constant__ float kCacheInv255 = 1.0f / 255.0f;    // the INT8 quantisers' "/ 255.0"

namespace {

constexpr int kPage = 64;

// Positions [0, head_len) come from head, the rest from tail (position
// head_len is tail's token 0).  Element strides (b, h, t); channels contiguous.
struct TokSrc {
    const void* head; int64_t hs[3];
    const void* tail; int64_t ts[3];
    int head_len;
    int dtype;
};

struct PageQuantParams {
    TokSrc k, v;
    bool do_k, k_codes, do_v;
    int B, H, n_tok;
    int tok_dst0;                       // destination token of position 0 (a page boundary for K)
    uint8_t* kp; int64_t kp_s[3];       // (b, h, t) byte strides
    void* ks; int64_t ks_s[3];          // (b, h, page) element strides; channels contiguous
    void* km; int64_t km_s[3];
    uint8_t* vp; int64_t vp_s[3];
    void* vs; int64_t vs_s[3];          // (b, h, t); groups contiguous
    void* vm; int64_t vm_s[3];
    int v_group;
    int meta_dtype;
};

FQ_DEV void load8(const TokSrc& s, int b, int h, int pos, int c8, float (&x)[8]) {
    const bool in_head = pos < s.head_len;
    const char* base = (const char*)(in_head ? s.head : s.tail);
    const int64_t* st = in_head ? s.hs : s.ts;
    const int t = in_head ? pos : pos - s.head_len;
    const int64_t e = b * st[0] + h * st[1] + t * st[2] + 8 * c8;
    if (s.dtype == FQ_F32) {
        const uint4 a = *(const uint4*)(base + e * 4), c = *(const uint4*)(base + e * 4 + 16);
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = __uint_as_float(w[i]);
    } else {
        const uint4 a = *(const uint4*)(base + e * 2);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = s.dtype == FQ_BF16 ? bf16_bits_to_f(w[i] & 0xFFFFu) : f16_bits_to_f(w[i] & 0xFFFFu);
            x[2 * i + 1] = s.dtype == FQ_BF16 ? bf16_bits_to_f(w[i] >> 16) : f16_bits_to_f(w[i] >> 16);
        }
    }
}

template <int BITS>
FQ_DEV uint32_t codeq(float v, float mn, float s) {
    float c = rintf(__fdiv_rn(v - mn, s));
    c = fminf(fmaxf(c, 0.f), (float)((1 << BITS) - 1));
    return (uint32_t)c;
}

// The 8 codes of a thread's channels: BITS 4 packs two per byte (4 bytes),
// BITS 8 one per byte (8 bytes), at byte 8 * c8 * BITS / 8 of the row.
template <int BITS>
FQ_DEV void store_codes(uint8_t* row, int c8, const uint32_t (&c)[8]) {
    if constexpr (BITS == 4) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) word |= c[i] << (4 * i);
        *(uint32_t*)(row + 4 * c8) = word;
    } else {
        *(uint2*)(row + 8 * c8) = make_uint2(c[0] | c[1] << 8 | c[2] << 16 | c[3] << 24,
                                             c[4] | c[5] << 8 | c[6] << 16 | c[7] << 24);
    }
}

FQ_DEV uint32_t meta_bits(float f, int dtype) {
    return dtype == FQ_BF16 ? f_to_bf16_bits(f) : f_to_f16_bits(f);
}

template <int D, int BITS>
__global__ __launch_bounds__(kThreads) void page_quant_kernel(PageQuantParams a) {
    constexpr int CPR = D / 8;                  // threads per token row
    constexpr int RPP = kThreads / CPR;         // token rows per pass
    constexpr int TPT = kPage / RPP;            // tokens per thread
    const int tid = threadIdx.x;
    const int c8 = tid % CPR, r = tid / CPR;
    const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const int pg = blockIdx.x;
    int pos[TPT];
    bool ok[TPT];
#pragma unroll
    for (int u = 0; u < TPT; ++u) {
        pos[u] = pg * kPage + r + RPP * u;
        ok[u] = pos[u] < a.n_tok;
    }

    if (a.do_k) {
        float x[TPT][8];
        float mn[8], mx[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) { mn[i] = INFINITY; mx[i] = -INFINITY; }
#pragma unroll
        for (int u = 0; u < TPT; ++u) {
            if (ok[u]) {
                load8(a.k, b, h, pos[u], c8, x[u]);
#pragma unroll
                for (int i = 0; i < 8; ++i) { mn[i] = fminf(mn[i], x[u][i]); mx[i] = fmaxf(mx[i], x[u][i]); }
            }
        }
        // rows of this wave: lanes c8 + CPR * j
#pragma unroll
        for (int off = CPR; off < 64; off <<= 1) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                mn[i] = fminf(mn[i], __shfl_xor(mn[i], off, 64));
                mx[i] = fmaxf(mx[i], __shfl_xor(mx[i], off, 64));
            }
        }
        __shared__ float s_red[kThreads / 64][CPR][16];
        const int w = tid >> 6;
        if ((tid & 63) < CPR) {
#pragma unroll
            for (int i = 0; i < 8; ++i) { s_red[w][c8][i] = mn[i]; s_red[w][c8][8 + i] = mx[i]; }
        }
        __syncthreads();
#pragma unroll
        for (int ww = 0; ww < kThreads / 64; ++ww) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                mn[i] = fminf(mn[i], s_red[ww][c8][i]);
                mx[i] = fmaxf(mx[i], s_red[ww][c8][8 + i]);
            }
        }
        // scale in the input dtype (kv_quant.py:131-149), as quant_k_kernel
        const int dt = a.k.dtype;
        float sc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float diff = round_to(mx[i] - mn[i], dt);
            float s = round_to(diff * (BITS == 8 ? kCacheInv255 : kCacheInv15), dt);
            sc[i] = round_to(fmaxf(s, kCacheEps), dt);
        }
        if (r == 0) {
            const int64_t p = a.tok_dst0 / kPage + pg;
            uint32_t sw[4], mw[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sw[j] = meta_bits(sc[2 * j], a.meta_dtype) | meta_bits(sc[2 * j + 1], a.meta_dtype) << 16;
                mw[j] = meta_bits(mn[2 * j], a.meta_dtype) | meta_bits(mn[2 * j + 1], a.meta_dtype) << 16;
            }
            *(uint4*)((uint16_t*)a.ks + b * a.ks_s[0] + h * a.ks_s[1] + p * a.ks_s[2] + 8 * c8) =
                make_uint4(sw[0], sw[1], sw[2], sw[3]);
            *(uint4*)((uint16_t*)a.km + b * a.km_s[0] + h * a.km_s[1] + p * a.km_s[2] + 8 * c8) =
                make_uint4(mw[0], mw[1], mw[2], mw[3]);
        }
        if (a.k_codes) {
#pragma unroll
            for (int u = 0; u < TPT; ++u) {
                if (!ok[u]) continue;
                uint32_t cd[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) cd[i] = codeq<BITS>(x[u][i], mn[i], sc[i]);
                store_codes<BITS>(a.kp + b * a.kp_s[0] + h * a.kp_s[1] + (int64_t)(a.tok_dst0 + pos[u]) * a.kp_s[2],
                                  c8, cd);
            }
        }
    }

    if (a.do_v) {
        const int lpg = a.v_group / 8;          // lanes per V group (a power of two <= CPR)
        const int g = (8 * c8) / a.v_group;
#pragma unroll
        for (int u = 0; u < TPT; ++u) {
            // every lane of the row takes part in the shuffles; invalid tokens are not stored
            float x[8];
            if (ok[u]) load8(a.v, b, h, pos[u], c8, x);
            else {
#pragma unroll
                for (int i = 0; i < 8; ++i) x[i] = 0.f;
            }
            float mn = x[0], mx = x[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) { mn = fminf(mn, x[i]); mx = fmaxf(mx, x[i]); }
            for (int off = 1; off < lpg; off <<= 1) {
                mn = fminf(mn, __shfl_xor(mn, off, 64));
                mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            }
            // fp32 (kv_quant.py:189-205; INT8: 78-89)
            const float s = fmaxf((mx - mn) * (BITS == 8 ? kCacheInv255 : kCacheInv15), kCacheEps);
            if (!ok[u]) continue;
            const int64_t t = a.tok_dst0 + pos[u];
            if (c8 % lpg == 0) {
                store_any(a.vs, a.meta_dtype, b * a.vs_s[0] + h * a.vs_s[1] + t * a.vs_s[2] + g, s);
                store_any(a.vm, a.meta_dtype, b * a.vm_s[0] + h * a.vm_s[1] + t * a.vm_s[2] + g, mn);
            }
            uint32_t cd[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) cd[i] = codeq<BITS>(x[i], mn, s);
            store_codes<BITS>(a.vp + b * a.vp_s[0] + h * a.vp_s[1] + t * a.vp_s[2], c8, cd);
        }
    }
}

// Tail staging: tokens [src_t0, src_t0 + n) of src -> [dst_t0, dst_t0 + n) of
// dst, 16 bytes per thread; blockIdx.y selects K (0) or V (1).
struct TailCopyParams {
    const void* src[2]; int64_t ss[2][3];
    void* dst[2]; int64_t ds[2][3];
    int src_t0, dst_t0, n, B, H, row_bytes, esize;
    int zero_rows;          // after the copy range, dst rows [dst_t0 + n, dst_t0 + n + zero_rows) are zeroed
};

__global__ __launch_bounds__(kThreads) void tail_copy_kernel(TailCopyParams a) {
    const int kv = blockIdx.y;
    const int chunks = a.row_bytes / 16;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int rows = a.n + a.zero_rows;
    const int64_t total = (int64_t)a.B * a.H * rows * chunks;
    if (idx >= total) return;
    const int ch = idx % chunks;
    const int t = (idx / chunks) % rows;
    const int bh = idx / ((int64_t)chunks * rows);
    const int b = bh / a.H, h = bh % a.H;
    char* d = (char*)a.dst[kv] +
              (b * a.ds[kv][0] + h * a.ds[kv][1] + (int64_t)(a.dst_t0 + t) * a.ds[kv][2]) * a.esize + 16 * ch;
    if (t >= a.n) {
        *(uint4*)d = make_uint4(0u, 0u, 0u, 0u);
        return;
    }
    const char* s = (const char*)a.src[kv] +
                    (b * a.ss[kv][0] + h * a.ss[kv][1] + (int64_t)(a.src_t0 + t) * a.ss[kv][2]) * a.esize + 16 * ch;
    *(uint4*)d = *(const uint4*)s;
}

// TurboQuant rows of positions [0, n_tok) of a two-source token stream into
// the planes / per-token scale at token tok_dst0 + position; one thread per
// (b, h, token), the arithmetic of turbo_quant_row.
struct TurboAppendParams {
    TokSrc src;
    int B, H, n_tok, tok_dst0;
    uint8_t* msb; int64_t msb_s[3];     // (b, h, t) byte strides; bytes of a row contiguous
    uint8_t* lsb; int64_t lsb_s[3];
    void* scale; int64_t s_s[3];        // (b, h, t) element strides (bf16)
};

template <int D>
__global__ __launch_bounds__(kThreads) void turbo_append_kernel(TurboAppendParams a) {
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.H * a.n_tok;
    if (idx >= total) return;
    const int pos = idx % a.n_tok;
    const int h = (idx / a.n_tok) % a.H;
    const int b = idx / ((int64_t)a.n_tok * a.H);
    float v[D];
#pragma unroll
    for (int c8 = 0; c8 < D / 8; ++c8) {
        float x[8];
        load8(a.src, b, h, pos, c8, x);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[8 * c8 + i] = x[i];
    }
    const int64_t t = a.tok_dst0 + pos;
    turbo_quant_row<D>(v, a.src.dtype, a.msb + b * a.msb_s[0] + h * a.msb_s[1] + t * a.msb_s[2], 1,
                       a.lsb + b * a.lsb_s[0] + h * a.lsb_s[1] + t * a.lsb_s[2], 1, a.scale,
                       b * a.s_s[0] + h * a.s_s[1] + t * a.s_s[2]);
}

bool rows16(const void* p, const int64_t* s, int n, int esize) {
    if ((uintptr_t)p & 15) return false;
    for (int i = 0; i < n; ++i)
        if ((s[i] * esize) % 16) return false;
    return true;
}

}  // namespace

bool page_quant_k_ok(int D, int page, int in_dtype, const void* k, const int64_t* k_s, const uint8_t* packed,
                     const int64_t* p_s, const void* scale, const int64_t* s_s, const void* mn, const int64_t* m_s) {
    if ((D != 64 && D != 128) || page != kPage) return false;
    const int es = in_dtype == FQ_F32 ? 4 : 2;
    if (k_s[3] != 1 || !rows16(k, k_s, 3, es)) return false;
    if (p_s[3] != 1 || ((uintptr_t)packed & 3) || p_s[0] % 4 || p_s[1] % 4 || p_s[2] % 4) return false;
    if (s_s[3] != 1 || m_s[3] != 1 || !rows16(scale, s_s, 3, 2) || !rows16(mn, m_s, 3, 2)) return false;
    return true;
}

bool page_quant_v_ok(int D, int group, int in_dtype, const void* v, const int64_t* v_s, const uint8_t* packed,
                     const int64_t* p_s, const int64_t* s_s, const int64_t* m_s) {
    if (D != 64 && D != 128) return false;
    if (group < 8 || group > D || (group & (group - 1))) return false;
    const int es = in_dtype == FQ_F32 ? 4 : 2;
    if (v_s[3] != 1 || !rows16(v, v_s, 3, es)) return false;
    if (p_s[3] != 1 || ((uintptr_t)packed & 3) || p_s[0] % 4 || p_s[1] % 4 || p_s[2] % 4) return false;
    if (D / group > 1 && (s_s[3] != 1 || m_s[3] != 1)) return false;
    return true;
}

// Quantise positions [0, n_tok) of (k, v) sources into the outputs at token
// tok_dst0 (K: whole pages, tok_dst0 a multiple of 64).
hipError_t launch_page_quant(const PageQuantParams& a, int D, hipStream_t st, int bits = 4) {
    if (a.n_tok <= 0 || a.B * a.H == 0) return hipSuccess;
    dim3 grid((a.n_tok + kPage - 1) / kPage, a.B * a.H);
    if (D == 128 && bits == 4) hipLaunchKernelGGL((page_quant_kernel<128, 4>), grid, dim3(kThreads), 0, st, a);
    else if (D == 64 && bits == 4) hipLaunchKernelGGL((page_quant_kernel<64, 4>), grid, dim3(kThreads), 0, st, a);
    else if (D == 128 && bits == 8) hipLaunchKernelGGL((page_quant_kernel<128, 8>), grid, dim3(kThreads), 0, st, a);
    else if (D == 64 && bits == 8) hipLaunchKernelGGL((page_quant_kernel<64, 8>), grid, dim3(kThreads), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_quant_k_pages(const void* k, int in_dtype, const int64_t* k_s, int B, int H, int S, int D,
                                uint8_t* packed, const int64_t* p_s, void* scale, const int64_t* s_s, void* mn,
                                const int64_t* m_s, int meta_dtype, hipStream_t st) {
    PageQuantParams a{};
    a.k = TokSrc{nullptr, {0, 0, 0}, k, {k_s[0], k_s[1], k_s[2]}, 0, in_dtype};
    a.do_k = true; a.k_codes = true;
    a.B = B; a.H = H; a.n_tok = S; a.tok_dst0 = 0;
    for (int i = 0; i < 3; ++i) { a.kp_s[i] = p_s[i]; a.ks_s[i] = s_s[i]; a.km_s[i] = m_s[i]; }
    a.kp = packed; a.ks = scale; a.km = mn; a.meta_dtype = meta_dtype;
    return launch_page_quant(a, D, st);
}

hipError_t launch_quant_v_pages(const void* v, int in_dtype, const int64_t* v_s, int B, int H, int S, int D,
                                int group, uint8_t* packed, const int64_t* p_s, void* scale, const int64_t* s_s,
                                void* mn, const int64_t* m_s, int meta_dtype, hipStream_t st) {
    PageQuantParams a{};
    a.v = TokSrc{nullptr, {0, 0, 0}, v, {v_s[0], v_s[1], v_s[2]}, 0, in_dtype};
    a.do_v = true;
    a.B = B; a.H = H; a.n_tok = S; a.tok_dst0 = 0;
    for (int i = 0; i < 3; ++i) { a.vp_s[i] = p_s[i]; a.vs_s[i] = s_s[i]; a.vm_s[i] = m_s[i]; }
    a.vp = packed; a.vs = scale; a.vm = mn; a.v_group = group; a.meta_dtype = meta_dtype;
    return launch_page_quant(a, D, st);
}

// Stage the tokens that remain after the completed pages in the partial-page
// tail: tokens [src_t0, src_t0 + n) of the new tokens -> tail rows
// [dst_t0, dst_t0 + n); zero_tail also clears the tail rows after them (the
// INT8 cache's convention, persistent_int8.py:129-132).
hipError_t stage_tail(int B, int H, int D, int page, void* kpart, const int64_t* kpart_s, void* vpart,
                      const int64_t* vpart_s, int64_t layer, const void* knew, const int64_t* kn_s, const void* vnew,
                      const int64_t* vn_s, int src_t0, int dst_t0, int n, bool zero_tail, hipStream_t st) {
    const int zero_rows = zero_tail ? page - (dst_t0 + n) : 0;
    if (n + zero_rows == 0 || B * H == 0) return hipSuccess;
    TailCopyParams t{};
    t.src[0] = knew; t.src[1] = vnew;
    t.dst[0] = (char*)kpart + layer * kpart_s[0] * 2;
    t.dst[1] = (char*)vpart + layer * vpart_s[0] * 2;
    for (int i = 0; i < 3; ++i) {
        t.ss[0][i] = kn_s[i]; t.ss[1][i] = vn_s[i];
        t.ds[0][i] = kpart_s[i + 1]; t.ds[1][i] = vpart_s[i + 1];
    }
    t.src_t0 = src_t0; t.dst_t0 = dst_t0; t.n = n; t.zero_rows = zero_rows;
    t.B = B; t.H = H; t.esize = 2; t.row_bytes = D * 2;
    const int64_t threads = (int64_t)B * H * (n + zero_rows) * (t.row_bytes / 16);
    hipLaunchKernelGGL(tail_copy_kernel, dim3((unsigned)((threads + kThreads - 1) / kThreads), 2), dim3(kThreads), 0,
                       st, t);
    return hipGetLastError();
}

// The page arithmetic of an append: `seen` tokens were in the layer, S_new
// arrive; the stream (old tail, new tokens) completes n_complete pages
// starting at token page_tok0, and `rest` tokens stay in the tail.
struct AppendPlan {
    int partial_len, n_complete, complete_len, page_tok0, rest;
};
AppendPlan plan_append(int seen, int S_new, int page) {
    AppendPlan p{};
    p.partial_len = seen % page;
    p.n_complete = (p.partial_len + S_new) / page;
    p.complete_len = p.n_complete * page;
    p.page_tok0 = seen - p.partial_len;
    p.rest = p.partial_len + S_new - p.complete_len;
    return p;
}

// Token sources of the stream: the layer's tail rows, then the new tokens.
TokSrc stream_src(const void* part, const int64_t* part_s, int64_t layer, const void* fresh, const int64_t* fresh_s,
                  int partial_len, int dtype) {
    return TokSrc{(const char*)part + layer * part_s[0] * 2, {part_s[1], part_s[2], part_s[3]}, fresh,
                  {fresh_s[0], fresh_s[1], fresh_s[2]}, partial_len, dtype};
}

// update_quantized of the INT4 cache (persistent_int4.py:69-132; bits 4) and
// of the INT8 cache (persistent_int8.py:72-135; bits 8, tail rows after the
// staged ones zeroed) for one layer: pages completed by the append are
// quantised from (partial tail, new tokens) into the cache, then the remaining
// tokens are staged in the tail.  The page kernel reads the old tail before
// the copy (stream order) overwrites it.
hipError_t launch_kv_append(const Int4Cache& c, int layer, void* kpart, const int64_t* kpart_s, void* vpart,
                            const int64_t* vpart_s, int part_dtype, const void* knew, const int64_t* kn_s,
                            const void* vnew, const int64_t* vn_s, int seen, int S_new, int bits, hipStream_t st) {
    const AppendPlan pl = plan_append(seen, S_new, c.page);
    const int64_t l = layer;
    if (pl.n_complete > 0) {
        PageQuantParams a{};
        a.k = stream_src(kpart, kpart_s, l, knew, kn_s, pl.partial_len, part_dtype);
        a.v = stream_src(vpart, vpart_s, l, vnew, vn_s, pl.partial_len, part_dtype);
        a.do_k = true; a.k_codes = true; a.do_v = true;
        a.B = c.B; a.H = c.Hkv; a.n_tok = pl.complete_len; a.tok_dst0 = pl.page_tok0;
        a.kp = (uint8_t*)c.kp + l * c.kp_s[0];
        a.vp = (uint8_t*)c.vp + l * c.vp_s[0];
        a.ks = (uint16_t*)c.ksc + l * c.ksc_s[0];
        a.km = (uint16_t*)c.kmn + l * c.kmn_s[0];
        a.vs = (uint16_t*)c.vsc + l * c.vsc_s[0];
        a.vm = (uint16_t*)c.vmn + l * c.vmn_s[0];
        for (int i = 0; i < 3; ++i) {
            a.kp_s[i] = c.kp_s[i + 1]; a.vp_s[i] = c.vp_s[i + 1];
            a.ks_s[i] = c.ksc_s[i + 1]; a.km_s[i] = c.kmn_s[i + 1];
            a.vs_s[i] = c.vsc_s[i + 1]; a.vm_s[i] = c.vmn_s[i + 1];
        }
        a.v_group = c.D / c.G;
        a.meta_dtype = c.meta_dtype;
        const hipError_t e = launch_page_quant(a, c.D, st, bits);
        if (e != hipSuccess) return e;
    }
    // without a completed page the new tokens extend the tail in place
    const bool done = pl.n_complete > 0;
    return stage_tail(c.B, c.Hkv, c.D, c.page, kpart, kpart_s, vpart, vpart_s, l, knew, kn_s, vnew, vn_s,
                      done ? S_new - pl.rest : 0, done ? 0 : pl.partial_len, done ? pl.rest : S_new, bits == 8, st);
}

// update_quantized of the TurboQuant cache (persistent_turbo.py:83-147) for
// one layer: for the completed pages, the un-rotated K's bf16 page scale/min
// (the INT4 metadata, no codes) and the K and V rotated 3-bit planes with
// their per-token scales; then the remaining tokens go to the tail.  raw:
// descriptor of K_scale_raw / K_mn_raw (ksc / kmn, element strides).
hipError_t launch_turbo_append(const fq_turbo_cache& tc, const Int4Cache& raw, int layer, void* kpart,
                               const int64_t* kpart_s, void* vpart, const int64_t* vpart_s, int part_dtype,
                               const void* knew, const int64_t* kn_s, const void* vnew, const int64_t* vn_s, int seen,
                               int S_new, hipStream_t st) {
    const AppendPlan pl = plan_append(seen, S_new, tc.page_size);
    const int64_t l = layer;
    if (pl.n_complete > 0) {
        PageQuantParams a{};
        a.k = stream_src(kpart, kpart_s, l, knew, kn_s, pl.partial_len, part_dtype);
        a.do_k = true; a.k_codes = false;
        a.B = tc.B; a.H = tc.H_kv; a.n_tok = pl.complete_len; a.tok_dst0 = pl.page_tok0;
        a.ks = (uint16_t*)raw.ksc + l * raw.ksc_s[0];
        a.km = (uint16_t*)raw.kmn + l * raw.kmn_s[0];
        for (int i = 0; i < 3; ++i) { a.ks_s[i] = raw.ksc_s[i + 1]; a.km_s[i] = raw.kmn_s[i + 1]; }
        a.meta_dtype = FQ_BF16;
        hipError_t e = launch_page_quant(a, tc.D, st, 4);
        if (e != hipSuccess) return e;
        for (int kv = 0; kv < 2; ++kv) {
            TurboAppendParams t{};
            t.src = kv == 0 ? a.k : stream_src(vpart, vpart_s, l, vnew, vn_s, pl.partial_len, part_dtype);
            t.B = tc.B; t.H = tc.H_kv; t.n_tok = pl.complete_len; t.tok_dst0 = pl.page_tok0;
            const uint8_t* msb = kv == 0 ? tc.k_msb : tc.v_msb;
            const uint8_t* lsb = kv == 0 ? tc.k_lsb : tc.v_lsb;
            const void* sc = kv == 0 ? tc.k_scale : tc.v_scale;
            const int64_t* ms = kv == 0 ? tc.kmsb_strides : tc.vmsb_strides;
            const int64_t* ls = kv == 0 ? tc.klsb_strides : tc.vlsb_strides;
            const int64_t* ss = kv == 0 ? tc.kst_strides : tc.vst_strides;
            t.msb = (uint8_t*)msb + l * ms[0];
            t.lsb = (uint8_t*)lsb + l * ls[0];
            t.scale = (uint16_t*)sc + l * ss[0];
            for (int i = 0; i < 3; ++i) { t.msb_s[i] = ms[i + 1]; t.lsb_s[i] = ls[i + 1]; t.s_s[i] = ss[i + 1]; }
            const int64_t n = (int64_t)t.B * t.H * t.n_tok;
            const dim3 grid((unsigned)((n + kThreads - 1) / kThreads));
            if (tc.D == 128) hipLaunchKernelGGL(turbo_append_kernel<128>, grid, dim3(kThreads), 0, st, t);
            else if (tc.D == 64) hipLaunchKernelGGL(turbo_append_kernel<64>, grid, dim3(kThreads), 0, st, t);
            else return hipErrorInvalidValue;
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
    }
    const bool done = pl.n_complete > 0;
    return stage_tail(tc.B, tc.H_kv, tc.D, tc.page_size, kpart, kpart_s, vpart, vpart_s, l, knew, kn_s, vnew, vn_s,
                      done ? S_new - pl.rest : 0, done ? 0 : pl.partial_len, done ? pl.rest : S_new, false, st);
}

}  // namespace fq
