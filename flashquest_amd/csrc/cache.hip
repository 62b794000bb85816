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

namespace fq {

constexpr float kCacheEps = 1e-6f;                      // kv_quant.py:14
__device__ __constant__ float kCacheInv15 = 1.0f / 15.0f;

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

FQ_DEV uint32_t code4(float v, float mn, float s) {
    float c = rintf(__fdiv_rn(v - mn, s));
    c = fminf(fmaxf(c, 0.f), 15.f);
    return (uint32_t)c;
}

FQ_DEV uint32_t meta_bits(float f, int dtype) {
    return dtype == FQ_BF16 ? f_to_bf16_bits(f) : f_to_f16_bits(f);
}

template <int D>
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
            float s = round_to(diff * kCacheInv15, dt);
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
                uint32_t word = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) word |= code4(x[u][i], mn[i], sc[i]) << (4 * i);
                *(uint32_t*)(a.kp + b * a.kp_s[0] + h * a.kp_s[1] + (int64_t)(a.tok_dst0 + pos[u]) * a.kp_s[2] +
                             4 * c8) = word;
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
            const float s = fmaxf((mx - mn) * kCacheInv15, kCacheEps);      // fp32 (kv_quant.py:189-205)
            if (!ok[u]) continue;
            const int64_t t = a.tok_dst0 + pos[u];
            if (c8 % lpg == 0) {
                store_any(a.vs, a.meta_dtype, b * a.vs_s[0] + h * a.vs_s[1] + t * a.vs_s[2] + g, s);
                store_any(a.vm, a.meta_dtype, b * a.vm_s[0] + h * a.vm_s[1] + t * a.vm_s[2] + g, mn);
            }
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) word |= code4(x[i], mn, s) << (4 * i);
            *(uint32_t*)(a.vp + b * a.vp_s[0] + h * a.vp_s[1] + t * a.vp_s[2] + 4 * c8) = word;
        }
    }
}

// Tail staging: tokens [src_t0, src_t0 + n) of src -> [dst_t0, dst_t0 + n) of
// dst, 16 bytes per thread; blockIdx.y selects K (0) or V (1).
struct TailCopyParams {
    const void* src[2]; int64_t ss[2][3];
    void* dst[2]; int64_t ds[2][3];
    int src_t0, dst_t0, n, B, H, row_bytes, esize;
};

__global__ __launch_bounds__(kThreads) void tail_copy_kernel(TailCopyParams a) {
    const int kv = blockIdx.y;
    const int chunks = a.row_bytes / 16;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.H * a.n * chunks;
    if (idx >= total) return;
    const int ch = idx % chunks;
    const int t = (idx / chunks) % a.n;
    const int bh = idx / ((int64_t)chunks * a.n);
    const int b = bh / a.H, h = bh % a.H;
    const char* s = (const char*)a.src[kv] +
                    (b * a.ss[kv][0] + h * a.ss[kv][1] + (int64_t)(a.src_t0 + t) * a.ss[kv][2]) * a.esize + 16 * ch;
    char* d = (char*)a.dst[kv] +
              (b * a.ds[kv][0] + h * a.ds[kv][1] + (int64_t)(a.dst_t0 + t) * a.ds[kv][2]) * a.esize + 16 * ch;
    *(uint4*)d = *(const uint4*)s;
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
hipError_t launch_page_quant(const PageQuantParams& a, int D, hipStream_t st) {
    if (a.n_tok <= 0 || a.B * a.H == 0) return hipSuccess;
    dim3 grid((a.n_tok + kPage - 1) / kPage, a.B * a.H);
    if (D == 128) hipLaunchKernelGGL(page_quant_kernel<128>, grid, dim3(kThreads), 0, st, a);
    else if (D == 64) hipLaunchKernelGGL(page_quant_kernel<64>, grid, dim3(kThreads), 0, st, a);
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

// update_quantized (persistent_int4.py:69-132) for one layer: pages completed
// by the append are quantised from (partial tail, new tokens) into the cache,
// then the remaining tokens are staged in the tail.  The page kernel reads the
// old tail before the copy (stream order) overwrites it.
hipError_t launch_int4_append(const Int4Cache& c, int layer, void* kpart, const int64_t* kpart_s, void* vpart,
                              const int64_t* vpart_s, int part_dtype, const void* knew, const int64_t* kn_s,
                              const void* vnew, const int64_t* vn_s, int seen, int S_new, hipStream_t st) {
    const int page = c.page;
    const int partial_len = seen % page;
    const int total = partial_len + S_new;
    const int n_complete = total / page;
    const int complete_len = n_complete * page;
    const int new_partial = total - complete_len;
    const int64_t l = layer;
    if (n_complete > 0) {
        PageQuantParams a{};
        const char* kp0 = (const char*)kpart + l * kpart_s[0] * 2;
        const char* vp0 = (const char*)vpart + l * vpart_s[0] * 2;
        a.k = TokSrc{kp0, {kpart_s[1], kpart_s[2], kpart_s[3]}, knew, {kn_s[0], kn_s[1], kn_s[2]}, partial_len,
                     part_dtype};
        a.v = TokSrc{vp0, {vpart_s[1], vpart_s[2], vpart_s[3]}, vnew, {vn_s[0], vn_s[1], vn_s[2]}, partial_len,
                     part_dtype};
        a.do_k = true; a.k_codes = true; a.do_v = true;
        a.B = c.B; a.H = c.Hkv; a.n_tok = complete_len; a.tok_dst0 = seen - partial_len;
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
        const hipError_t e = launch_page_quant(a, c.D, st);
        if (e != hipSuccess) return e;
    }
    const int n = n_complete > 0 ? new_partial : S_new;
    if (n == 0 || c.B * c.Hkv == 0) return hipSuccess;
    TailCopyParams t{};
    t.src[0] = knew; t.src[1] = vnew;
    t.dst[0] = (char*)kpart + l * kpart_s[0] * 2;
    t.dst[1] = (char*)vpart + l * vpart_s[0] * 2;
    for (int i = 0; i < 3; ++i) {
        t.ss[0][i] = kn_s[i]; t.ss[1][i] = vn_s[i];
        t.ds[0][i] = kpart_s[i + 1]; t.ds[1][i] = vpart_s[i + 1];
    }
    t.src_t0 = n_complete > 0 ? S_new - new_partial : 0;
    t.dst_t0 = n_complete > 0 ? 0 : partial_len;
    t.n = n; t.B = c.B; t.H = c.Hkv; t.esize = 2; t.row_bytes = c.D * 2;
    const int64_t threads = (int64_t)c.B * c.Hkv * n * (t.row_bytes / 16);
    hipLaunchKernelGGL(tail_copy_kernel, dim3((unsigned)((threads + kThreads - 1) / kThreads), 2), dim3(kThreads), 0,
                       st, t);
    return hipGetLastError();
}

}  // namespace fq
