// The memory-system ceiling of the decode step's access pattern: a kernel
// that reads exactly the bytes the single-launch INT4 decode reads, in the
// same order and granularity, and computes nothing.  One workgroup of 8 waves
// per KV group streams the K scale / min of every page (the scoring
// metadata, 16 bytes per lane and load), then its waves take the group's
// selected pages w, w + 8, ... and read each page's K and V codes, V scale /
// min and K scale / min.  Measurement only: bench.py times it beside the
// decode, so the gap between the two is what scoring, selection and the
// attention math add.  Every loaded word is folded into a value that is
// stored only if it hits an unlikely constant, so no load is dead.
//
// Built into its own library, libfq_probe.so (entries in fq_probe.h), which
// bench.py loads; the product library libfq_hip.so does not contain it.
//
// read_stream_kernel is the plainest read of the same byte count: one
// contiguous buffer, 2048 workgroups of 512 threads each streaming a
// contiguous slice with four 16-byte loads in flight per thread -- the rate
// HBM gives a read of this size with no access pattern at all.
#include "fq_probe.h"
#include "fused_common.h"

namespace fq {
namespace {

template <int G>
__global__ __launch_bounds__(512) void read_step_kernel(Int4Cache c, Workspace ws, unsigned* sink) {
    constexpr int NT = 512, NW = 8;
    const int g = blockIdx.x, tid = threadIdx.x, lane = lane_id(), w = wave_id();
    const int h = g % c.Hkv, b = (g / c.Hkv) % c.B, l = g / (c.Hkv * c.B);
    const char* ks = (const char*)((const uint16_t*)c.ksc + l * c.ksc_s[0] + b * c.ksc_s[1] + h * c.ksc_s[2]);
    const char* km = (const char*)((const uint16_t*)c.kmn + l * c.kmn_s[0] + b * c.kmn_s[1] + h * c.kmn_s[2]);
    uint32_t acc = 0;
    // scoring metadata: P pages x 256 bytes of K scale and of K min
    {
        const int n16 = c.P * 16;                  // 16-byte chunks per tensor
        for (int i = tid; i < n16; i += 4 * NT) {
            uint4 x[8];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = min(i + u * NT, n16 - 1);
                x[2 * u] = *(const uint4*)(ks + (int64_t)j * 16);
                x[2 * u + 1] = *(const uint4*)(km + (int64_t)j * 16);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) acc ^= x[u].x ^ x[u].w;
        }
    }
    __syncthreads();
    const uint8_t* kp = c.kp + l * c.kp_s[0] + b * c.kp_s[1] + h * c.kp_s[2];
    const uint8_t* vp = c.vp + l * c.vp_s[0] + b * c.vp_s[1] + h * c.vp_s[2];
    const char* vs = (const char*)((const uint16_t*)c.vsc + l * c.vsc_s[0] + b * c.vsc_s[1] + h * c.vsc_s[2]);
    const char* vm = (const char*)((const uint16_t*)c.vmn + l * c.vmn_s[0] + b * c.vmn_s[1] + h * c.vmn_s[2]);
    const int n = ws.n_sel[g];
    for (int i = w; i < n; i += NW) {
        const int p = ws.entries[(int64_t)g * c.P + i] & 0xFFFF;
        const int64_t t0 = (int64_t)p * 64;
        uint4 a[4], v[4];
#pragma unroll
        for (int T = 0; T < 4; ++T) {
            a[T] = *(const uint4*)(kp + t0 * 64 + T * 1024 + lane * 16);
            v[T] = *(const uint4*)(vp + t0 * 64 + T * 1024 + lane * 16);
        }
        uint32_t x = 0;
        if constexpr (G == 4) {
            const uint2 s = *(const uint2*)(vs + (t0 + lane) * 8), m = *(const uint2*)(vm + (t0 + lane) * 8);
            x = s.x ^ m.y;
        } else {
            x = *(const uint16_t*)(vs + (t0 + lane) * 2) ^ *(const uint16_t*)(vm + (t0 + lane) * 2);
        }
        const uint32_t ksv = *(const uint32_t*)(ks + (int64_t)p * 256 + lane * 4);
        const uint32_t kmv = *(const uint32_t*)(km + (int64_t)p * 256 + lane * 4);
#pragma unroll
        for (int T = 0; T < 4; ++T) x ^= a[T].x ^ v[T].y;
        acc ^= x ^ ksv ^ kmv;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

__global__ __launch_bounds__(512) void read_stream_kernel(const uint4* __restrict__ p, int64_t n16, int64_t per_wg,
                                                         unsigned* sink) {
    constexpr int NT = 512, U = 4;
    const int64_t base = (int64_t)blockIdx.x * per_wg, end = min(base + per_wg, n16);
    uint32_t acc = 0;
    for (int64_t i = base + threadIdx.x; i < end; i += NT * U) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t j = min(i + (int64_t)u * NT, end - 1);
            v[u] = p[j];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace

hipError_t launch_read_stream(const void* p, int64_t bytes, unsigned* sink, hipStream_t st) {
    const int64_t n16 = bytes / 16;
    constexpr int kWgs = 2048;
    const int64_t per = (n16 + kWgs - 1) / kWgs;
    timer_before_launch(st);
    hipLaunchKernelGGL(read_stream_kernel, dim3(kWgs), dim3(512), 0, st, (const uint4*)p, n16, per, sink);
    timer_after_launch(st);
    return hipGetLastError();
}

hipError_t launch_read_step(const Int4Cache& c, const Workspace& ws, unsigned* sink, hipStream_t st) {
    const int groups = c.L * c.B * c.Hkv;
    timer_before_launch(st);
    if (c.G == 4) hipLaunchKernelGGL(read_step_kernel<4>, dim3(groups), dim3(512), 0, st, c, ws, sink);
    else hipLaunchKernelGGL(read_step_kernel<1>, dim3(groups), dim3(512), 0, st, c, ws, sink);
    timer_after_launch(st);
    return hipGetLastError();
}

}  // namespace fq

using namespace fq;

extern "C" {

int fq_read_decode_pages(const fq_int4_cache* cache, const uint8_t* mask, const int64_t mask_strides[4],
                         int32_t H_q, uint32_t* sink, void* workspace, size_t workspace_bytes_, fq_stream_t stream) {
    Int4Cache c{};
    int st = check_cache(cache, &c);
    if (st) return st;
    if (H_q < 1 || H_q % c.Hkv) return fail(FQ_ERR_INVALID, "H_q=%d must be divisible by H_kv=%d", H_q, c.Hkv);
    if (c.D != 128 || c.page != 64 || (c.G != 1 && c.G != 4))
        return fail(FQ_ERR_UNSUPPORTED, "the read-only pass takes the matrix-core decode's layout");
    if (c.kp_s[3] != 64 || c.vp_s[3] != 64 || c.ksc_s[3] != 128 || c.kmn_s[3] != 128 || c.vsc_s[3] != c.G ||
        c.vmn_s[3] != c.G)
        return fail(FQ_ERR_UNSUPPORTED, "the read-only pass takes packed token / page rows");
    if (!mask || !sink) return fail(FQ_ERR_INVALID, "NULL mask or sink");
    const int G = c.L * c.B * c.Hkv, nrep = H_q / c.Hkv;
    const size_t need = workspace_bytes(G, c.P, nrep, nrep, c.D);
    if (!workspace || workspace_bytes_ < need)
        return fail(FQ_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, workspace_bytes_);
    Workspace ws = carve_workspace(workspace, G, c.P, nrep, nrep, c.D);
    hipStream_t s = (hipStream_t)stream;
    st = hip_status(fq::launch_union_from_mask(mask, mask_strides, c.L, c.B, c.Hkv, nrep, c.P, ws, s), "page union");
    if (st) return st;
    return hip_status(launch_read_step(c, ws, sink, s), "read decode pages");
}

int fq_read_stream(const void* buf, size_t bytes, uint32_t* sink, fq_stream_t stream) {
    if (!buf || !sink) return fail(FQ_ERR_INVALID, "NULL buffer or sink");
    if (((uintptr_t)buf & 15) || (bytes & 15) || bytes == 0)
        return fail(FQ_ERR_INVALID, "the stream read takes a 16-byte aligned buffer of a nonzero multiple of 16 bytes");
    return hip_status(launch_read_stream(buf, (int64_t)bytes, sink, (hipStream_t)stream), "read stream");
}

}  // extern "C"
