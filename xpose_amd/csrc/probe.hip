// Bandwidth probes: the ceiling the matvec and the token step are measured
// against (the reference's stream4, kernels/llm_matvec.cl:357-378), and a plain
// copy of known size whose counter readings calibrate rocprofv3's FETCH_SIZE /
// WRITE_SIZE (HBM bytes per dispatch) for the other kernels.
//
// stream_read: each workgroup reads one contiguous chunk with 16-byte
// nontemporal loads, four per thread in flight (the shape that measured
// highest in a sweep of chunked and grid-stride layouts on MI355X). As in the
// reference, the only store is guarded by a value the sum cannot take, so
// every load stays live and nothing is written.
#include "xp_device.hpp"
#include "xp_launch.hpp"

namespace xp {

constexpr int kProbeThreads = 256;
constexpr int kStreamThreads = 512;
constexpr int kStreamUnroll = 4;

__global__ __launch_bounds__(kStreamThreads) void stream_read_kernel(uint32_t* sink, const u32x4* src,
                                                                     size_t n) {
    const size_t per = (n + gridDim.x - 1) / gridDim.x;
    const size_t lo = size_t(blockIdx.x) * per;
    const size_t hi = lo + per < n ? lo + per : n;
    u32x4 acc = {0u, 0u, 0u, 0u};
    size_t i = lo + threadIdx.x;
    for (; i + (kStreamUnroll - 1) * kStreamThreads < hi; i += kStreamUnroll * kStreamThreads) {
        u32x4 v[kStreamUnroll];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) v[u] = ld_stream4(src + i + u * kStreamThreads);
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) acc += v[u];
    }
    for (; i < hi; i += kStreamThreads) acc += ld_stream4(src + i);
    const uint32_t s = acc.x + acc.y + acc.z + acc.w;
    if (s == 0xDEADBEEFu) sink[threadIdx.x & 3u] = s;
}

__global__ __launch_bounds__(kProbeThreads) void copy_kernel(u32x4* dst, const u32x4* src, size_t n) {
    const size_t stride = size_t(gridDim.x) * kProbeThreads;
    for (size_t i = size_t(blockIdx.x) * kProbeThreads + threadIdx.x; i < n; i += stride)
        __builtin_nontemporal_store(ld_stream4(src + i), dst + i);
}

namespace {
uint32_t n_cu() {
    DeviceScratch* s = scratch();
    return uint32_t(s && s->n_cu > 0 ? s->n_cu : 256);
}
}  // namespace

}  // namespace xp

using namespace xp;

extern "C" {

int xp_stream_read_timed(const void* buf, size_t bytes, uint32_t iters, xp_stream stream,
                         float* ms) {
    XP_REQUIRE(buf && ms, "null pointer");
    XP_REQUIRE(bytes >= 16 && bytes % 16 == 0, "bytes=%zu must be a positive multiple of 16",
               bytes);
    XP_REQUIRE((reinterpret_cast<uintptr_t>(buf) & 15u) == 0, "buffer must be 16-byte aligned");
    XP_REQUIRE(iters > 0, "iters must be positive");
    DeviceScratch* sc = scratch();
    if (!sc) return XP_E_HIP;
    if (!ensure_partial(sc, 4)) return XP_E_NOMEM;
    uint32_t* sink = reinterpret_cast<uint32_t*>(sc->partial);   // never written in practice
    hipStream_t st = as_stream(stream);
    const uint32_t grid = n_cu();   // one chunk per CU
    hipEvent_t e0 = nullptr, e1 = nullptr;
    XP_HIP(hipEventCreate(&e0));
    XP_HIP(hipEventCreate(&e1));
    int rc = XP_OK;
    hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(kStreamThreads), 0, st, sink,
                       static_cast<const u32x4*>(buf), bytes / 16);
    if (hipEventRecord(e0, st) != hipSuccess) rc = set_error(XP_E_HIP, "xp_stream_read_timed: event");
    for (uint32_t i = 0; i < iters && rc == XP_OK; ++i)
        hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(kStreamThreads), 0, st,
                           sink, static_cast<const u32x4*>(buf), bytes / 16);
    if (rc == XP_OK && hipGetLastError() != hipSuccess)
        rc = set_error(XP_E_HIP, "xp_stream_read_timed: launch failed");
    if (rc == XP_OK && hipEventRecord(e1, st) != hipSuccess)
        rc = set_error(XP_E_HIP, "xp_stream_read_timed: event");
    if (rc == XP_OK && hipEventSynchronize(e1) != hipSuccess)
        rc = set_error(XP_E_HIP, "xp_stream_read_timed: sync");
    if (rc == XP_OK && hipEventElapsedTime(ms, e0, e1) != hipSuccess)
        rc = set_error(XP_E_HIP, "xp_stream_read_timed: elapsed");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

int xp_stream_read_rot_timed(const void* const* bufs, uint32_t nbufs, size_t bytes, uint32_t grid,
                             uint32_t iters, xp_stream stream, float* ms) {
    XP_REQUIRE(bufs && ms && nbufs > 0, "null pointer or no buffers");
    XP_REQUIRE(bytes >= 16 && bytes % 16 == 0, "bytes=%zu must be a positive multiple of 16",
               bytes);
    for (uint32_t i = 0; i < nbufs; ++i)
        XP_REQUIRE(bufs[i] && (reinterpret_cast<uintptr_t>(bufs[i]) & 15u) == 0,
                   "buffer %u is null or not 16-byte aligned", i);
    XP_REQUIRE(iters > 0, "iters must be positive");
    XP_REQUIRE(grid <= 65536, "grid=%u > 65536", grid);
    DeviceScratch* sc = scratch();
    if (!sc) return XP_E_HIP;
    if (!ensure_partial(sc, 4)) return XP_E_NOMEM;
    uint32_t* sink = reinterpret_cast<uint32_t*>(sc->partial);   // never written in practice
    hipStream_t st = as_stream(stream);
    const uint32_t g = grid ? grid : n_cu();
    hipEvent_t e0 = nullptr, e1 = nullptr;
    XP_HIP(hipEventCreate(&e0));
    XP_HIP(hipEventCreate(&e1));
    int rc = XP_OK;
    for (uint32_t i = 0; i < nbufs; ++i)   // one untimed pass
        hipLaunchKernelGGL(stream_read_kernel, dim3(g), dim3(kStreamThreads), 0, st, sink,
                           static_cast<const u32x4*>(bufs[i]), bytes / 16);
    if (hipEventRecord(e0, st) != hipSuccess) rc = set_error(XP_E_HIP, "xp_stream_read_rot_timed: event");
    for (uint32_t i = 0; i < iters && rc == XP_OK; ++i)
        hipLaunchKernelGGL(stream_read_kernel, dim3(g), dim3(kStreamThreads), 0, st, sink,
                           static_cast<const u32x4*>(bufs[i % nbufs]), bytes / 16);
    if (rc == XP_OK && hipGetLastError() != hipSuccess)
        rc = set_error(XP_E_HIP, "xp_stream_read_rot_timed: launch failed");
    if (rc == XP_OK && hipEventRecord(e1, st) != hipSuccess)
        rc = set_error(XP_E_HIP, "xp_stream_read_rot_timed: event");
    if (rc == XP_OK && hipEventSynchronize(e1) != hipSuccess)
        rc = set_error(XP_E_HIP, "xp_stream_read_rot_timed: sync");
    if (rc == XP_OK && hipEventElapsedTime(ms, e0, e1) != hipSuccess)
        rc = set_error(XP_E_HIP, "xp_stream_read_rot_timed: elapsed");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

int xp_copy(void* dst, const void* src, size_t bytes, xp_stream stream) {
    XP_REQUIRE(dst && src, "null pointer");
    XP_REQUIRE(bytes % 16 == 0, "bytes=%zu must be a multiple of 16", bytes);
    XP_REQUIRE(((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15u) == 0,
               "buffers must be 16-byte aligned");
    if (bytes == 0) return XP_OK;
    hipLaunchKernelGGL(copy_kernel, dim3(n_cu() * 8u), dim3(kProbeThreads), 0, as_stream(stream),
                       static_cast<u32x4*>(dst), static_cast<const u32x4*>(src), bytes / 16);
    XP_LAUNCHED();
    return XP_OK;
}

}  // extern "C"
