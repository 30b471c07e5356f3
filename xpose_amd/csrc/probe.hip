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
#include <algorithm>
#include <vector>

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

// Exchange-latency chain: the token kernel's cross-workgroup hand-off
// measured alone. `stages` stages; stage s has `n` producer roles, each of
// which publishes a 64-float vector as 32 tagged 16-byte pairs; every role of
// stage s + 1 first waits until it has read all n vectors of stage s with the
// current tag (all 512 threads re-reading their pairs, as the token kernel's
// consumers do). Role r of stage s runs on workgroup ((s n + r) mod (grid /
// stride)) stride: stride 1 spreads the roles over all XCDs, stride 8 keeps
// them on the workgroups of one XCD (the hardware deals a launch's
// workgroups to the eight XCDs in turn). Stores are device-coherent (sc1),
// or with l2 set kept in the XCD's L2 (valid for stride 8 only). The grid
// must be resident at once (one 512-thread workgroup per CU); every wait is
// bounded and a timeout sets status. Each workgroup records the 100 MHz
// s_memrealtime of its first and last publish.
constexpr int kXcThreads = 512;
__device__ __forceinline__ uint32_t xcc_of_wave() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 0xFu;
}
struct XcArgs {
    u32x4* slots;                 // [stages][n][32] pairs
    unsigned long long* times;    // [grid][2]
    uint32_t* status;
    uint32_t stages, n, tag, stride, l2, spin_limit;
};

__global__ __launch_bounds__(kXcThreads) void exchange_chain_kernel(XcArgs a) {
    const uint32_t wg = blockIdx.x, tid = threadIdx.x;
    const uint32_t tag = a.tag;
    const rsrc_t rr = make_rsrc(a.slots, a.stages * a.n * 32u * 16u);
    const uint32_t n_slots = gridDim.x / a.stride;
    unsigned long long t_first = 0, t_last = 0;
    constexpr int M = 16;                                  // pairs per thread (n <= 256)
    for (uint32_t s = 0; s < a.stages; ++s) {
        for (uint32_t r = 0; r < a.n; ++r) {
            if (((s * a.n + r) % n_slots) * a.stride != wg) continue;
            if (s > 0) {
                const uint32_t np = a.n * 32u, base = (s - 1u) * a.n * 32u;
                const u32x4 ready = {0u, tag, 0u, tag};
                uint32_t off[M];
                bool act[M];
                u32x4 v[M];
#pragma unroll
                for (int i = 0; i < M; ++i) {
                    const uint32_t p = tid + uint32_t(i) * kXcThreads;
                    act[i] = p < np;
                    off[i] = (base + (act[i] ? p : 0u)) * 16u;
                }
#pragma unroll
                for (int i = 0; i < M; ++i) v[i] = act[i] ? ld_dev16(rr, off[i]) : ready;
                for (uint32_t spins = 0;; ++spins) {
                    bool ok = true;
#pragma unroll
                    for (int i = 0; i < M; ++i) ok &= (v[i].y == tag) & (v[i].w == tag);
                    if (ok) break;
                    if (spins > a.spin_limit) {
                        __hip_atomic_fetch_or((XP_GLOBAL uint32_t*)a.status, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    asm volatile("" ::: "memory");
#pragma unroll
                    for (int i = 0; i < M; ++i) v[i] = act[i] ? ld_dev16(rr, off[i]) : ready;
                }
                __syncthreads();
            }
            if (tid == 0 && t_first == 0) t_first = __builtin_amdgcn_s_memrealtime();
            if (tid < 32) {
                const uint32_t o = ((s * a.n + r) * 32u + tid) * 16u;
                const u32x4 val = {__float_as_uint(float(s)), tag, __float_as_uint(float(r)), tag};
                if (a.l2) __builtin_amdgcn_raw_buffer_store_b128(val, rr, int(o), 0, 0);
                else __builtin_amdgcn_raw_buffer_store_b128(val, rr, int(o), 0, kAuxDev);
            }
            if (tid == 0) t_last = __builtin_amdgcn_s_memrealtime();
        }
    }
    if (tid == 0) {
        a.times[2 * wg] = t_first;
        a.times[2 * wg + 1] = t_last;
    }
}

// Hand-off ping-pong: the token kernel's exchange reduced to two
// workgroups, to split a stage's wait into its parts. Workgroup 0 (ping)
// stores `np` tagged 16-byte pairs; workgroup `peer` (pong) has its 512
// threads poll all np pairs (device-scope loads) until every tag is the
// round's, passes a barrier, and answers with one pair, which ping's wave 0
// polls. Stores are device-scope (sc1) or, with l2, kept in the XCD's L2
// (pong on the same XCD only). A round trip is one payload hand-off plus one
// 16-byte one; every wait is bounded and a timeout sets status.
constexpr uint32_t kPpMaxPerThread = 8;   // pairs a pong thread polls (np <= 4096)
__global__ __launch_bounds__(512) void handoff_pingpong_kernel(u32x4* buf, uint32_t peer, uint32_t iters,
                                                               uint32_t np, uint32_t l2, uint32_t spin_limit,
                                                               unsigned long long* out, uint32_t* status) {
    const uint32_t wg = blockIdx.x, tid = threadIdx.x;
    if (wg != 0u && wg != peer) return;
    // [0, 2 x 4096) payload pairs of even / odd rounds, then the answers
    const rsrc_t r = make_rsrc(buf, (2u * 4096u + 2u) * 16u);
    __shared__ uint32_t sh_err[2];
    uint32_t err = 0;
    const bool ping = wg == 0u;
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t i = 1; i <= iters && !err; ++i) {
        const uint32_t base = (i & 1u) * 4096u, ans = 2u * 4096u + (i & 1u);
        const u32x4 val = {i, i, i, i};
        if (ping) {
            for (uint32_t p = tid; p < np; p += 512u) {
                if (l2) __builtin_amdgcn_raw_buffer_store_b128(val, r, int((base + p) * 16u), 0, 0);
                else __builtin_amdgcn_raw_buffer_store_b128(val, r, int((base + p) * 16u), 0, kAuxDev);
            }
            if (tid < 64u) {
                for (uint32_t s = 0;; ++s) {
                    asm volatile("" ::: "memory");
                    const u32x4 v = ld_dev16(r, ans * 16u);
                    if (__builtin_amdgcn_ballot_w64((v.y != i) | (v.w != i)) == 0ull) break;
                    if (s > spin_limit) { err = i; break; }
                }
            }
        } else {
            bool act[kPpMaxPerThread];
            uint32_t off[kPpMaxPerThread];
#pragma unroll
            for (uint32_t k = 0; k < kPpMaxPerThread; ++k) {
                const uint32_t p = tid + 512u * k;
                act[k] = p < np;
                off[k] = (base + (act[k] ? p : 0u)) * 16u;
            }
            for (uint32_t s = 0;; ++s) {
                asm volatile("" ::: "memory");
                bool ok = true;
#pragma unroll
                for (uint32_t k = 0; k < kPpMaxPerThread; ++k) {
                    const u32x4 v = act[k] ? ld_dev16(r, off[k]) : val;
                    ok &= (v.y == i) & (v.w == i);
                }
                if (ok) break;
                if (s > spin_limit) { err = i; break; }
            }
        }
        if (tid == 0u) sh_err[i & 1u] = 0u;
        __syncthreads();
        if (err) sh_err[i & 1u] = err;
        __syncthreads();
        err = sh_err[i & 1u];
        if (!ping && tid == 0u && !err) {
            if (l2) __builtin_amdgcn_raw_buffer_store_b128(val, r, int(ans * 16u), 0, 0);
            else __builtin_amdgcn_raw_buffer_store_b128(val, r, int(ans * 16u), 0, kAuxDev);
        }
    }
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    if (tid == 0u) {
        if (err)
            __hip_atomic_fetch_or((XP_GLOBAL uint32_t*)status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (ping) {
            out[0] = r1 - r0;
            out[1] = xcc_of_wave();
        } else {
            out[2] = xcc_of_wave();
        }
    }
}

// One lane walks a cyclic chain of dependent loads (next index in 4-byte
// words), plain or device-scope (sc1): clocks per load once warm.
__global__ void load_chase_kernel(const uint32_t* buf, uint32_t bytes, uint32_t steps, uint32_t dev,
                                  unsigned long long* out) {
    if (blockIdx.x != 0u || threadIdx.x != 0u) return;
    const rsrc_t r = make_rsrc(buf, bytes);
    uint32_t idx = 0;
    for (uint32_t i = 0; i < steps; ++i)
        idx = dev ? __builtin_amdgcn_raw_buffer_load_b32(r, int(idx * 4u), 0, kAuxDev)
                  : __builtin_amdgcn_raw_buffer_load_b32(r, int(idx * 4u), 0, 0);
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (uint32_t i = 0; i < steps; ++i)
        idx = dev ? __builtin_amdgcn_raw_buffer_load_b32(r, int(idx * 4u), 0, kAuxDev)
                  : __builtin_amdgcn_raw_buffer_load_b32(r, int(idx * 4u), 0, 0);
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    out[0] = t1 - t0;
    out[1] = idx;
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

int xp_stream_read_rot_batch_timed(const void* const* bufs, uint32_t nbufs, size_t bytes, uint32_t grid,
                                   uint32_t count, uint32_t reps, xp_stream stream, float* best_ms) {
    XP_REQUIRE(bufs && best_ms && nbufs > 0, "null pointer or no buffers");
    XP_REQUIRE(bytes >= 16 && bytes % 16 == 0, "bytes=%zu must be a positive multiple of 16",
               bytes);
    for (uint32_t i = 0; i < nbufs; ++i)
        XP_REQUIRE(bufs[i] && (reinterpret_cast<uintptr_t>(bufs[i]) & 15u) == 0,
                   "buffer %u is null or not 16-byte aligned", i);
    XP_REQUIRE(count > 0 && reps > 0, "count and reps must be positive");
    XP_REQUIRE(grid <= 65536, "grid=%u > 65536", grid);
    DeviceScratch* sc = scratch();
    if (!sc) return XP_E_HIP;
    if (!ensure_partial(sc, 4)) return XP_E_NOMEM;
    uint32_t* sink = reinterpret_cast<uint32_t*>(sc->partial);   // never written in practice
    const uint32_t g = grid ? grid : n_cu();
    return graph_batch_timed(
        [&](hipStream_t cs) {
            for (uint32_t i = 0; i < count; ++i)
                hipLaunchKernelGGL(stream_read_kernel, dim3(g), dim3(kStreamThreads), 0, cs, sink,
                                   static_cast<const u32x4*>(bufs[i % nbufs]), bytes / 16);
            if (hipGetLastError() != hipSuccess)
                return set_error(XP_E_HIP, "xp_stream_read_rot_batch_timed: launch failed");
            return int(XP_OK);
        },
        reps, as_stream(stream), best_ms);
}

int xp_exchange_chain_timed(uint32_t producers, uint32_t stages, uint32_t stride, int l2_local,
                            xp_stream stream, float* ns_per_stage) {
    XP_REQUIRE(ns_per_stage, "null pointer");
    XP_REQUIRE(stride == 1 || stride == 8, "stride=%u must be 1 or 8", stride);
    XP_REQUIRE(!l2_local || stride == 8, "l2_local needs stride 8 (one XCD)");
    XP_REQUIRE(stages >= 2 && stages <= 256, "stages=%u must be in [2, 256]", stages);
    const uint32_t grid = n_cu();
    XP_REQUIRE(producers >= 1 && producers <= 256 && producers <= grid / stride,
               "producers=%u must be in [1, min(256, %u)]", producers, grid / stride);
    const size_t lds = 96 * 1024;   // over half a CU's LDS: one workgroup per CU
    const void* fn = reinterpret_cast<const void*>(&exchange_chain_kernel);
    XP_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    int per_cu = 0;
    XP_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kXcThreads, lds));
    XP_REQUIRE(per_cu >= 1, "a CU cannot hold the probe's workgroup");
    hipStream_t st = as_stream(stream);
    const size_t slot_bytes = size_t(stages) * producers * 32u * 16u;
    char* mem = nullptr;
    const size_t tb = slot_bytes + size_t(grid) * 16u + 256u;
    XP_HIP(hipMalloc(&mem, tb));
    XcArgs a{};
    a.slots = reinterpret_cast<u32x4*>(mem);
    a.times = reinterpret_cast<unsigned long long*>(mem + slot_bytes);
    a.status = reinterpret_cast<uint32_t*>(mem + slot_bytes + size_t(grid) * 16u);
    a.stages = stages;
    a.n = producers;
    a.tag = 1u;
    a.stride = stride;
    a.l2 = l2_local ? 1u : 0u;
    a.spin_limit = 1u << 18;
    std::vector<unsigned long long> h(size_t(grid) * 2u);
    uint32_t status = 0;
    void* args[] = {&a};
    hipError_t e = hipMemsetAsync(mem, 0, tb, st);
    if (e == hipSuccess) e = hipLaunchKernel(fn, dim3(grid), dim3(kXcThreads), args, lds, st);
    if (e == hipSuccess) e = hipMemcpyAsync(h.data(), a.times, h.size() * 8u, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipMemcpyAsync(&status, a.status, 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    (void)hipFree(mem);
    if (e != hipSuccess) return set_error(XP_E_HIP, "xp_exchange_chain_timed: %s", hipGetErrorString(e));
    if (status != 0)
        return set_error(XP_E_DEVICE, "xp_exchange_chain_timed: a wait ran past its spin limit "
                         "(the grid was not resident at once)");
    unsigned long long lo = ~0ull, hi = 0;
    for (uint32_t w = 0; w < grid; ++w) {
        if (h[2u * w] == 0) continue;
        lo = h[2u * w] < lo ? h[2u * w] : lo;
        hi = h[2u * w + 1u] > hi ? h[2u * w + 1u] : hi;
    }
    *ns_per_stage = hi > lo ? float(double(hi - lo) * 10.0 / double(stages - 1u)) : 0.0f;
    return XP_OK;
}

int xp_handoff_pingpong_timed(uint32_t same_xcd, uint32_t payload_pairs, int l2_local, uint32_t iters,
                              xp_stream stream, float* ns_round_trip, uint32_t* xcc_pair) {
    XP_REQUIRE(ns_round_trip, "null pointer");
    XP_REQUIRE(payload_pairs >= 1 && payload_pairs <= 512u * kPpMaxPerThread,
               "payload_pairs=%u must be in [1, %u]", payload_pairs, 512u * kPpMaxPerThread);
    XP_REQUIRE(!l2_local || same_xcd, "l2_local needs the pong on ping's XCD");
    XP_REQUIRE(iters >= 1 && iters <= 100000, "iters=%u must be in [1, 100000]", iters);
    hipStream_t st = as_stream(stream);
    const size_t slot_bytes = (2u * 4096u + 2u) * 16u;
    char* mem = nullptr;
    XP_HIP(hipMalloc(&mem, slot_bytes + 64));
    u32x4* slots = reinterpret_cast<u32x4*>(mem);
    unsigned long long* out = reinterpret_cast<unsigned long long*>(mem + slot_bytes);
    uint32_t* status = reinterpret_cast<uint32_t*>(mem + slot_bytes + 32);
    // workgroups w and w + 8 share an XCD under the cyclic dealing (the
    // XCC ids are returned so the caller can see it held)
    const uint32_t peer = same_xcd ? 8u : 1u;
    unsigned long long h[3] = {};
    uint32_t stat = 0;
    hipError_t e = hipMemsetAsync(mem, 0, slot_bytes + 64, st);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(handoff_pingpong_kernel, dim3(16), dim3(512), 0, st, slots, peer, iters, payload_pairs,
                           uint32_t(l2_local ? 1 : 0), 1u << 18, out, status);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpyAsync(h, out, sizeof(h), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipMemcpyAsync(&stat, status, 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    (void)hipFree(mem);
    if (e != hipSuccess) return set_error(XP_E_HIP, "xp_handoff_pingpong_timed: %s", hipGetErrorString(e));
    if (stat) return set_error(XP_E_DEVICE, "xp_handoff_pingpong_timed: a wait ran past its spin limit");
    *ns_round_trip = float(double(h[0]) * 10.0 / iters);
    if (xcc_pair) *xcc_pair = uint32_t(h[1] & 0xFFu) | (uint32_t(h[2] & 0xFFu) << 8);
    return XP_OK;
}

int xp_load_latency(uint32_t bytes, uint32_t stride, int device_scope, xp_stream stream, float* clk_per_load) {
    XP_REQUIRE(clk_per_load, "null pointer");
    XP_REQUIRE(stride >= 4 && stride % 4 == 0 && bytes >= 2 * stride && bytes % stride == 0 &&
                   bytes <= (1u << 30),
               "bytes=%u / stride=%u: a multiple of stride, 2 nodes to 1 GiB, stride a multiple of 4", bytes,
               stride);
    const uint32_t n = bytes / stride, w = stride / 4;
    // a random cyclic order of the nodes (fixed seed): node order[i] points to order[i + 1]
    std::vector<uint32_t> order(n);
    for (uint32_t i = 0; i < n; ++i) order[i] = i;
    uint64_t x = 0x9E3779B97F4A7C15ull;
    for (uint32_t i = n - 1; i > 1; --i) {
        x ^= x << 13; x ^= x >> 7; x ^= x << 17;
        const uint32_t j = 1u + uint32_t(x % i);
        std::swap(order[i], order[j]);
    }
    std::vector<uint32_t> host(size_t(bytes) / 4, 0u);
    for (uint32_t i = 0; i < n; ++i) host[size_t(order[i]) * w] = order[(i + 1) % n] * w;
    hipStream_t st = as_stream(stream);
    char* mem = nullptr;
    XP_HIP(hipMalloc(&mem, size_t(bytes) + 16));
    unsigned long long* out = reinterpret_cast<unsigned long long*>(mem + bytes);
    unsigned long long h[2] = {};
    const uint32_t steps = 4096;
    hipError_t e = hipMemcpyAsync(mem, host.data(), bytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(load_chase_kernel, dim3(1), dim3(64), 0, st, reinterpret_cast<const uint32_t*>(mem), bytes,
                           steps, uint32_t(device_scope ? 1 : 0), out);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpyAsync(h, out, sizeof(h), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    (void)hipFree(mem);
    if (e != hipSuccess) return set_error(XP_E_HIP, "xp_load_latency: %s", hipGetErrorString(e));
    *clk_per_load = float(double(h[0]) / steps);
    return XP_OK;
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
