// Vocabulary reductions for sampling (kernels/llm_sampling.cl part 1).
//
// argmax: the reference needs a 3-level dispatch tree (262144 -> 4096 -> 64
// -> 1, llm_sampling.cl:42-48) because it has no workgroup memory. Here one
// launch does it: each workgroup reduces a contiguous slice with 16-byte
// loads and wave shuffles, and the last workgroup to finish (arrival ticket)
// reduces the per-workgroup winners. The comparison is (value, index)
// lexicographic — larger value, then lower index — and every slot starts at
// (-inf, 0), so the result equals the reference's serial scan
// (llm_transformer.cl:618-629) and its tree (llm_sampling.cl:50-56) for every
// input, NaNs included (a NaN never compares greater).
#include "xp_device.hpp"
#include "xp_launch.hpp"

namespace xp {

constexpr int kAmThreads = 256;

struct AmArgs {
    uint32_t* out_idx;
    float* out_val;
    const float* logits;
    uint32_t n;
    uint32_t per_wg;        // elements per workgroup (multiple of 4)
    float* pval;            // [gridDim.x]
    uint32_t* pidx;
    uint32_t* ticket;
    uint32_t* advance;      // when set, the last workgroup adds 1 here (a session's position)
};

__global__ __launch_bounds__(kAmThreads) void argmax_kernel(AmArgs a) {
    __shared__ float sv[kAmThreads / kWave];
    __shared__ uint32_t si[kAmThreads / kWave];
    __shared__ uint32_t last;
    const uint32_t tid = threadIdx.x;
    const uint32_t lo = blockIdx.x * a.per_wg;
    const uint32_t hi = min(lo + a.per_wg, a.n);
    float bv = -INFINITY;
    uint32_t bi = 0u;
    const uint32_t n4 = (hi > lo) ? (hi - lo) / 4 : 0;
    const float4* p4 = reinterpret_cast<const float4*>(a.logits + lo);
    for (uint32_t i = tid; i < n4; i += blockDim.x) {
        const float4 v = p4[i];
        const uint32_t k = lo + 4 * i;
        am_better(bv, bi, v.x, k);
        am_better(bv, bi, v.y, k + 1);
        am_better(bv, bi, v.z, k + 2);
        am_better(bv, bi, v.w, k + 3);
    }
    for (uint32_t k = lo + 4 * n4 + tid; k < hi; k += blockDim.x) am_better(bv, bi, a.logits[k], k);
    am_wave(bv, bi);
    if (tid % kWave == 0) { sv[tid / kWave] = bv; si[tid / kWave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kAmThreads / kWave; ++w) am_better(bv, bi, sv[w], si[w]);
        st_dev(a.pval + blockIdx.x, bv);
        st_dev(a.pidx + blockIdx.x, bi);
        wait_mem();
        last = take_ticket(a.ticket);
    }
    __syncthreads();
    if (last != gridDim.x - 1) return;
    bv = -INFINITY;
    bi = 0u;
    for (uint32_t w = tid; w < gridDim.x; w += blockDim.x)
        am_better(bv, bi, ld_dev(a.pval + w), ld_dev(a.pidx + w));
    am_wave(bv, bi);
    __syncthreads();
    if (tid % kWave == 0) { sv[tid / kWave] = bv; si[tid / kWave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kAmThreads / kWave; ++w) am_better(bv, bi, sv[w], si[w]);
        *a.out_idx = bi;
        if (a.out_val) *a.out_val = bv;
        if (a.advance) *a.advance += 1u;
        st_dev(a.ticket, 0u);
    }
}

// topk4_partial, llm_sampling.cl:318-347: one thread per strided chain
// e = p (mod nparts), best four by strict '>' (earliest index on ties),
// unfilled slots (-inf, 0xFFFFFFFF). Pure comparisons: bit-identical output.
// The chain's values are loaded kT4Batch at a time, all in flight together
// (one memory latency per batch, not one per element), then walked in chain
// order; past the end a slot holds -inf, which never enters the four.
constexpr uint32_t kT4Batch = 64;

__global__ __launch_bounds__(256) void topk4_kernel(float* cval, uint32_t* cidx, const float* x,
                                                    uint32_t n, uint32_t nparts) {
    x += size_t(blockIdx.y) * n;                 // batched rows (grid.y)
    cval += size_t(blockIdx.y) * nparts * 4u;
    cidx += size_t(blockIdx.y) * nparts * 4u;
    const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= nparts) return;
    float v0 = -INFINITY, v1 = -INFINITY, v2 = -INFINITY, v3 = -INFINITY;
    uint32_t i0 = 0xFFFFFFFFu, i1 = 0xFFFFFFFFu, i2 = 0xFFFFFFFFu, i3 = 0xFFFFFFFFu;
    for (size_t e0 = p; e0 < n; e0 += size_t(kT4Batch) * nparts) {
        float xv[kT4Batch];
#pragma unroll
        for (uint32_t j = 0; j < kT4Batch; ++j) {
            const size_t e = e0 + size_t(j) * nparts;
            xv[j] = e < n ? x[e] : -INFINITY;
        }
#pragma unroll
        for (uint32_t j = 0; j < kT4Batch; ++j) {
            // insertion by selects: v0 >= v1 >= v2 >= v3, so c0 implies c1
            // implies c2 implies c3, and the four selects below are the
            // branches "above v0 / v1 / v2 / v3" of the sequential insert
            // (NaN and -inf compare false everywhere and change nothing)
            const float v = xv[j];
            const uint32_t e = uint32_t(e0 + size_t(j) * nparts);
            const bool c0 = v > v0, c1 = v > v1, c2 = v > v2, c3 = v > v3;
            v3 = c2 ? v2 : (c3 ? v : v3);
            i3 = c2 ? i2 : (c3 ? e : i3);
            v2 = c1 ? v1 : (c2 ? v : v2);
            i2 = c1 ? i1 : (c2 ? e : i2);
            v1 = c0 ? v0 : (c1 ? v : v1);
            i1 = c0 ? i0 : (c1 ? e : i1);
            v0 = c0 ? v : v0;
            i0 = c0 ? e : i0;
        }
    }
    const uint32_t o = p * 4u;
    cval[o + 0] = v0; cidx[o + 0] = i0;
    cval[o + 1] = v1; cidx[o + 1] = i1;
    cval[o + 2] = v2; cidx[o + 2] = i2;
    cval[o + 3] = v3; cidx[o + 3] = i3;
}

// Shared with the decode session, which owns its own partial/ticket buffers.
int launch_argmax(uint32_t* out_idx, float* out_val, const float* logits, uint32_t n,
                  float* pval, uint32_t* pidx, uint32_t* ticket, hipStream_t st, uint32_t* advance) {
    AmArgs a{out_idx, out_val, logits, n, 0, pval, pidx, ticket, advance};
    uint32_t nwg = (n + 4095) / 4096;
    if (nwg > uint32_t(kAmMaxWg)) nwg = kAmMaxWg;
    if (nwg < 1) nwg = 1;
    a.per_wg = ((n + nwg - 1) / nwg + 3) & ~3u;
    nwg = (n + a.per_wg - 1) / a.per_wg;
    if (nwg < 1) nwg = 1;
    hipLaunchKernelGGL(argmax_kernel, dim3(nwg), dim3(kAmThreads), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "argmax: launch -> %s", hipGetErrorString(e));
    return XP_OK;
}

int launch_topk4(float* cval, uint32_t* cidx, const float* x, uint32_t n, uint32_t nparts,
                 hipStream_t st, uint32_t rows) {
    hipLaunchKernelGGL(topk4_kernel, dim3((nparts + 255) / 256, rows), dim3(256), 0, st, cval, cidx, x,
                       n, nparts);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "topk4: launch -> %s", hipGetErrorString(e));
    return XP_OK;
}

}  // namespace xp

using namespace xp;

extern "C" {

int xp_argmax(uint32_t* out_idx, float* out_val, const float* logits, uint32_t n,
              xp_stream stream) {
    XP_REQUIRE(out_idx && logits, "null pointer");
    XP_REQUIRE(n > 0, "n must be positive");
    XP_REQUIRE((reinterpret_cast<uintptr_t>(logits) & 15u) == 0, "logits must be 16-byte aligned");
    DeviceScratch* sc = scratch();
    if (!sc) return XP_E_HIP;
    if (!ensure_partial(sc, 2 * kAmMaxWg) || !ensure_tickets(sc, 1)) return XP_E_NOMEM;
    return launch_argmax(out_idx, out_val, logits, n, sc->partial,
                         reinterpret_cast<uint32_t*>(sc->partial + kAmMaxWg), sc->tickets,
                         as_stream(stream));
}

int xp_topk4_harvest(float* cval, uint32_t* cidx, const float* logits, uint32_t n,
                     uint32_t nparts, xp_stream stream) {
    XP_REQUIRE(cval && cidx && logits, "null pointer");
    XP_REQUIRE(nparts > 0, "nparts must be positive");
    return launch_topk4(cval, cidx, logits, n, nparts, as_stream(stream));
}

}  // extern "C"
