// int4 group-quantised matvec for gfx950 over the reference's KM4 packing.
//
// Semantics (kernels/llm_matvec.cl:187-200, :422-456):
//   out[j] = sum_b scale(b, j) * sum_{t<32} in[32b+t] * (nibble(32b+t, j) - 8)
//
// Mapping. The KM4 plane stores, for column group g (64 outputs) and block b,
// 64 consecutive uint4: one 16-byte quantisation block per output. A wave is
// one task = (group g, chunk of k): lane t owns output 64g+t and issues one
// global_load_dwordx4 per block, so a wave reads 1 KiB contiguous per block.
// No cross-lane reduction is needed inside a task. The activation chunk is
// staged once per workgroup in LDS (odd elements pre-scaled by 1/16, see
// nib8_dot) together with per-block sums of x, which fold the -8 nibble bias
// into one FMA per block.
//
// Split-k. Narrow matrices (1152 or 1536 outputs = 18-24 groups) cannot fill
// 256 CUs with one task per group, so k is split into `split` chunks of whole
// scale quads (the reference splits over quads for the same reason,
// llm_matvec.cl:436-438). Chunks write partials; the last chunk of a group to
// arrive (an arrival ticket, returned to zero afterwards) sums the partials
// in ascending chunk order, so the result does not depend on scheduling.
#include "xp_device.hpp"
#include "xp_launch.hpp"

namespace xp {

constexpr int kMvWaves   = 4;   // tasks (waves) per workgroup

struct MvMat {
    float*       out;
    const u32x4*  wq;
    const void*  sc;
    uint32_t     cols;
    uint32_t     grp0;   // first task-group index of this matrix
};

struct MvArgs {
    MvMat        m[kMvMaxMats];
    uint32_t     n_mats;
    const float* x;
    uint32_t     nblk;
    uint32_t     nquads;       // ceil(nblk / 4)
    uint32_t     split;
    uint32_t     qpc;          // quads per chunk
    uint32_t     groups;       // sum of cols/64 over matrices
    uint32_t     wg_per_chunk; // ceil(groups / kMvWaves)
    float*       partial;      // [split][groups * 64]
    uint32_t*    tickets;      // [groups], zero at rest
};

// Raw scale bits for one quad of blocks, held in registers across the load
// pipeline and decoded only when the quad is multiplied (decoding at load
// time would force a wait on the loads just issued).
template <int FMT>
struct QuadScales {
    u32x2 raw;      // F16 / BF16 quad planes: 4 x 16-bit scales
    float f[4];     // F32 plane
    __device__ __forceinline__ void load(const void* sc, uint32_t cols, uint32_t j, uint32_t b) {
        if constexpr (FMT == XP_SCALE_F32) {
            const float* p = reinterpret_cast<const float*>(sc) + size_t(b) * cols + j;
#pragma unroll
            for (int i = 0; i < 4; ++i) f[i] = __builtin_nontemporal_load(p + size_t(i) * cols);
        } else {
            raw = ld_stream2(reinterpret_cast<const u32x2*>(sc) + size_t(b >> 2) * cols + j);
        }
    }
    __device__ __forceinline__ float get(int i) const {
        if constexpr (FMT == XP_SCALE_F16_QUAD) {
            const uint32_t w = (i < 2) ? raw.x : raw.y;
            return f16_bits_to_f32((i & 1) ? (w >> 16) : w);
        } else if constexpr (FMT == XP_SCALE_BF16_QUAD) {
            const uint32_t w = (i < 2) ? raw.x : raw.y;
            return (i & 1) ? bf16hi(w) : bf16lo(w);
        } else {
            return f[i];
        }
    }
};

// One block: sum_t xs[t] * nibble_t over a 16-byte KM4 word group, with the
// -8 bias folded in via the block sum of x.
__device__ __forceinline__ float block_dot(const u32x4 w, const float* xb, float xsum) {
    float pa = 0.0f, pb = 0.0f;
    pa = nib8_dot(w.x, *reinterpret_cast<const float4*>(xb + 0),
                  *reinterpret_cast<const float4*>(xb + 4), pa);
    pb = nib8_dot(w.y, *reinterpret_cast<const float4*>(xb + 8),
                  *reinterpret_cast<const float4*>(xb + 12), pb);
    pa = nib8_dot(w.z, *reinterpret_cast<const float4*>(xb + 16),
                  *reinterpret_cast<const float4*>(xb + 20), pa);
    pb = nib8_dot(w.w, *reinterpret_cast<const float4*>(xb + 24),
                  *reinterpret_cast<const float4*>(xb + 28), pb);
    return (pa + pb) - 8.0f * xsum;
}

// SPLIT = false: one chunk covers all of k (the wide lm_head shape); no
// partials, no ticket. A separate instantiation so profiles name it apart.
template <int FMT, bool SPLIT>
__global__ __launch_bounds__(kMvWaves * kWave) void mv_int4_kernel(MvArgs a) {
    extern __shared__ float smem[];
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t s    = blockIdx.x / a.wg_per_chunk;
    const uint32_t gg   = (blockIdx.x % a.wg_per_chunk) * kMvWaves + wave;
    const uint32_t q0   = s * a.qpc;
    const uint32_t q1   = min(q0 + a.qpc, a.nquads);
    const uint32_t b0   = q0 * 4;
    const uint32_t b1   = min(q1 * 4, a.nblk);
    const uint32_t nkc  = (b1 - b0) * kBlk;

    float* xs   = smem;                    // [qpc*128] activations (odd /16)
    float* bsum = smem + a.qpc * 128;      // [qpc*4] per-block sum of x

    const float* xg = a.x + size_t(b0) * kBlk;
    for (uint32_t i = threadIdx.x; i < nkc; i += blockDim.x) {
        const float v = xg[i];
        xs[i] = (i & 1u) ? v * 0.0625f : v;
    }
    for (uint32_t bb = threadIdx.x; bb < b1 - b0; bb += blockDim.x) {
        float t = 0.0f;
        for (uint32_t k = 0; k < kBlk; ++k) t += xg[bb * kBlk + k];
        bsum[bb] = t;
    }
    __syncthreads();
    if (gg >= a.groups) return;

    float*       out = nullptr;
    const u32x4* wq  = nullptr;
    const void*  sc  = nullptr;
    uint32_t cols = 0, gl = 0;
#pragma unroll
    for (int i = 0; i < kMvMaxMats; ++i) {
        if (uint32_t(i) < a.n_mats && gg >= a.m[i].grp0) {
            out = a.m[i].out; wq = a.m[i].wq; sc = a.m[i].sc;
            cols = a.m[i].cols; gl = gg - a.m[i].grp0;
        }
    }
    const uint32_t j  = gl * kGrp + lane;
    const u32x4*   wp = wq + size_t(gl) * a.nblk * kGrp + lane;

    float acc = 0.0f;
    const uint32_t nfull = (b1 - b0) / 4;
    if (nfull > 0) {
        // Two-stage pipeline over whole quads: quad n+1's four 16-byte loads
        // and its scales are in flight while quad n is multiplied. The last
        // prefetch re-reads the final quad instead of branching.
        u32x4 w[4];
        QuadScales<FMT> qs;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = ld_stream4(wp + size_t(b0 + i) * kGrp);
        qs.load(sc, cols, j, b0);
        for (uint32_t qi = 0; qi < nfull; ++qi) {
            const uint32_t b  = b0 + 4 * qi;
            const uint32_t bn = (qi + 1 < nfull) ? b + 4 : b;
            u32x4 wn[4];
            QuadScales<FMT> qn;
#pragma unroll
            for (int i = 0; i < 4; ++i) wn[i] = ld_stream4(wp + size_t(bn + i) * kGrp);
            qn.load(sc, cols, j, bn);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lb = b - b0 + i;
                acc = fmaf(qs.get(i), block_dot(w[i], xs + lb * kBlk, bsum[lb]), acc);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = wn[i];
            qs = qn;
        }
    }
    if constexpr (FMT == XP_SCALE_F32) {
        // Blocks past the last whole quad (nblk % 4 != 0, fp32 plane only).
        for (uint32_t b = b0 + 4 * nfull; b < b1; ++b) {
            const uint32_t lb = b - b0;
            const u32x4 wb = ld_stream4(wp + size_t(b) * kGrp);
            const float sb = reinterpret_cast<const float*>(sc)[size_t(b) * cols + j];
            acc = fmaf(sb, block_dot(wb, xs + lb * kBlk, bsum[lb]), acc);
        }
    }

    if constexpr (!SPLIT) {
        out[j] = acc;
        return;
    }
    const size_t stride = size_t(a.groups) * kGrp;
    st_dev(a.partial + size_t(s) * stride + size_t(gg) * kGrp + lane, acc);
    wait_mem();
    uint32_t old = 0;
    if (lane == 0) old = take_ticket(&a.tickets[gg]);
    old = __shfl(old, 0, kWave);
    if (old != a.split - 1) return;
    // Batches of 8 independent loads, summed in ascending chunk order.
    const float* pp = a.partial + size_t(gg) * kGrp + lane;
    float sum = 0.0f;
    uint32_t p = 0;
    for (; p + 8 <= a.split; p += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = ld_dev(pp + size_t(p + i) * stride);
#pragma unroll
        for (int i = 0; i < 8; ++i) sum += v[i];
    }
    for (; p < a.split; ++p) sum += ld_dev(pp + size_t(p) * stride);
    out[j] = sum;
    if (lane == 0) st_dev(&a.tickets[gg], 0u);
}

__global__ void unpack_km4_kernel(int8_t* out, const u32x4* wq, uint32_t rows, uint32_t cols) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;   // column
    const uint32_t b = blockIdx.y;                              // block
    const uint32_t nblk = rows / kBlk;
    if (j >= cols) return;
    const u32x4 w = wq[(size_t(j / kGrp) * nblk + b) * kGrp + (j % kGrp)];
    const uint32_t c4[4] = {w.x, w.y, w.z, w.w};
    for (uint32_t t = 0; t < kBlk; ++t) {
        const uint32_t k = b * kBlk + t;
        const uint32_t nib = (c4[(t >> 3) & 3u] >> ((t & 7u) * 4u)) & 15u;
        out[size_t(k) * cols + j] = static_cast<int8_t>(int(nib) - 8);
    }
}

__global__ void fp16_decode_kernel(float* out, const uint16_t* src, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f16_bits_to_f32(src[i]);
}

namespace {

// Enough tasks to give every CU several waves, but at most 16 chunks: the
// last chunk of a group to finish reads every partial, in batches of 8
// loads at device-coherence latency, so its tail grows with the split.
uint32_t choose_split(uint32_t groups, uint32_t nquads, int n_cu) {
    const uint32_t target = uint32_t(n_cu > 0 ? n_cu : 256) * 8u;   // ~8 tasks per CU
    uint32_t split = (target + groups - 1) / groups;
    if (split > 16) split = 16;
    if (split < 1) split = 1;
    if (split > nquads) split = nquads;
    return split;
}

// Final (split, quads per chunk) for a shape: chunks are whole quads and
// empty trailing chunks are dropped.
void split_plan(uint32_t groups, uint32_t nquads, uint32_t split, int n_cu, uint32_t& out_split,
                uint32_t& qpc) {
    if (split == 0) split = choose_split(groups, nquads, n_cu);
    if (split > nquads) split = nquads;
    if (split < 1) split = 1;
    qpc = (nquads + split - 1) / split;
    out_split = (nquads + qpc - 1) / qpc;
}

}  // namespace

size_t mv_partial_floats(uint32_t rows, uint32_t total_cols, uint32_t split, int n_cu) {
    const uint32_t nquads = (rows / kBlk + 3) / 4, groups = total_cols / kGrp;
    uint32_t sp, qpc;
    split_plan(groups, nquads, split, n_cu, sp, qpc);
    return sp > 1 ? size_t(sp) * groups * kGrp : 0;
}

int launch_mv(const MvMatDesc* mats, uint32_t n, const float* x, int fmt, uint32_t rows,
              uint32_t split, float* partial, size_t partial_cap, uint32_t* tickets,
              size_t tickets_cap, hipStream_t st, const char* who) {
    if (!x) return set_error(XP_E_ARG, "%s: in is null", who);
    if (n < 1 || n > uint32_t(kMvMaxMats))
        return set_error(XP_E_ARG, "%s: %u matrices (1..%d)", who, n, kMvMaxMats);
    if (rows == 0 || rows % kBlk != 0)
        return set_error(XP_E_ARG, "%s: rows=%u must be a positive multiple of 32", who, rows);
    if (fmt != XP_SCALE_F16_QUAD && fmt != XP_SCALE_BF16_QUAD && fmt != XP_SCALE_F32)
        return set_error(XP_E_ARG, "%s: unknown scale_fmt %d", who, fmt);
    const uint32_t nblk = rows / kBlk;
    if (fmt != XP_SCALE_F32 && nblk % 4 != 0)
        return set_error(XP_E_ARG,
                         "%s: quad scale planes need rows %% 128 == 0 (rows=%u)", who, rows);
    MvArgs a{};
    uint32_t groups = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (!mats[i].out || !mats[i].wq || !mats[i].sc)
            return set_error(XP_E_ARG, "%s: matrix %u has a null pointer", who, i);
        if (mats[i].cols == 0 || mats[i].cols % kGrp != 0)
            return set_error(XP_E_ARG, "%s: cols=%u must be a positive multiple of 64", who,
                             mats[i].cols);
        if (mats[i].out == x)
            return set_error(XP_E_ARG, "%s: out aliases in", who);
        a.m[i] = MvMat{mats[i].out, reinterpret_cast<const u32x4*>(mats[i].wq), mats[i].sc,
                       mats[i].cols, groups};
        groups += mats[i].cols / kGrp;
    }
    int n_cu = 256;
    DeviceScratch* sc = nullptr;
    if (!partial || !tickets) {
        sc = scratch();
        if (!sc) return XP_E_HIP;
        n_cu = sc->n_cu;
    }
    a.n_mats = n;
    a.x = x;
    a.nblk = nblk;
    a.nquads = (nblk + 3) / 4;
    split_plan(groups, a.nquads, split, n_cu, a.split, a.qpc);
    a.groups = groups;
    a.wg_per_chunk = (groups + kMvWaves - 1) / kMvWaves;
    if (a.split > 1) {
        const size_t need = size_t(a.split) * groups * kGrp;
        if (sc) {
            if (!ensure_partial(sc, need)) return XP_E_NOMEM;
            if (!ensure_tickets(sc, groups)) return XP_E_NOMEM;
            a.partial = sc->partial;
            a.tickets = sc->tickets;
        } else {
            if (partial_cap < need || tickets_cap < groups)
                return set_error(XP_E_ARG, "%s: scratch too small (%zu < %zu floats or %zu < %u "
                                 "tickets)", who, partial_cap, need, tickets_cap, groups);
            a.partial = partial;
            a.tickets = tickets;
        }
    }
    const size_t lds = (size_t(a.qpc) * 128 + size_t(a.qpc) * 4) * sizeof(float);
    if (lds > 64 * 1024)
        return set_error(XP_E_ARG, "%s: k-chunk of %u quads needs %zu B of LDS (> 64 KiB); "
                         "pass a larger split", who, a.qpc, lds);
    const dim3 grid(a.wg_per_chunk * a.split), block(kMvWaves * kWave);
#define XP_MV_LAUNCH(F)                                                                    \
    if (a.split > 1)                                                                       \
        hipLaunchKernelGGL((mv_int4_kernel<F, true>), grid, block, lds, st, a);            \
    else                                                                                   \
        hipLaunchKernelGGL((mv_int4_kernel<F, false>), grid, block, lds, st, a);
    switch (fmt) {
        case XP_SCALE_F16_QUAD: XP_MV_LAUNCH(XP_SCALE_F16_QUAD) break;
        case XP_SCALE_BF16_QUAD: XP_MV_LAUNCH(XP_SCALE_BF16_QUAD) break;
        default: XP_MV_LAUNCH(XP_SCALE_F32) break;
    }
#undef XP_MV_LAUNCH
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "%s: launch -> %s", who, hipGetErrorString(e));
    return XP_OK;
}

}  // namespace xp

using namespace xp;

extern "C" {

int xp_mv_int4(float* out, const float* in, const void* wq, const void* scales, int scale_fmt,
               uint32_t rows, uint32_t cols, uint32_t split, xp_stream stream) {
    MvMatDesc m{out, wq, scales, cols};
    return launch_mv(&m, 1, in, scale_fmt, rows, split, nullptr, 0, nullptr, 0,
                     as_stream(stream), "xp_mv_int4");
}

int xp_mv_int4_multi(uint32_t n, float* const* outs, const float* in, const void* const* wqs,
                     const void* const* scales, const uint32_t* cols, int scale_fmt,
                     uint32_t rows, xp_stream stream) {
    XP_REQUIRE(n >= 1 && n <= uint32_t(kMvMaxMats), "n=%u must be in [1, %d]", n, kMvMaxMats);
    XP_REQUIRE(outs && wqs && scales && cols, "null array argument");
    MvMatDesc m[kMvMaxMats];
    for (uint32_t i = 0; i < n; ++i) m[i] = MvMatDesc{outs[i], wqs[i], scales[i], cols[i]};
    return launch_mv(m, n, in, scale_fmt, rows, 0, nullptr, 0, nullptr, 0, as_stream(stream),
                     "xp_mv_int4_multi");
}

int xp_mv_int4_timed(float* out, const float* in, const void* const* wqs,
                     const void* const* scales, uint32_t ncopies, int scale_fmt, uint32_t rows,
                     uint32_t cols, uint32_t split, uint32_t iters, xp_stream stream, float* ms) {
    XP_REQUIRE(wqs && scales && ms && ncopies > 0 && iters > 0, "bad arguments");
    hipStream_t st = as_stream(stream);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    XP_HIP(hipEventCreate(&e0));
    XP_HIP(hipEventCreate(&e1));
    int rc = XP_OK;
    // One untimed pass over every copy so scratch is sized before timing.
    for (uint32_t i = 0; i < ncopies && rc == XP_OK; ++i)
        rc = xp_mv_int4(out, in, wqs[i], scales[i], scale_fmt, rows, cols, split, stream);
    if (rc == XP_OK && hipStreamSynchronize(st) != hipSuccess) rc = set_error(XP_E_HIP, "sync");
    if (rc == XP_OK && hipEventRecord(e0, st) != hipSuccess) rc = set_error(XP_E_HIP, "event");
    for (uint32_t i = 0; i < iters && rc == XP_OK; ++i)
        rc = xp_mv_int4(out, in, wqs[i % ncopies], scales[i % ncopies], scale_fmt, rows, cols,
                        split, stream);
    if (rc == XP_OK && hipEventRecord(e1, st) != hipSuccess) rc = set_error(XP_E_HIP, "event");
    if (rc == XP_OK && hipEventSynchronize(e1) != hipSuccess) rc = set_error(XP_E_HIP, "sync");
    if (rc == XP_OK && hipEventElapsedTime(ms, e0, e1) != hipSuccess)
        rc = set_error(XP_E_HIP, "elapsed");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

int xp_unpack_km4(int8_t* out, const void* wq, uint32_t rows, uint32_t cols, xp_stream stream) {
    XP_REQUIRE(out && wq, "null pointer");
    XP_REQUIRE(rows > 0 && rows % kBlk == 0, "rows=%u must be a positive multiple of 32", rows);
    XP_REQUIRE(cols > 0 && cols % kGrp == 0, "cols=%u must be a positive multiple of 64", cols);
    const dim3 grid((cols + 255) / 256, rows / kBlk);
    hipLaunchKernelGGL(unpack_km4_kernel, grid, dim3(256), 0, as_stream(stream), out,
                       reinterpret_cast<const u32x4*>(wq), rows, cols);
    XP_LAUNCHED();
    return XP_OK;
}

int xp_fp16_decode(float* out, const uint16_t* src, uint32_t n, xp_stream stream) {
    XP_REQUIRE(out && src, "null pointer");
    if (n == 0) return XP_OK;
    hipLaunchKernelGGL(fp16_decode_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       as_stream(stream), out, src, n);
    XP_LAUNCHED();
    return XP_OK;
}

}  // extern "C"
