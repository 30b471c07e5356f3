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
// staged once per workgroup in LDS as 20-bit block fixed point (see
// block_dot), which turns the unpack-and-multiply into integer dot products.
//
// Split-k. Narrow matrices (1152 or 1536 outputs = 18-24 groups) cannot fill
// 256 CUs with one task per group, so k is split into `split` chunks of whole
// scale quads (the reference splits over quads for the same reason,
// llm_matvec.cl:436-438). Chunks write partials; the last chunk of a group to
// arrive (an arrival ticket, returned to zero afterwards) sums the partials
// in ascending chunk order, so the result does not depend on scheduling.
#include "xp_device.hpp"
#include "xp_launch.hpp"

#include <mutex>
#include <vector>

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
    // the column-slice kernel's input operation (MvIn; the mode is a
    // template argument of the kernel)
    const float* in_u;         // GeGLU: up; norm: y
    const float* in_wpost;
    const float* in_wpre;
    float*       in_xout;
    float        in_eps;
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

// One wave = one task = (column group, k-chunk). SPLIT = false: the chunk is
// all of k (the wide lm_head shape); no partials, no ticket. A separate
// instantiation so that profiles name the two apart. At most 128 VGPRs, so
// four tasks share each SIMD (the lm_head's 4096 tasks then run in one round
// on 256 CUs).
template <int FMT, bool SPLIT>
__global__ __launch_bounds__(kMvWaves * kWave) __attribute__((amdgpu_waves_per_eu(4)))
void mv_int4_kernel(MvArgs a) {
    extern __shared__ QxBlock smem_qx[];
    // The wave index is uniform across a wave; saying so keeps the task's
    // bookkeeping in scalar registers.
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t s    = blockIdx.x / a.wg_per_chunk;
    const uint32_t gg   = (blockIdx.x % a.wg_per_chunk) * kMvWaves + wave;
    const uint32_t q0   = s * a.qpc;
    const uint32_t q1   = min(q0 + a.qpc, a.nquads);
    const uint32_t b0   = q0 * 4;
    const uint32_t b1   = min(q1 * 4, a.nblk);
    const uint32_t nbc  = b1 - b0;
    QxBlock* qx = smem_qx;
    float*   sx = reinterpret_cast<float*>(smem_qx + a.qpc * 4);
    const float* xg = a.x + size_t(b0) * kBlk;

    // Staging tasks beyond the first blockDim.x (chunks over 64 blocks) go
    // first; the first batch's activations are loaded next, ahead of the
    // weight prefetch, so that waiting for them does not wait for weights.
    for (uint32_t i = threadIdx.x + blockDim.x; i < nbc * 4; i += blockDim.x)
        stage_x8(qx, sx, i, reinterpret_cast<const float4*>(xg)[2 * i],
                 reinterpret_cast<const float4*>(xg)[2 * i + 1]);
    float4 xv0 = {0.0f, 0.0f, 0.0f, 0.0f}, xv1 = xv0;
    if (threadIdx.x < nbc * 4) {
        xv0 = reinterpret_cast<const float4*>(xg)[2 * threadIdx.x];
        xv1 = reinterpret_cast<const float4*>(xg)[2 * threadIdx.x + 1];
    }

    // Waves past the last group (only in a chunk's last workgroup) prefetch
    // group 0 of matrix 0 like any other wave and drop the result, so every
    // wave issues the same loads and the wait counts stay exact.
    const bool active = gg < a.groups;
    uint32_t mi = 0;
#pragma unroll
    for (int i = 1; i < kMvMaxMats; ++i)
        if (uint32_t(i) < a.n_mats && gg >= a.m[i].grp0) mi = uint32_t(i);
    if (!active) mi = 0;
    float*       out = a.m[0].out;
    const u32x4* wq  = a.m[0].wq;
    const void*  sc  = a.m[0].sc;
    uint32_t cols = a.m[0].cols;
#pragma unroll
    for (int i = 1; i < kMvMaxMats; ++i) {
        if (uint32_t(i) == mi) {
            out = a.m[i].out; wq = a.m[i].wq; sc = a.m[i].sc; cols = a.m[i].cols;
        }
    }
    uint32_t grp0 = 0;
#pragma unroll
    for (int i = 1; i < kMvMaxMats; ++i)
        if (uint32_t(i) == mi) grp0 = a.m[i].grp0;
    const uint32_t gl = active ? gg - grp0 : 0u;
    const uint32_t j  = gl * kGrp + lane;
    const u32x4*   wp = wq + size_t(gl) * a.nblk * kGrp + lane;
    const uint32_t nq = nbc / 4;   // whole quads in the chunk

    // Three quads in flight: while quad n is multiplied, quads n+1 and n+2
    // (16 x 16-byte weight loads + their scales) are outstanding. Block
    // indices are clamped into the chunk, so a prefetch past its end (chunks
    // of fewer than three quads) re-reads the chunk's last block.
    u32x4 w[3][4];
    QuadScales<FMT> qs[3];
    const uint32_t blast = b1 - 1;
    auto load_quad = [&](int r, uint32_t q) {
        const uint32_t b = b0 + 4 * q;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[r][i] = ld_stream4(wp + size_t(min(b + i, blast)) * kGrp);
        qs[r].load(sc, cols, j, min(b, blast & ~3u));
    };
    auto mul_quad = [&](int r, uint32_t q, float& acc) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lb = 4 * q + i;
            const float f = qs[r].get(i) * sx[lb];
            acc = fmaf(f, float(block_dot(w[r][i], qx[lb])), acc);
        }
    };
    load_quad(0, 0);
    load_quad(1, 1);
    load_quad(2, 2);

    if (threadIdx.x < nbc * 4) stage_x8(qx, sx, threadIdx.x, xv0, xv1);
    __syncthreads();
    if (!active) return;

    float acc = 0.0f;
    uint32_t q = 0;
    // Steady state: every reload is in range. The scheduling barriers keep
    // each reload right after the multiply that frees its registers (left
    // alone, the scheduler sinks all three reloads to the end of the body).
    for (; q + 6 <= nq; q += 3) {
        mul_quad(0, q, acc);
        __builtin_amdgcn_sched_barrier(0);
        load_quad(0, q + 3);
        __builtin_amdgcn_sched_barrier(0);
        mul_quad(1, q + 1, acc);
        __builtin_amdgcn_sched_barrier(0);
        load_quad(1, q + 4);
        __builtin_amdgcn_sched_barrier(0);
        mul_quad(2, q + 2, acc);
        __builtin_amdgcn_sched_barrier(0);
        load_quad(2, q + 5);
        __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t rem = nq - q;    // 0..5 quads left; buffers hold q..q+2
    if (rem > 0) {
        mul_quad(0, q, acc);
        if (rem > 3) load_quad(0, q + 3);
    }
    if (rem > 1) {
        mul_quad(1, q + 1, acc);
        if (rem > 4) load_quad(1, q + 4);
    }
    if (rem > 2) mul_quad(2, q + 2, acc);
    if (rem > 3) mul_quad(0, q + 3, acc);
    if (rem > 4) mul_quad(1, q + 4, acc);
    if constexpr (FMT == XP_SCALE_F32) {
        // Blocks past the last whole quad (nblk % 4 != 0, fp32 plane only).
        for (uint32_t lb = 4 * nq; lb < nbc; ++lb) {
            const u32x4 wb = ld_stream4(wp + size_t(b0 + lb) * kGrp);
            const float sb = reinterpret_cast<const float*>(sc)[size_t(b0 + lb) * cols + j];
            acc = fmaf(sb * sx[lb], float(block_dot(wb, qx[lb])), acc);
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

// Workgroup tasks: one workgroup per (column group, k-chunk of at most 16
// quads), its eight waves splitting the chunk (wave w takes quads w and
// w + 8) and meeting in LDS, summed in wave order. Wide, shallow shapes
// (config 1: 108 column groups over 9 quads of k) take one chunk: no partial
// buffer, no ticket, one HBM round trip. Narrow, deep ones take at most eight
// chunks (SPLIT): partials, an arrival ticket and one batch of partial loads
// by the last chunk, summed in ascending chunk order. The activations are
// loaded ahead of the weights, so staging them overlaps the weight fetch.
// Quad scale planes only.
constexpr int kMvWgWaves = 8;
constexpr int kMvWgQuads = 2;                                 // quads per wave
constexpr uint32_t kMvWgChunk = kMvWgWaves * kMvWgQuads;      // quads per chunk
constexpr uint32_t kMvWgMaxSplit = 8;

template <int FMT, bool SPLIT>
__global__ __launch_bounds__(kMvWgWaves * kWave) void mv_int4_wg_kernel(MvArgs a) {
    extern __shared__ QxBlock smem_qx[];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t gg = blockIdx.x % a.groups, s = blockIdx.x / a.groups;
    const uint32_t q0 = s * a.qpc, nqc = min(a.qpc, a.nquads - q0), nbc = 4u * nqc;
    QxBlock* qx = smem_qx;
    float* sx = reinterpret_cast<float*>(smem_qx + 4u * a.qpc);
    float* red = sx + 4u * a.qpc;   // [kMvWgWaves][64]
    uint32_t mi = 0;
#pragma unroll
    for (int i = 1; i < kMvMaxMats; ++i)
        if (uint32_t(i) < a.n_mats && gg >= a.m[i].grp0) mi = uint32_t(i);
    float*       out = a.m[0].out;
    const u32x4* wq  = a.m[0].wq;
    const void*  sc  = a.m[0].sc;
    uint32_t cols = a.m[0].cols, grp0 = 0;
#pragma unroll
    for (int i = 1; i < kMvMaxMats; ++i) {
        if (uint32_t(i) == mi) {
            out = a.m[i].out; wq = a.m[i].wq; sc = a.m[i].sc; cols = a.m[i].cols; grp0 = a.m[i].grp0;
        }
    }
    const uint32_t gl = gg - grp0, j = gl * kGrp + lane;
    const u32x4* wp = wq + size_t(gl) * a.nblk * kGrp + lane;
    // the chunk's activations (at most 64 blocks: one staging task per thread)
    const float4* x4 = reinterpret_cast<const float4*>(a.x + size_t(4u * q0) * kBlk);
    const bool stager = threadIdx.x < nbc * 4u;
    float4 xv0 = {0.0f, 0.0f, 0.0f, 0.0f}, xv1 = xv0;
    if (stager) {
        xv0 = x4[2 * threadIdx.x];
        xv1 = x4[2 * threadIdx.x + 1];
    }
    u32x4 w[kMvWgQuads][4];
    QuadScales<FMT> qs[kMvWgQuads];
#pragma unroll
    for (int r = 0; r < kMvWgQuads; ++r) {
        const uint32_t b = 4u * (q0 + min(wave + uint32_t(kMvWgWaves) * r, nqc - 1u));
#pragma unroll
        for (int i = 0; i < 4; ++i) w[r][i] = ld_stream4(wp + size_t(b + i) * kGrp);
        qs[r].load(sc, cols, j, b);
    }
    if (stager) stage_x8(qx, sx, threadIdx.x, xv0, xv1);
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < kMvWgQuads; ++r) {
        const uint32_t lq = wave + uint32_t(kMvWgWaves) * r;
        if (lq < nqc) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lb = 4u * lq + i;
                acc = fmaf(qs[r].get(i) * sx[lb], float(block_dot(w[r][i], qx[lb])), acc);
            }
        }
    }
    red[wave * kGrp + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    float y = 0.0f;
#pragma unroll
    for (int v = 0; v < kMvWgWaves; ++v) y += red[v * kGrp + lane];
    if constexpr (!SPLIT) {
        out[j] = y;
        return;
    }
    const size_t stride = size_t(a.groups) * kGrp;
    st_dev(a.partial + size_t(s) * stride + size_t(gg) * kGrp + lane, y);
    wait_mem();
    uint32_t old = 0;
    if (lane == 0) old = take_ticket(&a.tickets[gg]);
    old = __shfl(old, 0, kWave);
    if (old != a.split - 1) return;
    // every partial in one batch (split <= 8), summed in ascending chunk order
    const float* pp = a.partial + size_t(gg) * kGrp + lane;
    float v[kMvWgMaxSplit];
#pragma unroll
    for (uint32_t p = 0; p < kMvWgMaxSplit; ++p) v[p] = p < a.split ? ld_dev(pp + size_t(p) * stride) : 0.0f;
    float sum = 0.0f;
#pragma unroll
    for (uint32_t p = 0; p < kMvWgMaxSplit; ++p)
        if (p < a.split) sum += v[p];
    out[j] = sum;
    if (lane == 0) st_dev(&a.tickets[gg], 0u);
}

// Column-slice workgroups: workgroup (column group g, slice h of S)
// computes the 64 / S columns 64 g + h 64 / S ... of all of k. Lane l of a
// wave takes column l % (64 / S) of the slice and block slot l / (64 / S) of
// each S-block step, so one wave load is S contiguous runs of 1024 / S
// bytes, and the grid holds S times as many workgroups as column groups
// (config 1: 108 groups, 216 workgroups at S = 2). Every workgroup stages
// all of x (at most 256 blocks, two staging tasks per thread); the eight
// waves take steps w, w + 8, ... (at most kMvSliceRounds each); their sums
// meet in LDS and are added in wave, then slot order (deterministic). No
// partials, no ticket: one HBM round trip, where a k-chunk plan's last
// arrival adds a ticket and a partial-sum round trip (measured on MI355X:
// q 1152 x 1024 2.9 us per launch against 5.7). Quad scale planes only.
constexpr uint32_t kMvSliceRounds = 8;
constexpr uint32_t kMvSliceMaxBlk = 256;

// GO (GeGLU output; S = 2, two matrices of equal width, gate then up): lane
// l takes column c of the gate (l < 32) or of the up matrix, both halves the
// same block each step (one block a step), and the workgroup writes
// gelu(gate) * up for its 32 columns into the first matrix's output.
template <int FMT, int S, int R, int XM = kMvInPlain, bool GO = false>
__global__ __launch_bounds__(kMvWgWaves * kWave) void mv_int4_slice_kernel(MvArgs a) {
    constexpr uint32_t CPS = kGrp / S;                                 // columns per slice
    static_assert(R >= 1 && R <= int(kMvSliceRounds), "steps per wave");
    static_assert(!GO || S == 2, "the GeGLU output pairs two 32-column halves");
    extern __shared__ QxBlock smem_qx[];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t gg = blockIdx.x / S, h = blockIdx.x % S;
    const uint32_t nblk = a.nblk, nsteps = GO ? nblk : (nblk + S - 1) / S;
    QxBlock* qx = smem_qx;
    float* sx = reinterpret_cast<float*>(smem_qx + nblk);
    float* red = sx + nblk;   // [kMvWgWaves][64]
    float* xs2 = red + kMvWgWaves * kGrp;   // [kMvWgWaves]: norm mode, the waves' sums of x_new^2
    uint32_t mi = 0;
#pragma unroll
    for (int i = 1; i < kMvMaxMats; ++i)
        if (uint32_t(i) < a.n_mats && gg >= a.m[i].grp0) mi = uint32_t(i);
    float*       out = a.m[0].out;
    const u32x4* wq  = a.m[0].wq;
    const void*  sc  = a.m[0].sc;
    uint32_t cols = a.m[0].cols, grp0 = 0;
#pragma unroll
    for (int i = 1; i < kMvMaxMats; ++i) {
        if (uint32_t(i) == mi) {
            out = a.m[i].out; wq = a.m[i].wq; sc = a.m[i].sc; cols = a.m[i].cols; grp0 = a.m[i].grp0;
        }
    }
    if constexpr (GO) {
        wq = lane < CPS ? a.m[0].wq : a.m[1].wq;
        sc = lane < CPS ? a.m[0].sc : a.m[1].sc;
    }
    const uint32_t gl = gg - grp0, c = h * CPS + lane % CPS, bs = GO ? 0u : lane / CPS;
    const uint32_t j = gl * kGrp + c;
    const u32x4* wp = wq + size_t(gl) * nblk * kGrp + c;
    // the block of step t for this lane (S blocks a step, or one with GO)
    auto blk_of = [&](uint32_t t) { return GO ? t : t * S + bs; };
    // all of x, staging tasks (8 elements each) i and i + 512 of thread i
    // (the second only past 128 blocks), loaded ahead of the weights
    constexpr uint32_t NT = kMvWgWaves * kWave;
    constexpr uint32_t NX = uint32_t(R) * kMvWgWaves * S > 128u ? 2u : 1u;
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    const uint32_t ntask = nblk * 4u;
    float4 xv[NX][2];
    [[maybe_unused]] float4 uv[NX][2], pv[NX][2], qv[NX][2];   // up or y; w_post; w_pre
    if constexpr (XM == kMvInPlain) {
#pragma unroll
        for (uint32_t k = 0; k < NX; ++k) {
            const uint32_t i = threadIdx.x + k * NT;
            xv[k][0] = xv[k][1] = float4{0.0f, 0.0f, 0.0f, 0.0f};
            if (i < ntask) {
                xv[k][0] = x4[2 * i];
                xv[k][1] = x4[2 * i + 1];
            }
        }
    } else {
        // every thread loads (past the last task, the last task again), so
        // that no use of these values is placed in a load's branch
        const float4* u4 = reinterpret_cast<const float4*>(a.in_u);
        const float4* p4 = reinterpret_cast<const float4*>(a.in_wpost);
        const float4* q4 = reinterpret_cast<const float4*>(a.in_wpre);
#pragma unroll
        for (uint32_t k = 0; k < NX; ++k) {
            const uint32_t i = min(threadIdx.x + k * NT, ntask - 1u);
            xv[k][0] = x4[2 * i];
            xv[k][1] = x4[2 * i + 1];
            uv[k][0] = u4[2 * i];
            uv[k][1] = u4[2 * i + 1];
            if constexpr (XM == kMvInNorm) {
                pv[k][0] = p4[2 * i];
                pv[k][1] = p4[2 * i + 1];
                qv[k][0] = q4[2 * i];
                qv[k][1] = q4[2 * i + 1];
            }
        }
    }
    // step t = wave + 8 r covers blocks S t .. S t + S - 1; this lane's block
    // is S t + bs, clamped (and weighted by zero) past the end
    u32x4 w[R];
    uint32_t sw[R];
    const uint32_t* sc32 = static_cast<const uint32_t*>(sc);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        // steps past the end load a valid block (clamped) and weigh it by zero
        const uint32_t t = min(wave + uint32_t(kMvWgWaves) * r, nsteps - 1u);
        const uint32_t b = min(blk_of(t), nblk - 1u);
        w[r] = ld_stream4(wp + size_t(b) * kGrp);
        // the 32-bit word holding scale b % 4 of quad b / 4 of column j
        sw[r] = __builtin_nontemporal_load(sc32 + (size_t(b >> 2) * cols + j) * 2u +
                                           ((b >> 1) & 1u));
    }
    [[maybe_unused]] float s2 = 0.0f;   // norm mode: this thread's sum of x_new^2
    if constexpr (XM == kMvInPlain) {
#pragma unroll
        for (uint32_t k = 0; k < NX; ++k) {
            const uint32_t i = threadIdx.x + k * NT;
            if (i < ntask) stage_x8(qx, sx, i, xv[k][0], xv[k][1]);
        }
    } else if constexpr (XM == kMvInGeglu) {
#pragma unroll
        for (uint32_t k = 0; k < NX; ++k) {
            const uint32_t i = threadIdx.x + k * NT;
            const float4 h0{gelu_hw(xv[k][0].x) * uv[k][0].x, gelu_hw(xv[k][0].y) * uv[k][0].y,
                            gelu_hw(xv[k][0].z) * uv[k][0].z, gelu_hw(xv[k][0].w) * uv[k][0].w};
            const float4 h1{gelu_hw(xv[k][1].x) * uv[k][1].x, gelu_hw(xv[k][1].y) * uv[k][1].y,
                            gelu_hw(xv[k][1].z) * uv[k][1].z, gelu_hw(xv[k][1].w) * uv[k][1].w};
            if (i < ntask) stage_x8(qx, sx, i, h0, h1);
        }
    } else {
        // x_new = x + y rsqrt(mean y^2 + eps) (1 + w_post): the sum of y^2
        // over the whole vector (every workgroup stages all of it)
        float ss = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < NX; ++k) {
            const float live = threadIdx.x + k * NT < ntask ? 1.0f : 0.0f;
            const float yy[8] = {uv[k][0].x, uv[k][0].y, uv[k][0].z, uv[k][0].w,
                                 uv[k][1].x, uv[k][1].y, uv[k][1].z, uv[k][1].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(yy[e] * live, yy[e], ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (uint32_t v = 0; v < uint32_t(kMvWgWaves); ++v) tot += red[v];
        const float post = rsq_hw(tot / float(nblk * kBlk) + a.in_eps);
#pragma unroll
        for (uint32_t k = 0; k < NX; ++k) {
            const uint32_t i = threadIdx.x + k * NT;
            const bool live = i < ntask;
            const float xx[8] = {xv[k][0].x, xv[k][0].y, xv[k][0].z, xv[k][0].w,
                                 xv[k][1].x, xv[k][1].y, xv[k][1].z, xv[k][1].w};
            const float yy[8] = {uv[k][0].x, uv[k][0].y, uv[k][0].z, uv[k][0].w,
                                 uv[k][1].x, uv[k][1].y, uv[k][1].z, uv[k][1].w};
            const float wp[8] = {pv[k][0].x, pv[k][0].y, pv[k][0].z, pv[k][0].w,
                                 pv[k][1].x, pv[k][1].y, pv[k][1].z, pv[k][1].w};
            const float wq8[8] = {qv[k][0].x, qv[k][0].y, qv[k][0].z, qv[k][0].w,
                                  qv[k][1].x, qv[k][1].y, qv[k][1].z, qv[k][1].w};
            float xn[8], st[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                xn[e] = xx[e] + yy[e] * post * (1.0f + wp[e]);
                s2 = fmaf(live ? xn[e] : 0.0f, xn[e], s2);
                st[e] = xn[e] * (1.0f + wq8[e]);
            }
            if (live && blockIdx.x == 0) {
                float4* xo = reinterpret_cast<float4*>(a.in_xout) + 2 * i;
                xo[0] = float4{xn[0], xn[1], xn[2], xn[3]};
                xo[1] = float4{xn[4], xn[5], xn[6], xn[7]};
            }
            if (live)
                stage_x8(qx, sx, i, float4{st[0], st[1], st[2], st[3]}, float4{st[4], st[5], st[6], st[7]});
        }
    }
    // while the staging completes: the nibbles as two's complement and each
    // step's weight scale (zero past the end)
    float ws[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t t = wave + uint32_t(kMvWgWaves) * r, b = blk_of(t);
        const uint32_t bb = min(b, nblk - 1u);
        const uint32_t hb = (sw[r] >> (16u * (bb & 1u))) & 0xFFFFu;
        const float scale = FMT == XP_SCALE_F16_QUAD ? f16_bits_to_f32(hb) : __uint_as_float(hb << 16);
        ws[r] = t < nsteps && b < nblk ? scale : 0.0f;
        w[r] ^= 0x88888888u;
    }
    __syncthreads();
    // The dots read the staged words through the lanes of a 16-lane row
    // (block_dot_bc): every lane of a row takes the same block (slot bs is
    // whole rows), lane jw < 10 holding words 2 jw, 2 jw + 1 of it. All of a
    // wave's words and block scales are read before any is used.
    const uint32_t jr = lane % 16u, jw = jr >= 2u * kQxPlanes ? jr - 2u * kQxPlanes : jr;
    u32x2 aw[R];
    float sxv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t t = min(wave + uint32_t(kMvWgWaves) * r, nsteps - 1u);
        const uint32_t bb = min(blk_of(t), nblk - 1u);
        sxv[r] = sx[bb];
        aw[r] = reinterpret_cast<const u32x2*>(&qx[bb])[jw];
    }
    __builtin_amdgcn_sched_barrier(0);
    // a DPP operation must follow an exec write by five wait states, which
    // the compiler does not provide for inline assembly: one s_nop 4 before
    // the first, ordered after the loads by the tied operands
#pragma unroll
    for (int r = 0; r < R; ++r) asm volatile("s_nop 4" : "+v"(aw[r].x), "+v"(aw[r].y));
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r += 2) {
        // steps of the whole wave past the end are skipped (t is uniform)
        if (wave + uint32_t(kMvWgWaves) * uint32_t(r) >= nsteps) break;
        if (r + 1 < R) {
            const u32x4 w2[2] = {w[r], w[r + 1]};
            const u32x2 a2[2] = {aw[r], aw[r + 1]};
            int32_t d[2];
            block_dot_bc<2>(w2, a2, d);
            acc = fmaf(ws[r] * sxv[r], float(d[0]), acc);
            acc = fmaf(ws[r + 1] * sxv[r + 1], float(d[1]), acc);
        } else {
            const u32x4 w1[1] = {w[r]};
            const u32x2 a1[1] = {aw[r]};
            int32_t d[1];
            block_dot_bc<1>(w1, a1, d);
            acc = fmaf(ws[r] * sxv[r], float(d[0]), acc);
        }
    }
    red[wave * kGrp + lane] = acc;
    if constexpr (XM == kMvInNorm) {
        const float w2 = wave_sum(s2);
        if (lane == 0) xs2[wave] = w2;
    }
    __syncthreads();
    if (wave != 0 || lane >= CPS) return;
    // the input norm's scalar rsqrt(mean x_new^2 + eps), applied here
    float nsc = 1.0f;
    if constexpr (XM == kMvInNorm) {
        float t2 = 0.0f;
#pragma unroll
        for (uint32_t v = 0; v < uint32_t(kMvWgWaves); ++v) t2 += xs2[v];
        nsc = rsq_hw(t2 / float(nblk * kBlk) + a.in_eps);
    }
    if constexpr (GO) {
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (uint32_t v = 0; v < uint32_t(kMvWgWaves); ++v) {
            g += red[v * kGrp + lane];
            u += red[v * kGrp + CPS + lane];
        }
        if constexpr (XM == kMvInNorm) {
            g *= nsc;
            u *= nsc;
        }
        out[j] = gelu_hw(g) * u;
    } else {
        float y = 0.0f;
#pragma unroll
        for (uint32_t v = 0; v < uint32_t(kMvWgWaves); ++v)
#pragma unroll
            for (uint32_t q = 0; q < uint32_t(S); ++q) y += red[v * kGrp + q * CPS + lane];
        if constexpr (XM == kMvInNorm) y *= nsc;
        out[j] = y;
    }
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

namespace {
// Column slices per group for the column-slice plan (0: the plan does not
// apply): two per group for wide shapes (>= 64 groups; config 1: 216
// workgroups), four for narrow ones, as long as each workgroup can hold its
// column group's whole k (at most kMvSliceRounds steps per wave).
uint32_t slice_count(uint32_t nblk, uint32_t groups, int fmt, int n_cu) {
    if (fmt == XP_SCALE_F32 || groups >= uint32_t(n_cu) * 8u) return 0;
    uint32_t S = groups >= 64 ? 2u : 4u;
    while (S < 4u && (nblk + S - 1) / S > kMvWgWaves * kMvSliceRounds) S *= 2u;
    if (nblk <= kMvSliceMaxBlk && (nblk + S - 1) / S <= kMvWgWaves * kMvSliceRounds) return S;
    return 0;
}
}  // namespace

bool mv_slice_plan(uint32_t rows, uint32_t total_cols, int fmt, int n_cu) {
    if (rows == 0 || rows % (4u * kBlk) != 0 || total_cols % kGrp != 0) return false;
    return slice_count(rows / kBlk, total_cols / kGrp, fmt, n_cu > 0 ? n_cu : 256) != 0;
}

bool mv_geglu_plan(uint32_t rows, uint32_t cols, int fmt, int n_cu) {
    // two 32-column halves a group (the two-slice plan of one matrix's
    // groups), one block a step: at most kMvSliceRounds steps a wave
    if (rows == 0 || rows % (4u * kBlk) != 0 || cols % kGrp != 0) return false;
    const uint32_t nblk = rows / kBlk;
    return slice_count(nblk, cols / kGrp, fmt, n_cu > 0 ? n_cu : 256) == 2u &&
           nblk <= kMvWgWaves * kMvSliceRounds;
}

int launch_mv(const MvMatDesc* mats, uint32_t n, const float* x, int fmt, uint32_t rows,
              uint32_t split, float* partial, size_t partial_cap, uint32_t* tickets,
              size_t tickets_cap, hipStream_t st, const char* who, int n_cu_hint, const MvIn* in) {
    if (!x) return set_error(XP_E_ARG, "%s: in is null", who);
    const int xm = in ? in->mode : kMvInPlain;
    if (xm != kMvInPlain && xm != kMvInGeglu && xm != kMvInNorm)
        return set_error(XP_E_ARG, "%s: input operation %d", who, xm);
    if (xm != kMvInPlain) {
        // GeGLU reads `up`, the norm `y` (and both weights, writing x_out)
        const float* u = xm == kMvInGeglu ? in->up : in->y;
        auto bad = [](const void* p) { return !p || (reinterpret_cast<uintptr_t>(p) & 15u); };
        if (bad(u) || (xm == kMvInNorm && (bad(in->w_post) || bad(in->w_pre) || bad(in->x_out))))
            return set_error(XP_E_ARG, "%s: the input operation's vectors must be non-null and 16-byte aligned",
                             who);
        if (xm == kMvInNorm && (in->x_out == x || in->x_out == u || !(in->eps >= 0.0f)))
            return set_error(XP_E_ARG, "%s: the norm's x_out aliases its inputs (or eps < 0)", who);
        for (uint32_t i = 0; i < n && i < uint32_t(kMvMaxMats); ++i)
            if (mats[i].out == u || (xm == kMvInNorm && mats[i].out == in->x_out))
                return set_error(XP_E_ARG, "%s: an output aliases the input operation's vectors", who);
    }
    if (reinterpret_cast<uintptr_t>(x) & 15u)
        return set_error(XP_E_ARG, "%s: in must be 16-byte aligned", who);
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
    int n_cu = n_cu_hint > 0 ? n_cu_hint : 256;
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
    a.groups = groups;
    // Automatic plan for a shape narrower than eight waves per CU (quad scale
    // planes): workgroup tasks, one chunk per column group when the whole k
    // fits one (and the groups alone give most CUs a task), else as many
    // chunks as give every CU a task, at most eight, each within kMvWgChunk
    // quads. A caller-provided partial buffer too small for that plan keeps
    // the split-k plan it was sized for.
    const bool go = in && in->geglu_out;
    if (go && (xm == kMvInGeglu || n != 2 || mats[0].cols != mats[1].cols || split != 0 ||
               !mv_geglu_plan(rows, mats[0].cols, fmt, n_cu)))
        return set_error(XP_E_ARG, "%s: the GeGLU output takes a gate and an up matrix of equal width "
                                   "within the column-slice plan", who);
    if (go && in->x_out && in->x_out == mats[0].out)
        return set_error(XP_E_ARG, "%s: the GeGLU output aliases the norm's x_out", who);
    if (xm != kMvInPlain && (split != 0 || slice_count(nblk, groups, fmt, n_cu) == 0))
        return set_error(XP_E_ARG, "%s: an input operation needs the column-slice plan", who);
    if (split == 0 && fmt != XP_SCALE_F32 && groups < uint32_t(n_cu) * 8u) {
        // Column slices (slice_count). Measured per launch on MI355X (back to
        // back, 2.8 us launch floor): config 1 3.3 us (one workgroup per
        // group: 3.9), q 2.9 us, o 2.9 us (k-chunks with a last-arrival sum:
        // 5.7, 6.1).
        const uint32_t S = go ? 2u : slice_count(nblk, groups, fmt, n_cu);
        if (S != 0) {
            a.split = 1;
            a.qpc = a.nquads;
            if (xm != kMvInPlain) {
                a.in_u = xm == kMvInGeglu ? in->up : in->y;
                a.in_wpost = in->w_post;
                a.in_wpre = in->w_pre;
                a.in_xout = in->x_out;
                a.in_eps = in->eps;
            }
            const size_t lds = size_t(nblk) * (sizeof(QxBlock) + sizeof(float)) +
                               size_t(kMvWgWaves) * (kGrp + 1) * sizeof(float);
            // GO: the gate's groups only, two workgroups each
            const dim3 grid((go ? mats[0].cols / kGrp : groups) * S), block(kMvWgWaves * kWave);
            // steps per wave, rounded up to 1, 2, 3, 4, 5 or 8 (one instance
            // each). A step past the end still loads (a clamped block, weighed
            // by zero): k = 1152 (18 steps) in 3 rounds instead of 4 loads 24
            // wave-blocks for 18 instead of 32, config 1 3.47 -> 3.31 us.
            const uint32_t steps = go ? nblk : (nblk + S - 1) / S;
            const uint32_t need = (steps + kMvWgWaves - 1) / kMvWgWaves;
            const uint32_t R = need <= 1 ? 1 : need <= 2 ? 2 : need <= 3 ? 3 : need <= 4 ? 4 : need <= 5 ? 5 : 8;
#define XP_MV_SLICE_R(F, SS, XX, GG)                                                                          \
    if (R == 1) hipLaunchKernelGGL((mv_int4_slice_kernel<F, SS, 1, XX, GG>), grid, block, lds, st, a);       \
    else if (R == 2) hipLaunchKernelGGL((mv_int4_slice_kernel<F, SS, 2, XX, GG>), grid, block, lds, st, a);  \
    else if (R == 3) hipLaunchKernelGGL((mv_int4_slice_kernel<F, SS, 3, XX, GG>), grid, block, lds, st, a);  \
    else if (R == 4) hipLaunchKernelGGL((mv_int4_slice_kernel<F, SS, 4, XX, GG>), grid, block, lds, st, a);  \
    else if (R == 5) hipLaunchKernelGGL((mv_int4_slice_kernel<F, SS, 5, XX, GG>), grid, block, lds, st, a);  \
    else hipLaunchKernelGGL((mv_int4_slice_kernel<F, SS, 8, XX, GG>), grid, block, lds, st, a);
#define XP_MV_SLICE_X(F, SS)                                         \
    if (xm == kMvInGeglu) { XP_MV_SLICE_R(F, SS, kMvInGeglu, false) } \
    else if (xm == kMvInNorm) { XP_MV_SLICE_R(F, SS, kMvInNorm, false) } \
    else { XP_MV_SLICE_R(F, SS, kMvInPlain, false) }
#define XP_MV_SLICE_LAUNCH(F)                                                    \
    if (go && xm == kMvInNorm) { XP_MV_SLICE_R(F, 2, kMvInNorm, true) }          \
    else if (go) { XP_MV_SLICE_R(F, 2, kMvInPlain, true) }                        \
    else if (S == 4) { XP_MV_SLICE_X(F, 4) }                                      \
    else { XP_MV_SLICE_X(F, 2) }
            if (fmt == XP_SCALE_F16_QUAD) {
                XP_MV_SLICE_LAUNCH(XP_SCALE_F16_QUAD)
            } else {
                XP_MV_SLICE_LAUNCH(XP_SCALE_BF16_QUAD)
            }
#undef XP_MV_SLICE_LAUNCH
#undef XP_MV_SLICE_X
#undef XP_MV_SLICE_R
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return set_error(XP_E_HIP, "%s: launch -> %s", who, hipGetErrorString(e));
            return XP_OK;
        }
        uint32_t sp = 1;
        if (a.nquads > kMvWgChunk || groups < 64) {
            sp = std::max(1u, std::min(kMvWgMaxSplit, uint32_t(n_cu) / groups));
            sp = std::max(sp, (a.nquads + kMvWgChunk - 1) / kMvWgChunk);
        }
        const uint32_t qpc = (a.nquads + sp - 1) / sp, nsp = (a.nquads + qpc - 1) / qpc;
        const size_t need = nsp > 1 ? size_t(nsp) * groups * kGrp : 0;
        bool ok = sp <= kMvWgMaxSplit;
        if (ok && nsp > 1) {
            if (sc) {
                if (!ensure_partial(sc, need)) return XP_E_NOMEM;
                if (!ensure_tickets(sc, groups)) return XP_E_NOMEM;
                a.partial = sc->partial;
                a.tickets = sc->tickets;
            } else if (partial_cap >= need && tickets_cap >= groups) {
                a.partial = partial;
                a.tickets = tickets;
            } else {
                ok = false;
            }
        }
        if (ok) {
            a.qpc = qpc;
            a.split = nsp;
            const size_t lds = size_t(4u * qpc) * (sizeof(QxBlock) + sizeof(float)) +
                               size_t(kMvWgWaves) * kGrp * sizeof(float);
            const dim3 grid(groups * nsp), block(kMvWgWaves * kWave);
#define XP_MV_WG_LAUNCH(F)                                                                 \
    if (nsp > 1)                                                                           \
        hipLaunchKernelGGL((mv_int4_wg_kernel<F, true>), grid, block, lds, st, a);         \
    else                                                                                   \
        hipLaunchKernelGGL((mv_int4_wg_kernel<F, false>), grid, block, lds, st, a);
            if (fmt == XP_SCALE_F16_QUAD) {
                XP_MV_WG_LAUNCH(XP_SCALE_F16_QUAD)
            } else {
                XP_MV_WG_LAUNCH(XP_SCALE_BF16_QUAD)
            }
#undef XP_MV_WG_LAUNCH
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return set_error(XP_E_HIP, "%s: launch -> %s", who, hipGetErrorString(e));
            return XP_OK;
        }
        a.partial = nullptr;
        a.tickets = nullptr;
    }
    split_plan(groups, a.nquads, split, n_cu, a.split, a.qpc);
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
                return set_error(XP_E_ARG, "%s: split %u of %u columns needs %zu partial floats "
                                 "and %u tickets; the scratch holds %zu and %zu", who, a.split,
                                 groups * kGrp, need, groups, partial_cap, tickets_cap);
            a.partial = partial;
            a.tickets = tickets;
        }
    }
    const size_t lds = size_t(a.qpc) * 4 * (sizeof(QxBlock) + sizeof(float));
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

// ---- allocation-free entry point -------------------------------------------------
// Scratch of xp_mv_int4_noalloc: split-k / k-chunk partial sums (words
// [0, kNaPartialFloats)), then the arrival tickets of the last-arrival
// reductions (zero at rest: every kernel that takes one returns it to zero).
// A file-scope device array, so each GPU the library runs on holds its own
// copy (1 MiB + 16 KiB) until the process ends; host code reaches it only
// through the address hipGetSymbolAddress returns for the current device.
constexpr size_t   kNaPartialFloats = size_t(1) << 18;
constexpr uint32_t kNaTickets       = 4096;

}  // namespace xp

static __device__ __align__(256) uint32_t scratch[xp::kNaPartialFloats + xp::kNaTickets];

namespace xp {

namespace {
__global__ void zero_words_kernel(uint32_t* p, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}
std::mutex g_na_mu;
std::vector<MvNoAlloc> g_na;   // per device; partial == nullptr until set up
}  // namespace

int mv_noalloc_setup(hipStream_t st, bool sync, MvNoAlloc* out) {
    int dev = 0;
    XP_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_na_mu);
    if (dev >= int(g_na.size())) g_na.resize(size_t(dev) + 1, MvNoAlloc{});
    MvNoAlloc& d = g_na[size_t(dev)];
    if (!d.partial) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch));
        if (e != hipSuccess || !p)
            return set_error(XP_E_HIP, "xp_mv_int4_noalloc: hipGetSymbolAddress(scratch) on device "
                             "%d -> %s", dev, hipGetErrorString(e));
        hipDeviceProp_t prop;
        XP_HIP(hipGetDeviceProperties(&prop, dev));
        uint32_t* words = static_cast<uint32_t*>(p);
        // Tickets start at zero. A fill kernel, not a memset: the first call
        // may be inside a caller's graph capture.
        hipLaunchKernelGGL(zero_words_kernel, dim3((kNaTickets + 255) / 256), dim3(256), 0, st,
                           words + kNaPartialFloats, kNaTickets);
        XP_HIP(hipGetLastError());
        if (sync) XP_HIP(hipStreamSynchronize(st));
        d.partial = reinterpret_cast<float*>(words);
        d.partial_floats = kNaPartialFloats;
        d.tickets = words + kNaPartialFloats;
        d.n_tickets = kNaTickets;
        d.n_cu = prop.multiProcessorCount;
    }
    *out = d;
    return XP_OK;
}

}  // namespace xp

using namespace xp;

extern "C" {

int xp_mv_int4_noalloc(float* out, const float* in, const void* wq, const void* scales,
                       int scale_fmt, uint32_t rows, uint32_t cols, uint32_t split,
                       xp_stream stream) {
    const hipStream_t st = as_stream(stream);
    MvNoAlloc d{};
    if (int rc = mv_noalloc_setup(st, false, &d); rc != XP_OK) return rc;
    MvMatDesc m{out, wq, scales, cols};
    return launch_mv(&m, 1, in, scale_fmt, rows, split, d.partial, d.partial_floats, d.tickets,
                     d.n_tickets, st, "xp_mv_int4_noalloc", d.n_cu);
}

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

int xp_mv_int4_batch_timed(float* out, const float* in, const void* const* wqs,
                           const void* const* scales, uint32_t ncopies, int scale_fmt, uint32_t rows,
                           uint32_t cols, uint32_t split, uint32_t count, uint32_t reps,
                           xp_stream stream, float* best_ms) {
    XP_REQUIRE(wqs && scales && best_ms && ncopies > 0 && count > 0 && reps > 0, "bad arguments");
    hipStream_t st = as_stream(stream);
    int rc = XP_OK;
    // One untimed pass over every copy: any scratch is sized before the capture.
    for (uint32_t i = 0; i < ncopies && rc == XP_OK; ++i)
        rc = xp_mv_int4(out, in, wqs[i], scales[i], scale_fmt, rows, cols, split, stream);
    if (rc != XP_OK) return rc;
    XP_HIP(hipStreamSynchronize(st));
    return graph_batch_timed(
        [&](hipStream_t cs) {
            for (uint32_t i = 0; i < count; ++i) {
                const int r = xp_mv_int4(out, in, wqs[i % ncopies], scales[i % ncopies], scale_fmt, rows,
                                         cols, split, reinterpret_cast<xp_stream>(cs));
                if (r != XP_OK) return r;
            }
            return int(XP_OK);
        },
        reps, st, best_ms);
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
