// Batched decode (up to 16 independent sequences per step) on gfx950.
//
// The token step's matvecs become M = 16 GEMMs on the matrix cores: rows are
// the sequences, and v_mfma_f32_16x16x32_bf16 takes one 32-wide quantisation
// block of k at a time, so every block's integer product is scaled by its own
// weight scale after the instruction. Weights stay in the packed KM4 layout;
// the nibbles are widened to bf16 in registers:
//
//   B operand  lane l holds column 16 t + l % 16 and k = 8 (l / 16) + 0..7,
//              i.e. word l / 16 of that column's 16-byte KM4 block, one dword
//              load per lane (a wave reads 256 contiguous bytes). Dword j of
//              the operand is ((w >> 4 j) & 0x000F000F) | 0x43004300: the
//              bf16 pair (128 + n_j, 128 + n_{j+4}), exact. Operand slot s
//              therefore holds nibble e(s) = s / 2 + 4 (s % 2).
//   A operand  lane l holds sequence l % 16 and the same eight k in the same
//              slot order, as two bf16 terms x = hi + lo (|x - hi - lo| <=
//              2^-18 |x|), staged once per step by bprep_kernel.
//   epilogue   C = A_hi B + A_lo B - 136 * sum_k (hi + lo) over the block
//              (the correction is the accumulator's start value, which saves
//              four VALU subtractions a tile and block), then
//              y += scale(block, column) * C, which removes the +128 magic
//              and the nibble bias of 8.
//
// Each wave owns one 64-column KM4 group (four 16-column MFMA tiles); the four
// waves of a workgroup share a k chunk whose staged A blocks pass through LDS.
// Chunks are split-K partials reduced in ascending order by the workgroup that
// arrives last, so results are deterministic.
#include "xp_device.hpp"
#include "xp_launch.hpp"

#include "xp_bmm_device.hpp"

namespace xp {

namespace {
constexpr uint32_t kPrepThreads = 1024;
}  // namespace

// ---- staging (bprep: modes in xp_bmm_device.hpp) ------------------------------------
__global__ __launch_bounds__(kPrepThreads) void bprep_kernel(BprepArgs a) {
    __shared__ float red[2][kPrepThreads / kWave];
    prep_row<kPrepThreads, false>(a, blockIdx.x, red);
}

// ---- M = 16 int4 GEMM (the tile in xp_bmm_device.hpp) ------------------------------
template <int FMT, int T, int AM, bool GE = false, int KC = 0>
__global__ __launch_bounds__(kBmmThreads) void bmm_int4_kernel(BmmArgs a) {
    __shared__ BmmSmem<T> sm;
    (void)bmm_tile<FMT, T, AM, GE, false, KC>(a, blockIdx.x, blockIdx.y, gridDim.x, sm);
}

// Streamed M = 16 GEMM for wide matrices (the batched lm_head: 4096 column
// groups of a 1152-long k): a persistent grid of one workgroup per CU takes
// column groups wg, wg + grid, ...; wave w keeps the staged operand of its
// k blocks (nblk / 8 or one more, at most 5: at most two scale quads) in
// registers for every group and keeps the weights of the next group in
// flight while it multiplies the current ones, so the stream never waits on
// a workgroup's launch or reduction. The eight waves' partial tiles meet in
// LDS, double buffered (one barrier a group), and are added in wave order
// as bmm_int4_kernel adds them. The groups rotate through two weight
// buffers in an unrolled ring so that each keeps fixed registers.
template <int FMT>
__global__ __launch_bounds__(kBmmThreads) void bmm_stream_kernel(BmmArgs a) {
    constexpr int MB = int(kBmmMaxPerWave);
    constexpr int NBUF = 2;                           // 3 spills registers
    constexpr uint32_t NO = 1024;                      // 16 rows x 64 columns
    static_assert(MB <= 5, "a wave's blocks span at most two scale quads");
    __shared__ float red[2][kBmmWaves][NO];
    // the wave index as a uniform value: the blocks, quads and scalar load
    // offsets derived from it then stay in scalar registers (derived from a
    // per-lane value, every raw buffer load with such an offset compiled to
    // a loop over the offset's distinct values, one pass at run time but
    // ~10 instructions and a branch per load)
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave;
    const uint32_t col16 = lane % 16u, wsel = lane / 16u;
    const uint32_t nblk = a.nblk, base = nblk / kBmmWaves, rem = nblk % kBmmWaves;
    const uint32_t nbw = base + (wave < rem ? 1u : 0u);       // this wave's blocks
    const uint32_t kb0 = wave * base + min(wave, rem);
    const uint32_t q0 = kb0 / 4u;                               // its first scale quad
    const u32x4* A = static_cast<const u32x4*>(a.a);
    u32x4 ahi[MB], alo[MB];
    float4 as[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) {
        const uint32_t blk = kb0 + min(uint32_t(j), nbw - 1u);
        ahi[j] = A[(size_t(blk) * 2 + 0) * 64 + lane];
        alo[j] = A[(size_t(blk) * 2 + 1) * 64 + lane];
        as[j] = *reinterpret_cast<const float4*>(a.asum + size_t(blk) * 16 + 4u * wsel);
    }
    const uint32_t cols = a.mats[0].cols, ng = cols / kGrp;
    const uint32_t nq = (nblk + 3u) / 4u;
    const uint32_t* wq = static_cast<const uint32_t*>(a.mats[0].wq);
    const u32x2* sq = static_cast<const u32x2*>(a.mats[0].sc);
    float* out = a.mats[0].out;
    const NibConst nk = nib_const();
    struct Wt {
        uint32_t w[MB][4];
        u32x2 sc[2][4];                                 // scale quads q0, q0 + 1
    };
    // raw buffer loads: a fixed per-lane offset and a per-group (and block)
    // scalar offset, no 64-bit address per lane and load
    const rsrc_t rw = make_rsrc(wq, cols * nblk * 16u), rs = make_rsrc(sq, nq * cols * 8u);
    auto load = [&](Wt& o, uint32_t g) {
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            const uint32_t blk = kb0 + min(uint32_t(j), nbw - 1u);
#pragma unroll
            for (int t = 0; t < 4; ++t)
                o.w[j][t] = __builtin_amdgcn_raw_buffer_load_b32(rw, int((16u * t + col16) * 16u + wsel * 4u),
                                                                 int((g * nblk + blk) * 1024u), 2);
        }
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
            const uint32_t q = min(q0 + uint32_t(qq), nq - 1u);
#pragma unroll
            for (int t = 0; t < 4; ++t)
                o.sc[qq][t] = __builtin_amdgcn_raw_buffer_load_b64(rs, int((16u * t + col16) * 8u),
                                                                   int((q * cols + g * kGrp) * 8u), 0);
        }
    };
    auto group = [&](const Wt& cur, uint32_t g, float (&rd)[kBmmWaves][NO]) {
        f32x4 acc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            if (uint32_t(j) >= nbw) break;
            const uint32_t blk = kb0 + uint32_t(j);
            const bf16x8 hi = as_bf16x8(ahi[j]), lo = as_bf16x8(alo[j]);
            const float corr[4] = {136.0f * as[j].x, 136.0f * as[j].y, 136.0f * as[j].z, 136.0f * as[j].w};
            const bool second = blk / 4u != q0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bf16x8 bw = as_bf16x8(widen_nibbles(cur.w[j][t], nk));
                f32x4 c = {-corr[0], -corr[1], -corr[2], -corr[3]};   // bias correction as the start value
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, bw, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, bw, c, 0, 0, 0);
                const float f = quad_scale<FMT>(second ? cur.sc[1][t] : cur.sc[0][t], blk % 4u);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(f, c[r], acc[t][r]);
            }
        }
        // o = lane * 16 + t * 4 + r  <->  row 4 (lane / 16) + r, column 16 t + lane % 16
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) rd[wave][lane * 16u + t * 4 + r] = acc[t][r];
        __syncthreads();
#pragma unroll
        for (uint32_t jo = 0; jo < NO / kBmmThreads; ++jo) {
            const uint32_t o = tid + jo * kBmmThreads;
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < int(kBmmWaves); ++w) sum += rd[w][o];
            const uint32_t ol = o / 16u, ot = (o % 16u) / 4u, orr = o % 4u;
            const uint32_t row = 4u * (ol / 16u) + orr, col = g * kGrp + 16u * ot + ol % 16u;
            if (row < a.rows) out[size_t(row) * cols + col] = sum;
        }
    };
    // Every prefetch is issued, past the last group as a repeat of it: a
    // load under a condition leaves the compiler's wait counts unable to
    // tell whether it was issued, and it then waits for all of them.
    Wt wb[NBUF];
    const uint32_t step = gridDim.x;
    uint32_t g = blockIdx.x;
#pragma unroll
    for (int b = 0; b < NBUF - 1; ++b) load(wb[b], min(g + uint32_t(b) * step, ng - 1u));
    // group i uses buffer i % NBUF and LDS half i % 2: the ring is unrolled
    // over 2 NBUF groups so that both are fixed
    for (;;) {
#pragma unroll
        for (int b = 0; b < 2 * NBUF; ++b) {
            if (g >= ng) return;
            load(wb[(b + NBUF - 1) % NBUF], min(g + uint32_t(NBUF - 1) * step, ng - 1u));
            group(wb[b % NBUF], g, red[b % 2]);
            g += step;
        }
    }
}

// ---- launchers --------------------------------------------------------------------
int launch_bprep(const BprepArgs& a, uint32_t batch, hipStream_t st) {
    if (a.K % 32 || a.K == 0 || a.K > 8 * kPrepThreads)
        return set_error(XP_E_ARG, "bprep: K=%u must be a multiple of 32, at most %u", a.K, 8 * kPrepThreads);
    if (batch == 0 || batch > 16) return set_error(XP_E_ARG, "bprep: batch %u outside [1, 16]", batch);
    hipLaunchKernelGGL(bprep_kernel, dim3(batch), dim3(kPrepThreads), 0, st, a);
    XP_LAUNCHED();
    return XP_OK;
}

// At most kBmmMaxPerWave blocks per wave; splits only when eight waves cannot
// cover k that way (the 6912-long down projection).
uint32_t bmm_split(uint32_t total_cols, uint32_t nblk, int n_cu) {
    (void)total_cols;
    (void)n_cu;
    return (nblk + kBmmWaves * kBmmMaxPerWave - 1) / (kBmmWaves * kBmmMaxPerWave);
}

size_t bmm_partial_floats(uint32_t total_cols, uint32_t nblk, int n_cu) {
    const uint32_t s = bmm_split(total_cols, nblk, n_cu);
    return s > 1 ? size_t(s) * (total_cols / kGrp) * kGrp * 16u : 0;
}

int plan_bmm(BmmArgs& a, int fmt, int n_cu, const char* who, uint32_t* n_blocks, bool* quarter_out) {
    if (a.n_mats == 0 || a.n_mats > 4) return set_error(XP_E_ARG, "%s: 1..4 matrices", who);
    if (a.rows == 0 || a.rows > 16) return set_error(XP_E_ARG, "%s: rows %u outside [1, 16]", who, a.rows);
    a.groups[0] = 0;
    for (uint32_t i = 0; i < a.n_mats; ++i) {
        if (a.mats[i].cols % kGrp) return set_error(XP_E_ARG, "%s: cols %u not a multiple of 64", who, a.mats[i].cols);
        a.groups[i + 1] = a.groups[i] + a.mats[i].cols / kGrp;
    }
    const uint32_t total = a.groups[a.n_mats] * kGrp;
    a.n_colwg = a.groups[a.n_mats];
    a.nsplit = bmm_split(total, a.nblk, n_cu);
    a.kc = (a.nblk + kBmmWaves * a.nsplit - 1) / (kBmmWaves * a.nsplit);
    a.nsplit = (a.nblk + kBmmWaves * a.kc - 1) / (kBmmWaves * a.kc);
    if (a.nsplit > 1) {
        if (!a.part || a.part_cap < size_t(a.nsplit) * a.n_colwg * kGrp * 16u)
            return set_error(XP_E_ARG, "%s: split-K partial buffer too small", who);
        if (!a.tickets || a.tickets_cap < a.n_colwg) return set_error(XP_E_ARG, "%s: too few tickets", who);
    }
    // Quarter-group column blocks (one MFMA tile per wave) when the groups
    // alone would give fewer than half the CUs a workgroup.
    const bool quarter = a.n_colwg * a.nsplit * 2u < uint32_t(n_cu > 0 ? n_cu : 256);
    const uint32_t nblocks = a.n_colwg * (quarter ? 4u : 1u);
    if (a.nsplit > 1 && a.tickets_cap < nblocks)
        return set_error(XP_E_ARG, "%s: too few tickets (%u < %u)", who, a.tickets_cap, nblocks);
    if (a.amode != 0 && a.amode != 2 && a.amode != 3)
        return set_error(XP_E_ARG, "%s: operand mode %u", who, a.amode);
    if (a.amode != 0 && (!a.xa || (a.amode == 3 && !a.xu) || a.lda < a.nblk * kBlk ||
                         ((reinterpret_cast<uintptr_t>(a.xa) | reinterpret_cast<uintptr_t>(a.xu)) & 15u) ||
                         a.lda % 4u))
        return set_error(XP_E_ARG, "%s: fp32 operand rows must be 16-byte aligned, lda >= k", who);
    if (fmt != XP_SCALE_F16_QUAD && fmt != XP_SCALE_BF16_QUAD)
        return set_error(XP_E_ARG, "%s: the batched GEMM takes fp16 or bf16 quad scales", who);
    if (a.geglu) {
        if (a.n_mats != 2 || a.mats[0].cols != a.mats[1].cols || a.nsplit != 1 || a.amode != 0 ||
            !a.a_out || !a.asum_out || a.a_out == a.a || a.asum_out == a.asum)
            return set_error(XP_E_ARG, "%s: the GeGLU epilogue takes two equal-width matrices, one "
                             "k split, a staged operand and separate output buffers", who);
    }
    *n_blocks = a.geglu ? a.mats[0].cols / 32u : nblocks;
    *quarter_out = !a.geglu && quarter;
    return XP_OK;
}

int launch_bmm(BmmArgs a, int fmt, int n_cu, hipStream_t st, const char* who) {
    uint32_t nblocks = 0;
    bool quarter = false;
    if (int rc = plan_bmm(a, fmt, n_cu, who, &nblocks, &quarter); rc != XP_OK) return rc;
    if (a.geglu) {
        const dim3 ggrid(nblocks, 1);
#define XP_BMM_GE(F)                                                                                           \
    if (a.kc == 5) hipLaunchKernelGGL((bmm_int4_kernel<F, 4, 0, true, 5>), ggrid, dim3(kBmmThreads), 0, st, a);      \
    else if (a.kc == 4) hipLaunchKernelGGL((bmm_int4_kernel<F, 4, 0, true, 4>), ggrid, dim3(kBmmThreads), 0, st, a); \
    else hipLaunchKernelGGL((bmm_int4_kernel<F, 4, 0, true>), ggrid, dim3(kBmmThreads), 0, st, a);
        if (fmt == XP_SCALE_F16_QUAD) {
            XP_BMM_GE(XP_SCALE_F16_QUAD)
        } else {
            XP_BMM_GE(XP_SCALE_BF16_QUAD)
        }
#undef XP_BMM_GE
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_error(XP_E_HIP, "%s: launch -> %s", who, hipGetErrorString(e));
        return XP_OK;
    }
    // Wide single matrices (the lm_head) stream through a persistent grid.
    if (a.n_mats == 1 && a.amode == 0 && a.nsplit == 1 && n_cu > 0 && a.n_colwg >= 4u * uint32_t(n_cu) &&
        a.nblk >= kBmmWaves && a.nblk <= kBmmWaves * kBmmMaxPerWave) {
        const dim3 sgrid{static_cast<uint32_t>(n_cu)};
        if (fmt == XP_SCALE_F16_QUAD)
            hipLaunchKernelGGL((bmm_stream_kernel<XP_SCALE_F16_QUAD>), sgrid, dim3(kBmmThreads), 0, st, a);
        else
            hipLaunchKernelGGL((bmm_stream_kernel<XP_SCALE_BF16_QUAD>), sgrid, dim3(kBmmThreads), 0, st, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_error(XP_E_HIP, "%s: launch -> %s", who, hipGetErrorString(e));
        return XP_OK;
    }
    const dim3 grid(nblocks, a.nsplit);
    // blocks per wave 4 and 5 (every Gemma-3 shape: k = 1024, 1152, 6912)
    // as compile-time counts, other counts under the chunk test
#define XP_BMM_KC(F, TT, AM)                                                                               \
    if (a.kc == 5) hipLaunchKernelGGL((bmm_int4_kernel<F, TT, AM, false, 5>), grid, dim3(kBmmThreads), 0, st, a);      \
    else if (a.kc == 4) hipLaunchKernelGGL((bmm_int4_kernel<F, TT, AM, false, 4>), grid, dim3(kBmmThreads), 0, st, a); \
    else hipLaunchKernelGGL((bmm_int4_kernel<F, TT, AM>), grid, dim3(kBmmThreads), 0, st, a);
#define XP_BMM_AM(F, TT)                                  \
    if (a.amode == 2) { XP_BMM_KC(F, TT, 2) }             \
    else if (a.amode == 3) { XP_BMM_KC(F, TT, 3) }        \
    else { XP_BMM_KC(F, TT, 0) }
    if (fmt == XP_SCALE_F16_QUAD) {
        if (quarter) { XP_BMM_AM(XP_SCALE_F16_QUAD, 1) } else { XP_BMM_AM(XP_SCALE_F16_QUAD, 4) }
    } else {
        if (quarter) { XP_BMM_AM(XP_SCALE_BF16_QUAD, 1) } else { XP_BMM_AM(XP_SCALE_BF16_QUAD, 4) }
    }
#undef XP_BMM_AM
#undef XP_BMM_KC
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "%s: launch -> %s", who, hipGetErrorString(e));
    return XP_OK;
}

}  // namespace xp
