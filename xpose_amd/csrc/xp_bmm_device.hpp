// Device code of the batched decode step (up to 16 sequences, M = 16 MFMA
// GEMMs on int4 weights), shared by its per-op kernels (batch_kernels.hip)
// and the persistent step kernel (batch_step.hip). The layout of the
// operands and the epilogue are described in batch_kernels.hip.
//
// Functions with a DEV template switch write their outputs with device-scope
// stores when DEV is set: the persistent kernel's consumers are other
// workgroups of the same launch, possibly on other XCDs, which read them
// after a completion counter says they are complete.
#pragma once

#include "xp_device.hpp"
#include "xp_launch.hpp"

namespace xp {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kBmmThreads = 512;       // eight waves share one column group

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// The constants of widen_nibbles in registers the compiler cannot fold: the
// mask in a scalar register, the bf16 128 pair in a vector register. Then
// (w & mask) | magic is one v_and_or_b32 (gfx9's three-operand encoding has
// no literal and takes one scalar operand, so with both constants as
// literals it became a separate AND and OR). The bias correction's 136 is
// held the same way: a block's operands are loaded under a test of the
// wave's chunk, and a product of a loaded value with a literal was moved by
// the compiler into that test's branch (an operation on a phi with one
// loaded and one undefined input is folded into the input's block), where
// it waited for the block's operands before the next block's loads could
// issue: one memory round trip per block, in series.
struct NibConst {
    uint32_t mask, magic;
    float bias;
};
__device__ __forceinline__ NibConst nib_const() {
    NibConst k{0x000F000Fu, 0x43004300u, 136.0f};
    asm volatile("" : "+s"(k.mask));
    asm volatile("" : "+v"(k.magic));
    asm volatile("" : "+s"(k.bias));
    return k;
}
// The eight B-operand bf16 (128 + nibble) of one KM4 word, slot s = nibble e(s).
__device__ __forceinline__ u32x4 widen_nibbles(uint32_t w, NibConst k) {
    u32x4 d;
    d.x = (w & k.mask) | k.magic;
    d.y = ((w >> 4) & k.mask) | k.magic;
    d.z = ((w >> 8) & k.mask) | k.magic;
    d.w = ((w >> 12) & k.mask) | k.magic;
    return d;
}

// The 32-bit word of lane 4 (l / 4) + R, as a float, in every lane l.
template <int R>
__device__ __forceinline__ float dpp_quad_bcast(uint32_t v) {
    return __uint_as_float(uint32_t(__builtin_amdgcn_mov_dpp(int(v), R * 0x55, 0xF, 0xF, false)));
}

template <int FMT>
__device__ __forceinline__ float quad_scale(u32x2 raw, uint32_t i) {
    const uint32_t w = (i & 2u) ? raw.y : raw.x;
    const uint32_t h = (w >> (16u * (i & 1u))) & 0xFFFFu;
    if constexpr (FMT == XP_SCALE_F16_QUAD) return f16_bits_to_f32(h);
    else return __uint_as_float(h << 16);
}

__device__ __forceinline__ uint32_t bf16_bits_rn(float f) {
    return uint32_t(__builtin_bit_cast(uint16_t, __bf16(f)));
}



// ---- staging -------------------------------------------------------------------
// Word c of staged block blk for row b from its eight elements v (k = 32 blk +
// 8 c + 0..7): the hi / lo bf16 operand of lane b + 16 c in slot order
// (slot s <- element s / 2 + 4 (s % 2)), and, from the four words of the
// block held by four adjacent lanes (c = lane % 4, whole quads active), the
// block's sum of hi + lo for row b.
template <bool DEV = false>
__device__ __forceinline__ void stage_word(u32x4* A, float* asum, uint32_t blk, uint32_t c, uint32_t b,
                                           const float (&v)[8]) {
    uint32_t hi[8], lo[8];
    float sum = 0.0f;
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
        const float t = v[sl / 2 + 4 * (sl % 2)];
        const uint32_t h = bf16_bits_rn(t);
        const float hf = __uint_as_float(h << 16);
        const uint32_t l = bf16_bits_rn(t - hf);
        hi[sl] = h;
        lo[sl] = l;
        sum += hf + __uint_as_float(l << 16);
    }
    const u32x4 H{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16), hi[4] | (hi[5] << 16),
                  hi[6] | (hi[7] << 16)};
    const u32x4 L{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16), lo[4] | (lo[5] << 16),
                  lo[6] | (lo[7] << 16)};
    const uint32_t lane = b + 16u * c;
    st_u4<DEV>(A + (size_t(blk) * 2 + 0) * 64 + lane, H);
    st_u4<DEV>(A + (size_t(blk) * 2 + 1) * 64 + lane, L);
    sum += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0xB1, 0xF, 0xF, false));
    sum += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0x4E, 0xF, 0xF, false));
    if (c == 0) st_f<DEV>(asum + size_t(blk) * 16 + b, sum);
}

// One workgroup per sequence b; thread i holds elements 8 p .. 8 p + 7 for p =
// i, i + 1024, ... (every width here is one pass) in registers from the load
// through the norms to the staged operand. Modes (x, y: [batch][K] fp32, row b):
//   0  stage rmsnorm(x) (1 + w_pre)
//   1  x += rmsnorm(y) (1 + w_post) (written back), then stage rmsnorm(x) (1 + w_pre)
//   2  stage y
//   3  stage gelu_tanh(y) * u
// Staged: A[blk][0 / 1][lane] = the hi / lo bf16 operand of lane l = b + 16 c
// for k = 32 blk + 8 c + e(s); asum[blk][b] = sum of hi + lo over the block.
__device__ __forceinline__ void ld8f(float (&v)[8], const float* p) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <uint32_t NT, bool DEV>
__device__ __forceinline__ void prep_row(const BprepArgs& a, uint32_t b, float (&red)[2][NT / kWave]) {
    const uint32_t tid = DEV ? opaque_tid() : threadIdx.x;
    const uint32_t K = a.K, npair = K / 8;    // (block, word) pairs of eight elements
    const uint32_t p = tid;
    const bool own = p < npair;
    float* x = a.x ? a.x + size_t(b) * K : nullptr;
    const float* y = a.y ? a.y + size_t(b) * K : nullptr;
    const float* u = a.u ? a.u + size_t(b) * K : nullptr;
    auto bsum = [&](float v, int slot) {
        v = wave_sum(v);
        if (tid % kWave == 0) red[slot][tid / kWave] = v;
        __syncthreads();
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < int(NT / kWave); ++w) t += red[slot][w];
        return t;
    };
    float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (a.mode <= 1) {
        float xv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f}, wpre[8];
        if (own && a.mode == 0 && a.tok) {
            // the embedding (decode.cpp:1618-1627): elements 8p .. 8p + 7 are
            // one word of the table column's block
            uint32_t t = a.tok[b];
            if (t >= a.vocab) t = 0;
            if (a.etable) {
                ld8f(xv, a.etable + size_t(t) * K + 8 * p);
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[e] = xv[e] * a.escale;
            } else {
                const uint32_t nblk = K / kBlk, blk = (8 * p) / kBlk, i0 = (8 * p) % kBlk;
                const uint32_t word = static_cast<const uint32_t*>(
                    a.ewq)[((size_t(t / kGrp) * nblk + blk) * kGrp + (t % kGrp)) * 4 + i0 / 8];
                const uint16_t h = static_cast<const uint16_t*>(a.esc)[(size_t(blk / 4) * a.vocab + t) * 4 + blk % 4];
                const float sc = a.efmt == XP_SCALE_F16_QUAD ? f16_bits_to_f32(h) : __uint_as_float(uint32_t(h) << 16);
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[e] = (float(int((word >> (4 * e)) & 15u) - 8) * sc) * a.escale;
            }
            float4* xo = reinterpret_cast<float4*>(x + 8 * p);
            st_u4<DEV>(reinterpret_cast<u32x4*>(xo), u32x4{__float_as_uint(xv[0]), __float_as_uint(xv[1]),
                                                           __float_as_uint(xv[2]), __float_as_uint(xv[3])});
            st_u4<DEV>(reinterpret_cast<u32x4*>(xo + 1), u32x4{__float_as_uint(xv[4]), __float_as_uint(xv[5]),
                                                               __float_as_uint(xv[6]), __float_as_uint(xv[7])});
            ld8f(wpre, a.w_pre + 8 * p);
        } else if (own) {
            ld8f(xv, x + 8 * p);
            ld8f(wpre, a.w_pre + 8 * p);
        }
        if (a.mode == 1) {
            float yv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f}, wpost[8];
            if (own) {
                ld8f(yv, y + 8 * p);
                ld8f(wpost, a.w_post + 8 * p);
            }
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(yv[e], yv[e], ss);
            const float post = rsq_hw(bsum(ss, 0) / float(K) + a.eps);
            if (own) {
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[e] = xv[e] + yv[e] * post * (1.0f + wpost[e]);
                float4* xo = reinterpret_cast<float4*>(a.x_out ? a.x_out + size_t(b) * K + 8 * p : x + 8 * p);
                st_u4<DEV>(reinterpret_cast<u32x4*>(xo),
                           u32x4{__float_as_uint(xv[0]), __float_as_uint(xv[1]), __float_as_uint(xv[2]),
                                 __float_as_uint(xv[3])});
                st_u4<DEV>(reinterpret_cast<u32x4*>(xo + 1),
                           u32x4{__float_as_uint(xv[4]), __float_as_uint(xv[5]), __float_as_uint(xv[6]),
                                 __float_as_uint(xv[7])});
            }
        }
        float sx = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sx = fmaf(xv[e], xv[e], sx);
        const float pre = rsq_hw(bsum(sx, 1) / float(K) + a.eps);
        if (own) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = xv[e] * pre * (1.0f + wpre[e]);
        }
    } else if (own) {
        ld8f(v, y + 8 * p);
        if (a.mode == 3) {
            float uv[8];
            ld8f(uv, u + 8 * p);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = gelu_hw(v[e]) * uv[e];
        }
    }
    if (!own) return;
    stage_word<DEV>(static_cast<u32x4*>(a.a), a.asum, p / 4u, p % 4u, b, v);
}

// ---- M = 16 int4 GEMM ------------------------------------------------------------
// Workgroup (cb, s): a block of 16 T columns (T MFMA tiles: 4 = one 64-column
// KM4 group, 1 = a quarter of one, for narrow shapes whose groups alone would
// leave most CUs idle), k split s; its eight waves take consecutive chunks of
// kc <= kBmmMaxPerWave blocks, load every operand of their chunk at once (one
// memory latency per wave, not one per block), and sum their 16 x 16 T
// results through LDS in wave order. With nsplit > 1 the splits publish
// partials and the last to arrive (ticket per column block) adds them in
// split order.
constexpr uint32_t kBmmWaves = 8;
constexpr uint32_t kBmmMaxPerWave = 5;

// The staged operand of one block from fp32 rows, in registers (the same
// values and slot order bprep_kernel writes): lane l holds row l % 16 and k =
// 32 blk + 8 (l / 16) + e(s); as = the block sums of rows 4 (l / 16) + 0..3.
__device__ __forceinline__ void stage_regs(u32x4& H, u32x4& L, float4& as, const float (&v)[8],
                                           uint32_t wsel) {
    uint32_t hi[8], lo[8];
    float sum = 0.0f;
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
        const float t = v[sl / 2 + 4 * (sl % 2)];
        const uint32_t h = bf16_bits_rn(t);
        const float hf = __uint_as_float(h << 16);
        const uint32_t l = bf16_bits_rn(t - hf);
        hi[sl] = h;
        lo[sl] = l;
        sum += hf + __uint_as_float(l << 16);
    }
    H = u32x4{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16), hi[4] | (hi[5] << 16), hi[6] | (hi[7] << 16)};
    L = u32x4{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16), lo[4] | (lo[5] << 16), lo[6] | (lo[7] << 16)};
    // the row's block sum over its four 8-element groups (lanes 16 apart),
    // added as bprep_kernel adds them: (g0 + g1) + (g2 + g3)
    sum += __shfl_xor(sum, 16, kWave);
    sum = add_xor32(sum);
    as = float4{__shfl(sum, int(4 * wsel + 0), kWave), __shfl(sum, int(4 * wsel + 1), kWave),
                __shfl(sum, int(4 * wsel + 2), kWave), __shfl(sum, int(4 * wsel + 3), kWave)};
}

template <int T>
struct BmmSmem {
    float red[kBmmWaves][256u * T];
    uint32_t last;
};

// One workgroup's tile: column block cb (of ncb) and k split s. Returns true
// when this workgroup wrote final outputs (every tile without k splits; with
// splits, the last split of its column block to arrive). DEV: outputs go out
// with device-scope stores (read by other workgroups of the same launch).
// KC > 0: every wave loads exactly KC blocks (a.kc == KC), its blocks past
// its chunk re-reading its last one (not multiplied), so the loads are
// unconditional and each block's multiply waits for that block's operands
// only. KC = 0: blocks loaded under the chunk test; the compiler cannot then
// count the loads issued after a block, and the first multiply waited for
// nearly every load of the wave.
template <int FMT, int T, int AM, bool GE, bool DEV, int KC = 0>
__device__ __forceinline__ bool bmm_tile(const BmmArgs& a, uint32_t cb, uint32_t s, uint32_t ncb,
                                         BmmSmem<T>& sm) {
    constexpr uint32_t NO = 256u * T;            // outputs of a workgroup: 16 rows x 16 T columns
    constexpr uint32_t PER = (NO + kBmmThreads - 1) / kBmmThreads;
    constexpr uint32_t SUBS = 4u / T;            // column blocks per 64-column group
    static_assert(!GE || (T == 4 && AM == 0), "the GeGLU epilogue takes four tiles of staged A");
    auto& red = sm.red;
    uint32_t& last = sm.last;
    const uint32_t tid = DEV ? opaque_tid() : threadIdx.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave;
    // GE: columns 32 (cb % 2) .. + 31 of group cb / 2 of both matrices;
    // tiles 0, 1 from the gate, 2, 3 from the up projection
    const uint32_t gg = GE ? cb / 2u : cb / SUBS;
    const uint32_t c16 = GE ? (cb % 2u) * 32u : (cb % SUBS) * 16u * T;   // first column in the group
    // the matrix of column group gg, chosen without indexing the argument
    // arrays by a variable (so that a copy of them can live in registers)
    MvMatDesc md = a.mats[0];
    uint32_t g0 = 0;
    if constexpr (!GE) {
#pragma unroll
        for (uint32_t i = 1; i < 4; ++i)
            if (i < a.n_mats && gg >= a.groups[i]) {
                md = a.mats[i];
                g0 = a.groups[i];
            }
    }
    const uint32_t g = gg - g0;
    const uint32_t cols = md.cols;
    const uint32_t col16 = lane % 16u, wsel = lane / 16u;
    const uint32_t kb0 = min((s * kBmmWaves + wave) * a.kc, a.nblk);
    const uint32_t kb1 = min(kb0 + a.kc, a.nblk);
    f32x4 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // Every operand is read through a raw buffer: a fixed per-lane offset
    // and a per-block offset that is the same for the whole wave (a scalar),
    // so no 64-bit address is formed per lane and load (the GEMM is
    // VALU-bound at M = 16). Weights stream past the caches (nt).
    constexpr int kNt = 2;
    const uint32_t nblk = a.nblk, wbytes = cols * nblk * 16u, sbytes = ((nblk + 3u) / 4u) * cols * 8u;
    rsrc_t rw[GE ? 2 : 1], rs[GE ? 2 : 1];
    if constexpr (GE) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            rw[i] = make_rsrc(a.mats[i].wq, wbytes);
            rs[i] = make_rsrc(a.mats[i].sc, sbytes);
        }
    } else {
        rw[0] = make_rsrc(md.wq, wbytes);
        rs[0] = make_rsrc(md.sc, sbytes);
    }
    // operands of one block (raw fp32 rows in AM 2 / 3, staged after the loads)
    constexpr int NR = AM == 3 ? 4 : (AM == 2 ? 2 : 1);
    struct Ops {
        u32x4 hi, lo;
        float4 as;
        uint32_t asr;   // AM 0: lane l's word of the block sums, row 4 (l / 16) + l % 4
        float4 raw[NR];
        uint32_t w[T];
    };
    const rsrc_t ra = make_rsrc(a.a, nblk * 2u * 64u * 16u), rsum = make_rsrc(a.asum, nblk * 16u * 4u);
    // fp32 rows: sequences past a.rows lie past the buffer's end and read as zeros
    const rsrc_t rxa = make_rsrc(a.xa, a.rows * a.lda * 4u), rxu = make_rsrc(a.xu, a.rows * a.lda * 4u);
    const uint32_t vx = (col16 * a.lda + 8u * wsel) * 4u;
    auto ldx4 = [&](rsrc_t r, uint32_t voff, uint32_t soff) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), int(soff), 0);
        return float4{__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
    };
    auto load = [&](Ops& o, uint32_t blk) {
        if constexpr (AM == 0) {
            o.hi = __builtin_amdgcn_raw_buffer_load_b128(ra, int(lane * 16u), int(blk * 2048u), 0);
            o.lo = __builtin_amdgcn_raw_buffer_load_b128(ra, int(lane * 16u), int(blk * 2048u + 1024u), 0);
            // one word a lane; the four rows of its quad are read by DPP
            o.asr = __builtin_amdgcn_raw_buffer_load_b32(rsum, int(wsel * 16u + (lane % 4u) * 4u),
                                                         int(blk * 64u), 0);
        } else {
            // row col16, k 32 blk + 8 wsel ..
            o.raw[0] = ldx4(rxa, vx, blk * 128u);
            o.raw[1] = ldx4(rxa, vx + 16u, blk * 128u);
            if constexpr (AM == 3) {
                o.raw[2] = ldx4(rxu, vx, blk * 128u);
                o.raw[3] = ldx4(rxu, vx + 16u, blk * 128u);
            }
        }
        // block blk of column group g: weights at ((g nblk + blk) 64 + column) 16 + word 4
        const uint32_t sw = (g * nblk + blk) * 1024u;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const uint32_t mt = GE ? uint32_t(t) / 2u : 0u;
            const uint32_t cg = GE ? c16 + 16u * (uint32_t(t) % 2u) + col16 : c16 + 16u * t + col16;
            o.w[t] = __builtin_amdgcn_raw_buffer_load_b32(rw[mt], int(cg * 16u + wsel * 4u), int(sw), kNt);
        }
    };
    const NibConst nk = nib_const();
    // The scale quads of the wave's blocks (at most kBmmMaxPerWave = 5
    // consecutive blocks: two quads), each loaded once: quad q of column
    // group g at ((q cols + 64 g + column) 8.
    const uint32_t nq = (nblk + 3u) / 4u, q0 = min(kb0 / 4u, nq - 1u);
    u32x2 scq[2][T];
#pragma unroll
    for (uint32_t qq = 0; qq < 2; ++qq) {
        const uint32_t ss = (min(q0 + qq, nq - 1u) * cols + g * kGrp) * 8u;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const uint32_t mt = GE ? uint32_t(t) / 2u : 0u;
            const uint32_t cg = GE ? c16 + 16u * (uint32_t(t) % 2u) + col16 : c16 + 16u * t + col16;
            scq[qq][t] = __builtin_amdgcn_raw_buffer_load_b64(rs[mt], int(cg * 8u), int(ss), 0);
        }
    }
    static_assert(KC >= 0 && KC <= int(kBmmMaxPerWave), "blocks per wave");
    constexpr uint32_t NB = KC > 0 ? uint32_t(KC) : kBmmMaxPerWave;
    Ops ops[NB];
    if constexpr (KC > 0) {
        const uint32_t blast = kb1 > kb0 ? kb1 - 1u : nblk - 1u;
#pragma unroll
        for (uint32_t j = 0; j < NB; ++j) {
            load(ops[j], min(kb0 + j, blast));
            // in block order, and all before the first multiply (the
            // scheduler would otherwise group the loads by kind, putting a
            // block's last operand near the end, or move later blocks' loads
            // behind earlier blocks' waits)
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
#pragma unroll
        for (uint32_t j = 0; j < NB; ++j)
            if (kb0 + j < kb1) load(ops[j], kb0 + j);
    }
#pragma unroll
    for (uint32_t j = 0; j < NB; ++j) {
        if (kb0 + j >= kb1) break;
        const uint32_t blk = kb0 + j;
        Ops& cur = ops[j];
        if constexpr (AM != 0) {
            float v[8] = {cur.raw[0].x, cur.raw[0].y, cur.raw[0].z, cur.raw[0].w,
                          cur.raw[1].x, cur.raw[1].y, cur.raw[1].z, cur.raw[1].w};
            if constexpr (AM == 3) {
                const float u[8] = {cur.raw[2].x, cur.raw[2].y, cur.raw[2].z, cur.raw[2].w,
                                    cur.raw[3].x, cur.raw[3].y, cur.raw[3].z, cur.raw[3].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = gelu_hw(v[e]) * u[e];
            }
            stage_regs(cur.hi, cur.lo, cur.as, v, wsel);
        } else {
            cur.as = float4{dpp_quad_bcast<0>(cur.asr), dpp_quad_bcast<1>(cur.asr), dpp_quad_bcast<2>(cur.asr),
                            dpp_quad_bcast<3>(cur.asr)};
        }
        const bf16x8 ahi = as_bf16x8(cur.hi), alo = as_bf16x8(cur.lo);
        const float corr[4] = {nk.bias * cur.as.x, nk.bias * cur.as.y, nk.bias * cur.as.z, nk.bias * cur.as.w};
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const bf16x8 bw = as_bf16x8(widen_nibbles(cur.w[t], nk));
            // the bias correction enters as the accumulator's start value
            f32x4 c = {-corr[0], -corr[1], -corr[2], -corr[3]};
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, bw, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, bw, c, 0, 0, 0);
            const float f = quad_scale<FMT>(blk / 4u != q0 ? scq[1][t] : scq[0][t], blk % 4u);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(f, c[r], acc[t][r]);
        }
    }
    // o = lane * 4 T + t * 4 + r  <->  row 4 (lane / 16) + r, column 16 t + lane % 16
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][lane * 4u * T + t * 4 + r] = acc[t][r];
    __syncthreads();
    if constexpr (GE) {
        // h[row][j] = gelu_tanh(gate) * up for the 16 rows x 32 columns, one
        // per thread (gate tile j / 16 at o, up tile j / 16 + 2 at o + 8),
        // each summed over the waves in order; then staged as operand block
        // cb of the following GEMM (rows past a.rows as zeros)
        float* hb = &red[0][0];   // [16][32] after the barrier below
        const uint32_t row = tid / 32u, j = tid % 32u;
        const uint32_t ol = 16u * (row / 4u) + j % 16u, t = j / 16u;
        const uint32_t og = ol * 4u * T + t * 4u + row % 4u;
        float gs = 0.0f, us = 0.0f;
#pragma unroll
        for (int w = 0; w < int(kBmmWaves); ++w) {
            gs += red[w][og];
            us += red[w][og + 8u];
        }
        const float h = row < a.rows ? gelu_hw(gs) * us : 0.0f;
        __syncthreads();
        hb[row * 32u + j] = h;
        __syncthreads();
        if (tid < 64u) {
            const uint32_t b = tid / 4u, c = tid % 4u;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = hb[b * 32u + 8u * c + e];
            stage_word<DEV>(static_cast<u32x4*>(const_cast<void*>(a.a_out)), a.asum_out, cb, c, b, v);
        }
        return true;
    }
    float v[PER];
    uint32_t row[PER], col[PER];
    bool own[PER];
#pragma unroll
    for (uint32_t j = 0; j < PER; ++j) {
        const uint32_t o = tid + j * kBmmThreads;
        own[j] = o < NO;
        const uint32_t oc = own[j] ? o : 0u;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < int(kBmmWaves); ++w) sum += red[w][oc];
        v[j] = sum;
        const uint32_t ol = oc / (4u * T), ot = (oc % (4u * T)) / 4u, orr = oc % 4u;
        row[j] = 4u * (ol / 16u) + orr;
        col[j] = g * kGrp + c16 + 16u * ot + ol % 16u;
    }
    float* out = md.out;
    if (a.nsplit == 1) {
#pragma unroll
        for (uint32_t j = 0; j < PER; ++j)
            if (own[j] && row[j] < a.rows) st_f<DEV>(out + size_t(row[j]) * cols + col[j], v[j]);
        return true;
    }
    float* part = a.part + (size_t(s) * ncb + cb) * NO;
#pragma unroll
    for (uint32_t j = 0; j < PER; ++j)
        if (own[j]) st_dev(part + tid + j * kBmmThreads, v[j]);
    wait_mem();
    __syncthreads();
    if (tid == 0) last = take_ticket(a.tickets + cb);
    __syncthreads();
    if (last != a.nsplit - 1) return false;
    // last arrival: every split's partial, loaded together, added in split order
#pragma unroll
    for (uint32_t j = 0; j < PER; ++j) {
        if (!own[j]) continue;
        float sum = 0.0f;
        for (uint32_t p0 = 0; p0 < a.nsplit; p0 += 8) {
            float pv[8];
#pragma unroll
            for (uint32_t q = 0; q < 8; ++q)
                pv[q] = p0 + q < a.nsplit
                            ? ld_dev(a.part + (size_t(p0 + q) * ncb + cb) * NO + tid + j * kBmmThreads)
                            : 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < 8; ++q)
                if (p0 + q < a.nsplit) sum += pv[q];
        }
        if (row[j] < a.rows) st_f<DEV>(out + size_t(row[j]) * cols + col[j], sum);
    }
    if (tid == 0) st_dev(a.tickets + cb, 0u);
    return true;
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

}  // namespace

}  // namespace xp
