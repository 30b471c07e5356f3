// Native-format weights on gfx950: GGUF's Q8_0 / Q5_0 / Q4_K / Q6_K blocks.
//
// Native layout (kernels/llm_quant.cl:83-322): the file's blocks, read in
// place. dequant_native_kernel writes the element values with the host
// dequantiser's fp32 operations, uncontracted, so the two agree bit for bit.
// mv_native_kernel is the fused matvec: one wave per output row, lanes over
// the row's 32-element sub-blocks, fp32 accumulation and a wave sum. The
// blocks are 22 / 34 / 144 / 210 bytes, so from the second block on most
// fields sit at odd word offsets: every field is read with 16-bit loads
// (every block field is at an even offset), and this path is the reference
// the repacked one is checked against, not the fast one.
//
// Repacked layout (llm_quant.cl:340-615, quant_repack.cpp): slot idx =
// (g nkb + kb) 64 + t holds k-block kb of output row 64 g + t, so a wave
// (64 rows) reads each plane contiguously, one 16-byte nibble word per lane
// and block — the int4 KM4 plane's shape. mv_rq_kernel follows the int4
// matvec (matvec.hip): a wave is one task = (row group, k-chunk), the chunk's
// activations are staged once per workgroup in LDS as 20-bit block fixed
// point, and every block product is an exact integer:
//   Q4_K  sum q x        = D + 8 S                     (q the unsigned nibble)
//   Q5_0  sum (q - 16) x = D + 16 H - 8 S              (H: the fifth bits)
//   Q6_K  sum (q - 32) x = D + 16 H - 24 S per 16-element half
//   Q8_0  sum q x        = sum_p 256^p sum_k q_k e_pk  (sdot4 on the int8 bytes)
// where D = sum (n - 8) q_x is the int4 block dot (v_dot8_i32_i4 over five
// digit planes), S = sum q_x, and H = sum h q_x uses the high bits spread to
// one nibble per weight. Per block the fp32 work is one or two multiplies.
#include <algorithm>
#include <string>

#include "xp_device.hpp"
#include "xp_launch.hpp"

namespace xp {
namespace {

constexpr int kRqWaves = 4;
constexpr uint32_t kRqMaxSplit = 16;
constexpr uint32_t kQ80 = XP_GGML_Q8_0, kQ50 = XP_GGML_Q5_0, kQ4K = XP_GGML_Q4_K,
                   kQ6K = XP_GGML_Q6_K;

// ---- native layout --------------------------------------------------------------

__device__ __forceinline__ uint32_t u16at(const uint8_t* p, size_t off) {
    return ldg16(p + off);
}
__device__ __forceinline__ uint32_t u8at(const uint8_t* p, size_t off) {
    const uint32_t w = u16at(p, off & ~size_t(1));
    return (off & 1) ? (w >> 8) : (w & 0xFFu);
}
__device__ __forceinline__ float h16at(const uint8_t* p, size_t off) {
    return f16_bits_to_f32(u16at(p, off));
}

// Q4_K sub-block j's six-bit scale and min from the 12 packed bytes at s.
__device__ __forceinline__ void k4_pair(const uint8_t* p, size_t s, uint32_t j, uint32_t& sc,
                                        uint32_t& mn) {
    if (j < 4) {
        sc = u8at(p, s + j) & 63u;
        mn = u8at(p, s + j + 4) & 63u;
    } else {
        sc = (u8at(p, s + j + 4) & 15u) | ((u8at(p, s + j - 4) >> 6) << 4);
        mn = (u8at(p, s + j + 4) >> 4) | ((u8at(p, s + j) >> 6) << 4);
    }
}

// Element i of a native tensor, with the host dequantiser's operations and
// rounding order (no contraction).
template <uint32_t T>
__device__ float native_value(const uint8_t* p, uint64_t i) {
#pragma clang fp contract(off)
    if constexpr (T == kQ80) {
        const size_t b = size_t(i / 32) * 34;
        const int q = int(int8_t(u8at(p, b + 2 + i % 32)));
        return float(q) * h16at(p, b);
    } else if constexpr (T == kQ50) {
        const size_t b = size_t(i / 32) * 22;
        const uint32_t e = uint32_t(i % 32);
        const uint32_t qh = u16at(p, b + 2) | (u16at(p, b + 4) << 16);
        const uint32_t byte = u8at(p, b + 6 + (e & 15u));
        const uint32_t lo = e < 16 ? (byte & 15u) : (byte >> 4);
        const int q = int(lo | (((qh >> e) & 1u) << 4)) - 16;
        return float(q) * h16at(p, b);
    } else if constexpr (T == kQ4K) {
        const size_t b = size_t(i / 256) * 144;
        const uint32_t e = uint32_t(i % 256), run = e / 64, hi = (e % 64) / 32, l = e % 32;
        uint32_t sc, mn;
        k4_pair(p, b + 4, 2 * run + hi, sc, mn);
        const uint32_t q = (u8at(p, b + 16 + 32 * run + l) >> (4 * hi)) & 15u;
        return h16at(p, b) * float(sc) * float(q) - h16at(p, b + 2) * float(mn);
    } else {
        const size_t b = size_t(i / 256) * 210;
        const uint32_t e = uint32_t(i % 256), h = e / 128, t = (e % 128) / 32, l = e % 32;
        const uint32_t lo = (u8at(p, b + 64 * h + l + 32 * (t & 1u)) >> (4 * (t >> 1))) & 15u;
        const uint32_t up = (u8at(p, b + 128 + 32 * h + l) >> (2 * t)) & 3u;
        const int q = int(lo | (up << 4)) - 32;
        const int sc = int(int8_t(u8at(p, b + 192 + 8 * h + 2 * t + l / 16)));
        return h16at(p, b + 208) * float(sc) * float(q);
    }
}

template <uint32_t T>
__global__ void dequant_native_kernel(float* out, const uint8_t* src, uint64_t n) {
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = native_value<T>(src, i);
}

// Sub-block u (32 elements) of a native row at `row` against x[32u ..].
template <uint32_t T>
__device__ float native_unit(const uint8_t* row, const float* x, uint32_t u) {
    const float4* xv = reinterpret_cast<const float4*>(x + size_t(u) * 32);
    float xs[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 v = xv[i];
        xs[4 * i] = v.x; xs[4 * i + 1] = v.y; xs[4 * i + 2] = v.z; xs[4 * i + 3] = v.w;
    }
    if constexpr (T == kQ80) {
        const size_t b = size_t(u) * 34;
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; e += 2) {
            const uint32_t w = u16at(row, b + 2 + e);
            s = fmaf(xs[e], float(int(int8_t(w & 0xFFu))), s);
            s = fmaf(xs[e + 1], float(int(int8_t(w >> 8))), s);
        }
        return h16at(row, b) * s;
    } else if constexpr (T == kQ50) {
        const size_t b = size_t(u) * 22;
        const uint32_t qh = u16at(row, b + 2) | (u16at(row, b + 4) << 16);
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
            const uint32_t w = u16at(row, b + 6 + e);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const uint32_t byte = (w >> (8 * k)) & 0xFFu;
                const int lo = int((byte & 15u) | (((qh >> (e + k)) & 1u) << 4)) - 16;
                const int hi = int((byte >> 4) | (((qh >> (e + k + 16)) & 1u) << 4)) - 16;
                s = fmaf(xs[e + k], float(lo), s);
                s = fmaf(xs[e + k + 16], float(hi), s);
            }
        }
        return h16at(row, b) * s;
    } else if constexpr (T == kQ4K) {
        const size_t b = size_t(u / 8) * 144;
        const uint32_t j = u % 8;
        uint32_t sc, mn;
        k4_pair(row, b + 4, j, sc, mn);
        const size_t qs = b + 16 + (j / 2) * 32;
        const uint32_t sh = 4 * (j & 1u);
        float sq = 0.0f, sx = 0.0f;
#pragma unroll
        for (int l = 0; l < 32; l += 2) {
            const uint32_t w = u16at(row, qs + l);
            sq = fmaf(xs[l], float((w >> sh) & 15u), sq);
            sq = fmaf(xs[l + 1], float((w >> (8 + sh)) & 15u), sq);
            sx += xs[l] + xs[l + 1];
        }
        return h16at(row, b) * float(sc) * sq - h16at(row, b + 2) * float(mn) * sx;
    } else {
        const size_t b = size_t(u / 8) * 210;
        const uint32_t j = u % 8, h = j / 4, t = j % 4;
        const size_t ql = b + 64 * h + 32 * (t & 1u), qh = b + 128 + 32 * h;
        const uint32_t lsh = 4 * (t >> 1), hsh = 2 * t;
        float acc = 0.0f;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float s = 0.0f;
#pragma unroll
            for (int l = 16 * half; l < 16 * half + 16; l += 2) {
                const uint32_t wl = u16at(row, ql + l), wh = u16at(row, qh + l);
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const uint32_t lo = (wl >> (8 * k + lsh)) & 15u;
                    const uint32_t up = (wh >> (8 * k + hsh)) & 3u;
                    s = fmaf(xs[l + k], float(int(lo | (up << 4)) - 32), s);
                }
            }
            acc = fmaf(float(int(int8_t(u8at(row, b + 192 + 8 * h + 2 * t + half)))), s, acc);
        }
        return h16at(row, b + 208) * acc;
    }
}

template <uint32_t T>
__global__ __launch_bounds__(256) void mv_native_kernel(float* out, const float* x,
                                                       const uint8_t* src, uint32_t rows,
                                                       uint32_t cols, size_t row_bytes) {
    const uint32_t r = blockIdx.x * 4 + threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    if (r >= rows) return;   // whole waves
    const uint8_t* row = src + size_t(r) * row_bytes;
    float acc = 0.0f;
    for (uint32_t u = lane; u < cols / 32; u += kWave) acc += native_unit<T>(row, x, u);
    acc = wave_sum(acc);
    if (lane == 0) out[r] = acc;
}

// ---- repacked layout ------------------------------------------------------------

struct RqArgs {
    float*          out;
    const float*    x;
    const u32x4*    quant;
    const uint32_t* high;
    const float*    scale;
    const float*    bias;
    uint32_t        rows;           // logical outputs
    uint32_t        nkb;            // k-blocks per row
    uint32_t        groups;         // padded rows / 64
    uint32_t        split;
    uint32_t        kpc;            // k-blocks per chunk
    uint32_t        wg_per_chunk;
    float*          partial;        // [split][groups * 64]
    uint32_t*       tickets;        // [groups], zero at rest
};

// LDS per staged k-block: five nibble digit planes + four word sums
// (Q4_K / Q5_0 / Q6_K) or three byte digit planes (Q8_0), and the scale.
constexpr uint32_t kRqLdsPerBlock = 100;

// Nibble digit planes as stage_x8 makes them, plus the sum of the eight
// quantised values of this task's word.
__device__ __forceinline__ void stage_nib(QxBlock* qx, int32_t* wsum, float* sx, uint32_t i,
                                          float4 v0, float4 v1) {
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[e]));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    const float r = m > 0.0f ? kQxRange / m : 0.0f;
    uint32_t t[8];
    int32_t s = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int32_t q = __float2int_rn(v[e] * r);
        s += q;
        t[e] = uint32_t(q + int32_t(kQxBias)) ^ kQxBias;
    }
    const uint32_t lb = i >> 2, c = i & 3u;
#pragma unroll
    for (int p = 0; p < kQxPlanes; ++p) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) word |= ((t[e] >> (4 * p)) & 15u) << (4 * e);
        reinterpret_cast<uint32_t*>(&qx[lb].p[p])[c] = word;
    }
    wsum[i] = s;
    if (c == 0) sx[lb] = m * (1.0f / kQxRange);
}

// Byte digit planes for Q8_0: q = sum_p 256^p e_p with signed bytes e_p
// (q + 0x808080 has bytes e_p + 128). Plane p, word w of a block packs the
// digits of k = 4w .. 4w + 3 at byte positions 0..3, the positions the Q8_0
// quant word gives those k.
__device__ __forceinline__ void stage_b8(uint32_t* pl, float* sx, uint32_t i, float4 v0,
                                         float4 v1) {
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[e]));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    const float r = m > 0.0f ? kQxRange / m : 0.0f;
    uint32_t u[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) u[e] = uint32_t(__float2int_rn(v[e] * r) + 0x808080);
    const uint32_t lb = i >> 2, c = i & 3u;
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            w0 |= (((u[e] >> (8 * p)) & 0xFFu) ^ 0x80u) << (8 * e);
            w1 |= (((u[e + 4] >> (8 * p)) & 0xFFu) ^ 0x80u) << (8 * e);
        }
        pl[(lb * 3 + p) * 8 + 2 * c] = w0;
        pl[(lb * 3 + p) * 8 + 2 * c + 1] = w1;
    }
    if (c == 0) sx[lb] = m * (1.0f / kQxRange);
}

// sum over words C0 .. C0 + N - 1 of v's nibbles times the staged values, exact.
template <int C0, int N>
__device__ __forceinline__ int32_t nib_dot(u32x4 v, const QxBlock& q) {
    uint32_t d = 0;
#pragma unroll
    for (int p = 0; p < kQxPlanes; ++p) {
        int32_t s = 0;
#pragma unroll
        for (int c = C0; c < C0 + N; ++c) s = __builtin_amdgcn_sdot8(int32_t(v[c]), int32_t(q.p[p][c]), s, false);
        d += uint32_t(s) << (4 * p);
    }
    return int32_t(d);
}

// Bits 0..7 of b to nibbles 0..7 (values 0 / 1).
__device__ __forceinline__ uint32_t spread1(uint32_t b) {
    uint32_t x = b & 0xFFu;
    x = (x | (x << 12)) & 0x000F000Fu;
    x = (x | (x << 6)) & 0x03030303u;
    return (x | (x << 3)) & 0x11111111u;
}
// Two-bit fields 0..7 (bits 0..15) of f to nibbles 0..7 (values 0..3).
__device__ __forceinline__ uint32_t spread2(uint32_t f) {
    uint32_t x = f & 0xFFFFu;
    x = (x | (x << 8)) & 0x00FF00FFu;
    x = (x | (x << 4)) & 0x0F0F0F0Fu;
    return (x | (x << 2)) & 0x33333333u;
}

struct RqLds {
    const QxBlock*  qx;
    const int32_t*  wsum;
    const uint32_t* b8;
    const float*    sx;
};

template <uint32_t T> struct RqFmt;

template <> struct RqFmt<kQ4K> {
    static constexpr int kU = 4;   // blocks per pipeline stage
    struct Blk { u32x4 w; float s, b; };
    __device__ static void load(Blk& k, const RqArgs& a, size_t idx) {
        k.w = ld_stream4(a.quant + idx);
        k.s = __builtin_nontemporal_load(a.scale + idx);
        k.b = __builtin_nontemporal_load(a.bias + idx);
    }
    __device__ static float dot(const Blk& k, const RqLds& x, uint32_t lb) {
        const int4 ws = reinterpret_cast<const int4*>(x.wsum)[lb];
        const int32_t s = ws.x + ws.y + ws.z + ws.w;
        const int32_t d = nib_dot<0, 4>(k.w ^ 0x88888888u, x.qx[lb]);
        return x.sx[lb] * (k.s * float(d + 8 * s) - k.b * float(s));
    }
};

template <> struct RqFmt<kQ50> {
    static constexpr int kU = 4;
    struct Blk { u32x4 w; uint32_t h; float s; };
    __device__ static void load(Blk& k, const RqArgs& a, size_t idx) {
        k.w = ld_stream4(a.quant + idx);
        k.h = __builtin_nontemporal_load(a.high + idx);
        k.s = __builtin_nontemporal_load(a.scale + idx);
    }
    __device__ static float dot(const Blk& k, const RqLds& x, uint32_t lb) {
        const int4 ws = reinterpret_cast<const int4*>(x.wsum)[lb];
        const int32_t s = ws.x + ws.y + ws.z + ws.w;
        const QxBlock& q = x.qx[lb];
        const int32_t d = nib_dot<0, 4>(k.w ^ 0x88888888u, q);
        const u32x4 hv = {spread1(k.h), spread1(k.h >> 8), spread1(k.h >> 16), spread1(k.h >> 24)};
        const int32_t h = nib_dot<0, 4>(hv, q);
        return x.sx[lb] * (k.s * float(d + 16 * h - 8 * s));
    }
};

template <> struct RqFmt<kQ6K> {
    static constexpr int kU = 3;
    struct Blk { u32x4 w; u32x2 h; u32x2 s; };
    __device__ static void load(Blk& k, const RqArgs& a, size_t idx) {
        k.w = ld_stream4(a.quant + idx);
        k.h = ld_stream2(reinterpret_cast<const u32x2*>(a.high) + idx);
        k.s = ld_stream2(reinterpret_cast<const u32x2*>(a.scale) + idx);
    }
    __device__ static float dot(const Blk& k, const RqLds& x, uint32_t lb) {
        const int4 ws = reinterpret_cast<const int4*>(x.wsum)[lb];
        const QxBlock& q = x.qx[lb];
        const u32x4 w = k.w ^ 0x88888888u;
        const u32x4 hv = {spread2(k.h.x), spread2(k.h.x >> 16), spread2(k.h.y),
                          spread2(k.h.y >> 16)};
        const int32_t p0 = nib_dot<0, 2>(w, q) + 16 * nib_dot<0, 2>(hv, q) - 24 * (ws.x + ws.y);
        const int32_t p1 = nib_dot<2, 2>(w, q) + 16 * nib_dot<2, 2>(hv, q) - 24 * (ws.z + ws.w);
        return x.sx[lb] * (__uint_as_float(k.s.x) * float(p0) + __uint_as_float(k.s.y) * float(p1));
    }
};

template <> struct RqFmt<kQ80> {
    static constexpr int kU = 2;
    struct Blk { u32x4 a, b; float s; };
    __device__ static void load(Blk& k, const RqArgs& a, size_t idx) {
        k.a = ld_stream4(a.quant + 2 * idx);
        k.b = ld_stream4(a.quant + 2 * idx + 1);
        k.s = __builtin_nontemporal_load(a.scale + idx);
    }
    __device__ static float dot(const Blk& k, const RqLds& x, uint32_t lb) {
        const u32x4* pl = reinterpret_cast<const u32x4*>(x.b8) + lb * 6;   // [plane][2] u32x4
        uint32_t d = 0;
#pragma unroll
        for (int p = 0; p < 3; ++p) {
            const u32x4 e0 = pl[2 * p], e1 = pl[2 * p + 1];
            int32_t s = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) s = __builtin_amdgcn_sdot4(int32_t(k.a[c]), int32_t(e0[c]), s, false);
#pragma unroll
            for (int c = 0; c < 4; ++c) s = __builtin_amdgcn_sdot4(int32_t(k.b[c]), int32_t(e1[c]), s, false);
            d += uint32_t(s) << (8 * p);
        }
        return x.sx[lb] * (k.s * float(int32_t(d)));
    }
};

// One wave = one task = (row group, k-chunk). As in the int4 matvec: three
// pipeline stages of kU blocks in flight; waves past the last group load
// group 0 and drop the result; SPLIT: partials, an arrival ticket, and the
// last chunk of the group sums the partials in ascending chunk order.
template <uint32_t T, bool SPLIT>
__global__ __launch_bounds__(kRqWaves * kWave) __attribute__((amdgpu_waves_per_eu(4)))
void mv_rq_kernel(RqArgs a) {
    using F = RqFmt<T>;
    constexpr int U = F::kU;
    extern __shared__ QxBlock smem_rq[];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t s    = blockIdx.x / a.wg_per_chunk;
    const uint32_t gg   = (blockIdx.x % a.wg_per_chunk) * kRqWaves + wave;
    const uint32_t kb0  = s * a.kpc;
    const uint32_t kb1  = min(kb0 + a.kpc, a.nkb);
    const uint32_t nkc  = kb1 - kb0;
    RqLds x;
    float* sx;
    if constexpr (T == kQ80) {
        uint32_t* pl = reinterpret_cast<uint32_t*>(smem_rq);
        sx = reinterpret_cast<float*>(pl + size_t(a.kpc) * 24);
        x = RqLds{nullptr, nullptr, pl, sx};
    } else {
        int32_t* ws = reinterpret_cast<int32_t*>(smem_rq + a.kpc);
        sx = reinterpret_cast<float*>(ws + size_t(a.kpc) * 4);
        x = RqLds{smem_rq, ws, nullptr, sx};
    }
    const float* xg = a.x + size_t(kb0) * kBlk;
    auto stage = [&](uint32_t i, float4 v0, float4 v1) {
        if constexpr (T == kQ80)
            stage_b8(const_cast<uint32_t*>(x.b8), sx, i, v0, v1);
        else
            stage_nib(const_cast<QxBlock*>(x.qx), const_cast<int32_t*>(x.wsum), sx, i, v0, v1);
    };
    for (uint32_t i = threadIdx.x + blockDim.x; i < nkc * 4; i += blockDim.x)
        stage(i, reinterpret_cast<const float4*>(xg)[2 * i], reinterpret_cast<const float4*>(xg)[2 * i + 1]);
    float4 xv0 = {0.0f, 0.0f, 0.0f, 0.0f}, xv1 = xv0;
    if (threadIdx.x < nkc * 4) {
        xv0 = reinterpret_cast<const float4*>(xg)[2 * threadIdx.x];
        xv1 = reinterpret_cast<const float4*>(xg)[2 * threadIdx.x + 1];
    }

    const bool active = gg < a.groups;
    const uint32_t gl = active ? gg : 0u;
    const size_t slot0 = size_t(gl) * a.nkb * kGrp + lane;
    const uint32_t klast = kb1 - 1;
    const uint32_t nst = (nkc + U - 1) / U;
    typename F::Blk buf[3][U];
    auto load_stage = [&](int r, uint32_t st) {
#pragma unroll
        for (int u = 0; u < U; ++u)
            F::load(buf[r][u], a, slot0 + size_t(min(kb0 + st * U + u, klast)) * kGrp);
    };
    auto mul_stage = [&](int r, uint32_t st, float& acc) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t lb = st * U + u;
            if (lb < nkc) acc += F::dot(buf[r][u], x, lb);
        }
    };
    load_stage(0, 0);
    load_stage(1, 1);
    load_stage(2, 2);
    if (threadIdx.x < nkc * 4) stage(threadIdx.x, xv0, xv1);
    __syncthreads();
    if (!active) return;

    float acc = 0.0f;
    uint32_t st = 0;
    for (; st + 6 <= nst; st += 3) {
        mul_stage(0, st, acc);
        __builtin_amdgcn_sched_barrier(0);
        load_stage(0, st + 3);
        __builtin_amdgcn_sched_barrier(0);
        mul_stage(1, st + 1, acc);
        __builtin_amdgcn_sched_barrier(0);
        load_stage(1, st + 4);
        __builtin_amdgcn_sched_barrier(0);
        mul_stage(2, st + 2, acc);
        __builtin_amdgcn_sched_barrier(0);
        load_stage(2, st + 5);
        __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t rem = nst - st;   // 0..5 stages left; buffers hold st .. st + 2
    if (rem > 0) {
        mul_stage(0, st, acc);
        if (rem > 3) load_stage(0, st + 3);
    }
    if (rem > 1) {
        mul_stage(1, st + 1, acc);
        if (rem > 4) load_stage(1, st + 4);
    }
    if (rem > 2) mul_stage(2, st + 2, acc);
    if (rem > 3) mul_stage(0, st + 3, acc);
    if (rem > 4) mul_stage(1, st + 4, acc);

    const uint32_t row = gl * kGrp + lane;
    if constexpr (!SPLIT) {
        if (row < a.rows) a.out[row] = acc;
        return;
    }
    const size_t stride = size_t(a.groups) * kGrp;
    st_dev(a.partial + size_t(s) * stride + size_t(gg) * kGrp + lane, acc);
    wait_mem();
    uint32_t old = 0;
    if (lane == 0) old = take_ticket(&a.tickets[gg]);
    old = __shfl(old, 0, kWave);
    if (old != a.split - 1) return;
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
    if (row < a.rows) a.out[row] = sum;
    if (lane == 0) st_dev(&a.tickets[gg], 0u);
}

bool native_type(uint32_t t) { return t == kQ80 || t == kQ50 || t == kQ4K || t == kQ6K; }

uint32_t native_block_elems(uint32_t t) { return (t == kQ4K || t == kQ6K) ? 256u : 32u; }
uint32_t native_block_bytes(uint32_t t) {
    return t == kQ80 ? 34u : t == kQ50 ? 22u : t == kQ4K ? 144u : 210u;
}

}  // namespace

// Workgroup tasks: one workgroup per (row group, k-chunk of at most 40
// k-blocks), its eight waves splitting the chunk's blocks (wave w takes
// blocks w, w + 8, ...) and meeting in LDS, summed in wave order. Wide,
// shallow shapes (Q5_0 6912 x 1152: 108 row groups, 36 k-blocks) take one
// chunk: no partials, no ticket. Narrow, deep ones (Q4_K / Q6_K 1152 x 6912:
// 18 row groups, 216 k-blocks) take at most eight chunks (SPLIT): the
// partials, an arrival ticket and one batch of partial loads by the last
// chunk, summed in ascending chunk order. The activations are loaded ahead
// of the weights.
constexpr int kRqWgWaves = 8;
constexpr int kRqWgBlk = 5;                                 // k-blocks per wave
constexpr uint32_t kRqWgChunk = kRqWgWaves * kRqWgBlk;      // k-blocks per chunk
constexpr uint32_t kRqWgMaxSplit = 8;

template <uint32_t T, bool SPLIT>
__global__ __launch_bounds__(kRqWgWaves * kWave) void mv_rq_wg_kernel(RqArgs a) {
    using F = RqFmt<T>;
    extern __shared__ QxBlock smem_rq[];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t gg = blockIdx.x % a.groups, s = blockIdx.x / a.groups;
    const uint32_t kb0 = s * a.kpc, nkc = min(a.kpc, a.nkb - kb0);
    RqLds x;
    float* sx;
    if constexpr (T == kQ80) {
        uint32_t* pl = reinterpret_cast<uint32_t*>(smem_rq);
        sx = reinterpret_cast<float*>(pl + size_t(a.kpc) * 24);
        x = RqLds{nullptr, nullptr, pl, sx};
    } else {
        int32_t* ws = reinterpret_cast<int32_t*>(smem_rq + a.kpc);
        sx = reinterpret_cast<float*>(ws + size_t(a.kpc) * 4);
        x = RqLds{smem_rq, ws, nullptr, sx};
    }
    float* red = reinterpret_cast<float*>(reinterpret_cast<char*>(smem_rq) +
                                          ((size_t(a.kpc) * kRqLdsPerBlock + 15u) & ~size_t(15)));
    const float4* x4 = reinterpret_cast<const float4*>(a.x + size_t(kb0) * kBlk);
    const bool stager = threadIdx.x < nkc * 4u;
    float4 xv0 = {0.0f, 0.0f, 0.0f, 0.0f}, xv1 = xv0;
    if (stager) {
        xv0 = x4[2 * threadIdx.x];
        xv1 = x4[2 * threadIdx.x + 1];
    }
    const size_t slot0 = (size_t(gg) * a.nkb + kb0) * kGrp + lane;
    typename F::Blk buf[kRqWgBlk];
#pragma unroll
    for (int r = 0; r < kRqWgBlk; ++r)
        F::load(buf[r], a, slot0 + size_t(min(wave + uint32_t(kRqWgWaves) * r, nkc - 1u)) * kGrp);
    if (stager) {
        if constexpr (T == kQ80)
            stage_b8(const_cast<uint32_t*>(x.b8), sx, threadIdx.x, xv0, xv1);
        else
            stage_nib(const_cast<QxBlock*>(x.qx), const_cast<int32_t*>(x.wsum), sx, threadIdx.x, xv0, xv1);
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < kRqWgBlk; ++r) {
        const uint32_t lb = wave + uint32_t(kRqWgWaves) * r;
        if (lb < nkc) acc += F::dot(buf[r], x, lb);
    }
    red[wave * kGrp + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    float y = 0.0f;
#pragma unroll
    for (int v = 0; v < kRqWgWaves; ++v) y += red[v * kGrp + lane];
    const uint32_t row = gg * kGrp + lane;
    if constexpr (!SPLIT) {
        if (row < a.rows) a.out[row] = y;
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
    float v[kRqWgMaxSplit];
#pragma unroll
    for (uint32_t p = 0; p < kRqWgMaxSplit; ++p) v[p] = p < a.split ? ld_dev(pp + size_t(p) * stride) : 0.0f;
    float sum = 0.0f;
#pragma unroll
    for (uint32_t p = 0; p < kRqWgMaxSplit; ++p)
        if (p < a.split) sum += v[p];
    if (row < a.rows) a.out[row] = sum;
    if (lane == 0) st_dev(&a.tickets[gg], 0u);
}

int launch_mv_rq(float* out, const float* x, const xp_rq_tensor& w, uint32_t split,
                 hipStream_t st, const char* who) {
    if (!out || !x) return set_error(XP_E_ARG, "%s: null pointer", who);
    xp_rq_layout l;
    if (xp_rq_layout_of(w.type, w.rows, w.cols, &l) != XP_OK) {
        const std::string why = xp_last_error();
        return set_error(XP_E_ARG, "%s: %s", who, why.c_str());
    }
    if (!w.quant || !w.scale || (l.high_bytes && !w.high) || (l.bias_bytes && !w.bias))
        return set_error(XP_E_ARG, "%s: a plane of the type-%u tensor is null", who, w.type);
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w.quant)) & 15u)
        return set_error(XP_E_ARG, "%s: in and quant must be 16-byte aligned", who);
    if ((reinterpret_cast<uintptr_t>(w.scale) | reinterpret_cast<uintptr_t>(w.high)) & 7u)
        return set_error(XP_E_ARG, "%s: scale and high must be 8-byte aligned", who);
    if (out == x) return set_error(XP_E_ARG, "%s: out aliases in", who);
    DeviceScratch* sc = scratch();
    if (!sc) return XP_E_HIP;
    RqArgs a{};
    a.out = out;
    a.x = x;
    a.quant = reinterpret_cast<const u32x4*>(w.quant);
    a.high = w.high;
    a.scale = w.scale;
    a.bias = w.bias;
    a.rows = w.rows;
    a.nkb = l.nkb;
    a.groups = l.padded_rows / kGrp;
    // Enough tasks for ~8 waves per CU, at most kRqMaxSplit chunks, and every
    // chunk's staged activations within 64 KiB of LDS.
    const uint32_t lds_min = (a.nkb * kRqLdsPerBlock + 65535u) / 65536u;
    const uint32_t n_cu = uint32_t(sc->n_cu > 0 ? sc->n_cu : 256);
    // Automatic plan for a shape narrower than eight waves per CU: workgroup
    // tasks, one chunk per row group when the whole k fits one (and the
    // groups alone give most CUs a task), else as many chunks as give every
    // CU a task, at most eight, each within kRqWgChunk blocks.
    if (split == 0 && a.groups < n_cu * 8u) {
        uint32_t sp = 1;
        if (a.nkb > kRqWgChunk || a.groups < 64) {
            sp = std::max(1u, std::min(kRqWgMaxSplit, n_cu / a.groups));
            sp = std::max(sp, (a.nkb + kRqWgChunk - 1) / kRqWgChunk);
        }
        if (sp <= kRqWgMaxSplit) {
            a.kpc = (a.nkb + sp - 1) / sp;
            a.split = (a.nkb + a.kpc - 1) / a.kpc;
            if (a.split > 1) {
                if (!ensure_partial(sc, size_t(a.split) * a.groups * kGrp)) return XP_E_NOMEM;
                if (!ensure_tickets(sc, a.groups)) return XP_E_NOMEM;
                a.partial = sc->partial;
                a.tickets = sc->tickets;
            }
            const size_t lds = ((size_t(a.kpc) * kRqLdsPerBlock + 15u) & ~size_t(15)) +
                               size_t(kRqWgWaves) * kGrp * sizeof(float);
            const dim3 grid(a.groups * a.split), block(kRqWgWaves * kWave);
#define XP_RQ_WG_LAUNCH(T)                                                                  \
    if (a.split > 1)                                                                        \
        hipLaunchKernelGGL((mv_rq_wg_kernel<T, true>), grid, block, lds, st, a);            \
    else                                                                                    \
        hipLaunchKernelGGL((mv_rq_wg_kernel<T, false>), grid, block, lds, st, a);
            switch (w.type) {
                case kQ80: XP_RQ_WG_LAUNCH(kQ80) break;
                case kQ50: XP_RQ_WG_LAUNCH(kQ50) break;
                case kQ4K: XP_RQ_WG_LAUNCH(kQ4K) break;
                default: XP_RQ_WG_LAUNCH(kQ6K) break;
            }
#undef XP_RQ_WG_LAUNCH
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return set_error(XP_E_HIP, "%s: launch -> %s", who, hipGetErrorString(e));
            return XP_OK;
        }
    }
    if (split == 0) {
        const uint32_t target = uint32_t(sc->n_cu > 0 ? sc->n_cu : 256) * 8u;
        split = (target + a.groups - 1) / a.groups;
        split = std::max(1u, std::min(split, kRqMaxSplit));
        split = std::max(split, lds_min);
    }
    split = std::min(split, a.nkb);
    if (split < lds_min)
        return set_error(XP_E_ARG, "%s: a k-chunk of %u blocks needs more than 64 KiB of LDS; "
                         "pass split >= %u", who, (a.nkb + split - 1) / split, lds_min);
    a.kpc = (a.nkb + split - 1) / split;
    a.split = (a.nkb + a.kpc - 1) / a.kpc;
    a.wg_per_chunk = (a.groups + kRqWaves - 1) / kRqWaves;
    if (a.split > 1) {
        if (!ensure_partial(sc, size_t(a.split) * a.groups * kGrp)) return XP_E_NOMEM;
        if (!ensure_tickets(sc, a.groups)) return XP_E_NOMEM;
        a.partial = sc->partial;
        a.tickets = sc->tickets;
    }
    const size_t lds = size_t(a.kpc) * kRqLdsPerBlock;
    const dim3 grid(a.wg_per_chunk * a.split), block(kRqWaves * kWave);
#define XP_RQ_LAUNCH(T)                                                                   \
    if (a.split > 1)                                                                      \
        hipLaunchKernelGGL((mv_rq_kernel<T, true>), grid, block, lds, st, a);             \
    else                                                                                  \
        hipLaunchKernelGGL((mv_rq_kernel<T, false>), grid, block, lds, st, a);
    switch (w.type) {
        case kQ80: XP_RQ_LAUNCH(kQ80) break;
        case kQ50: XP_RQ_LAUNCH(kQ50) break;
        case kQ4K: XP_RQ_LAUNCH(kQ4K) break;
        default: XP_RQ_LAUNCH(kQ6K) break;
    }
#undef XP_RQ_LAUNCH
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "%s: launch -> %s", who, hipGetErrorString(e));
    return XP_OK;
}

}  // namespace xp

using namespace xp;

extern "C" {

int xp_mv_rq(float* out, const float* in, const xp_rq_tensor* w, uint32_t split,
             xp_stream stream) {
    XP_REQUIRE(w, "null tensor");
    return launch_mv_rq(out, in, *w, split, as_stream(stream), "xp_mv_rq");
}

int xp_mv_rq_timed(float* out, const float* in, const xp_rq_tensor* ws, uint32_t ncopies,
                   uint32_t split, uint32_t iters, xp_stream stream, float* ms) {
    XP_REQUIRE(ws && ms && ncopies > 0 && iters > 0, "bad arguments");
    hipStream_t st = as_stream(stream);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    XP_HIP(hipEventCreate(&e0));
    XP_HIP(hipEventCreate(&e1));
    int rc = XP_OK;
    for (uint32_t i = 0; i < ncopies && rc == XP_OK; ++i)
        rc = launch_mv_rq(out, in, ws[i], split, st, "xp_mv_rq_timed");
    if (rc == XP_OK && hipStreamSynchronize(st) != hipSuccess) rc = set_error(XP_E_HIP, "sync");
    if (rc == XP_OK && hipEventRecord(e0, st) != hipSuccess) rc = set_error(XP_E_HIP, "event");
    for (uint32_t i = 0; i < iters && rc == XP_OK; ++i)
        rc = launch_mv_rq(out, in, ws[i % ncopies], split, st, "xp_mv_rq_timed");
    if (rc == XP_OK && hipEventRecord(e1, st) != hipSuccess) rc = set_error(XP_E_HIP, "event");
    if (rc == XP_OK && hipEventSynchronize(e1) != hipSuccess) rc = set_error(XP_E_HIP, "sync");
    if (rc == XP_OK && hipEventElapsedTime(ms, e0, e1) != hipSuccess)
        rc = set_error(XP_E_HIP, "elapsed");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

int xp_dequant_native(float* out, const void* src, uint32_t type, uint64_t n, xp_stream stream) {
    XP_REQUIRE(out && src, "null pointer");
    XP_REQUIRE(native_type(type), "type %u is not Q8_0, Q5_0, Q4_K or Q6_K", type);
    XP_REQUIRE(n % native_block_elems(type) == 0, "%llu elements are not whole blocks",
               static_cast<unsigned long long>(n));
    XP_REQUIRE((reinterpret_cast<uintptr_t>(src) & 1u) == 0, "src must be 2-byte aligned");
    if (n == 0) return XP_OK;
    const uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 65536);
    const auto* p = static_cast<const uint8_t*>(src);
    hipStream_t st = as_stream(stream);
    switch (type) {
        case kQ80: hipLaunchKernelGGL(dequant_native_kernel<kQ80>, dim3(blocks), dim3(256), 0, st, out, p, n); break;
        case kQ50: hipLaunchKernelGGL(dequant_native_kernel<kQ50>, dim3(blocks), dim3(256), 0, st, out, p, n); break;
        case kQ4K: hipLaunchKernelGGL(dequant_native_kernel<kQ4K>, dim3(blocks), dim3(256), 0, st, out, p, n); break;
        default: hipLaunchKernelGGL(dequant_native_kernel<kQ6K>, dim3(blocks), dim3(256), 0, st, out, p, n); break;
    }
    XP_LAUNCHED();
    return XP_OK;
}

int xp_mv_native(float* out, const float* in, const void* src, uint32_t type, uint32_t rows,
                 uint32_t cols, xp_stream stream) {
    XP_REQUIRE(out && in && src, "null pointer");
    XP_REQUIRE(native_type(type), "type %u is not Q8_0, Q5_0, Q4_K or Q6_K", type);
    XP_REQUIRE(rows > 0 && cols > 0 && cols % native_block_elems(type) == 0,
               "%u x %u: cols must be a positive multiple of %u", rows, cols,
               native_block_elems(type));
    XP_REQUIRE((reinterpret_cast<uintptr_t>(src) & 1u) == 0, "src must be 2-byte aligned");
    XP_REQUIRE((reinterpret_cast<uintptr_t>(in) & 15u) == 0, "in must be 16-byte aligned");
    XP_REQUIRE(out != in, "out aliases in");
    const size_t rb = size_t(cols / native_block_elems(type)) * native_block_bytes(type);
    const auto* p = static_cast<const uint8_t*>(src);
    const dim3 grid((rows + 3) / 4), block(256);
    hipStream_t st = as_stream(stream);
    switch (type) {
        case kQ80: hipLaunchKernelGGL(mv_native_kernel<kQ80>, grid, block, 0, st, out, in, p, rows, cols, rb); break;
        case kQ50: hipLaunchKernelGGL(mv_native_kernel<kQ50>, grid, block, 0, st, out, in, p, rows, cols, rb); break;
        case kQ4K: hipLaunchKernelGGL(mv_native_kernel<kQ4K>, grid, block, 0, st, out, in, p, rows, cols, rb); break;
        default: hipLaunchKernelGGL(mv_native_kernel<kQ6K>, grid, block, 0, st, out, in, p, rows, cols, rb); break;
    }
    XP_LAUNCHED();
    return XP_OK;
}

}  // extern "C"
