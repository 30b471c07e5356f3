// Device-side helpers shared by the gfx950 kernels: fp16/bf16 scale decode,
// the int4 block dot, and wave-level reductions. Wave size is 64 throughout.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <type_traits>

namespace xp {

constexpr int kWave = 64;

// Native clang vectors: the nontemporal-load builtin needs them (HIP's uint4
// is a struct).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Streaming loads: weights are read exactly once per token.
__device__ __forceinline__ u32x4 ld_stream4(const u32x4* p) {
    return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ u32x2 ld_stream2(const u32x2* p) {
    return __builtin_nontemporal_load(p);
}
// Global-address-space views. Pointers read out of device memory (a layer
// table) are generic to the compiler, which then emits FLAT accesses; FLAT
// loads also count against lgkmcnt, so every later LDS or scalar wait would
// wait for them. These casts keep such accesses on the global path.
#define XP_GLOBAL __attribute__((address_space(1)))
__device__ __forceinline__ u32x4 ldg_stream4(const u32x4* p) {
    return __builtin_nontemporal_load((const XP_GLOBAL u32x4*)p);
}
__device__ __forceinline__ u32x2 ldg_stream2(const u32x2* p) {
    return __builtin_nontemporal_load((const XP_GLOBAL u32x2*)p);
}
__device__ __forceinline__ u32x4 ldg4(const void* p) { return *(const XP_GLOBAL u32x4*)p; }
__device__ __forceinline__ uint32_t ldg32(const void* p) { return *(const XP_GLOBAL uint32_t*)p; }
__device__ __forceinline__ uint16_t ldg16(const void* p) { return *(const XP_GLOBAL uint16_t*)p; }
__device__ __forceinline__ float ldgf(const float* p) { return *(const XP_GLOBAL float*)p; }
__device__ __forceinline__ void stg16(void* p, uint16_t v) { *(XP_GLOBAL uint16_t*)p = v; }

constexpr uint32_t kBlk = 32;   // quantisation block along k (BLK, llm_matvec.cl:25)
constexpr uint32_t kGrp = 64;   // KM4 column-group width (GRP, llm_matvec.cl:26)

// fp16 bits -> fp32. The hardware conversion is exact for every finite fp16
// and for +-inf, which is what the reference's bit-surgery decoder computes
// (kernels/llm_quant.cl:56-77); NaNs stay NaNs.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(h & 0xFFFFu)));
}

// bf16 is the top half of an fp32 word (bf16lo/bf16hi, llm_matvec.cl:407-408).
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// fp32 -> fp16 bits, round to nearest even (v_cvt_f16_f32 under the default
// round-to-nearest mode).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __half_as_ushort(__float2half_rn(f));
}

// Activation staging. Each workgroup stores its k-chunk of x in LDS as 20-bit
// block fixed point: for block b, sx_b = max|x| / 2^18 and q_k = rint(x_k /
// sx_b), so |q_k| <= 2^18 and |x_k - sx_b q_k| <= 2^-19 max|x|. q_k is kept as
// five planes of signed 4-bit digits (q = sum_p d_p 16^p, d_p in [-8, 7]):
// plane p, word c of a block packs the digits of k = 32b + 8c .. 32b + 8c + 7
// at nibble positions 0..7, which are the positions the KM4 word gives the
// weights of those k. The signed weight nibble - 8 is (nibble ^ 8) read as a
// two's-complement nibble, so one v_dot8_i32_i4 per (word, plane) multiplies
// eight weights by eight digits exactly, and the block product
// sum_k (n_k - 8) q_k is an exact int32 (|.| <= 2^26). Per block that is 4
// XORs, 20 dot8 and 4 shift-adds for 2048 multiply-adds per wave, against
// two conversions and one FMA per weight in fp32.
#ifndef XP_QX_PLANES
#define XP_QX_PLANES 5
#endif
constexpr int      kQxPlanes = XP_QX_PLANES;
static_assert(kQxPlanes == 4 || kQxPlanes == 5, "16- or 20-bit block fixed point");
constexpr float    kQxRange  = kQxPlanes == 5 ? 262144.0f : 16384.0f;   // 2^(4 planes - 2)
constexpr uint32_t kQxBias   = kQxPlanes == 5 ? 0x88888u : 0x8888u;     // 8 * sum of 16^p

struct QxBlock {
    u32x4 p[kQxPlanes];
};

// sum_k (nibble_k - 8) * q_k over one block, exact. Horner's rule over the
// digit planes in two chains (even and odd planes, 8-bit steps): each plane's
// four dot8 accumulate onto the chain so far shifted left by 8, so no
// per-plane zeroing, shift and add. |sum over one plane| <= 32 * 8 * 8 =
// 2048, so every partial fits in int32.
__device__ __forceinline__ int32_t plane_dot(u32x4 w, u32x4 q, int32_t acc) {
    acc = __builtin_amdgcn_sdot8(int32_t(w.x), int32_t(q.x), acc, false);
    acc = __builtin_amdgcn_sdot8(int32_t(w.y), int32_t(q.y), acc, false);
    acc = __builtin_amdgcn_sdot8(int32_t(w.z), int32_t(q.z), acc, false);
    return __builtin_amdgcn_sdot8(int32_t(w.w), int32_t(q.w), acc, false);
}
// block_dot_signed: w holds two's-complement nibbles (the stored nibbles
// xor 0x88888888); block_dot takes the stored (biased) nibbles.
__device__ __forceinline__ int32_t block_dot_signed(u32x4 w, const QxBlock& q) {
    constexpr int PE = (kQxPlanes - 1) & ~1, PO = (kQxPlanes - 2) | 1;   // top even / odd plane
    int32_t e = plane_dot(w, q.p[PE], 0);
#pragma unroll
    for (int p = PE - 2; p >= 0; p -= 2) e = plane_dot(w, q.p[p], e * 256);
    int32_t o = plane_dot(w, q.p[PO], 0);
#pragma unroll
    for (int p = PO - 2; p >= 1; p -= 2) o = plane_dot(w, q.p[p], o * 256);
    return e + o * 16;
}
__device__ __forceinline__ int32_t block_dot(u32x4 w, const QxBlock& q) {
    return block_dot_signed(w ^ 0x88888888u, q);
}

// The dot of one block with the staged planes, its activation words taken
// from the lanes of the row: lane j < 2 P of each 16-lane row holds words
// 2 j, 2 j + 1 of the block's 4 P plane words (plane p's word c is word
// 4 p + c), and v_dot8c_i32_i4 with DPP row_newbcast:n reads lane n of the
// row. A wave's lanes then read 8 bytes each from LDS for a block, not its
// 16 P bytes. (The DPP form is inline assembly: the compiler does not fold a
// DPP move into v_dot8c. Its sources come straight from LDS loads; see
// the callers for the exec hazard.)
template <int N>
__device__ __forceinline__ int32_t dot8_bc(int32_t acc, uint32_t a, uint32_t w);
#define XP_DOT8_BC(N)                                                                               \
    template <>                                                                                    \
    __device__ __forceinline__ int32_t dot8_bc<N>(int32_t acc, uint32_t a, uint32_t w) {           \
        asm("v_dot8c_i32_i4_dpp %0, %1, %2 row_newbcast:" #N " row_mask:0xf bank_mask:0xf"         \
            : "+v"(acc)                                                                            \
            : "v"(a), "v"(w));                                                                     \
        return acc;                                                                                \
    }
XP_DOT8_BC(0)
XP_DOT8_BC(1)
XP_DOT8_BC(2)
XP_DOT8_BC(3)
XP_DOT8_BC(4)
XP_DOT8_BC(5)
XP_DOT8_BC(6)
XP_DOT8_BC(7)
XP_DOT8_BC(8)
XP_DOT8_BC(9)
#undef XP_DOT8_BC
// Word C of plane P (word 4 P + C: lane 2 P + C / 2 of the row, component C % 2).
template <int P, int C>
__device__ __forceinline__ int32_t wdot_bc(int32_t acc, u32x4 w, u32x2 a) {
    static_assert(P >= 0 && P < kQxPlanes && C >= 0 && C < 4, "plane word");
    const uint32_t wv = C == 0 ? w.x : C == 1 ? w.y : C == 2 ? w.z : w.w;
    return dot8_bc<2 * P + C / 2>(acc, C % 2 ? a.y : a.x, wv);
}
// sum_k w_k q_k = sum_p 16^p D_p (D_p the dot with digit plane p) for
// two's-complement nibbles w, over NB = 1 or 2 blocks at once, in three
// chains a block: X = D_{P-1} 2^12 + D_{P-4}, Y = D_{P-2} 2^12 + D_{P-5}
// (absent when P = 4), Z = D_{P-3}, combined as 16^(P-4) X + ... below.
// The chains of both blocks are interleaved word by word, so consecutive
// dots of one chain are at least four instructions apart: no wait states
// for the compiler to insert (it keeps two between a VALU write and any
// operand of a following DPP operation in inline assembly). |D_p| <= 2^11.
template <int NB>
__device__ __forceinline__ void block_dot_bc(const u32x4 (&w)[NB], const u32x2 (&a)[NB], int32_t (&out)[NB]) {
    static_assert(kQxPlanes == 5 || kQxPlanes == 4, "4 or 5 digit planes");
    constexpr int P = kQxPlanes;
    int32_t X[NB], Y[NB], Z[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) X[b] = Y[b] = Z[b] = 0;
    // first pass: planes P - 1, P - 2, P - 3
    auto round1 = [&](auto cc) {
        constexpr int C = decltype(cc)::value;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            X[b] = wdot_bc<P - 1, C>(X[b], w[b], a[b]);
            Y[b] = wdot_bc<P - 2, C>(Y[b], w[b], a[b]);
            Z[b] = wdot_bc<P - 3, C>(Z[b], w[b], a[b]);
        }
    };
    round1(std::integral_constant<int, 0>{});
    round1(std::integral_constant<int, 1>{});
    round1(std::integral_constant<int, 2>{});
    round1(std::integral_constant<int, 3>{});
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        X[b] <<= 12;
        if constexpr (P == 5) Y[b] <<= 12;
    }
    // second pass: plane P - 4 onto X, plane P - 5 (P = 5) onto Y
    auto round2 = [&](auto cc) {
        constexpr int C = decltype(cc)::value;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            X[b] = wdot_bc<P - 4, C>(X[b], w[b], a[b]);
            if constexpr (P == 5) Y[b] = wdot_bc<0, C>(Y[b], w[b], a[b]);
        }
    };
    round2(std::integral_constant<int, 0>{});
    round2(std::integral_constant<int, 1>{});
    round2(std::integral_constant<int, 2>{});
    round2(std::integral_constant<int, 3>{});
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if constexpr (P == 5) out[b] = (X[b] << 4) + Y[b] + (Z[b] << 8);   // 16 X + Y + 256 Z
        else out[b] = X[b] + (Y[b] << 8) + (Z[b] << 4);                  // X + 256 Y + 16 Z
    }
}

// Quantises eight consecutive activations (task i = (block i/4, word i%4))
// into the five digit-plane words of that block and, for word 0, the block
// scale. The four tasks of a block are adjacent lanes of one wave.
__device__ __forceinline__ void stage_x8(QxBlock* qx, float* sx, uint32_t i, float4 v0,
                                         float4 v1) {
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[e]));
    // max over the block's four tasks (one lane quad): quad_perm xor 1, xor 2
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    const float r = m > 0.0f ? kQxRange / m : 0.0f;
    uint32_t t[8];
    // q + bias has hex digits d_p + 8; xor-ing the bias back gives each
    // digit as a two's-complement nibble.
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = uint32_t(__float2int_rn(v[e] * r) + int32_t(kQxBias)) ^ kQxBias;
    const uint32_t lb = i >> 2, c = i & 3u;
#pragma unroll
    for (int p = 0; p < kQxPlanes; ++p) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) word |= ((t[e] >> (4 * p)) & 15u) << (4 * e);
        reinterpret_cast<uint32_t*>(&qx[lb].p[p])[c] = word;
    }
    if (c == 0) sx[lb] = m * (1.0f / kQxRange);
}

// Cross-workgroup hand-off without an L2 flush. An agent-scope fence on
// gfx950 writes back and invalidates the whole L2 (buffer_wbl2 / buffer_inv
// sc1), which serialises when every wave does it. Instead, data another
// workgroup will read is stored with agent-scope relaxed atomics (sc1,
// written through to the device coherence point), the writer waits for its
// stores to complete before taking an arrival ticket, and the reader loads
// with agent-scope relaxed atomics (sc1, re-read from the coherence point).
__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store((XP_GLOBAL float*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
    __hip_atomic_store((XP_GLOBAL uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load((XP_GLOBAL float*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
    return __hip_atomic_load((XP_GLOBAL uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev64(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store((XP_GLOBAL unsigned long long*)p, v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_dev64(const unsigned long long* p) {
    return __hip_atomic_load((XP_GLOBAL unsigned long long*)p, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
// v through an opaque copy in a vector register. A variable that is a
// loaded value on one path and v on the other then has no constant input,
// and the compiler leaves an operation on it where the source puts it (with
// a constant input it folds the operation into the loading branch, and the
// wait for the load lands right after the load).
template <typename T>
__device__ __forceinline__ T opaque_v(T v) {
    asm volatile("" : "+v"(v));
    return v;
}

// threadIdx.x through an opaque copy: values derived from it are computed
// where they are used, not hoisted out of an enclosing loop by the compiler
// (a persistent kernel that runs many different tiles in a loop would
// otherwise keep every tile's per-thread offsets live at once).
__device__ __forceinline__ uint32_t opaque_tid() {
    uint32_t v = threadIdx.x;
    asm volatile("" : "+v"(v));
    return v;
}

// A store that is plain (DEV false) or device-scope (DEV true: read by
// other workgroups of the same launch after a completion signal); 16 bytes
// as two 8-byte device-scope stores.
template <bool DEV>
__device__ __forceinline__ void st_f(float* p, float v) {
    if constexpr (DEV) st_dev(p, v);
    else *p = v;
}
template <bool DEV>
__device__ __forceinline__ void st_u4(u32x4* p, u32x4 v) {
    if constexpr (DEV) {
        unsigned long long* q = reinterpret_cast<unsigned long long*>(p);
        st_dev64(q, (static_cast<unsigned long long>(v.y) << 32) | v.x);
        st_dev64(q + 1, (static_cast<unsigned long long>(v.w) << 32) | v.z);
    } else {
        *p = v;
    }
}

// Raw buffer resources for 16-byte device-scope accesses. Cache policy sc1
// (aux 16) writes through to, and reads from, the point where all XCDs are
// coherent; word 3 describes a raw (untyped, unswizzled) gfx9 buffer.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kAuxDev    = 16;
constexpr int kRsrcWord3 = 0x00020000;
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), short(0), int(bytes), kRsrcWord3);
}
__device__ __forceinline__ u32x4 ld_dev16(rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, int(byte_off), 0, kAuxDev);
}
// Blocks until every memory operation this wave issued has completed.
__device__ __forceinline__ void wait_mem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Arrival ticket: returns the number of arrivals before this one.
__device__ __forceinline__ uint32_t take_ticket(uint32_t* t) {
    return __hip_atomic_fetch_add((XP_GLOBAL uint32_t*)t, 1u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
}

// Wave-wide sum / max with DPP row operations (a few cycles per step, no LDS
// round trip): xor 1 and xor 2 inside quads, the half-row and row mirrors
// for 8 and 16 lanes, then row_bcast:15 / row_bcast:31 fold the four rows
// into lane 63, whose value is read back as a wave-uniform scalar.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float v, float old) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL,
                                                      ROW_MASK, 0xF, false));
}
// Sum over each row of 16 lanes, left in every lane of the row.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1, 0xF>(v, 0.0f);    // quad_perm [1,0,3,2]
    v += dpp_f<0x4E, 0xF>(v, 0.0f);    // quad_perm [2,3,0,1]
    v += dpp_f<0x141, 0xF>(v, 0.0f);   // row_half_mirror
    v += dpp_f<0x140, 0xF>(v, 0.0f);   // row_mirror
    return v;
}
// x + (x of lane ^ 32) through v_permlane32_swap (a VALU op; ds_bpermute
// would take the LDS pipe): the swap of x with itself hands lane l < 32
// (x[l], x[l + 32]) and lane l + 32 (x[l], x[l + 32]), so every lane gets
// the pair's sum, bit-identical to x + __shfl_xor(x, 32) (fp addition
// commutes).
__device__ __forceinline__ float add_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The value of lane l + 32 in lanes l < 32 (lanes 32..63 get their own).
__device__ __forceinline__ float from_lane_plus32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[1]);
}
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    v += dpp_f<0x142, 0xA>(v, 0.0f);   // row_bcast:15 -> rows 1, 3
    v += dpp_f<0x143, 0xC>(v, 0.0f);   // row_bcast:31 -> rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Lanes a step does not write read -inf, the max identity.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1, 0xF>(v, -INFINITY));
    v = fmaxf(v, dpp_f<0x4E, 0xF>(v, -INFINITY));
    v = fmaxf(v, dpp_f<0x141, 0xF>(v, -INFINITY));
    v = fmaxf(v, dpp_f<0x140, 0xF>(v, -INFINITY));
    v = fmaxf(v, dpp_f<0x142, 0xA>(v, -INFINITY));
    v = fmaxf(v, dpp_f<0x143, 0xC>(v, -INFINITY));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// (value, index) argmax step: larger value wins, then the lower index
// (kernels/llm_sampling.cl:50-56).
__device__ __forceinline__ void am_better(float& bv, uint32_t& bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__device__ __forceinline__ void am_wave(float& bv, uint32_t& bi) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v = __shfl_xor(bv, o, kWave);
        const uint32_t i = __shfl_xor(bi, o, kWave);
        am_better(bv, bi, v, i);
    }
}

// gelu_pytorch_tanh with the reference's clamped-exp tanh
// (kernels/llm_transformer.cl:213-231). expf is the device libm exp; the
// quotient uses the hardware reciprocal (1 ulp), not a correctly rounded
// division.
// The hardware reciprocal and reciprocal square root (v_rcp_f32, v_rsq_f32:
// about 1 ulp) and e^v as 2^(v log2 e) on v_exp_f32 (relative error ~1e-6
// for |v| <= 20, from the rounding of the product), for the latency-bound
// kernels: each replaces a correctly rounded sequence of 15-30 dependent
// instructions. exp_hw is used where v <= 0 (softmax weights, rescale
// factors) or |v| <= 20 (GeGLU).
__device__ __forceinline__ float rcp_hw(float v) { return __builtin_amdgcn_rcpf(v); }
__device__ __forceinline__ float rsq_hw(float v) { return __builtin_amdgcn_rsqf(v); }
__device__ __forceinline__ float exp_hw(float v) { return __builtin_amdgcn_exp2f(v * 1.4426950408889634f); }

__device__ __forceinline__ float gelu_tanh(float g) {
    float z = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    z = fminf(fmaxf(z, -10.0f), 10.0f);
    const float e = expf(-2.0f * z);
    const float t = (1.0f - e) * __builtin_amdgcn_rcpf(1.0f + e);
    return 0.5f * g * (1.0f + t);
}
// The same GELU on exp_hw / rcp_hw (the decode kernels' critical paths).
__device__ __forceinline__ float gelu_hw(float g) {
    float z = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    z = fminf(fmaxf(z, -10.0f), 10.0f);
    const float e = exp_hw(-2.0f * z);
    const float t = (1.0f - e) * rcp_hw(1.0f + e);
    return 0.5f * g * (1.0f + t);
}

}  // namespace xp
