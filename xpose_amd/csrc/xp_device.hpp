// Device-side helpers shared by the gfx950 kernels: fp16/bf16 scale decode,
// the int4 block dot, and wave-level reductions. Wave size is 64 throughout.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>

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

// Cross-workgroup hand-off without an L2 flush. An agent-scope fence on
// gfx950 writes back and invalidates the whole L2 (buffer_wbl2 / buffer_inv
// sc1), which serialises when every wave does it. Instead, data another
// workgroup will read is stored with agent-scope relaxed atomics (sc1,
// written through to the device coherence point), the writer waits for its
// stores to complete before taking an arrival ticket, and the reader loads
// with agent-scope relaxed atomics (sc1, re-read from the coherence point).
__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
// Blocks until every memory operation this wave issued has completed.
__device__ __forceinline__ void wait_mem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Arrival ticket: returns the number of arrivals before this one.
__device__ __forceinline__ uint32_t take_ticket(uint32_t* t) {
    return __hip_atomic_fetch_add(t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave-wide sum / max via DPP-backed shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// gelu_pytorch_tanh with the reference's clamped-exp tanh
// (kernels/llm_transformer.cl:213-231). expf is the device libm exp.
__device__ __forceinline__ float gelu_tanh(float g) {
    float z = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    z = fminf(fmaxf(z, -10.0f), 10.0f);
    const float e = expf(-2.0f * z);
    const float t = (1.0f - e) / (1.0f + e);
    return 0.5f * g * (1.0f + t);
}

}  // namespace xp
