// Small kernels that exist only for the decode session's token step.
//
//  embed_norm       the token's embedding row (the model's fp32 row, or the
//                   tied int4 table's, dequantised) scaled by sqrt(hidden),
//                   and the first layer's input norm, in one launch — the
//                   reference forms the row on the CPU from the GGUF mapping
//                   and uploads it (decode.cpp:1618-1627); here the token id
//                   is read from device memory so a whole token step can be
//                   replayed from one captured graph.
//  norm_res_norm    x += rmsnorm(y) * (1 + w_post); out = rmsnorm(x) * (1 +
//                   w_pre): the post-sublayer norm, the residual add and the
//                   next sublayer's pre-norm of record_token
//                   (decode.cpp:1739-1751, 1668) in one workgroup.
//  advance          position += 1 after a step (the greedy step's argmax
//                   does it itself).
#include "xp_device.hpp"
#include "xp_launch.hpp"

namespace xp {

__device__ __forceinline__ float blk_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
    const int nw = (blockDim.x + kWave - 1) / kWave;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

// Element k of token tok's embedding row: the model's fp32 row when it has
// one, else the tied int4 table's column, dequantised; times embed_scale.
__device__ __forceinline__ float embed_value(uint32_t k, uint32_t tok, const u32x4* wq, const void* sc,
                                             int fmt, uint32_t hidden, uint32_t vocab, float embed_scale,
                                             const float* table) {
    if (table) return table[size_t(tok) * hidden + k] * embed_scale;
    const uint32_t nblk = hidden / kBlk, b = k / kBlk;
    const u32x4 w = wq[(size_t(tok / kGrp) * nblk + b) * kGrp + (tok % kGrp)];
    const uint32_t t = k % kBlk;
    const uint32_t word = (t < 8) ? w.x : (t < 16) ? w.y : (t < 24) ? w.z : w.w;
    const float q = float(int((word >> ((t & 7u) * 4u)) & 15u) - 8);
    float s;
    if (fmt == XP_SCALE_F32) {
        s = reinterpret_cast<const float*>(sc)[size_t(b) * vocab + tok];
    } else {
        const uint16_t h = reinterpret_cast<const uint16_t*>(sc)[(size_t(b / 4) * vocab + tok) * 4 +
                                                                 (b % 4)];
        s = (fmt == XP_SCALE_F16_QUAD) ? f16_bits_to_f32(h) : __uint_as_float(uint32_t(h) << 16);
    }
    return (q * s) * embed_scale;
}

// The embedding row and the first layer's input norm in one workgroup:
// x = the row, xn = rmsnorm(x) (1 + w_pre), the sums in norm_res_norm's order
// (the same bits as writing the row and then norm_res_norm without y).
// state[0] = position, state[1] = token to run.
__global__ __launch_bounds__(1024) void embed_norm_kernel(float* x, float* xn, const float* w_pre, float eps,
                                                          const u32x4* wq, const void* sc, int fmt,
                                                          uint32_t hidden, uint32_t vocab, float embed_scale,
                                                          const uint32_t* state, uint32_t* hist,
                                                          const float* table) {
    __shared__ float red[16];
    constexpr int kMaxPer = 8;   // hidden <= 8 * 1024
    const uint32_t pos = state[0];
    uint32_t tok = state[1];
    if (tok >= vocab) tok = 0;
    if (threadIdx.x == 0) hist[pos] = tok;
    float xv[kMaxPer];
    int c = 0;
    for (uint32_t i = threadIdx.x; i < hidden; i += blockDim.x, ++c) {
        xv[c] = embed_value(i, tok, wq, sc, fmt, hidden, vocab, embed_scale, table);
        x[i] = xv[c];
    }
    float ss = 0.0f;
    for (int j = 0; j < c; ++j) ss += xv[j] * xv[j];
    ss = blk_sum(ss, red);
    const float scale = rsq_hw(ss / float(hidden) + eps);
    c = 0;
    for (uint32_t i = threadIdx.x; i < hidden; i += blockDim.x, ++c)
        xn[i] = xv[c] * scale * (1.0f + w_pre[i]);
}

// y == nullptr: out = rmsnorm(x) * (1 + w_pre) only.
__global__ __launch_bounds__(1024) void norm_res_norm_kernel(float* x, const float* y,
                                                             const float* w_post,
                                                             const float* w_pre, float* out,
                                                             uint32_t n, float eps) {
    __shared__ float red[16];
    constexpr int kMaxPer = 8;   // n <= 8 * 1024
    float xv[kMaxPer];
    int c = 0;
    if (y) {
        float ss = 0.0f;
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) ss += y[i] * y[i];
        ss = blk_sum(ss, red);
        const float scale = rsq_hw(ss / float(n) + eps);
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x, ++c) {
            const float v = x[i] + y[i] * scale * (1.0f + w_post[i]);
            x[i] = v;
            xv[c] = v;
        }
    } else {
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x, ++c) xv[c] = x[i];
    }
    float ss = 0.0f;
    for (int j = 0; j < c; ++j) ss += xv[j] * xv[j];
    ss = blk_sum(ss, red);
    const float scale = rsq_hw(ss / float(n) + eps);
    c = 0;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x, ++c)
        out[i] = xv[c] * scale * (1.0f + w_pre[i]);
}

__global__ void advance_kernel(uint32_t* state) { state[0] += 1u; }

int launch_embed_norm(float* x, float* xn, const float* w_pre, float eps, const void* wq, const void* sc,
                      int fmt, uint32_t hidden, uint32_t vocab, float embed_scale, const uint32_t* state,
                      uint32_t* hist, const float* table, hipStream_t st) {
    if (hidden > 8 * 1024) return set_error(XP_E_ARG, "embed_norm: hidden=%u > 8192", hidden);
    hipLaunchKernelGGL(embed_norm_kernel, dim3(1), dim3(1024), 0, st, x, xn, w_pre, eps,
                       reinterpret_cast<const u32x4*>(wq), sc, fmt, hidden, vocab, embed_scale, state, hist,
                       table);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "embed_norm: launch -> %s", hipGetErrorString(e));
    return XP_OK;
}

int launch_norm_res_norm(float* x, const float* y, const float* w_post, const float* w_pre,
                         float* out, uint32_t n, float eps, hipStream_t st) {
    if (n > 8 * 1024) return set_error(XP_E_ARG, "norm_res_norm: n=%u > 8192", n);
    hipLaunchKernelGGL(norm_res_norm_kernel, dim3(1), dim3(1024), 0, st, x, y, w_post, w_pre, out,
                       n, eps);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "norm_res_norm: launch -> %s",
                                          hipGetErrorString(e));
    return XP_OK;
}

int launch_advance(uint32_t* state, hipStream_t st) {
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, st, state);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "advance: launch -> %s", hipGetErrorString(e));
    return XP_OK;
}

}  // namespace xp
