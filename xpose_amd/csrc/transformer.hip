// The non-matvec ops of the decode step (kernels/llm_transformer.cl): Gemma
// RMSNorm, QK-norm + RoPE + fp16 KV append (fused), split-span decode
// attention over the fp16 cache, GeGLU and the residual add.
//
// Each op here is one launch; the reference needs two to seven dispatches for
// the same work because it has no workgroup-shared memory
// (llm_transformer.cl:10-19). On gfx950 a 1152-element reduction is one
// workgroup with LDS, so the two-pass RMSNorm (rmsnorm_sumsq +
// rmsnorm_apply_gemma) becomes one kernel, and the six per-layer QK-norm /
// RoPE / kv_append dispatches become one.
#include "xp_device.hpp"
#include "xp_launch.hpp"

#include <cmath>

namespace xp {

// theta^(-2d/head_dim) for d < head_dim/2, evaluated on the host with the
// reference's formula exp2(-log2(theta) * frac) (llm_transformer.cl:168-169),
// passed by value so a captured launch replays it unchanged.
struct RopeFreq {
    float inv[kMaxHeadDim / 2];
};

static void rope_freq(RopeFreq& f, uint32_t head_dim, float theta) {
    for (uint32_t d = 0; d < head_dim / 2; ++d) {
        const float frac = float(2u * d) / float(head_dim);
        f.inv[d] = std::exp2f(-std::log2f(theta) * frac);
    }
}

// Block-wide sum for blockDim.x <= 1024, result broadcast to every thread.
__device__ __forceinline__ float block_sum(float v, float* red) {
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

// ---- RMSNorm (Gemma (1 + w)), one workgroup --------------------------------
__global__ __launch_bounds__(1024) void rmsnorm_gemma_kernel(float* out, const float* in,
                                                             const float* w, uint32_t n,
                                                             float eps) {
    __shared__ float red[16];
    float ss = 0.0f;
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) ss += in[k] * in[k];
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / float(n) + eps);
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) out[i] = in[i] * scale * (1.0f + w[i]);
}

// ---- per-head RMSNorm (QK-norm), one workgroup per head --------------------
__global__ __launch_bounds__(256) void rmsnorm_heads_kernel(float* out, const float* in,
                                                            const float* w, uint32_t head_dim,
                                                            float eps) {
    __shared__ float red[16];
    const float* x = in + size_t(blockIdx.x) * head_dim;
    float ss = 0.0f;
    for (uint32_t k = threadIdx.x; k < head_dim; k += blockDim.x) ss += x[k] * x[k];
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / float(head_dim) + eps);
    for (uint32_t d = threadIdx.x; d < head_dim; d += blockDim.x)
        out[size_t(blockIdx.x) * head_dim + d] = x[d] * scale * (1.0f + w[d]);
}

// ---- RoPE, rotate-half, in place -------------------------------------------
__device__ __forceinline__ void rope_pair(float& lo, float& hi, float inv, uint32_t pos) {
    const float ang = float(pos) * inv;
    float s, c;
    sincosf(ang, &s, &c);
    const float a = lo, b = hi;
    lo = a * c - b * s;
    hi = a * s + b * c;
}

__global__ void rope_kernel(float* x, uint32_t n_heads, uint32_t head_dim, uint32_t pos,
                            RopeFreq f) {
    const uint32_t half = head_dim >> 1;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_heads * half) return;
    const uint32_t h = i / half, d = i - h * half;
    const size_t base = size_t(h) * head_dim + d;
    float lo = x[base], hi = x[base + half];
    rope_pair(lo, hi, f.inv[d], pos);
    x[base] = lo;
    x[base + half] = hi;
}

// ---- fused QK-norm + RoPE + fp16 KV append ----------------------------------
// Workgroup h < n_heads: q head h. n_heads <= h < n_heads + kv_heads: k head
// (normed, rotated, stored to k_out and kcache[pos]) and the matching v head
// (stored to vcache[pos]). One thread per pair (d, d + head_dim/2).

__global__ __launch_bounds__(256) void qk_norm_rope_append_kernel(QkArgs a, RopeFreq f) {
    __shared__ float red[16];
    const uint32_t half = a.head_dim >> 1;
    const uint32_t pos = a.pos_dev ? *a.pos_dev : a.pos;
    const bool is_q = blockIdx.x < a.n_heads;
    const uint32_t h = is_q ? blockIdx.x : blockIdx.x - a.n_heads;
    const float* x = (is_q ? a.q_raw : a.k_raw) + size_t(h) * a.head_dim;
    const float* w = is_q ? a.qw : a.kw;
    const uint32_t d = threadIdx.x;   // pair index, blockDim.x == half
    float lo = x[d], hi = x[d + half];
    const float ss = block_sum(lo * lo + hi * hi, red);
    const float scale = 1.0f / sqrtf(ss / float(a.head_dim) + a.eps);
    lo = lo * scale * (1.0f + w[d]);
    hi = hi * scale * (1.0f + w[d + half]);
    rope_pair(lo, hi, f.inv[d], pos);
    const size_t o = size_t(h) * a.head_dim;
    if (is_q) {
        a.q_out[o + d] = lo;
        a.q_out[o + d + half] = hi;
    } else {
        a.k_out[o + d] = lo;
        a.k_out[o + d + half] = hi;
        const size_t c = (size_t(pos) * a.kv_heads + h) * a.head_dim;
        a.kcache[c + d] = f32_to_f16_bits(lo);
        a.kcache[c + d + half] = f32_to_f16_bits(hi);
        const float* v = a.v + o;
        a.vcache[c + d] = f32_to_f16_bits(v[d]);
        a.vcache[c + d + half] = f32_to_f16_bits(v[d + half]);
    }
}

// ---- decode attention (split-span, fp16 KV) ----------------------------------
// Grid: (nsplit, kv_heads). Workgroup (s, g) scores keys
// [kv_start + s*chunk, ...) against the `group` query heads that share kv head
// g, reading each key and value once (the mq4 idea, llm_transformer.cl:
// 418-464, 499-557). It writes per-split (max, sum of exp, unnormalised o);
// the last workgroup of kv head g to finish (arrival ticket) combines the
// splits in ascending order — the online-softmax rescale of
// softmax_rows_finish (llm_transformer.cl:385-405).
constexpr int kAttnThreads = 256;
constexpr int kAttnChunk   = 32;    // keys per workgroup
constexpr int kAttnMaxGrp  = 8;     // query heads per kv head


__device__ __forceinline__ void attn_range(const AttnArgs& a, uint32_t& span, uint32_t& kv0) {
    if (a.pos_dev) {
        const uint32_t seq = *a.pos_dev + 1u;
        kv0 = (a.window == 0 || seq <= a.window) ? 0u : seq - a.window;
        span = seq - kv0;
    } else {
        span = a.span;
        kv0 = a.kv_start;
    }
}

__global__ __launch_bounds__(kAttnThreads) void attention_decode_kernel(AttnArgs a) {
    __shared__ float qs[kAttnMaxGrp * kMaxHeadDim];
    __shared__ float ps[kAttnMaxGrp * kAttnChunk];
    __shared__ float stat[kAttnMaxGrp * 2];
    __shared__ uint32_t last;
    uint32_t span, kv0;
    attn_range(a, span, kv0);
    const uint32_t g = blockIdx.y, s = blockIdx.x;
    const uint32_t G = a.group, hd = a.head_dim;
    const uint32_t chunk = (span + a.nsplit - 1) / a.nsplit;
    const uint32_t j0 = s * chunk;
    const uint32_t j1 = min(j0 + chunk, span);
    const uint32_t nk = j1 > j0 ? j1 - j0 : 0;
    const uint32_t tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const uint32_t rowlen = 2 + hd;
    float* part = a.part + (size_t(g) * a.nsplit + s) * G * rowlen;

    for (uint32_t i = tid; i < G * hd; i += blockDim.x)
        qs[i] = a.q[size_t(g) * G * hd + i];   // heads g*G .. g*G+G-1 are contiguous
    __syncthreads();

    // Scores: each wave takes keys j0+wave, j0+wave+4, ...; a lane covers
    // head_dim/64 consecutive dims of the key.
    const uint32_t per = hd / kWave;   // dims per lane (4 for head_dim 256)
    for (uint32_t jj = wave; jj < nk; jj += kAttnThreads / kWave) {
        const uint16_t* kr = a.kc + (size_t(kv0 + j0 + jj) * a.kv_heads + g) * hd + lane * per;
        float kf[kMaxHeadDim / kWave];
        for (uint32_t e = 0; e < per; ++e) kf[e] = f16_bits_to_f32(kr[e]);
        for (uint32_t h = 0; h < G; ++h) {
            float acc = 0.0f;
            for (uint32_t e = 0; e < per; ++e) acc = fmaf(qs[h * hd + lane * per + e], kf[e], acc);
            acc = wave_sum(acc);
            if (lane == 0) ps[h * kAttnChunk + jj] = acc * a.scale;
        }
    }
    __syncthreads();
    // Chunk softmax statistics per head (unnormalised).
    if (tid < G) {
        float m = -INFINITY;
        for (uint32_t jj = 0; jj < nk; ++jj) m = fmaxf(m, ps[tid * kAttnChunk + jj]);
        float l = 0.0f;
        for (uint32_t jj = 0; jj < nk; ++jj) {
            const float e = expf(ps[tid * kAttnChunk + jj] - m);
            ps[tid * kAttnChunk + jj] = e;
            l += e;
        }
        stat[2 * tid] = m;
        stat[2 * tid + 1] = l;
    }
    __syncthreads();
    // Weighted values: thread d accumulates dim d for every head.
    for (uint32_t d = tid; d < hd; d += blockDim.x) {
        float o[kAttnMaxGrp];
        for (uint32_t h = 0; h < G; ++h) o[h] = 0.0f;
        for (uint32_t jj = 0; jj < nk; ++jj) {
            const float v = f16_bits_to_f32(a.vc[(size_t(kv0 + j0 + jj) * a.kv_heads + g) * hd + d]);
            for (uint32_t h = 0; h < G; ++h) o[h] = fmaf(ps[h * kAttnChunk + jj], v, o[h]);
        }
        for (uint32_t h = 0; h < G; ++h) part[h * rowlen + 2 + d] = o[h];
    }
    if (tid < G) {
        part[tid * rowlen] = stat[2 * tid];
        part[tid * rowlen + 1] = stat[2 * tid + 1];
    }

    // Last workgroup of this kv head combines every split.
    __threadfence();
    __syncthreads();
    if (tid == 0) last = atomicAdd(&a.tickets[g], 1u);
    __syncthreads();
    if (last != a.nsplit - 1) return;
    __threadfence();
    const float* base = a.part + size_t(g) * a.nsplit * G * rowlen;
    for (uint32_t i = tid; i < G * hd; i += blockDim.x) {
        const uint32_t h = i / hd, d = i % hd;
        float M = -INFINITY;
        for (uint32_t p = 0; p < a.nsplit; ++p) {
            const float* r = base + (size_t(p) * G + h) * rowlen;
            if (__builtin_nontemporal_load(r + 1) > 0.0f) M = fmaxf(M, __builtin_nontemporal_load(r));
        }
        float L = 0.0f, o = 0.0f;
        for (uint32_t p = 0; p < a.nsplit; ++p) {
            const float* r = base + (size_t(p) * G + h) * rowlen;
            const float l = __builtin_nontemporal_load(r + 1);
            if (!(l > 0.0f)) continue;
            const float f = expf(__builtin_nontemporal_load(r) - M);
            L += l * f;
            o += __builtin_nontemporal_load(r + 2 + d) * f;
        }
        a.out[(size_t(g) * G + h) * hd + d] = o / L;
    }
    if (tid == 0) a.tickets[g] = 0u;
}

// ---- elementwise ------------------------------------------------------------
__global__ void geglu_kernel(float* out, const float* gate, const float* up, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = gelu_tanh(gate[i]) * up[i];
}

__global__ void add_residual_kernel(float* x, const float* y, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] += y[i];
}

__global__ void kv_append_f16_kernel(uint16_t* cache, const float* src, uint32_t n, uint32_t pos) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) cache[size_t(pos) * n + i] = f32_to_f16_bits(src[i]);
}

// ---- launch helpers shared with the decode session ---------------------------
int launch_qk(const QkArgs& a, float theta, hipStream_t st) {
    if (a.head_dim == 0 || a.head_dim % 2 || a.head_dim > uint32_t(kMaxHeadDim) ||
        a.head_dim / 2 > 256)
        return set_error(XP_E_ARG, "qk_norm_rope_append: head_dim=%u must be even and <= 512",
                         a.head_dim);
    if (a.n_heads == 0 || a.kv_heads == 0)
        return set_error(XP_E_ARG, "qk_norm_rope_append: empty head count");
    RopeFreq f;
    rope_freq(f, a.head_dim, theta);
    hipLaunchKernelGGL(qk_norm_rope_append_kernel, dim3(a.n_heads + a.kv_heads),
                       dim3(a.head_dim / 2), 0, st, a, f);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "qk_norm_rope_append: launch -> %s",
                                          hipGetErrorString(e));
    return XP_OK;
}

uint32_t attn_splits(uint32_t span) {
    uint32_t n = (span + kAttnChunk - 1) / kAttnChunk;
    return n < 1 ? 1 : n;
}

size_t attn_partial_floats(uint32_t kv_heads, uint32_t n_heads, uint32_t head_dim,
                           uint32_t max_span) {
    return size_t(kv_heads) * attn_splits(max_span) * (n_heads / kv_heads) * (2 + head_dim);
}

int launch_attention(AttnArgs a, uint32_t max_span, hipStream_t st) {
    if (a.head_dim == 0 || a.head_dim % kWave || a.head_dim > uint32_t(kMaxHeadDim))
        return set_error(XP_E_ARG, "attention: head_dim=%u must be a multiple of 64, <= %d",
                         a.head_dim, kMaxHeadDim);
    if (a.kv_heads == 0 || a.n_heads % a.kv_heads)
        return set_error(XP_E_ARG, "attention: n_heads=%u not a multiple of kv_heads=%u",
                         a.n_heads, a.kv_heads);
    a.group = a.n_heads / a.kv_heads;
    if (a.group > uint32_t(kAttnMaxGrp))
        return set_error(XP_E_ARG, "attention: %u query heads per kv head (max %d)", a.group,
                         kAttnMaxGrp);
    a.nsplit = attn_splits(max_span);
    if (!a.part || !a.tickets) {
        DeviceScratch* sc = scratch();
        if (!sc) return XP_E_HIP;
        const size_t need = size_t(a.kv_heads) * a.nsplit * a.group * (2 + a.head_dim);
        if (!ensure_partial(sc, need) || !ensure_tickets(sc, a.kv_heads)) return XP_E_NOMEM;
        a.part = sc->partial;
        a.tickets = sc->tickets;
    }
    hipLaunchKernelGGL(attention_decode_kernel, dim3(a.nsplit, a.kv_heads), dim3(kAttnThreads),
                       0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "attention: launch -> %s", hipGetErrorString(e));
    return XP_OK;
}

}  // namespace xp

using namespace xp;

extern "C" {

int xp_rmsnorm_gemma(float* out, const float* in, const float* w, uint32_t n, float eps,
                     xp_stream stream) {
    XP_REQUIRE(out && in && w, "null pointer");
    XP_REQUIRE(n > 0, "n must be positive");
    hipLaunchKernelGGL(rmsnorm_gemma_kernel, dim3(1), dim3(1024), 0, as_stream(stream), out, in,
                       w, n, eps);
    XP_LAUNCHED();
    return XP_OK;
}

int xp_rmsnorm_heads_gemma(float* out, const float* in, const float* w, uint32_t n_heads,
                           uint32_t head_dim, float eps, xp_stream stream) {
    XP_REQUIRE(out && in && w, "null pointer");
    XP_REQUIRE(n_heads > 0 && head_dim > 0, "empty shape");
    XP_REQUIRE(out != in, "out must not alias in (threads of one head are unordered)");
    hipLaunchKernelGGL(rmsnorm_heads_kernel, dim3(n_heads), dim3(256), 0, as_stream(stream), out,
                       in, w, head_dim, eps);
    XP_LAUNCHED();
    return XP_OK;
}

int xp_rope(float* x, uint32_t n_heads, uint32_t head_dim, uint32_t pos, float theta,
            xp_stream stream) {
    XP_REQUIRE(x != nullptr, "x is null");
    XP_REQUIRE(head_dim > 0 && head_dim % 2 == 0 && head_dim <= uint32_t(kMaxHeadDim),
               "head_dim=%u must be even and <= %d", head_dim, kMaxHeadDim);
    RopeFreq f;
    rope_freq(f, head_dim, theta);
    const uint32_t n = n_heads * (head_dim / 2);
    if (n == 0) return XP_OK;
    hipLaunchKernelGGL(rope_kernel, dim3((n + 255) / 256), dim3(256), 0, as_stream(stream), x,
                       n_heads, head_dim, pos, f);
    XP_LAUNCHED();
    return XP_OK;
}

int xp_qk_norm_rope_append(float* q_out, float* k_out, const float* q_raw, const float* k_raw,
                           const float* v, const float* q_norm_w, const float* k_norm_w,
                           uint16_t* kcache, uint16_t* vcache, uint32_t n_heads,
                           uint32_t kv_heads, uint32_t head_dim, uint32_t pos, float theta,
                           float eps, xp_stream stream) {
    XP_REQUIRE(q_out && k_out && q_raw && k_raw && v && q_norm_w && k_norm_w && kcache && vcache,
               "null pointer");
    XP_REQUIRE(q_out != q_raw && k_out != k_raw, "outputs must not alias inputs");
    QkArgs a{q_out, k_out, q_raw, k_raw, v, q_norm_w, k_norm_w, kcache, vcache,
             n_heads, kv_heads, head_dim, eps, nullptr, pos};
    return launch_qk(a, theta, as_stream(stream));
}

int xp_attention_decode(float* out, const float* q, const uint16_t* kcache,
                        const uint16_t* vcache, uint32_t n_heads, uint32_t kv_heads,
                        uint32_t head_dim, uint32_t span, uint32_t kv_start, float scale,
                        xp_stream stream) {
    XP_REQUIRE(out && q && kcache && vcache, "null pointer");
    XP_REQUIRE(span > 0, "span must be positive (the query attends at least to itself)");
    AttnArgs a{};
    a.out = out; a.q = q; a.kc = kcache; a.vc = vcache;
    a.n_heads = n_heads; a.kv_heads = kv_heads; a.head_dim = head_dim;
    a.span = span; a.kv_start = kv_start; a.scale = scale;
    return launch_attention(a, span, as_stream(stream));
}

int xp_geglu(float* out, const float* gate, const float* up, uint32_t n, xp_stream stream) {
    XP_REQUIRE(out && gate && up, "null pointer");
    if (n == 0) return XP_OK;
    hipLaunchKernelGGL(geglu_kernel, dim3((n + 255) / 256), dim3(256), 0, as_stream(stream), out,
                       gate, up, n);
    XP_LAUNCHED();
    return XP_OK;
}

int xp_add_residual(float* x, const float* y, uint32_t n, xp_stream stream) {
    XP_REQUIRE(x && y, "null pointer");
    if (n == 0) return XP_OK;
    hipLaunchKernelGGL(add_residual_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       as_stream(stream), x, y, n);
    XP_LAUNCHED();
    return XP_OK;
}

int xp_kv_append_f16(uint16_t* cache, const float* src, uint32_t n, uint32_t pos,
                     xp_stream stream) {
    XP_REQUIRE(cache && src, "null pointer");
    if (n == 0) return XP_OK;
    hipLaunchKernelGGL(kv_append_f16_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       as_stream(stream), cache, src, n, pos);
    XP_LAUNCHED();
    return XP_OK;
}

}  // extern "C"
