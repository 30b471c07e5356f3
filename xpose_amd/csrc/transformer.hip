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
    const uint32_t b = blockIdx.y;   // batched sequence
    a.q_raw += size_t(b) * a.bq;
    a.q_out += size_t(b) * a.bq;
    a.k_raw += size_t(b) * a.bkv;
    a.k_out += size_t(b) * a.bkv;
    a.v += size_t(b) * a.bkv;
    a.kcache += b * a.bcache;
    a.vcache += b * a.bcache;
    const uint32_t pos = a.pos_dev ? a.pos_dev[b] : a.pos;
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
// Grid: (nsplit, kv_heads). Workgroup (s, g) takes a contiguous chunk of the
// attended keys [kv_start + s*chunk, ...) for the G query heads that share kv
// head g, reading every key and value once for all G heads (the mq4 idea,
// llm_transformer.cl:418-464, 499-557):
//   scores  head_dim/8 threads per key, 16-byte fp16 loads, q held in
//           registers, shuffle reduction; several keys in flight per thread
//   softmax one wave per head over the chunk (max, exp, sum)
//   values  head_dim/2 threads per key, 4-byte loads, several keys in flight
// Each split publishes (max, sum of exp, unnormalised o) per head; the last
// workgroup of kv head g to arrive (arrival ticket) rescales and sums the
// splits in ascending order — softmax_rows_finish's online combine
// (llm_transformer.cl:385-405). One split writes the normalised output.
constexpr int kAttnThreads  = 256;
constexpr int kAttnMinChunk = 32;    // keys per workgroup at short spans
constexpr int kAttnChunk    = 128;   // most keys one workgroup takes
constexpr int kAttnMaxSplit = 64;    // workgroups per kv head

__device__ __forceinline__ void attn_range(const AttnArgs& a, uint32_t& span, uint32_t& kv0) {
    if (a.pos_dev) {
        const uint32_t seq = a.pos_dev[blockIdx.z] + 1u;
        kv0 = (a.window == 0 || seq <= a.window) ? 0u : seq - a.window;
        span = seq - kv0;
    } else {
        span = a.span;
        kv0 = a.kv_start;
    }
}

template <int G, int HD>
__global__ __launch_bounds__(kAttnThreads) void attention_decode_kernel(AttnArgs a) {
    constexpr int TPK = HD / 8;                 // threads per key (scores)
    constexpr int KPP = kAttnThreads / TPK;     // keys per pass (scores)
    constexpr int TPV = HD / 2;                 // threads per key (values)
    constexpr int KPV = kAttnThreads / TPV;     // keys per pass (values)
    constexpr int ROW = 2 + HD;
    __shared__ float ps[G * kAttnChunk];
    __shared__ float red[KPV * G * HD];
    __shared__ float mstat[G], lstat[G];
    __shared__ float fs[kAttnMaxSplit * G];
    __shared__ float ls[kAttnMaxSplit * G];
    __shared__ uint32_t last;
    {   // batched sequence blockIdx.z
        const uint32_t b = blockIdx.z;
        a.q += size_t(b) * a.bq;
        a.out += size_t(b) * a.bq;
        a.kc += b * a.bcache;
        a.vc += b * a.bcache;
        if (a.part) a.part += b * a.bpart;
        if (a.tickets) a.tickets += size_t(b) * a.kv_heads;
    }
    uint32_t span, kv0;
    attn_range(a, span, kv0);
    const uint32_t g = blockIdx.y, s = blockIdx.x;
    const uint32_t chunk = (span + a.nsplit - 1) / a.nsplit;
    const uint32_t j0 = s * chunk;
    const uint32_t j1 = min(j0 + chunk, span);
    const int nk = j1 > j0 ? int(j1 - j0) : 0;
    const int tid = threadIdx.x;
    const size_t rowstride = size_t(a.kv_heads) * HD;   // fp16 elements per cache row
    const uint16_t* kbase = a.kc + size_t(kv0 + j0) * rowstride + size_t(g) * HD;
    const uint16_t* vbase = a.vc + size_t(kv0 + j0) * rowstride + size_t(g) * HD;

    // ---- scores
    {
        const int sub = tid % TPK, kp = tid / TPK;
        float q[G][8];
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) q[h][e] = a.q[(size_t(g) * G + h) * HD + sub * 8 + e];
        for (int base = 0; base < nk; base += 4 * KPP) {
            u32x4 kw[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = base + u * KPP + kp;
                kw[u] = (j < nk) ? *reinterpret_cast<const u32x4*>(kbase + size_t(j) * rowstride + sub * 8)
                                 : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = base + u * KPP + kp;
                float kf[8];
                kf[0] = f16_bits_to_f32(kw[u].x); kf[1] = f16_bits_to_f32(kw[u].x >> 16);
                kf[2] = f16_bits_to_f32(kw[u].y); kf[3] = f16_bits_to_f32(kw[u].y >> 16);
                kf[4] = f16_bits_to_f32(kw[u].z); kf[5] = f16_bits_to_f32(kw[u].z >> 16);
                kf[6] = f16_bits_to_f32(kw[u].w); kf[7] = f16_bits_to_f32(kw[u].w >> 16);
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    float d = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) d = fmaf(q[h][e], kf[e], d);
#pragma unroll
                    for (int o = TPK / 2; o > 0; o >>= 1) d += __shfl_xor(d, o, kWave);
                    if (sub == 0 && j < nk) ps[h * kAttnChunk + j] = d * a.scale;
                }
            }
        }
    }
    __syncthreads();
    // ---- chunk softmax, one wave per head
    for (int h = tid / kWave; h < G; h += kAttnThreads / kWave) {
        const int l = tid % kWave;
        float m = -INFINITY;
        for (int j = l; j < nk; j += kWave) m = fmaxf(m, ps[h * kAttnChunk + j]);
        m = wave_max(m);
        float sum = 0.0f;
        for (int j = l; j < nk; j += kWave) {
            const float e = expf(ps[h * kAttnChunk + j] - m);
            ps[h * kAttnChunk + j] = e;
            sum += e;
        }
        sum = wave_sum(sum);
        if (l == 0) { mstat[h] = m; lstat[h] = sum; }
    }
    __syncthreads();
    // ---- weighted values
    {
        const int dp = tid % TPV, ks = tid / TPV;
        float o[G][2];
#pragma unroll
        for (int h = 0; h < G; ++h) o[h][0] = o[h][1] = 0.0f;
        for (int base = 0; base < nk; base += 4 * KPV) {
            uint32_t vw[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = base + u * KPV + ks;
                vw[u] = (j < nk) ? *reinterpret_cast<const uint32_t*>(vbase + size_t(j) * rowstride + dp * 2)
                                 : 0u;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = base + u * KPV + ks;
                if (j < nk) {
                    const float v0 = f16_bits_to_f32(vw[u]), v1 = f16_bits_to_f32(vw[u] >> 16);
#pragma unroll
                    for (int h = 0; h < G; ++h) {
                        const float p = ps[h * kAttnChunk + j];
                        o[h][0] = fmaf(p, v0, o[h][0]);
                        o[h][1] = fmaf(p, v1, o[h][1]);
                    }
                }
            }
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            red[(ks * G + h) * HD + dp * 2] = o[h][0];
            red[(ks * G + h) * HD + dp * 2 + 1] = o[h][1];
        }
    }
    __syncthreads();
    if (a.nsplit == 1) {
        for (int i = tid; i < G * HD; i += kAttnThreads) {
            const int h = i / HD;
            float acc = 0.0f;
            for (int k2 = 0; k2 < KPV; ++k2) acc += red[k2 * G * HD + i];
            a.out[size_t(g) * G * HD + i] = acc / lstat[h];
        }
        return;
    }
    float* part = a.part + (size_t(g) * a.nsplit + s) * G * ROW;
    for (int i = tid; i < G * HD; i += kAttnThreads) {
        const int h = i / HD, d = i % HD;
        float acc = 0.0f;
        for (int k2 = 0; k2 < KPV; ++k2) acc += red[k2 * G * HD + i];
        st_dev(part + h * ROW + 2 + d, acc);
    }
    if (tid < G) {
        st_dev(part + tid * ROW, nk > 0 ? mstat[tid] : -INFINITY);
        st_dev(part + tid * ROW + 1, nk > 0 ? lstat[tid] : 0.0f);
    }
    wait_mem();
    __syncthreads();
    if (tid == 0) last = take_ticket(&a.tickets[g]);
    __syncthreads();
    if (last != a.nsplit - 1) return;

    // ---- combine (last workgroup): factors f[p][h] = exp(m_p - M) in LDS
    const float* base = a.part + size_t(g) * a.nsplit * G * ROW;
    for (uint32_t i = tid; i < a.nsplit * G; i += kAttnThreads) {
        const float* r = base + size_t(i) * ROW;   // i = p * G + h
        const float m = ld_dev(r), l = ld_dev(r + 1);
        fs[i] = l > 0.0f ? m : -INFINITY;
        ls[i] = l;
    }
    __syncthreads();
    if (tid < G) {
        float M = -INFINITY;
        for (uint32_t p = 0; p < a.nsplit; ++p) M = fmaxf(M, fs[p * G + tid]);
        float L = 0.0f;
        for (uint32_t p = 0; p < a.nsplit; ++p) {
            const float m = fs[p * G + tid];
            const float f = (m == -INFINITY) ? 0.0f : expf(m - M);
            L += ls[p * G + tid] * f;
            fs[p * G + tid] = f;
        }
        lstat[tid] = L;
    }
    __syncthreads();
    const size_t pstride = size_t(G) * ROW;
    for (int i = tid; i < G * HD; i += kAttnThreads) {
        const int h = i / HD, d = i % HD;
        const float* col = base + size_t(h) * ROW + 2 + d;
        float o = 0.0f;
        uint32_t p = 0;
        for (; p + 8 <= a.nsplit; p += 8) {
            float v[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) v[q] = ld_dev(col + (p + q) * pstride);
#pragma unroll
            for (int q = 0; q < 8; ++q) o = fmaf(v[q], fs[(p + q) * G + h], o);
        }
        for (; p < a.nsplit; ++p) o = fmaf(ld_dev(col + p * pstride), fs[p * G + h], o);
        a.out[size_t(g) * G * HD + i] = o / lstat[h];
    }
    if (tid == 0) st_dev(&a.tickets[g], 0u);
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
    hipLaunchKernelGGL(qk_norm_rope_append_kernel, dim3(a.n_heads + a.kv_heads, a.batch ? a.batch : 1),
                       dim3(a.head_dim / 2), 0, st, a, f);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "qk_norm_rope_append: launch -> %s",
                                          hipGetErrorString(e));
    return XP_OK;
}

uint32_t attn_splits(uint32_t span) {
    uint32_t n = (span + kAttnMinChunk - 1) / kAttnMinChunk;
    if (n > uint32_t(kAttnMaxSplit)) n = kAttnMaxSplit;
    return n < 1 ? 1 : n;
}

size_t attn_partial_floats(uint32_t kv_heads, uint32_t n_heads, uint32_t head_dim,
                           uint32_t max_span) {
    return size_t(kv_heads) * attn_splits(max_span) * (n_heads / kv_heads) * (2 + head_dim);
}

int launch_attention(AttnArgs a, uint32_t max_span, hipStream_t st) {
    if (a.head_dim != 64 && a.head_dim != 128 && a.head_dim != 256 && a.head_dim != 512)
        return set_error(XP_E_ARG, "attention: head_dim=%u must be 64, 128, 256 or 512",
                         a.head_dim);
    if (a.kv_heads == 0 || a.n_heads % a.kv_heads)
        return set_error(XP_E_ARG, "attention: n_heads=%u not a multiple of kv_heads=%u",
                         a.n_heads, a.kv_heads);
    if (max_span == 0 || max_span > uint32_t(kAttnMaxSplit * kAttnChunk))
        return set_error(XP_E_ARG, "attention: span %u outside [1, %d]", max_span,
                         kAttnMaxSplit * kAttnChunk);
    a.group = a.n_heads / a.kv_heads;
    const uint32_t G = a.group;
    if (G != 1 && G != 2 && G != 4 && G != 8)
        return set_error(XP_E_ARG, "attention: %u query heads per kv head (1, 2, 4 or 8)", G);
    a.nsplit = attn_splits(max_span);
    if (a.batch == 0) a.batch = 1;
    if (a.batch > 1 && a.nsplit > 1 && (!a.part || !a.tickets || a.bpart == 0))
        return set_error(XP_E_ARG, "attention: a batch needs its own partials and tickets");
    if (a.nsplit > 1 && (!a.part || !a.tickets)) {
        DeviceScratch* sc = scratch();
        if (!sc) return XP_E_HIP;
        const size_t need = size_t(a.kv_heads) * a.nsplit * G * (2 + a.head_dim);
        if (!ensure_partial(sc, need) || !ensure_tickets(sc, a.kv_heads)) return XP_E_NOMEM;
        a.part = sc->partial;
        a.tickets = sc->tickets;
    }
    const dim3 grid(a.nsplit, a.kv_heads, a.batch), block(kAttnThreads);
#define XP_ATTN(GG, HH)                                                                    \
    if (G == GG && a.head_dim == HH) {                                                     \
        hipLaunchKernelGGL((attention_decode_kernel<GG, HH>), grid, block, 0, st, a);      \
        hipError_t e = hipGetLastError();                                                  \
        if (e != hipSuccess)                                                               \
            return set_error(XP_E_HIP, "attention: launch -> %s", hipGetErrorString(e));   \
        return XP_OK;                                                                      \
    }
    XP_ATTN(1, 64) XP_ATTN(1, 128) XP_ATTN(1, 256) XP_ATTN(1, 512)
    XP_ATTN(2, 64) XP_ATTN(2, 128) XP_ATTN(2, 256) XP_ATTN(2, 512)
    XP_ATTN(4, 64) XP_ATTN(4, 128) XP_ATTN(4, 256) XP_ATTN(4, 512)
    XP_ATTN(8, 64) XP_ATTN(8, 128) XP_ATTN(8, 256)
#undef XP_ATTN
    return set_error(XP_E_ARG, "attention: no kernel for %u heads/kv head at head_dim %u", G,
                     a.head_dim);
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
