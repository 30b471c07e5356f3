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
#include "xp_attn_device.hpp"
#include <algorithm>
#include <vector>

#include "xp_device.hpp"
#include "xp_launch.hpp"

#include <cmath>
#include <cstdlib>

namespace xp {

// theta^(-2d/head_dim) for d < head_dim/2, evaluated on the host with the
// reference's formula exp2(-log2(theta) * frac) (llm_transformer.cl:168-169),
// passed by value so a captured launch replays it unchanged.

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
    const float scale = rsq_hw(ss / float(n) + eps);
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
    const float scale = rsq_hw(ss / float(head_dim) + eps);
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
    const float scale = rsq_hw(ss / float(a.head_dim) + a.eps);
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

// ---- decode attention (split-span, fp16 KV; the tile in xp_attn_device.hpp) ----
template <int G, int U, bool FQ>
__global__ __launch_bounds__(kAttnThreads) void attention_decode_kernel(AttnArgs a, RopeFreq f) {
    __shared__ AttnSmem<G, U> sm;
    (void)attn_tile<G, U, FQ, false>(a, f, blockIdx.x, blockIdx.y, blockIdx.z, sm);
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

uint32_t attn_splits(uint32_t max_span, uint32_t batch, uint32_t kv_heads) {
    // Enough workgroups to give every CU one (256), at most two 128-key passes
    // per split, at least kAttnMinChunk keys per split, at most kAttnSplitCap.
    const uint32_t units = (batch ? batch : 1) * (kv_heads ? kv_heads : 1);
    uint32_t n = (256 + units - 1) / units;
    const uint32_t by_len = (max_span + 2 * kAttnMaxPass - 1) / (2 * kAttnMaxPass);
    // Where a few more splits than kAttnFan would be needed for two passes
    // each but the CUs are shared out in kAttnFan or fewer, splits of up to
    // three passes keep one combine level and one workgroup a CU (config 5's
    // global layers: 16 sequences x 16 splits instead of x 17).
    const bool three = n <= uint32_t(kAttnFan) && by_len > n &&
                       (max_span + 3 * kAttnMaxPass - 1) / (3 * kAttnMaxPass) <= uint32_t(kAttnFan);
    if (three) n = kAttnFan;
    else if (n < by_len) n = by_len;
    const uint32_t most = (max_span + kAttnMinChunk - 1) / kAttnMinChunk;
    if (n > most) n = most;
    // At most 128 splits: past that the splits' exchange (each split reads
    // every split's statistics) costs more than the longer chunks (one
    // sequence at span 8192: 256 x 32 keys 13.4 us, 128 x 64 keys 11.9 us).
    if (n > kAttnSplitCap) n = kAttnSplitCap;
    return n < 1 ? 1 : n;
}

size_t attn_partial_floats(uint32_t kv_heads, uint32_t n_heads, uint32_t head_dim) {
    (void)head_dim;
    return size_t(kv_heads) * attn_head_floats(kv_heads ? n_heads / kv_heads : 1);
}

int plan_attention(AttnArgs& a, uint32_t max_span, bool allow_xchg, int* U_out, RopeFreq* f_out) {
    if (a.head_dim != uint32_t(kAttnHD))
        return set_error(XP_E_ARG, "attention: head_dim=%u must be %d", a.head_dim, kAttnHD);
    if (a.kv_heads == 0 || a.n_heads % a.kv_heads)
        return set_error(XP_E_ARG, "attention: n_heads=%u not a multiple of kv_heads=%u",
                         a.n_heads, a.kv_heads);
    if (max_span == 0) return set_error(XP_E_ARG, "attention: empty span");
    a.group = a.n_heads / a.kv_heads;
    const uint32_t G = a.group;
    if (G != 1 && G != 2 && G != 4)
        return set_error(XP_E_ARG, "attention: %u query heads per kv head (1, 2 or 4)", G);
    if (a.batch == 0) a.batch = 1;
    a.nsplit = attn_splits(max_span, a.batch, a.kv_heads);
    if (a.batch > 1 && a.nsplit > 1 && (!a.part || !a.tickets || a.bpart == 0))
        return set_error(XP_E_ARG, "attention: a batch needs its own partials and tickets");
    // Exchange mode: more splits than one ticket level combines (the ticket
    // chain would take two levels) and the launch's workgroups at most one a
    // CU, so all are resident at once and may wait for each other (bounded).
    // Measured: one sequence at span 4096 (128 splits) 12.2 -> 10.9 us, 8192
    // (256) 14.3 -> 13.5 us; 16 sequences x 16 splits (one ticket level)
    // 1.461 -> 1.472 ms a batched step, so those keep the tickets.
    // XP_ATTN_EXCHANGE=0 in the environment turns it off.
    static const bool xchg_on = [] {
        const char* e = std::getenv("XP_ATTN_EXCHANGE");
        return !(e && e[0] == '0');
    }();
    {
        DeviceScratch* sc = scratch();
        if (!sc) return XP_E_HIP;
        const uint64_t wgs = uint64_t(a.nsplit) * a.kv_heads * a.batch;
        a.xchg = allow_xchg && xchg_on && a.nsplit > uint32_t(kAttnFan) && sc->n_cu > 0 &&
                 wgs <= uint64_t(sc->n_cu) && a.nsplit <= kAttnSplitCap ? 1u : 0u;
        if (a.xchg && (!a.part || !a.tickets)) {
            // the exchange mode's own zeroed buffers, not the shared scratch
            if (!ensure_attn_x(sc, attn_partial_floats(a.kv_heads, a.n_heads, a.head_dim),
                               size_t(a.kv_heads) * kAttnTicketsPerHead))
                return XP_E_NOMEM;
            a.part = sc->attn_x;
            a.tickets = sc->attn_state;
        }
    }
    if (a.nsplit > 1 && (!a.part || !a.tickets)) {
        DeviceScratch* sc = scratch();
        if (!sc) return XP_E_HIP;
        const size_t need = attn_partial_floats(a.kv_heads, a.n_heads, a.head_dim);
        if (!ensure_partial(sc, need) || !ensure_tickets(sc, size_t(a.kv_heads) * kAttnTicketsPerHead))
            return XP_E_NOMEM;
        a.part = sc->partial;
        a.tickets = sc->tickets;
    }
    // keys per lane per pass: a quarter pass for 32-key chunks, a half for
    // 64, a whole 128-key pass beyond
    uint32_t chunk = (max_span + a.nsplit - 1) / a.nsplit;
    if (chunk < uint32_t(kAttnMinChunk)) chunk = kAttnMinChunk;
    const int U = chunk <= 32 ? 2 : (chunk <= 64 ? 4 : 8);
    const bool fq = a.q_raw != nullptr;
    RopeFreq f{};
    if (fq) {
        if (!a.pos_dev || !a.k_raw || !a.v_raw || !a.qw || !a.kw || !(a.theta > 0.0f))
            return set_error(XP_E_ARG, "attention: the fused QK-norm / RoPE form needs pos_dev, k_raw, "
                                       "v_raw, both norm weights and theta > 0");
        rope_freq(f, a.head_dim, a.theta);
    } else if (!a.q) {
        return set_error(XP_E_ARG, "attention: null q");
    }
    *U_out = U;
    *f_out = f;
    return XP_OK;
}

int launch_attention(AttnArgs a, uint32_t max_span, hipStream_t st, bool allow_xchg) {
    int U = 0;
    RopeFreq f{};
    if (int rc = plan_attention(a, max_span, allow_xchg, &U, &f); rc != XP_OK) return rc;
    const bool fq = a.q_raw != nullptr;
    const uint32_t G = a.group;
    const dim3 grid(a.nsplit, a.kv_heads, a.batch), block(kAttnThreads);
#define XP_ATTN_U(GG, FF)                                                                                 \
    if (U == 2) hipLaunchKernelGGL((attention_decode_kernel<GG, 2, FF>), grid, block, 0, st, a, f);      \
    else if (U == 4) hipLaunchKernelGGL((attention_decode_kernel<GG, 4, FF>), grid, block, 0, st, a, f); \
    else hipLaunchKernelGGL((attention_decode_kernel<GG, 8, FF>), grid, block, 0, st, a, f);
#define XP_ATTN_LAUNCH(GG)        \
    if (fq) { XP_ATTN_U(GG, true) } \
    else { XP_ATTN_U(GG, false) }
    if (G == 1) {
        XP_ATTN_LAUNCH(1)
    } else if (G == 2) {
        XP_ATTN_LAUNCH(2)
    } else {
        XP_ATTN_LAUNCH(4)
    }
#undef XP_ATTN_LAUNCH
#undef XP_ATTN_U
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(XP_E_HIP, "attention: launch -> %s", hipGetErrorString(e));
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

}  // extern "C"

namespace {
// One decode attention on the library's own split records. xchg: the
// exchange mode may be chosen (its error word is then the caller's to check,
// attention_xchg_check); otherwise the splits combine through the arrival
// tickets, which reset themselves.
int attention_call(float* out, const float* q, const uint16_t* kcache, const uint16_t* vcache,
                   uint32_t n_heads, uint32_t kv_heads, uint32_t head_dim, uint32_t span,
                   uint32_t kv_start, float scale, hipStream_t st, bool xchg) {
    XP_REQUIRE(out && q && kcache && vcache, "null pointer");
    XP_REQUIRE(span > 0, "span must be positive (the query attends at least to itself)");
    AttnArgs a{};
    a.out = out; a.q = q; a.kc = kcache; a.vc = vcache;
    a.n_heads = n_heads; a.kv_heads = kv_heads; a.head_dim = head_dim;
    a.span = span; a.kv_start = kv_start; a.scale = scale;
    return launch_attention(a, span, st, xchg);
}
// After the stream has been synchronised: XP_E_DEVICE when an exchange-mode
// wait on the library's records timed out (another kernel held CUs, so the
// splits were not all resident at once); the records, epochs and error
// words then start over from zero.
int attention_xchg_check(uint32_t kv_heads) {
    DeviceScratch* sc = scratch();
    if (!sc || !sc->attn_state) return XP_OK;
    const size_t words = std::min(sc->attn_state_words, size_t(kv_heads) * kAttnTicketsPerHead);
    std::vector<uint32_t> h(words);
    XP_HIP(hipMemcpy(h.data(), sc->attn_state, words * 4, hipMemcpyDeviceToHost));
    uint32_t err = 0;
    for (size_t g = 0; g * kAttnTicketsPerHead + kAttnXErrWord < words; ++g)
        err |= h[g * kAttnTicketsPerHead + kAttnXErrWord];
    if (!err) return XP_OK;
    XP_HIP(hipMemset(sc->attn_x, 0, sc->attn_x_floats * sizeof(float)));
    XP_HIP(hipMemset(sc->attn_state, 0, sc->attn_state_words * 4));
    XP_HIP(hipDeviceSynchronize());
    return set_error(XP_E_DEVICE, "attention: an exchange-mode wait ran past its spin limit (the "
                     "splits were not resident at once); the output holds NaN");
}
}  // namespace

extern "C" {

int xp_attention_decode(float* out, const float* q, const uint16_t* kcache,
                        const uint16_t* vcache, uint32_t n_heads, uint32_t kv_heads,
                        uint32_t head_dim, uint32_t span, uint32_t kv_start, float scale,
                        xp_stream stream) {
    return attention_call(out, q, kcache, vcache, n_heads, kv_heads, head_dim, span, kv_start,
                          scale, as_stream(stream), false);
}

int xp_attention_decode_timed(float* out, const float* q, const uint16_t* const* kcaches,
                              const uint16_t* const* vcaches, uint32_t ncopies, uint32_t n_heads,
                              uint32_t kv_heads, uint32_t head_dim, uint32_t span,
                              uint32_t kv_start, float scale, uint32_t iters, xp_stream stream,
                              float* ms) {
    XP_REQUIRE(kcaches && vcaches && ms && ncopies > 0 && iters > 0, "bad arguments");
    hipStream_t st = as_stream(stream);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    XP_HIP(hipEventCreate(&e0));
    XP_HIP(hipEventCreate(&e1));
    int rc = XP_OK;
    // One untimed pass over every copy so the split scratch is sized before
    // timing. The timed launches may take the exchange mode: its error word
    // is checked once the stream has drained.
    for (uint32_t i = 0; i < ncopies && rc == XP_OK; ++i)
        rc = attention_call(out, q, kcaches[i], vcaches[i], n_heads, kv_heads, head_dim, span,
                            kv_start, scale, st, true);
    if (rc == XP_OK && hipStreamSynchronize(st) != hipSuccess) rc = set_error(XP_E_HIP, "sync");
    if (rc == XP_OK && hipEventRecord(e0, st) != hipSuccess) rc = set_error(XP_E_HIP, "event");
    for (uint32_t i = 0; i < iters && rc == XP_OK; ++i)
        rc = attention_call(out, q, kcaches[i % ncopies], vcaches[i % ncopies], n_heads, kv_heads,
                            head_dim, span, kv_start, scale, st, true);
    if (rc == XP_OK && hipEventRecord(e1, st) != hipSuccess) rc = set_error(XP_E_HIP, "event");
    if (rc == XP_OK && hipEventSynchronize(e1) != hipSuccess) rc = set_error(XP_E_HIP, "sync");
    if (rc == XP_OK && hipEventElapsedTime(ms, e0, e1) != hipSuccess)
        rc = set_error(XP_E_HIP, "elapsed");
    if (rc == XP_OK) rc = attention_xchg_check(kv_heads);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
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
