// Prefill-shaped twins of the decode kernels (kernels/llm_sampling.cl:496-736):
// row-indexed softmax, causal / sliding-window attention scores and apply,
// row RMSNorm, per-head row QK-norm, per-row-position RoPE, KV row append and
// embedding row gather, each behind its own C-ABI entry.
//
// The reference gives row reductions one thread per row (serial loops over
// the columns); here a row is one wave: lanes stride over the columns and DPP
// wave reductions combine them. Elementwise kernels are grid-stride loops,
// scores and apply one thread per output element with 16-byte loads along
// head_dim (scores) or lanes along head_dim (apply, coalesced over v rows).
// Layouts are the reference's, row-major: row r occupies [r n_cols, (r + 1)
// n_cols); q, scores and outputs are [head][query][...]; caches [t][kv_head][d]
// in fp32.
#include <algorithm>
#include <cmath>

#include "xp_device.hpp"
#include "xp_launch.hpp"

namespace xp {
namespace {

constexpr int kPfThreads = 256;
constexpr int kPfWaves = kPfThreads / kWave;

uint32_t pf_blocks(size_t n) {
    return uint32_t(std::min<size_t>((n + kPfThreads - 1) / kPfThreads, 65536));
}
uint32_t pf_row_blocks(size_t rows) { return uint32_t((rows + kPfWaves - 1) / kPfWaves); }

// softmax_rows_stats (llm_sampling.cl:527-547): one wave per row.
__global__ __launch_bounds__(kPfThreads) void softmax_rows_stats_kernel(float* stats, const float* x,
                                                                       uint32_t n_rows, uint32_t n_cols) {
    const uint32_t r = blockIdx.x * kPfWaves + threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (r >= n_rows) return;   // whole waves
    const float* row = x + size_t(r) * n_cols;
    float m = -INFINITY;
    for (uint32_t j = lane; j < n_cols; j += kWave) m = fmaxf(m, row[j]);
    m = wave_max(m);
    if (!isfinite(m)) {
        if (lane == 0) {
            stats[2 * size_t(r)] = 0.0f;
            stats[2 * size_t(r) + 1] = 1.0f;
        }
        return;
    }
    float s = 0.0f;
    for (uint32_t j = lane; j < n_cols; j += kWave) s += expf(row[j] - m);
    s = wave_sum(s);
    if (lane == 0) {
        stats[2 * size_t(r)] = m;
        stats[2 * size_t(r) + 1] = s;
    }
}

// softmax_rows_apply (llm_sampling.cl:549-556).
__global__ void softmax_rows_apply_kernel(float* x, const float* stats, uint32_t n_cols, size_t total) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += size_t(gridDim.x) * blockDim.x) {
        const size_t r = i / n_cols;
        x[i] = expf(x[i] - stats[2 * r]) / stats[2 * r + 1];
    }
}

// attention_scores_prefill (llm_sampling.cl:574-600): causal and window
// masks folded in; one thread per score, head_dim in 16-byte steps.
__global__ void attention_scores_prefill_kernel(float* scores, const float* q, const float* kc,
                                                uint32_t n_heads, uint32_t kv_heads, uint32_t head_dim,
                                                uint32_t n_query, uint32_t seq_len, uint32_t q_offset,
                                                uint32_t window, float scale, size_t total) {
    const uint32_t group = n_heads / kv_heads;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += size_t(gridDim.x) * blockDim.x) {
        const uint32_t t = uint32_t(i % seq_len);
        const size_t hq = i / seq_len;
        const uint32_t qi = uint32_t(hq % n_query), h = uint32_t(hq / n_query);
        const uint32_t qpos = q_offset + qi;
        if (t > qpos || (window != 0u && t + window <= qpos)) {
            scores[i] = -INFINITY;
            continue;
        }
        const float4* qv = reinterpret_cast<const float4*>(q + (size_t(h) * n_query + qi) * head_dim);
        const float4* kv = reinterpret_cast<const float4*>(kc + (size_t(t) * kv_heads + h / group) * head_dim);
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        for (uint32_t d = 0; d < head_dim / 4; ++d) {
            const float4 x = qv[d], y = kv[d];
            a0 = fmaf(x.x, y.x, a0);
            a1 = fmaf(x.y, y.y, a1);
            a2 = fmaf(x.z, y.z, a2);
            a3 = fmaf(x.w, y.w, a3);
        }
        scores[i] = ((a0 + a1) + (a2 + a3)) * scale;
    }
}

// attention_apply_prefill (llm_sampling.cl:605-627): one thread per output
// element, lanes along head_dim (coalesced v rows, probs broadcast).
__global__ void attention_apply_prefill_kernel(float* out, const float* probs, const float* vc,
                                               uint32_t n_heads, uint32_t kv_heads, uint32_t head_dim,
                                               uint32_t n_query, uint32_t seq_len, size_t total) {
    const uint32_t group = n_heads / kv_heads, vstride = kv_heads * head_dim;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += size_t(gridDim.x) * blockDim.x) {
        const uint32_t d = uint32_t(i % head_dim);
        const size_t hq = i / head_dim;
        const uint32_t qi = uint32_t(hq % n_query), h = uint32_t(hq / n_query);
        const float* p = probs + (size_t(h) * n_query + qi) * seq_len;
        const float* v = vc + size_t(h / group) * head_dim + d;
        float a0 = 0.0f, a1 = 0.0f;
        uint32_t t = 0;
        for (; t + 2 <= seq_len; t += 2) {
            a0 = fmaf(p[t], v[size_t(t) * vstride], a0);
            a1 = fmaf(p[t + 1], v[size_t(t + 1) * vstride], a1);
        }
        if (t < seq_len) a0 = fmaf(p[t], v[size_t(t) * vstride], a0);
        out[i] = a0 + a1;
    }
}

// rmsnorm_rows_sumsq (llm_sampling.cl:634-642): one wave per row.
__global__ __launch_bounds__(kPfThreads) void rmsnorm_rows_sumsq_kernel(float* rowss, const float* in,
                                                                       uint32_t n_rows, uint32_t n) {
    const uint32_t r = blockIdx.x * kPfWaves + threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (r >= n_rows) return;
    const float* row = in + size_t(r) * n;
    float ss = 0.0f;
    for (uint32_t j = lane; j < n; j += kWave) ss = fmaf(row[j], row[j], ss);
    ss = wave_sum(ss);
    if (lane == 0) rowss[r] = ss;
}

// rmsnorm_rows_apply_gemma (llm_sampling.cl:645-656).
__global__ void rmsnorm_rows_apply_gemma_kernel(float* out, const float* in, const float* w,
                                                const float* rowss, uint32_t n, float eps, size_t total) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += size_t(gridDim.x) * blockDim.x) {
        const size_t r = i / n;
        const float scale = rsq_hw(rowss[r] / float(n) + eps);
        out[i] = in[i] * scale * (1.0f + w[i - r * n]);
    }
}

// rmsnorm_heads_rows_gemma (llm_sampling.cl:659-672): one wave per
// (token, head) row of head_dim.
__global__ __launch_bounds__(kPfThreads) void rmsnorm_heads_rows_gemma_kernel(
    float* out, const float* in, const float* w, uint32_t n_rows, uint32_t head_dim, float eps) {
    const uint32_t r = blockIdx.x * kPfWaves + threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (r >= n_rows) return;
    const float* row = in + size_t(r) * head_dim;
    float ss = 0.0f;
    for (uint32_t j = lane; j < head_dim; j += kWave) ss = fmaf(row[j], row[j], ss);
    const float scale = rsq_hw(wave_sum(ss) / float(head_dim) + eps);
    for (uint32_t j = lane; j < head_dim; j += kWave) out[size_t(r) * head_dim + j] = row[j] * scale * (1.0f + w[j]);
}

// rope_prefill (llm_sampling.cl:687-708): one thread per rotated pair, token
// ti at position pos0 + ti, with the decode rope's inverse frequencies, so a
// row rotates exactly as xp_rope rotates it at that position.
__global__ void rope_prefill_kernel(float* x, uint32_t n_heads, uint32_t head_dim, uint32_t pos0,
                                    RopeFreq f, size_t total) {
    const uint32_t hdhalf = head_dim / 2u;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += size_t(gridDim.x) * blockDim.x) {
        const uint32_t d = uint32_t(i % hdhalf);
        const size_t th = i / hdhalf;
        const uint32_t ti = uint32_t(th / n_heads);
        const size_t base = th * head_dim + d;
        const float ang = float(pos0 + ti) * f.inv[d];
        float s, c;
        sincosf(ang, &s, &c);
        const float a = x[base], b = x[base + hdhalf];
        x[base] = a * c - b * s;
        x[base + hdhalf] = b * c + a * s;
    }
}

// kv_append_rows (llm_sampling.cl:714-721).
__global__ void kv_append_rows_kernel(float* dst, const float* src, size_t total) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += size_t(gridDim.x) * blockDim.x)
        dst[i] = src[i];
}

// embed_lookup_rows (llm_sampling.cl:728-736); an id past the table writes
// zeros instead of reading past it.
__global__ void embed_lookup_rows_kernel(float* out, const float* table, const uint32_t* tokens,
                                         uint32_t n, uint32_t vocab, size_t total) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += size_t(gridDim.x) * blockDim.x) {
        const size_t ti = i / n;
        const uint32_t tok = tokens[ti];
        out[i] = tok < vocab ? table[size_t(tok) * n + (i - ti * n)] : 0.0f;
    }
}

int launched(const char* who) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "%s: launch -> %s", who, hipGetErrorString(e));
    return XP_OK;
}

}  // namespace
}  // namespace xp

using namespace xp;

extern "C" {

int xp_softmax_rows_stats(float* stats, const float* x, uint32_t n_rows, uint32_t n_cols,
                          xp_stream stream) {
    XP_REQUIRE(stats && x, "null pointer");
    XP_REQUIRE(n_rows > 0 && n_cols > 0, "empty shape %u x %u", n_rows, n_cols);
    hipLaunchKernelGGL(softmax_rows_stats_kernel, dim3(pf_row_blocks(n_rows)), dim3(kPfThreads), 0,
                       as_stream(stream), stats, x, n_rows, n_cols);
    return launched("xp_softmax_rows_stats");
}

int xp_softmax_rows_apply(float* x, const float* stats, uint32_t n_rows, uint32_t n_cols,
                          xp_stream stream) {
    XP_REQUIRE(stats && x, "null pointer");
    XP_REQUIRE(n_rows > 0 && n_cols > 0, "empty shape %u x %u", n_rows, n_cols);
    const size_t total = size_t(n_rows) * n_cols;
    hipLaunchKernelGGL(softmax_rows_apply_kernel, dim3(pf_blocks(total)), dim3(kPfThreads), 0,
                       as_stream(stream), x, stats, n_cols, total);
    return launched("xp_softmax_rows_apply");
}

int xp_attention_scores_prefill(float* scores, const float* q, const float* kcache, uint32_t n_heads,
                                uint32_t kv_heads, uint32_t head_dim, uint32_t n_query,
                                uint32_t seq_len, uint32_t q_offset, uint32_t window, float scale,
                                xp_stream stream) {
    XP_REQUIRE(scores && q && kcache, "null pointer");
    XP_REQUIRE(n_heads > 0 && kv_heads > 0 && n_heads % kv_heads == 0,
               "n_heads=%u must be a positive multiple of kv_heads=%u", n_heads, kv_heads);
    XP_REQUIRE(head_dim > 0 && head_dim % 4 == 0, "head_dim=%u must be a positive multiple of 4", head_dim);
    XP_REQUIRE(n_query > 0 && seq_len > 0, "n_query=%u, seq_len=%u must be positive", n_query, seq_len);
    XP_REQUIRE(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kcache)) & 15u) == 0,
               "q and kcache must be 16-byte aligned");
    const size_t total = size_t(n_heads) * n_query * seq_len;
    hipLaunchKernelGGL(attention_scores_prefill_kernel, dim3(pf_blocks(total)), dim3(kPfThreads), 0,
                       as_stream(stream), scores, q, kcache, n_heads, kv_heads, head_dim, n_query,
                       seq_len, q_offset, window, scale, total);
    return launched("xp_attention_scores_prefill");
}

int xp_attention_apply_prefill(float* out, const float* probs, const float* vcache, uint32_t n_heads,
                               uint32_t kv_heads, uint32_t head_dim, uint32_t n_query,
                               uint32_t seq_len, xp_stream stream) {
    XP_REQUIRE(out && probs && vcache, "null pointer");
    XP_REQUIRE(n_heads > 0 && kv_heads > 0 && n_heads % kv_heads == 0,
               "n_heads=%u must be a positive multiple of kv_heads=%u", n_heads, kv_heads);
    XP_REQUIRE(head_dim > 0 && n_query > 0 && seq_len > 0, "empty shape");
    const size_t total = size_t(n_heads) * n_query * head_dim;
    hipLaunchKernelGGL(attention_apply_prefill_kernel, dim3(pf_blocks(total)), dim3(kPfThreads), 0,
                       as_stream(stream), out, probs, vcache, n_heads, kv_heads, head_dim, n_query,
                       seq_len, total);
    return launched("xp_attention_apply_prefill");
}

int xp_rmsnorm_rows_sumsq(float* rowss, const float* in, uint32_t n_rows, uint32_t n,
                          xp_stream stream) {
    XP_REQUIRE(rowss && in, "null pointer");
    XP_REQUIRE(n_rows > 0 && n > 0, "empty shape %u x %u", n_rows, n);
    hipLaunchKernelGGL(rmsnorm_rows_sumsq_kernel, dim3(pf_row_blocks(n_rows)), dim3(kPfThreads), 0,
                       as_stream(stream), rowss, in, n_rows, n);
    return launched("xp_rmsnorm_rows_sumsq");
}

int xp_rmsnorm_rows_apply_gemma(float* out, const float* in, const float* w, const float* rowss,
                                uint32_t n_rows, uint32_t n, float eps, xp_stream stream) {
    XP_REQUIRE(out && in && w && rowss, "null pointer");
    XP_REQUIRE(n_rows > 0 && n > 0, "empty shape %u x %u", n_rows, n);
    const size_t total = size_t(n_rows) * n;
    hipLaunchKernelGGL(rmsnorm_rows_apply_gemma_kernel, dim3(pf_blocks(total)), dim3(kPfThreads), 0,
                       as_stream(stream), out, in, w, rowss, n, eps, total);
    return launched("xp_rmsnorm_rows_apply_gemma");
}

int xp_rmsnorm_heads_rows_gemma(float* out, const float* in, const float* w, uint32_t n_tokens,
                                uint32_t n_heads, uint32_t head_dim, float eps, xp_stream stream) {
    XP_REQUIRE(out && in && w, "null pointer");
    XP_REQUIRE(n_tokens > 0 && n_heads > 0 && head_dim > 0, "empty shape");
    XP_REQUIRE(out != in, "out must not alias in (each row is read after other lanes write)");
    const size_t rows = size_t(n_tokens) * n_heads;
    XP_REQUIRE(rows <= 0xFFFFFFFFull, "too many rows");
    hipLaunchKernelGGL(rmsnorm_heads_rows_gemma_kernel, dim3(pf_row_blocks(rows)), dim3(kPfThreads), 0,
                       as_stream(stream), out, in, w, uint32_t(rows), head_dim, eps);
    return launched("xp_rmsnorm_heads_rows_gemma");
}

int xp_rope_prefill(float* x, uint32_t n_tokens, uint32_t n_heads, uint32_t head_dim, uint32_t pos0,
                    float theta, xp_stream stream) {
    XP_REQUIRE(x, "null pointer");
    XP_REQUIRE(n_tokens > 0 && n_heads > 0 && head_dim > 0 && head_dim % 2 == 0 &&
                   head_dim <= uint32_t(kMaxHeadDim),
               "empty shape, or head_dim=%u odd or above %d", head_dim, kMaxHeadDim);
    XP_REQUIRE(theta > 0.0f, "theta=%g must be positive", double(theta));
    RopeFreq f;
    rope_freq(f, head_dim, theta);
    const size_t total = size_t(n_tokens) * n_heads * (head_dim / 2);
    hipLaunchKernelGGL(rope_prefill_kernel, dim3(pf_blocks(total)), dim3(kPfThreads), 0,
                       as_stream(stream), x, n_heads, head_dim, pos0, f, total);
    return launched("xp_rope_prefill");
}

int xp_kv_append_rows(float* cache, const float* src, uint32_t n_tokens, uint32_t row, uint32_t pos0,
                      xp_stream stream) {
    XP_REQUIRE(cache && src, "null pointer");
    XP_REQUIRE(n_tokens > 0 && row > 0, "empty shape");
    const size_t total = size_t(n_tokens) * row;
    hipLaunchKernelGGL(kv_append_rows_kernel, dim3(pf_blocks(total)), dim3(kPfThreads), 0,
                       as_stream(stream), cache + size_t(pos0) * row, src, total);
    return launched("xp_kv_append_rows");
}

int xp_embed_lookup_rows(float* out, const float* table, const uint32_t* tokens, uint32_t n_tokens,
                         uint32_t n, uint32_t vocab, xp_stream stream) {
    XP_REQUIRE(out && table && tokens, "null pointer");
    XP_REQUIRE(n_tokens > 0 && n > 0 && vocab > 0, "empty shape");
    const size_t total = size_t(n_tokens) * n;
    hipLaunchKernelGGL(embed_lookup_rows_kernel, dim3(pf_blocks(total)), dim3(kPfThreads), 0,
                       as_stream(stream), out, table, tokens, n, vocab, total);
    return launched("xp_embed_lookup_rows");
}

}  // extern "C"
