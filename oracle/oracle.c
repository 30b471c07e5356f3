/*
 * oracle.c — CPU restatement of the reference Gemma-3 decode arithmetic.
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for libxpose and the
 * timed CPU baseline in bench.py; never linked into the product.
 *
 * Line citations are into /root/reference (badnikhil/Xpose). Parallel loops
 * (OpenMP) only split independent output elements; each element's arithmetic
 * is the reference's sequential order, so results do not depend on the
 * thread count.
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

static int g_threads = 0;   /* 0 = OpenMP default */
static int nthreads(void) { return g_threads > 0 ? g_threads : omp_get_max_threads(); }

/* ------------------------------------------------------------------ */
/* Scalar formats                                                       */
/* ------------------------------------------------------------------ */

static float as_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t as_uint(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* fp16_to_fp32, kernels/llm_quant.cl:56-77: integer bit surgery, subnormals
 * normalised by a shift loop, Inf/NaN mantissa kept. */
float xo_fp16_to_fp32(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0u) {
        if (mant == 0u) {
            bits = sign;
        } else {
            uint32_t m = mant;
            int e = -1;
            do { m <<= 1; e++; } while ((m & 0x400u) == 0u);
            m &= 0x3FFu;
            bits = sign | ((uint32_t)(112 - e) << 23) | (m << 13);
        }
    } else if (exp == 31u) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    return as_float(bits);
}

/* Round-to-nearest-even fp32 -> fp16 (the build's KV-cache store; the
 * reference keeps fp32 KV, decode.cpp:1544-1545). */
uint16_t xo_fp32_to_fp16(float f) {
    uint32_t x = as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax >= 0x38800000u) {
        uint32_t r = ax - ((127u - 15u) << 23);
        r = (r + 0x0FFFu + ((r >> 13) & 1u)) >> 13;
        return (uint16_t)(sign | r);
    }
    if (ax <= 0x33000000u) return (uint16_t)sign;
    uint32_t e = ax >> 23;
    uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e;
    uint32_t m = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (m & 1u))) ++m;
    return (uint16_t)(sign | m);
}

/* bf16lo, kernels/llm_matvec.cl:407. */
float xo_bf16_to_fp32(uint32_t h) { return as_float((h & 0xFFFFu) << 16); }

/* ------------------------------------------------------------------ */
/* int4 matvec                                                          */
/* ------------------------------------------------------------------ */

/* q4dot8, kernels/llm_matvec.cl:54-65. */
float xo_q4dot8(uint32_t w, const float* v) {
    float s;
    s  = v[0] * ((float)((w      ) & 15u) - 8.0f);
    s += v[1] * ((float)((w >>  4) & 15u) - 8.0f);
    s += v[2] * ((float)((w >>  8) & 15u) - 8.0f);
    s += v[3] * ((float)((w >> 12) & 15u) - 8.0f);
    s += v[4] * ((float)((w >> 16) & 15u) - 8.0f);
    s += v[5] * ((float)((w >> 20) & 15u) - 8.0f);
    s += v[6] * ((float)((w >> 24) & 15u) - 8.0f);
    s += v[7] * ((float)((w >> 28) & 15u) - 8.0f);
    return s;
}

/* q4dot32, kernels/llm_matvec.cl:68-72. */
float xo_q4dot32(const uint32_t* w4, const float* v) {
    return xo_q4dot8(w4[0], v) + xo_q4dot8(w4[1], v + 8) +
           xo_q4dot8(w4[2], v + 16) + xo_q4dot8(w4[3], v + 24);
}

/* Scale of (block b, column j). fp16 / bf16 quad planes follow the Km4Bf16
 * arrangement sc[(b/4)*cols + j] holding blocks 4q..4q+3 (decode.hpp:369-370,
 * llm_matvec.cl:412-419); fp32 is [b][col] (llm_matvec.cl:187-200). */
float xo_scale_at(const void* sc, int fmt, uint32_t cols, uint32_t b, uint32_t j) {
    if (fmt == 2) return ((const float*)sc)[(size_t)b * cols + j];
    uint32_t h = ((const uint16_t*)sc)[((size_t)(b / 4) * cols + j) * 4 + (b % 4)];
    return fmt == 0 ? xo_fp16_to_fp32(h) : xo_bf16_to_fp32(h);
}

/* part[c] = q4dot32(block of column c) for the 64 columns of one KM4 group
 * block: the reference order per column, vectorisable across columns. */
static void block_dot64(float* part, const uint32_t* blk, const float* v) {
    float d[4][64];
    for (int comp = 0; comp < 4; ++comp) {
        const float* vv = v + 8 * comp;
        float* s = d[comp];
        for (int c = 0; c < 64; ++c)
            s[c] = vv[0] * ((float)(blk[4 * c + comp] & 15u) - 8.0f);
        for (int i = 1; i < 8; ++i)
            for (int c = 0; c < 64; ++c)
                s[c] += vv[i] * ((float)((blk[4 * c + comp] >> (4 * i)) & 15u) - 8.0f);
    }
    for (int c = 0; c < 64; ++c) part[c] = ((d[0][c] + d[1][c]) + d[2][c]) + d[3][c];
}

/* mv_km4, kernels/llm_matvec.cl:187-200 (acc += q4dot32 * scale per block),
 * over a block range of one group; acc carried by the caller. */
static void km4_group(float* acc, const float* in, const uint32_t* wq, const void* sc, int fmt,
                      uint32_t nblk, uint32_t cols, uint32_t g, uint32_t b0, uint32_t b1) {
    float part[64];
    for (uint32_t b = b0; b < b1; ++b) {
        block_dot64(part, wq + ((size_t)g * nblk + b) * 256, in + (size_t)b * 32);
        for (int c = 0; c < 64; ++c) acc[c] += part[c] * xo_scale_at(sc, fmt, cols, b, g * 64 + c);
    }
}

void xo_mv_km4(float* out, const float* in, const uint32_t* wq, const void* sc, int fmt,
               uint32_t rows, uint32_t cols) {
    const uint32_t nblk = rows / 32, G = cols / 64;
#pragma omp parallel for schedule(static) num_threads(nthreads())
    for (int64_t g = 0; g < (int64_t)G; ++g) {
        float acc[64] = {0};
        km4_group(acc, in, wq, sc, fmt, nblk, cols, (uint32_t)g, 0, nblk);
        memcpy(out + g * 64, acc, sizeof acc);
    }
}

/* mv_km4_bs + km4_quad, kernels/llm_matvec.cl:412-434: a quad of scaled
 * block dots is summed first, then added to acc. */
void xo_mv_km4_bs(float* out, const float* in, const uint32_t* wq, const void* sc, int fmt,
                  uint32_t rows, uint32_t cols) {
    const uint32_t nblk = rows / 32, G = cols / 64, nq = nblk / 4;
#pragma omp parallel for schedule(static) num_threads(nthreads())
    for (int64_t g = 0; g < (int64_t)G; ++g) {
        float acc[64] = {0}, a[64], part[64];
        for (uint32_t q = 0; q < nq; ++q) {
            for (uint32_t i = 0; i < 4; ++i) {
                const uint32_t b = q * 4 + i;
                block_dot64(part, wq + ((size_t)g * nblk + b) * 256, in + (size_t)b * 32);
                for (int c = 0; c < 64; ++c) {
                    const float p = part[c] * xo_scale_at(sc, fmt, cols, b, (uint32_t)g * 64 + c);
                    a[c] = i == 0 ? p : a[c] + p;
                }
            }
            for (int c = 0; c < 64; ++c) acc[c] += a[c];
        }
        memcpy(out + g * 64, acc, sizeof acc);
    }
}

/* mv_km4_split, kernels/llm_matvec.cl:339-356: block ranges
 * per = ceil(nblk/split), partial[p*cols + j]. */
void xo_mv_km4_split(float* partial, const float* in, const uint32_t* wq, const void* sc,
                     int fmt, uint32_t rows, uint32_t cols, uint32_t split) {
    const uint32_t nblk = rows / 32, G = cols / 64;
    const uint32_t per = (nblk + split - 1u) / split;
#pragma omp parallel for schedule(static) num_threads(nthreads())
    for (int64_t t = 0; t < (int64_t)G * split; ++t) {
        const uint32_t g = (uint32_t)(t % G), p = (uint32_t)(t / G);
        const uint32_t s0 = p * per, s1 = s0 + per < nblk ? s0 + per : nblk;
        float acc[64] = {0};
        if (s0 < nblk) km4_group(acc, in, wq, sc, fmt, nblk, cols, g, s0, s1);
        memcpy(partial + (size_t)p * cols + (size_t)g * 64, acc, sizeof acc);
    }
}

/* mv_reduce, kernels/llm_matvec.cl:128-135. */
void xo_mv_reduce(float* out, const float* partial, uint32_t cols, uint32_t split) {
    for (uint32_t j = 0; j < cols; ++j) {
        float acc = 0.0f;
        for (uint32_t p = 0; p < split; ++p) acc += partial[(size_t)p * cols + j];
        out[j] = acc;
    }
}

/* matvec_q4 (COL layout), kernels/llm.cl:488-513: the reference's gold. */
void xo_matvec_q4_col(float* out, const float* in, const uint32_t* wq, const float* scale,
                      uint32_t rows, uint32_t cols) {
    const uint32_t nblk = rows / 32;
#pragma omp parallel for schedule(static) num_threads(nthreads())
    for (int64_t jj = 0; jj < (int64_t)cols; ++jj) {
        const uint32_t j = (uint32_t)jj;
        const uint32_t shift = (j & 7u) * 4u;
        float acc = 0.0f;
        for (uint32_t b = 0; b < nblk; ++b) {
            const float s = scale[(size_t)b * cols + j];
            float part = 0.0f;
            for (uint32_t t = 0; t < 32; ++t) {
                const uint32_t k = b * 32 + t;
                const uint32_t word = wq[((size_t)k * cols + j) >> 3];
                const float wv = (float)((word >> shift) & 0x0Fu) - 8.0f;
                part += in[k] * wv;
            }
            acc += part * s;
        }
        out[j] = acc;
    }
}

/* nib(k, j), examples/llm/matvec_bench.cpp:45-55. */
uint32_t xo_nib_hash(uint32_t k, uint32_t j) {
    uint32_t h = k * 2654435761u ^ (j + 0x9e3779b9u) * 2246822519u;
    h ^= h >> 15;
    h *= 2654435761u;
    h ^= h >> 13;
    return h & 15u;
}

/* pack_km4, matvec_bench.cpp:88-99. */
void xo_pack_km4_hash(uint32_t* wq, uint32_t rows, uint32_t cols) {
    const size_t nblk = rows / 32;
    memset(wq, 0, (size_t)rows * cols / 2);
    for (uint32_t j = 0; j < cols; ++j) {
        const size_t base = ((size_t)(j / 64) * nblk * 64 + (j % 64)) * 4;
        for (uint32_t k = 0; k < rows; ++k)
            wq[base + (size_t)(k / 32) * 64 * 4 + ((k >> 3) & 3u)] |=
                xo_nib_hash(k, j) << ((k & 7u) * 4u);
    }
}

/* pack_col, matvec_bench.cpp:58-64. */
void xo_pack_col_hash(uint32_t* wq, uint32_t rows, uint32_t cols) {
    memset(wq, 0, (size_t)rows * cols / 2);
    for (uint32_t k = 0; k < rows; ++k)
        for (uint32_t j = 0; j < cols; ++j)
            wq[((size_t)k * cols + j) >> 3] |= xo_nib_hash(k, j) << ((j & 7u) * 4u);
}

/* KM4 unpack, decode.hpp:46-48: out[k*cols + j] = nibble - 8. */
void xo_unpack_km4(int8_t* out, const uint32_t* wq, uint32_t rows, uint32_t cols) {
    const size_t nblk = rows / 32;
    for (uint32_t j = 0; j < cols; ++j) {
        const size_t base = ((size_t)(j / 64) * nblk * 64 + (j % 64)) * 4;
        for (uint32_t k = 0; k < rows; ++k) {
            const uint32_t w = wq[base + (size_t)(k / 32) * 256 + ((k >> 3) & 3u)];
            out[(size_t)k * cols + j] = (int8_t)((int)((w >> ((k & 7u) * 4u)) & 15u) - 8);
        }
    }
}

/* ------------------------------------------------------------------ */
/* Transformer ops (kernels/llm_transformer.cl)                         */
/* ------------------------------------------------------------------ */

static float rsqrt_ref(float x) { return 1.0f / sqrtf(x); }

/* rmsnorm_sumsq, llm_transformer.cl:96-103. */
void xo_rmsnorm_sumsq(float* partial, const float* in, uint32_t n, uint32_t nparts) {
    for (uint32_t p = 0; p < nparts; ++p) {
        float acc = 0.0f;
        for (uint32_t k = p; k < n; k += nparts) acc += in[k] * in[k];
        partial[p] = acc;
    }
}

/* rmsnorm_apply_gemma, llm_transformer.cl:106-116. */
void xo_rmsnorm_apply_gemma(float* out, const float* in, const float* w, const float* partial,
                            uint32_t n, uint32_t nparts, float eps) {
    float ss = 0.0f;
    for (uint32_t p = 0; p < nparts; ++p) ss += partial[p];
    const float scale = rsqrt_ref(ss / (float)n + eps);
    for (uint32_t i = 0; i < n; ++i) out[i] = in[i] * scale * (1.0f + w[i]);
}

void xo_rmsnorm_gemma2(float* out, const float* in, const float* w, uint32_t n,
                       uint32_t nparts, float eps) {
    float partial[1024];
    if (nparts > 1024) nparts = 1024;
    xo_rmsnorm_sumsq(partial, in, n, nparts);
    xo_rmsnorm_apply_gemma(out, in, w, partial, n, nparts, eps);
}

/* rmsnorm_heads_gemma, llm_transformer.cl:122-134. */
void xo_rmsnorm_heads_gemma(float* out, const float* in, const float* w, uint32_t n_heads,
                            uint32_t head_dim, float eps) {
    for (uint32_t h = 0; h < n_heads; ++h) {
        const uint32_t base = h * head_dim;
        float ss = 0.0f;
        for (uint32_t k = 0; k < head_dim; ++k) ss += in[base + k] * in[base + k];
        const float scale = rsqrt_ref(ss / (float)head_dim + eps);
        for (uint32_t d = 0; d < head_dim; ++d)
            out[base + d] = in[base + d] * scale * (1.0f + w[d]);
    }
}

/* rope, llm_transformer.cl:158-179 (rotate-half, angle via exp2/log2). */
void xo_rope(float* x, uint32_t n_heads, uint32_t head_dim, uint32_t pos, float theta) {
    const uint32_t half_dim = head_dim >> 1;
    for (uint32_t h = 0; h < n_heads; ++h)
        for (uint32_t d = 0; d < half_dim; ++d) {
            const uint32_t base = h * head_dim + d;
            const float frac = (float)(2u * d) / (float)head_dim;
            const float inv = exp2f(-log2f(theta) * frac);
            const float ang = (float)pos * inv;
            const float c = cosf(ang), s = sinf(ang);
            const float lo = x[base], hi = x[base + half_dim];
            x[base] = lo * c - hi * s;
            x[base + half_dim] = lo * s + hi * c;
        }
}

/* tanh_approx + geglu, llm_transformer.cl:213-231. */
static float tanh_approx(float z) {
    z = fminf(fmaxf(z, -10.0f), 10.0f);
    const float e = expf(-2.0f * z);
    return (1.0f - e) / (1.0f + e);
}

void xo_geglu(float* out, const float* gate, const float* up, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) {
        const float g = gate[i];
        const float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
        const float gelu = 0.5f * g * (1.0f + tanh_approx(inner));
        out[i] = gelu * up[i];
    }
}

/* add_residual, llm_transformer.cl:564-568. */
void xo_add_residual(float* x, const float* y, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) x[i] += y[i];
}

/* kv_append, llm_transformer.cl:590-595, into an fp16 cache. */
void xo_kv_append_f16(uint16_t* cache, const float* src, uint32_t n, uint32_t pos) {
    for (uint32_t i = 0; i < n; ++i) cache[(size_t)pos * n + i] = xo_fp32_to_fp16(src[i]);
}

/* attention_scores, llm_transformer.cl:287-305. */
void xo_attention_scores(float* scores, const float* q, const float* kcache, uint32_t n_heads,
                         uint32_t kv_heads, uint32_t head_dim, uint32_t span, float scale,
                         uint32_t kv_start) {
    const uint32_t group = n_heads / kv_heads;
    for (uint32_t h = 0; h < n_heads; ++h)
        for (uint32_t j = 0; j < span; ++j) {
            const uint32_t kvh = h / group;
            const size_t qb = (size_t)h * head_dim;
            const size_t kb = ((size_t)(kv_start + j) * kv_heads + kvh) * head_dim;
            float acc = 0.0f;
            for (uint32_t d = 0; d < head_dim; ++d) acc += q[qb + d] * kcache[kb + d];
            scores[(size_t)h * span + j] = acc * scale;
        }
}

/* softmax_rows, llm_transformer.cl:318-335. */
void xo_softmax_rows(float* x, uint32_t n_rows, uint32_t n_cols) {
    for (uint32_t r = 0; r < n_rows; ++r) {
        float* row = x + (size_t)r * n_cols;
        float m = -INFINITY;
        for (uint32_t j = 0; j < n_cols; ++j) m = fmaxf(m, row[j]);
        float sum = 0.0f;
        for (uint32_t j = 0; j < n_cols; ++j) {
            const float e = expf(row[j] - m);
            row[j] = e;
            sum += e;
        }
        const float inv = 1.0f / sum;
        for (uint32_t j = 0; j < n_cols; ++j) row[j] *= inv;
    }
}

/* attention_apply, llm_transformer.cl:478-497. */
void xo_attention_apply(float* out, const float* probs, const float* vcache, uint32_t n_heads,
                        uint32_t kv_heads, uint32_t head_dim, uint32_t span, uint32_t kv_start) {
    const uint32_t group = n_heads / kv_heads;
    const uint32_t vstride = kv_heads * head_dim;
    for (uint32_t h = 0; h < n_heads; ++h)
        for (uint32_t d = 0; d < head_dim; ++d) {
            const uint32_t kvh = h / group;
            const size_t pb = (size_t)h * span;
            const size_t vb = ((size_t)kv_start * kv_heads + kvh) * head_dim + d;
            float acc = 0.0f;
            for (uint32_t j = 0; j < span; ++j) acc += probs[pb + j] * vcache[vb + (size_t)j * vstride];
            out[(size_t)h * head_dim + d] = acc;
        }
}

void xo_attention_f16(float* out, const float* q, const uint16_t* kcache, const uint16_t* vcache,
                      uint32_t n_heads, uint32_t kv_heads, uint32_t head_dim, uint32_t span,
                      uint32_t kv_start, float scale) {
    const size_t row = (size_t)kv_heads * head_dim;
    const size_t n = (size_t)span * row;
    float* k = (float*)malloc(n * sizeof(float));
    float* v = (float*)malloc(n * sizeof(float));
    float* sc = (float*)malloc((size_t)n_heads * span * sizeof(float));
    for (size_t i = 0; i < n; ++i) {
        k[i] = xo_fp16_to_fp32(kcache[(size_t)kv_start * row + i]);
        v[i] = xo_fp16_to_fp32(vcache[(size_t)kv_start * row + i]);
    }
    xo_attention_scores(sc, q, k, n_heads, kv_heads, head_dim, span, scale, 0);
    xo_softmax_rows(sc, n_heads, span);
    xo_attention_apply(out, sc, v, n_heads, kv_heads, head_dim, span, 0);
    free(k);
    free(v);
    free(sc);
}

/* ------------------------------------------------------------------ */
/* Sampling (kernels/llm_sampling.cl, decode.cpp:1873-1917)             */
/* ------------------------------------------------------------------ */

/* argmax_partial, llm_sampling.cl:57-70: strict > keeps the earliest k. */
void xo_argmax_partial(float* pval, uint32_t* pidx, const float* logits, uint32_t n,
                       uint32_t nparts) {
    for (uint32_t p = 0; p < nparts; ++p) {
        float bv = -INFINITY;
        uint32_t bi = 0u;
        for (uint32_t k = p; k < n; k += nparts) {
            const float v = logits[k];
            if (v > bv) { bv = v; bi = k; }
        }
        pval[p] = bv;
        pidx[p] = bi;
    }
}

/* argmax_reduce, llm_sampling.cl:84-98: (value, index) lexicographic. */
void xo_argmax_reduce(float* oval, uint32_t* oidx, const float* pval, const uint32_t* pidx,
                      uint32_t n, uint32_t nparts) {
    for (uint32_t p = 0; p < nparts; ++p) {
        float bv = -INFINITY;
        uint32_t bi = 0xFFFFFFFFu;
        for (uint32_t k = p; k < n; k += nparts) {
            const float v = pval[k];
            const uint32_t e = pidx[k];
            if (v > bv || (v == bv && e < bi)) { bv = v; bi = e; }
        }
        oval[p] = bv;
        oidx[p] = bi;
    }
}

/* argmax_final, llm_sampling.cl:106-123. */
void xo_argmax_final(float* out, uint32_t* idx_out, const float* pval, const uint32_t* pidx,
                     uint32_t nparts) {
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t p = 0; p < nparts; ++p) {
        const float v = pval[p];
        const uint32_t k = pidx[p];
        if (v > bv || (v == bv && k < bi)) { bv = v; bi = k; }
    }
    out[0] = (float)bi;
    out[1] = bv;
    idx_out[0] = bi;
}

/* vocab -> 4096 -> 64 -> 1 (decode.cpp:1766-1773, decode.hpp argmax_parts). */
uint32_t xo_argmax_tree(const float* logits, uint32_t n, float* val_out) {
    static float v1[4096], v2[64];
    static uint32_t i1[4096], i2[64];
    float out[2];
    uint32_t idx;
    xo_argmax_partial(v1, i1, logits, n, 4096);
    xo_argmax_reduce(v2, i2, v1, i1, 4096, 64);
    xo_argmax_final(out, &idx, v2, i2, 64);
    if (val_out) *val_out = out[1];
    return idx;
}

/* topk4_partial, llm_sampling.cl:318-347. */
void xo_topk4_partial(float* cval, uint32_t* cidx, const float* x, uint32_t n, uint32_t nparts) {
    for (uint32_t p = 0; p < nparts; ++p) {
        float v0 = -INFINITY, v1 = -INFINITY, v2 = -INFINITY, v3 = -INFINITY;
        uint32_t i0 = 0xFFFFFFFFu, i1 = 0xFFFFFFFFu, i2 = 0xFFFFFFFFu, i3 = 0xFFFFFFFFu;
        for (uint32_t e = p; e < n; e += nparts) {
            const float v = x[e];
            if (!(v > v3)) continue;
            if (v > v0) {
                v3 = v2; i3 = i2; v2 = v1; i2 = i1; v1 = v0; i1 = i0; v0 = v; i0 = e;
            } else if (v > v1) {
                v3 = v2; i3 = i2; v2 = v1; i2 = i1; v1 = v; i1 = e;
            } else if (v > v2) {
                v3 = v2; i3 = i2; v2 = v; i2 = e;
            } else {
                v3 = v; i3 = e;
            }
        }
        const uint32_t o = p * 4u;
        cval[o + 0] = v0; cidx[o + 0] = i0;
        cval[o + 1] = v1; cidx[o + 1] = i1;
        cval[o + 2] = v2; cidx[o + 2] = i2;
        cval[o + 3] = v3; cidx[o + 3] = i3;
    }
}

/* topk_partial, llm_sampling.cl:257-281 (k <= 64). */
void xo_topk_partial(float* cval, uint32_t* cidx, const float* x, uint32_t n, uint32_t nparts,
                     uint32_t k) {
    if (k > 64u) k = 64u;
    for (uint32_t p = 0; p < nparts; ++p) {
        float bv[64];
        uint32_t bi[64];
        for (uint32_t j = 0; j < k; ++j) { bv[j] = -INFINITY; bi[j] = 0xFFFFFFFFu; }
        for (uint32_t e = p; e < n; e += nparts) {
            const float v = x[e];
            if (!(v > bv[k - 1u])) continue;
            uint32_t j = k - 1u;
            while (j > 0u && v > bv[j - 1u]) {
                bv[j] = bv[j - 1u];
                bi[j] = bi[j - 1u];
                --j;
            }
            bv[j] = v;
            bi[j] = e;
        }
        for (uint32_t j = 0; j < k; ++j) {
            cval[p * k + j] = bv[j];
            cidx[p * k + j] = bi[j];
        }
    }
}

/* topk_rank_select, llm_sampling.cl:349-369. */
void xo_topk_rank_select(float* oval, uint32_t* oidx, const float* cval, const uint32_t* cidx,
                         uint32_t ncand, uint32_t k) {
    for (uint32_t i = 0; i < ncand; ++i) {
        const float v = cval[i];
        const uint32_t d = cidx[i];
        if (d == 0xFFFFFFFFu) continue;
        uint32_t rank = 0u;
        for (uint32_t j = 0; j < ncand; ++j) {
            const float w = cval[j];
            const uint32_t e = cidx[j];
            if (e == 0xFFFFFFFFu) continue;
            if (w > v || (w == v && e < d)) ++rank;
        }
        if (rank < k) { oval[rank] = v; oidx[rank] = d; }
    }
}

/* topp_cutoff, llm_sampling.cl:399-415. */
void xo_topp_cutoff(float* w, uint32_t k, float p) {
    float total = 0.0f;
    for (uint32_t j = 0; j < k; ++j) total += w[j];
    if (!(total > 0.0f)) return;
    float cum = 0.0f;
    for (uint32_t j = 0; j < k; ++j) {
        if (cum >= p * total) w[j] = 0.0f;
        else cum += w[j];
    }
}

/* multinomial_sample, llm_sampling.cl:424-446. */
void xo_multinomial_sample(float* out, uint32_t* idx_out, const float* w, const uint32_t* idx,
                           uint32_t k, float u) {
    float total = 0.0f;
    for (uint32_t j = 0; j < k; ++j) total += w[j];
    const float target = u * total;
    float cum = 0.0f;
    uint32_t chosen = 0u;
    float cw = 0.0f;
    for (uint32_t j = 0; j < k; ++j) {
        cum += w[j];
        if (w[j] > 0.0f) { chosen = idx[j]; cw = w[j]; }
        if (cum > target) break;
    }
    out[0] = (float)chosen;
    out[1] = cw;
    idx_out[0] = chosen;
}

/* ---- full-vocabulary sampling chain, llm_sampling.cl:130-206, 380-386, 455-488 ---- */

/* apply_temperature, llm_sampling.cl:130-134. */
void xo_apply_temperature(float* logits, float inv_temp, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) logits[i] = logits[i] * inv_temp;
}

/* reduce_max_partial, llm_sampling.cl:156-163: max of strided chain p. */
void xo_reduce_max_partial(float* pmax, const float* x, uint32_t n, uint32_t nparts) {
    for (uint32_t p = 0; p < nparts; ++p) {
        float m = -INFINITY;
        for (uint32_t k = p; k < n; k += nparts) m = fmaxf(m, x[k]);
        pmax[p] = m;
    }
}

/* reduce_max_final, llm_sampling.cl:165-172. */
void xo_reduce_max_final(float* stats, const float* pmax, uint32_t nparts) {
    float m = -INFINITY;
    for (uint32_t p = 0; p < nparts; ++p) m = fmaxf(m, pmax[p]);
    stats[0] = m;
}

/* softmax_exp_partial, llm_sampling.cl:175-191: out[k] = exp(x[k] - max),
 * psum[p] = chain p's sum in chain order. out may alias x. */
void xo_softmax_exp_partial(float* out, float* psum, const float* x, const float* stats,
                            uint32_t n, uint32_t nparts) {
    const float m = stats[0];
    for (uint32_t p = 0; p < nparts; ++p) {
        float sum = 0.0f;
        for (uint32_t k = p; k < n; k += nparts) {
            const float e = expf(x[k] - m);
            out[k] = e;
            sum += e;
        }
        psum[p] = sum;
    }
}

/* reduce_sum_partial, llm_sampling.cl:202-209. */
void xo_reduce_sum_partial(float* out, const float* in, uint32_t n, uint32_t nparts) {
    for (uint32_t p = 0; p < nparts; ++p) {
        float sum = 0.0f;
        for (uint32_t k = p; k < n; k += nparts) sum += in[k];
        out[p] = sum;
    }
}

/* reduce_sum_final, llm_sampling.cl:211-218. */
void xo_reduce_sum_final(float* stats, const float* psum, uint32_t nparts) {
    float sum = 0.0f;
    for (uint32_t p = 0; p < nparts; ++p) sum += psum[p];
    stats[1] = sum;
}

/* softmax_normalize, llm_sampling.cl:220-225. */
void xo_softmax_normalize(float* out, const float* stats, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) out[i] = out[i] / stats[1];
}

/* topk_mask, llm_sampling.cl:380-386: logits below topk_val[k-1] -> -inf. */
void xo_topk_mask(float* logits, const float* topk_val, uint32_t k, uint32_t n) {
    const float t = topk_val[k - 1u];
    for (uint32_t i = 0; i < n; ++i)
        if (logits[i] < t) logits[i] = -INFINITY;
}

/* multinomial_strided, llm_sampling.cl:462-488: walk the chain sums to the
 * owning chain, then that chain's elements; a permuted CDF of w. */
void xo_multinomial_strided(float* out, uint32_t* idx_out, const float* w, const float* psum,
                            const float* stats, uint32_t n, uint32_t nparts, float u) {
    const float target = u * stats[1];
    float cum = 0.0f;
    uint32_t chain = nparts - 1u;
    for (uint32_t p = 0; p < nparts; ++p) {
        const float sp = psum[p];
        if (cum + sp > target) { chain = p; break; }
        cum += sp;
    }
    uint32_t chosen = chain;
    for (uint32_t k = chain; k < n; k += nparts) {
        chosen = k;
        cum += w[k];
        if (cum > target) break;
    }
    out[0] = (float)chosen;
    out[1] = w[chosen];
    idx_out[0] = chosen;
}

/* Philox4x32-10 (Salmon et al., SC'11). */
void xo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        if (r) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c0 = n0; c1 = (uint32_t)p1; c2 = n2; c3 = (uint32_t)p0;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

double xo_philox_uniform(uint32_t seed, uint32_t seq, uint32_t step) {
    const uint32_t c[4] = {step, 0u, 0u, 0u}, k[2] = {seed, seq};
    uint32_t o[4];
    xo_philox4x32_10(c, k, o);
    const uint64_t m = ((uint64_t)o[0] << 21) | (o[1] >> 11);
    return (double)m * (1.0 / 9007199254740992.0);
}

static int better(float av, uint32_t ai, float bv, uint32_t bi) {
    return av > bv || (av == bv && ai < bi);
}

/* Insertion sort by (value desc, index asc): n <= a few hundred here. */
static void sort_cand(float* v, uint32_t* ix, uint32_t n) {
    for (uint32_t i = 1; i < n; ++i) {
        const float cv = v[i];
        const uint32_t ci = ix[i];
        uint32_t j = i;
        while (j > 0 && better(cv, ci, v[j - 1], ix[j - 1])) {
            v[j] = v[j - 1];
            ix[j] = ix[j - 1];
            --j;
        }
        v[j] = cv;
        ix[j] = ci;
    }
}

/* DecodeSession::draw, decode.cpp:1873-1917. The top-k selection keeps the
 * reference's set (nth_element by (value desc, index asc)); the kept set is
 * then walked in that sorted order, where the reference walks nth_element's
 * unspecified order unless top-p sorts it. */
uint32_t xo_draw(float* val, uint32_t* idx, uint32_t n, float temperature, uint32_t top_k,
                 float top_p, double u) {
    if (n == 0) return 0;
    const float t = temperature > 0.0f ? temperature : 1.0f;
    sort_cand(val, idx, n);
    const uint32_t k = top_k ? (top_k < n ? top_k : n) : n;
    n = k;
    float maxl = -INFINITY;
    for (uint32_t i = 0; i < n; ++i) maxl = fmaxf(maxl, val[i]);
    double sum = 0;
    for (uint32_t i = 0; i < n; ++i) {
        val[i] = expf((val[i] - maxl) / t);
        sum += val[i];
    }
    if (top_p > 0.0f && top_p < 1.0f && sum > 0) {
        double acc = 0, cut = top_p * sum;
        uint32_t keep = 0;
        for (; keep < n; ++keep) {
            acc += val[keep];
            if (acc >= cut) break;
        }
        n = n < keep + 1 ? n : keep + 1;
        sum = 0;
        for (uint32_t i = 0; i < n; ++i) sum += val[i];
    }
    double r = u * sum;
    for (uint32_t i = 0; i < n; ++i) {
        r -= val[i];
        if (r <= 0) return idx[i];
    }
    return idx[n - 1];
}

/* ------------------------------------------------------------------ */
/* Full decode step                                                     */
/* ------------------------------------------------------------------ */

static int g_fmt = 0;   /* scale format of the model in xo_forward */
static void mv(float* out, const float* in, const xo_qweight* w) {
    xo_mv_km4(out, in, w->wq, w->sc, g_fmt, w->rows, w->cols);
}

void xo_embed(float* x, const xo_model* m, uint32_t token) {
    if (m->embed) {   /* the GGUF row (RowReader::read), times the scale */
        const float sc = sqrtf((float)m->hidden);
        for (uint32_t k = 0; k < m->hidden; ++k) x[k] = m->embed[(size_t)token * m->hidden + k] * sc;
        return;
    }
    const xo_qweight* e = &m->lm_head;
    const uint32_t nblk = e->rows / 32;
    const size_t base = ((size_t)(token / 64) * nblk * 64 + (token % 64)) * 4;
    const float sc = sqrtf((float)m->hidden);
    for (uint32_t k = 0; k < e->rows; ++k) {
        const uint32_t w = e->wq[base + (size_t)(k / 32) * 256 + ((k >> 3) & 3u)];
        const float q = (float)((int)((w >> ((k & 7u) * 4u)) & 15u) - 8);
        const float v = q * xo_scale_at(e->sc, m->scale_fmt, e->cols, k / 32, token);
        x[k] = v * sc;
    }
}

static float* g_x = NULL;   /* residual stream carried between calls */
static uint32_t g_x_n = 0;

int xo_forward(const xo_model* m, uint32_t token, uint32_t pos, float* logits, int threads) {
    const uint32_t H = m->hidden, F = m->ffn, hd = m->head_dim;
    const uint32_t qd = m->n_heads * hd, kvd = m->n_kv_heads * hd;
    const uint32_t seq_len = pos + 1;
    const float eps = m->rms_eps;
    const float ascale = 1.0f / sqrtf((float)hd);
    if (pos >= m->max_seq || token >= m->vocab) return -1;
    g_threads = threads;
    g_fmt = m->scale_fmt;

    float* x = (float*)malloc(H * sizeof(float));
    float* xb = (float*)malloc((H > qd ? H : qd) * sizeof(float));
    float* xb2 = (float*)malloc(H * sizeof(float));
    float* q_raw = (float*)malloc(qd * sizeof(float));
    float* q = (float*)malloc(qd * sizeof(float));
    float* k_raw = (float*)malloc(kvd * sizeof(float));
    float* k = (float*)malloc(kvd * sizeof(float));
    float* v = (float*)malloc(kvd * sizeof(float));
    float* att = (float*)malloc(qd * sizeof(float));
    float* g = (float*)malloc(F * sizeof(float));
    float* u = (float*)malloc(F * sizeof(float));
    float* hb = (float*)malloc(F * sizeof(float));

    xo_embed(x, m, token);   /* write_embedding, decode.cpp:1618-1627 */
    for (uint32_t l = 0; l < m->n_layers; ++l) {
        const xo_layer* w = &m->layers[l];
        const int global = m->global_every == 0 || (l + 1) % m->global_every == 0;
        const float theta = global ? m->theta_global : m->theta_local;
        const uint32_t win = global ? 0u : m->sliding_window;
        const uint32_t kv_start = (win == 0 || seq_len <= win) ? 0u : seq_len - win;
        const uint32_t span = seq_len - kv_start;

        xo_rmsnorm_gemma2(xb, x, w->attn_norm, H, 64, eps);
        mv(q_raw, xb, &w->q);
        mv(k_raw, xb, &w->k);
        mv(v, xb, &w->v);
        xo_rmsnorm_heads_gemma(q, q_raw, w->q_norm, m->n_heads, hd, eps);
        xo_rmsnorm_heads_gemma(k, k_raw, w->k_norm, m->n_kv_heads, hd, eps);
        xo_rope(q, m->n_heads, hd, pos, theta);
        xo_rope(k, m->n_kv_heads, hd, pos, theta);
        xo_kv_append_f16(w->kcache, k, kvd, pos);
        xo_kv_append_f16(w->vcache, v, kvd, pos);
        xo_attention_f16(att, q, w->kcache, w->vcache, m->n_heads, m->n_kv_heads, hd, span,
                         kv_start, ascale);
        mv(xb, att, &w->o);
        xo_rmsnorm_gemma2(xb2, xb, w->post_attn_norm, H, 64, eps);
        xo_add_residual(x, xb2, H);

        xo_rmsnorm_gemma2(xb, x, w->ffn_norm, H, 64, eps);
        mv(g, xb, &w->gate);
        mv(u, xb, &w->up);
        xo_geglu(hb, g, u, F);
        mv(xb, hb, &w->down);
        xo_rmsnorm_gemma2(xb2, xb, w->post_ffn_norm, H, 64, eps);
        xo_add_residual(x, xb2, H);
    }
    xo_rmsnorm_gemma2(xb, x, m->final_norm, H, 64, eps);
    if (logits) mv(logits, xb, &m->lm_head);

    if (g_x_n < H) {
        free(g_x);
        g_x = (float*)malloc(H * sizeof(float));
        g_x_n = H;
    }
    memcpy(g_x, x, H * sizeof(float));
    free(x); free(xb); free(xb2); free(q_raw); free(q); free(k_raw); free(k); free(v);
    free(att); free(g); free(u); free(hb);
    return 0;
}

int xo_generate_greedy(const xo_model* m, const uint32_t* prompt, uint32_t n_prompt,
                       uint32_t n_gen, uint32_t* out, int threads) {
    if (n_prompt == 0) return -1;
    float* logits = (float*)malloc((size_t)m->vocab * sizeof(float));
    uint32_t pos = 0;
    int rc = 0;
    for (uint32_t i = 0; i < n_prompt && rc == 0; ++i, ++pos)
        rc = xo_forward(m, prompt[i], pos, i + 1 == n_prompt ? logits : NULL, threads);
    for (uint32_t s = 0; s < n_gen && rc == 0; ++s, ++pos) {
        const uint32_t tok = xo_argmax_tree(logits, m->vocab, NULL);   /* sample first */
        out[s] = tok;
        rc = xo_forward(m, tok, pos, logits, threads);
    }
    free(logits);
    return rc;
}

/* ------------------------------------------------------------------ */
/* GGUF load path                                                       */
/* ------------------------------------------------------------------ */

static uint16_t rd_u16(const uint8_t* p) { uint16_t v; memcpy(&v, p, 2); return v; }
static float rd_half(const uint8_t* p) { return xo_fp16_to_fp32(rd_u16(p)); }

/* get_scale_min_k4, gguf.cpp:436-446. */
static void k4_scale_min(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* GGUFFile::dequantize, gguf.cpp:448-645, in the reference's loop order. */
int xo_dequantize(uint32_t type, const void* src, float* dst, uint64_t n) {
    const uint8_t* p = (const uint8_t*)src;
    uint64_t b, i;
    int j, l;
    switch (type) {
        case 0: /* F32, :456-458 */
            memcpy(dst, p, (size_t)n * 4);
            return 0;
        case 1: /* F16, :460-466 */
            for (i = 0; i < n; ++i) dst[i] = rd_half(p + i * 2);
            return 0;
        case 30: /* BF16, :468-476 */
            for (i = 0; i < n; ++i) dst[i] = as_float((uint32_t)rd_u16(p + i * 2) << 16);
            return 0;
        case 2: /* Q4_0, :478-494 */
            if (n % 32) return -1;
            for (b = 0; b < n / 32; ++b) {
                const uint8_t* blk = p + b * 18;
                const float d = rd_half(blk);
                const uint8_t* qs = blk + 2;
                float* y = dst + b * 32;
                for (j = 0; j < 16; ++j) {
                    y[j] = (float)((int)(qs[j] & 0x0F) - 8) * d;
                    y[j + 16] = (float)((int)(qs[j] >> 4) - 8) * d;
                }
            }
            return 0;
        case 3: /* Q4_1, :496-512 */
            if (n % 32) return -1;
            for (b = 0; b < n / 32; ++b) {
                const uint8_t* blk = p + b * 20;
                const float d = rd_half(blk), m = rd_half(blk + 2);
                const uint8_t* qs = blk + 4;
                float* y = dst + b * 32;
                for (j = 0; j < 16; ++j) {
                    y[j] = (float)(qs[j] & 0x0F) * d + m;
                    y[j + 16] = (float)(qs[j] >> 4) * d + m;
                }
            }
            return 0;
        case 6: /* Q5_0, :514-549 */
        case 7: /* Q5_1 */ {
            const int is_1 = type == 7;
            const size_t stride = is_1 ? 24 : 22;
            if (n % 32) return -1;
            for (b = 0; b < n / 32; ++b) {
                const uint8_t* blk = p + b * stride;
                const float d = rd_half(blk);
                const float m = is_1 ? rd_half(blk + 2) : 0.0f;
                uint32_t qh;
                memcpy(&qh, blk + (is_1 ? 4 : 2), 4);
                const uint8_t* qs = blk + (is_1 ? 8 : 6);
                float* y = dst + b * 32;
                for (j = 0; j < 16; ++j) {
                    const uint8_t xh0 = (uint8_t)(((qh >> (j + 0)) << 4) & 0x10);
                    const uint8_t xh1 = (uint8_t)((qh >> (j + 12)) & 0x10);
                    const int q0 = (int)((qs[j] & 0x0F) | xh0);
                    const int q1 = (int)((qs[j] >> 4) | xh1);
                    if (is_1) {
                        y[j] = (float)q0 * d + m;
                        y[j + 16] = (float)q1 * d + m;
                    } else {
                        y[j] = (float)(q0 - 16) * d;
                        y[j + 16] = (float)(q1 - 16) * d;
                    }
                }
            }
            return 0;
        }
        case 8: /* Q8_0, :551-562 */
            if (n % 32) return -1;
            for (b = 0; b < n / 32; ++b) {
                const uint8_t* blk = p + b * 34;
                const float d = rd_half(blk);
                const int8_t* qs = (const int8_t*)(blk + 2);
                for (j = 0; j < 32; ++j) dst[b * 32 + j] = (float)qs[j] * d;
            }
            return 0;
        case 12: /* Q4_K, :564-595 */
            if (n % 256) return -1;
            for (b = 0; b < n / 256; ++b) {
                const uint8_t* blk = p + b * 144;
                const float d = rd_half(blk), dmin = rd_half(blk + 2);
                const uint8_t* scales = blk + 4;
                const uint8_t* qs = blk + 16;
                float* y = dst + b * 256;
                int is = 0;
                for (j = 0; j < 256; j += 64) {
                    uint8_t sc, m;
                    k4_scale_min(is + 0, scales, &sc, &m);
                    const float d1 = d * sc, m1 = dmin * m;
                    k4_scale_min(is + 1, scales, &sc, &m);
                    const float d2 = d * sc, m2 = dmin * m;
                    for (l = 0; l < 32; ++l) *y++ = d1 * (float)(qs[l] & 0xF) - m1;
                    for (l = 0; l < 32; ++l) *y++ = d2 * (float)(qs[l] >> 4) - m2;
                    qs += 32;
                    is += 2;
                }
            }
            return 0;
        case 14: /* Q6_K, :597-631 */
            if (n % 256) return -1;
            for (b = 0; b < n / 256; ++b) {
                const uint8_t* blk = p + b * 210;
                const uint8_t* ql = blk;
                const uint8_t* qh = blk + 128;
                const int8_t* sc = (const int8_t*)(blk + 192);
                const float d = rd_half(blk + 208);
                float* y = dst + b * 256;
                int n2;
                for (n2 = 0; n2 < 256; n2 += 128) {
                    for (l = 0; l < 32; ++l) {
                        const int is = l / 16;
                        const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        y[l + 0] = d * sc[is + 0] * (float)q1;
                        y[l + 32] = d * sc[is + 2] * (float)q2;
                        y[l + 64] = d * sc[is + 4] * (float)q3;
                        y[l + 96] = d * sc[is + 6] * (float)q4;
                    }
                    y += 128;
                    ql += 64;
                    qh += 32;
                    sc += 8;
                }
            }
            return 0;
        default:
            return -1;
    }
}

/* quantise, decode.cpp:101-104: round half away from zero, +8, clamp. */
uint32_t xo_quantise(float v, float inv_scale) {
    long r = lroundf(v * inv_scale);
    int q = (int)r + 8;
    return (uint32_t)(q < 0 ? 0 : (q > 15 ? 15 : q));
}

/* best_bf16_scale, decode.cpp:127-151: the two bf16 values around s0 (s0
 * truncated, and one bf16 ulp up), the one with the smaller double-precision
 * squared block error, the lower on a tie. */
static double bf16_err(const float* blk, float s) {
    if (!(s > 0.0f)) return INFINITY;
    const float inv = 1.0f / s;
    double e = 0.0;
    for (int t = 0; t < 32; ++t) {
        const double d = (double)((int)xo_quantise(blk[t], inv) - 8) * (double)s - (double)blk[t];
        e += d * d;
    }
    return e;
}

float xo_best_bf16_scale(const float* blk, float s0) {
    if (!(s0 > 0.0f)) return 0.0f;
    const uint32_t ulo = as_uint(s0) & 0xFFFF0000u;
    const float lo = as_float(ulo), hi = as_float(ulo + 0x10000u);
    return bf16_err(blk, lo) <= bf16_err(blk, hi) ? lo : hi;
}

/* pack_group (decode.cpp:177-229, Km4 branch) over every column group, then
 * pack_scales_bf16_cols (:157-172) for the bf16 plane. */
void xo_pack_int4(const float* w, uint32_t rows, uint32_t cols, int bf16, uint32_t* wq,
                  void* scv) {
    const uint32_t nblk = rows / 32;
    float* scales = (float*)malloc((size_t)nblk * cols * sizeof(float));
    for (uint32_t group = 0; group < cols / 64; ++group) {
        const float* cols64 = w + (size_t)group * 64 * rows;
        const uint32_t j0 = group * 64;
        float inv[64];
        for (uint32_t b = 0; b < nblk; ++b) {
            for (uint32_t c = 0; c < 64; ++c) {
                const float* r = cols64 + (size_t)c * rows + b * 32;
                float amax = 0.0f;
                for (uint32_t t = 0; t < 32; ++t) {
                    const float a = fabsf(r[t]);
                    if (a > amax) amax = a;
                }
                const float s = bf16 ? xo_best_bf16_scale(r, amax / 7.0f) : amax / 7.0f;
                scales[(size_t)b * cols + j0 + c] = s;
                inv[c] = s > 0.0f ? 1.0f / s : 0.0f;
            }
            const size_t base = ((size_t)group * nblk + b) * 64;
            for (uint32_t c = 0; c < 64; ++c) {
                uint32_t v4[4] = {0, 0, 0, 0};
                for (uint32_t t = 0; t < 32; ++t) {
                    const uint32_t k = b * 32 + t;
                    v4[(t >> 3) & 3u] |= xo_quantise(cols64[(size_t)c * rows + k], inv[c])
                                         << ((t & 7u) * 4);
                }
                uint32_t* d = wq + (base + c) * 4;
                d[0] = v4[0]; d[1] = v4[1]; d[2] = v4[2]; d[3] = v4[3];
            }
        }
    }
    if (bf16) {
        uint32_t* out = (uint32_t*)scv;
        for (uint32_t q = 0; q < nblk / 4; ++q)
            for (uint32_t j = 0; j < cols; ++j) {
                const size_t d = ((size_t)q * cols + j) * 2;
                out[d] = 0;
                out[d + 1] = 0;
                for (uint32_t i = 0; i < 4; ++i) {
                    const uint32_t bits = as_uint(scales[(size_t)(q * 4 + i) * cols + j]) >> 16;
                    out[d + (i >> 1)] |= bits << ((i & 1u) * 16);
                }
            }
    } else {
        memcpy(scv, scales, (size_t)nblk * cols * sizeof(float));
    }
    free(scales);
}

/* ------------------------------------------------------------------ */
/* Native-format repack (examples/llm/quant_repack.cpp)                 */
/* ------------------------------------------------------------------ */

/* quant_repack.cpp's fp16() (:8-28) is llm_quant.cl's decoder again:
 * xo_fp16_to_fp32. get_scale_min_k4 (:35-43): k4_scale_min above. */

/* extract_q8_0 / _q5_0 / _q4_k / _q6_k, quant_repack.cpp:62-127: one row's
 * raw (unbiased) quants, its scales (granularity 32, Q6_K 16) and, for Q4_K,
 * its biases. */
static void rq_extract(uint32_t type, const uint8_t* row, uint32_t cols, uint8_t* qraw,
                       float* scale, float* bias) {
    uint32_t b, j, s, l, h, g;
    switch (type) {
        case 8:
            for (b = 0; b < cols / 32; ++b) {
                const uint8_t* blk = row + (size_t)b * 34;
                scale[b] = rd_half(blk);
                for (j = 0; j < 32; ++j) qraw[b * 32 + j] = blk[2 + j];
            }
            break;
        case 6:
            for (b = 0; b < cols / 32; ++b) {
                const uint8_t* blk = row + (size_t)b * 22;
                uint32_t qh;
                scale[b] = rd_half(blk);
                qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                     ((uint32_t)blk[5] << 24);
                for (j = 0; j < 32; ++j) {
                    const uint32_t byte = blk[6 + j % 16];
                    const uint32_t lo = j < 16 ? (byte & 0xF) : (byte >> 4);
                    qraw[b * 32 + j] = (uint8_t)(lo | (((qh >> j) & 1u) << 4));
                }
            }
            break;
        case 12:
            for (b = 0; b < cols / 256; ++b) {
                const uint8_t* blk = row + (size_t)b * 144;
                const float dd = rd_half(blk), dmin = rd_half(blk + 2);
                for (s = 0; s < 8; ++s) {
                    uint8_t sc, mn;
                    k4_scale_min((int)s, blk + 4, &sc, &mn);
                    scale[b * 8 + s] = dd * (float)sc;
                    bias[b * 8 + s] = dmin * (float)mn;
                    for (l = 0; l < 32; ++l) {
                        const uint32_t byte = blk[16 + (s / 2) * 32 + l];
                        qraw[b * 256 + s * 32 + l] = (uint8_t)((s & 1) ? (byte >> 4) : (byte & 0xF));
                    }
                }
            }
            break;
        case 14:
            for (b = 0; b < cols / 256; ++b) {
                const uint8_t* blk = row + (size_t)b * 210;
                const float dd = rd_half(blk + 208);
                for (h = 0; h < 2; ++h)
                    for (g = 0; g < 4; ++g)
                        for (l = 0; l < 32; ++l) {
                            const uint32_t byte = blk[h * 64 + l + (g & 1) * 32];
                            const uint32_t lo = g < 2 ? (byte & 0xF) : (byte >> 4);
                            const uint32_t hi = (blk[128 + h * 32 + l] >> (2 * g)) & 3u;
                            const uint32_t r = h * 128 + g * 32 + l;
                            qraw[b * 256 + r] = (uint8_t)(lo | (hi << 4));
                            if (l % 16 == 0)
                                scale[(b * 256 + r) / 16] =
                                    dd * (float)(int8_t)blk[192 + h * 8 + l / 16 + 2 * g];
                        }
            }
            break;
    }
}

/* repack(), quant_repack.cpp:135-217: the planes (sized for the padded
 * rows) are zeroed, then each row's extract is interleaved at slot
 * idx = (g nkb + kb) 64 + t. Returns -1 where repack() returns false. */
int xo_rq_repack(uint32_t type, const void* src, uint32_t rows, uint32_t cols, uint32_t* quant,
                 uint32_t* high, float* scale, float* bias) {
    uint32_t gran = 32, qwords = 4, hwords = 0, nkb, padded, r, kb, j;
    int has_bias = 0;
    size_t slots, row_bytes;
    uint8_t* qraw;
    float *rs, *rb;
    if (cols == 0 || cols % 32 != 0 || rows == 0) return -1;
    switch (type) {
        case 8: qwords = 8; row_bytes = (size_t)(cols / 32) * 34; break;
        case 6: hwords = 1; row_bytes = (size_t)(cols / 32) * 22; break;
        case 12:
            if (cols % 256) return -1;
            has_bias = 1;
            row_bytes = (size_t)(cols / 256) * 144;
            break;
        case 14:
            if (cols % 256) return -1;
            hwords = 2;
            gran = 16;
            row_bytes = (size_t)(cols / 256) * 210;
            break;
        default: return -1;
    }
    nkb = cols / 32;
    padded = (rows + 63) / 64 * 64;
    slots = (size_t)(padded / 64) * nkb * 64;
    memset(quant, 0, slots * qwords * 4);
    if (hwords) memset(high, 0, slots * hwords * 4);
    memset(scale, 0, slots * (32 / gran) * 4);
    if (has_bias) memset(bias, 0, slots * 4);
    qraw = (uint8_t*)malloc(cols);
    rs = (float*)malloc((size_t)(cols / gran) * 4);
    rb = (float*)malloc((size_t)(cols / 32) * 4);
    for (r = 0; r < rows; ++r) {
        const uint32_t g = r / 64, t = r % 64;
        rq_extract(type, (const uint8_t*)src + (size_t)r * row_bytes, cols, qraw, rs, rb);
        for (kb = 0; kb < nkb; ++kb) {
            const size_t idx = ((size_t)g * nkb + kb) * 64 + t;
            for (j = 0; j < 32; ++j) {
                const uint32_t q = qraw[kb * 32 + j];
                if (type == 8) {
                    quant[idx * 8 + j / 4] |= q << (8 * (j % 4));
                } else {
                    quant[idx * 4 + j / 8] |= (q & 0xFu) << (4 * (j % 8));
                    if (type == 6) high[idx] |= ((q >> 4) & 1u) << j;
                    else if (type == 14) high[idx * 2 + j / 16] |= ((q >> 4) & 3u) << (2 * (j % 16));
                }
            }
            if (gran == 16) {
                scale[idx * 2] = rs[kb * 2];
                scale[idx * 2 + 1] = rs[kb * 2 + 1];
            } else {
                scale[idx] = rs[kb];
            }
            if (has_bias) bias[idx] = rb[kb];
        }
    }
    free(qraw);
    free(rs);
    free(rb);
    return 0;
}

/* reconstruct(), quant_repack.cpp:219-239. */
float xo_rq_reconstruct(uint32_t type, uint32_t nkb, const uint32_t* quant, const uint32_t* high,
                        const float* scale, const float* bias, uint32_t r, uint32_t k) {
    const uint32_t g = r / 64, tt = r % 64, kb = k / 32, j = k % 32;
    const size_t idx = ((size_t)g * nkb + kb) * 64 + tt;
    uint32_t q;
    if (type == 8) {
        const uint32_t byte = (quant[idx * 8 + j / 4] >> (8 * (j % 4))) & 0xFFu;
        return scale[idx] * (float)((int)(byte ^ 0x80u) - 128);
    }
    q = (quant[idx * 4 + j / 8] >> (4 * (j % 8))) & 0xFu;
    if (type == 6) {
        q |= ((high[idx] >> j) & 1u) << 4;
        return scale[idx] * (float)((int)q - 16);
    }
    if (type == 14) {
        q |= ((high[idx * 2 + j / 16] >> (2 * (j % 16))) & 3u) << 4;
        return scale[idx * 2 + j / 16] * (float)((int)q - 32);
    }
    return scale[idx] * (float)q - bias[idx];
}

/* ------------------------------------------------------------------ */
/* Prefill shapes (kernels/llm_sampling.cl:496-736), row-indexed twins  */
/* ------------------------------------------------------------------ */

/* softmax_rows_stats, llm_sampling.cl:527-547: per row max and sum of exp;
 * a row with no finite maximum gives (0, 1). */
void xo_softmax_rows_stats(float* stats, const float* x, uint32_t n_rows, uint32_t n_cols) {
    uint32_t r, j;
    for (r = 0; r < n_rows; ++r) {
        const float* row = x + (size_t)r * n_cols;
        float m = -INFINITY, s = 0.0f;
        for (j = 0; j < n_cols; ++j) m = fmaxf(m, row[j]);
        if (!isfinite(m)) {
            stats[2 * r] = 0.0f;
            stats[2 * r + 1] = 1.0f;
            continue;
        }
        for (j = 0; j < n_cols; ++j) s += expf(row[j] - m);
        stats[2 * r] = m;
        stats[2 * r + 1] = s;
    }
}

/* softmax_rows_apply, llm_sampling.cl:549-556. */
void xo_softmax_rows_apply(float* x, const float* stats, uint32_t n_rows, uint32_t n_cols) {
    size_t i;
    for (i = 0; i < (size_t)n_rows * n_cols; ++i) {
        const size_t r = i / n_cols;
        x[i] = expf(x[i] - stats[2 * r]) / stats[2 * r + 1];
    }
}

/* attention_scores_prefill, llm_sampling.cl:574-600: scores[h][qi][t],
 * causal (t <= q_offset + qi) and, when window != 0, t + window > qpos;
 * masked entries are -inf. */
void xo_attention_scores_prefill(float* scores, const float* q, const float* kcache,
                                 uint32_t n_heads, uint32_t kv_heads, uint32_t head_dim,
                                 uint32_t n_query, uint32_t seq_len, uint32_t q_offset,
                                 uint32_t window, float scale) {
    const size_t total = (size_t)n_heads * n_query * seq_len;
    const uint32_t group = n_heads / kv_heads;
    size_t i;
    for (i = 0; i < total; ++i) {
        const uint32_t t = (uint32_t)(i % seq_len);
        const uint32_t hq = (uint32_t)(i / seq_len);
        const uint32_t qi = hq % n_query, h = hq / n_query;
        const uint32_t qpos = q_offset + qi;
        const size_t qb = ((size_t)h * n_query + qi) * head_dim;
        const size_t kb = ((size_t)t * kv_heads + h / group) * head_dim;
        float acc = 0.0f;
        uint32_t d;
        if (t > qpos || (window != 0u && t + window <= qpos)) {
            scores[i] = -INFINITY;
            continue;
        }
        for (d = 0; d < head_dim; ++d) acc += q[qb + d] * kcache[kb + d];
        scores[i] = acc * scale;
    }
}

/* attention_apply_prefill, llm_sampling.cl:605-627:
 * out[h][qi][d] = sum_t probs[h][qi][t] v[t][kv_head(h)][d]. */
void xo_attention_apply_prefill(float* out, const float* probs, const float* vcache,
                                uint32_t n_heads, uint32_t kv_heads, uint32_t head_dim,
                                uint32_t n_query, uint32_t seq_len) {
    const size_t total = (size_t)n_heads * n_query * head_dim;
    const uint32_t group = n_heads / kv_heads, vstride = kv_heads * head_dim;
    size_t i;
    for (i = 0; i < total; ++i) {
        const uint32_t d = (uint32_t)(i % head_dim);
        const uint32_t hq = (uint32_t)(i / head_dim);
        const uint32_t qi = hq % n_query, h = hq / n_query;
        const size_t pb = ((size_t)h * n_query + qi) * seq_len;
        const uint32_t vb = (h / group) * head_dim + d;
        float acc = 0.0f;
        uint32_t t;
        for (t = 0; t < seq_len; ++t) acc += probs[pb + t] * vcache[(size_t)t * vstride + vb];
        out[i] = acc;
    }
}

/* rmsnorm_rows_sumsq, llm_sampling.cl:634-642. */
void xo_rmsnorm_rows_sumsq(float* rowss, const float* in, uint32_t n_rows, uint32_t n) {
    uint32_t r, j;
    for (r = 0; r < n_rows; ++r) {
        float ss = 0.0f;
        for (j = 0; j < n; ++j) {
            const float v = in[(size_t)r * n + j];
            ss += v * v;
        }
        rowss[r] = ss;
    }
}

/* rmsnorm_rows_apply_gemma, llm_sampling.cl:645-656. */
void xo_rmsnorm_rows_apply_gemma(float* out, const float* in, const float* w, const float* rowss,
                                 uint32_t n_rows, uint32_t n, float eps) {
    size_t i;
    for (i = 0; i < (size_t)n_rows * n; ++i) {
        const size_t r = i / n, j = i - r * n;
        const float scale = rsqrt_ref(rowss[r] / (float)n + eps);
        out[i] = in[i] * scale * (1.0f + w[j]);
    }
}

/* rmsnorm_heads_rows_gemma, llm_sampling.cl:659-672: [token][head][head_dim]. */
void xo_rmsnorm_heads_rows_gemma(float* out, const float* in, const float* w, uint32_t n_tokens,
                                 uint32_t n_heads, uint32_t head_dim, float eps) {
    const size_t total = (size_t)n_tokens * n_heads * head_dim;
    size_t i;
    for (i = 0; i < total; ++i) {
        const uint32_t d = (uint32_t)(i % head_dim);
        const size_t base = (i / head_dim) * head_dim;
        float ss = 0.0f;
        uint32_t j;
        for (j = 0; j < head_dim; ++j) {
            const float v = in[base + j];
            ss += v * v;
        }
        out[i] = in[i] * rsqrt_ref(ss / (float)head_dim + eps) * (1.0f + w[d]);
    }
}

/* rope_prefill, llm_sampling.cl:687-708: rotate-half, token ti at pos0 + ti. */
void xo_rope_prefill(float* x, uint32_t n_tokens, uint32_t n_heads, uint32_t head_dim,
                     uint32_t pos0, float theta) {
    const uint32_t hdhalf = head_dim / 2u;
    const size_t total = (size_t)n_tokens * n_heads * hdhalf;
    size_t i;
    for (i = 0; i < total; ++i) {
        const uint32_t d = (uint32_t)(i % hdhalf);
        const size_t th = i / hdhalf;
        const uint32_t ti = (uint32_t)(th / n_heads);
        const size_t base = th * head_dim + d;
        const float frac = (float)(2u * d) / (float)head_dim;
        const float inv = exp2f(-log2f(theta) * frac);
        const float ang = (float)(pos0 + ti) * inv;
        const float c = cosf(ang), s = sinf(ang);
        const float a = x[base], b = x[base + hdhalf];
        x[base] = a * c - b * s;
        x[base + hdhalf] = b * c + a * s;
    }
}

/* kv_append_rows, llm_sampling.cl:714-721 (fp32 cache [t][row]). */
void xo_kv_append_rows(float* cache, const float* src, uint32_t n_tokens, uint32_t row,
                       uint32_t pos0) {
    memcpy(cache + (size_t)pos0 * row, src, (size_t)n_tokens * row * 4);
}

/* embed_lookup_rows, llm_sampling.cl:728-736. */
void xo_embed_lookup_rows(float* out, const float* table, const uint32_t* tokens,
                          uint32_t n_tokens, uint32_t n) {
    uint32_t t;
    for (t = 0; t < n_tokens; ++t)
        memcpy(out + (size_t)t * n, table + (size_t)tokens[t] * n, (size_t)n * 4);
}
