/*
 * oracle.h — CPU restatement of the reference (badnikhil/Xpose "Vulkore")
 * Gemma-3 decode arithmetic. TEST INFRASTRUCTURE ONLY: tests/, the graft
 * entry's smoke() and bench.py's cpu_baseline leg may load it, as the checker
 * or the timed CPU baseline. The product (libxpose) never calls it.
 *
 * Every function follows the reference source line for line in its
 * arithmetic (operation order, which products are rounded, tie rules); each
 * cites the file:line it restates. Built with -ffp-contract=off so each
 * written a*b+c rounds twice, as OpenCL C without contraction does.
 *
 * Pinning (what checks each function beyond restating it; the CPU tests in
 * tests/test_matvec.py, test_transformer.py, test_sampling.py, test_session.py):
 *  xo_fp16_to_fp32          all 65536 patterns vs numpy float16 (exact)
 *  xo_q4dot8/32, mv_*       nibble closed form; float64 brute force; COL gold
 *                           == KM4 on the reference's nib() fixture
 *                           (matvec_bench.cpp:45-55) at all six shapes
 *  xo_rmsnorm_*             numpy closed form (rtol 1e-5)
 *  xo_rope                  rotation invariants (norm kept, pos 0 identity,
 *                           composition pos a then b == a+b)
 *  xo_geglu                 numpy tanh-GELU
 *  attention                numpy softmax(q.K)V, rows sum to 1, window
 *                           negative control (kernel_tests.cpp:483-621)
 *  argmax / topk            planted max 190037 (kernel_tests.cpp:695-711),
 *                           ties -> lowest index (sampling_test.cpp:171-178),
 *                           sort-based top-k with duplicates (:427-480)
 *  topp / multinomial       known answers of sampling_test.cpp:537-607
 *  vocab softmax chain      numpy float64 softmax (rtol 1e-5), rows sum to 1,
 *                           chain max/sum vs numpy over the same strides,
 *                           max-subtraction invariance (x + c gives the same
 *                           probabilities); temperature = exact fp32 product
 *  topk_mask                survivors == elements >= the k-th largest (numpy)
 *  multinomial_strided      float64 walk of the chain-permuted CDF at u away
 *                           from boundaries; draw frequencies vs weights
 *  xo_forward               numpy re-derivation of one layer; greedy token
 *                           ids are pinned by this oracle only (parity
 *                           unpinned against the reference itself: no
 *                           reference-held end-to-end fixture exists).
 */
#ifndef XPOSE_ORACLE_H
#define XPOSE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar formats ---- */
float    xo_fp16_to_fp32(uint32_t h);
uint16_t xo_fp32_to_fp16(float f);
float    xo_bf16_to_fp32(uint32_t h);

/* ---- int4 matvec ---- */
float xo_q4dot8(uint32_t w, const float* v);
float xo_q4dot32(const uint32_t* w4, const float* v);
/* scale_fmt: 0 fp16 quad plane, 1 bf16 quad plane, 2 fp32 [b][col]. */
float xo_scale_at(const void* sc, int scale_fmt, uint32_t cols, uint32_t b, uint32_t j);
void  xo_mv_km4(float* out, const float* in, const uint32_t* wq, const void* sc,
                int scale_fmt, uint32_t rows, uint32_t cols);
void  xo_mv_km4_bs(float* out, const float* in, const uint32_t* wq, const void* sc,
                   int scale_fmt, uint32_t rows, uint32_t cols);
void  xo_mv_km4_split(float* partial, const float* in, const uint32_t* wq, const void* sc,
                      int scale_fmt, uint32_t rows, uint32_t cols, uint32_t split);
void  xo_mv_reduce(float* out, const float* partial, uint32_t cols, uint32_t split);
void  xo_matvec_q4_col(float* out, const float* in, const uint32_t* wq,
                       const float* scale, uint32_t rows, uint32_t cols);
uint32_t xo_nib_hash(uint32_t k, uint32_t j);
void  xo_pack_km4_hash(uint32_t* wq, uint32_t rows, uint32_t cols);
void  xo_pack_col_hash(uint32_t* wq, uint32_t rows, uint32_t cols);
void  xo_unpack_km4(int8_t* out, const uint32_t* wq, uint32_t rows, uint32_t cols);

/* ---- transformer ops ---- */
void xo_rmsnorm_sumsq(float* partial, const float* in, uint32_t n, uint32_t nparts);
void xo_rmsnorm_apply_gemma(float* out, const float* in, const float* w,
                            const float* partial, uint32_t n, uint32_t nparts, float eps);
void xo_rmsnorm_gemma2(float* out, const float* in, const float* w, uint32_t n,
                       uint32_t nparts, float eps);
void xo_rmsnorm_heads_gemma(float* out, const float* in, const float* w,
                            uint32_t n_heads, uint32_t head_dim, float eps);
void xo_rope(float* x, uint32_t n_heads, uint32_t head_dim, uint32_t pos, float theta);
void xo_geglu(float* out, const float* gate, const float* up, uint32_t n);
void xo_add_residual(float* x, const float* y, uint32_t n);
void xo_kv_append_f16(uint16_t* cache, const float* src, uint32_t n, uint32_t pos);
void xo_attention_scores(float* scores, const float* q, const float* kcache,
                         uint32_t n_heads, uint32_t kv_heads, uint32_t head_dim,
                         uint32_t span, float scale, uint32_t kv_start);
void xo_softmax_rows(float* x, uint32_t n_rows, uint32_t n_cols);
void xo_attention_apply(float* out, const float* probs, const float* vcache,
                        uint32_t n_heads, uint32_t kv_heads, uint32_t head_dim,
                        uint32_t span, uint32_t kv_start);
/* scores -> softmax -> apply over fp16 caches (widened exactly). */
void xo_attention_f16(float* out, const float* q, const uint16_t* kcache,
                      const uint16_t* vcache, uint32_t n_heads, uint32_t kv_heads,
                      uint32_t head_dim, uint32_t span, uint32_t kv_start, float scale);

/* ---- sampling ---- */
void xo_argmax_partial(float* pval, uint32_t* pidx, const float* logits, uint32_t n,
                       uint32_t nparts);
void xo_argmax_reduce(float* oval, uint32_t* oidx, const float* pval, const uint32_t* pidx,
                      uint32_t n, uint32_t nparts);
void xo_argmax_final(float* out, uint32_t* idx_out, const float* pval, const uint32_t* pidx,
                     uint32_t nparts);
/* The decode path's tree: n -> 4096 -> 64 -> 1. */
uint32_t xo_argmax_tree(const float* logits, uint32_t n, float* val_out);
void xo_topk4_partial(float* cval, uint32_t* cidx, const float* x, uint32_t n,
                      uint32_t nparts);
void xo_topk_partial(float* cval, uint32_t* cidx, const float* x, uint32_t n,
                     uint32_t nparts, uint32_t k);
void xo_topk_rank_select(float* oval, uint32_t* oidx, const float* cval,
                         const uint32_t* cidx, uint32_t ncand, uint32_t k);
void xo_topp_cutoff(float* w, uint32_t k, float p);
void xo_multinomial_sample(float* out, uint32_t* idx_out, const float* w,
                           const uint32_t* idx, uint32_t k, float u);
/* Host draw (decode.cpp:1873-1917) over (value, index) candidates, modified
 * in place; u in [0,1) replaces the reference's mt19937_64 draw. */
uint32_t xo_draw(float* val, uint32_t* idx, uint32_t n, float temperature, uint32_t top_k,
                 float top_p, double u);
/* Philox-derived uniform for sequence `seq` at step `step` (53-bit, [0,1)). */
/* full-vocabulary sampling chain (llm_sampling.cl:130-225, 380-386, 455-488) */
void xo_apply_temperature(float* logits, float inv_temp, uint32_t n);
void xo_reduce_max_partial(float* pmax, const float* x, uint32_t n, uint32_t nparts);
void xo_reduce_max_final(float* stats, const float* pmax, uint32_t nparts);
void xo_softmax_exp_partial(float* out, float* psum, const float* x, const float* stats,
                            uint32_t n, uint32_t nparts);
void xo_reduce_sum_partial(float* out, const float* in, uint32_t n, uint32_t nparts);
void xo_reduce_sum_final(float* stats, const float* psum, uint32_t nparts);
void xo_softmax_normalize(float* out, const float* stats, uint32_t n);
void xo_topk_mask(float* logits, const float* topk_val, uint32_t k, uint32_t n);
void xo_multinomial_strided(float* out, uint32_t* idx_out, const float* w, const float* psum,
                            const float* stats, uint32_t n, uint32_t nparts, float u);
double xo_philox_uniform(uint32_t seed, uint32_t seq, uint32_t step);
void xo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* ---- full decode step (record_token order, decode.cpp:1634-1780) ---- */
typedef struct {
    const uint32_t* wq;   /* KM4 nibble plane */
    const void* sc;       /* scale plane in the model's scale_fmt */
    uint32_t rows, cols;
} xo_qweight;

typedef struct {
    xo_qweight q, k, v, o, gate, up, down;
    const float* attn_norm;      /* all norm weights stored as multiplier - 1 */
    const float* post_attn_norm;
    const float* ffn_norm;
    const float* post_ffn_norm;
    const float* q_norm;
    const float* k_norm;
    uint16_t* kcache;            /* [max_seq][kv_heads*head_dim] fp16 */
    uint16_t* vcache;
} xo_layer;

typedef struct {
    uint32_t n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim, vocab, max_seq;
    uint32_t global_every, sliding_window;
    float rms_eps, theta_global, theta_local;
    const xo_layer* layers;
    xo_qweight lm_head;          /* tied: rows = hidden, cols = vocab */
    const float* final_norm;
    int32_t scale_fmt;           /* 0 fp16 quad, 1 bf16 quad, 2 fp32 [b][cols] */
    const float* embed;          /* optional fp32 [vocab][hidden] embedding rows */
} xo_model;

/* Embedding of `token` times sqrt(float(hidden)) (decode.cpp:1618-1627): row
 * `token` of m->embed when given (the GGUF row, as the reference reads it),
 * else column token of the tied int4 table, dequantised. */
void xo_embed(float* x, const xo_model* m, uint32_t token);
/* One forward pass at `pos` on `token`; appends K/V at pos. Writes vocab
 * logits when logits != NULL (the lm_head is skipped otherwise). Uses
 * `threads` OpenMP threads for the matvecs (0 = runtime default). */
int xo_forward(const xo_model* m, uint32_t token, uint32_t pos, float* logits,
               int threads);
/* Greedy generation: prefill `n_prompt` ids from pos 0, then `n_gen`
 * sample-first decode steps (decode.cpp:1790-1866). out receives n_gen ids. */
int xo_generate_greedy(const xo_model* m, const uint32_t* prompt, uint32_t n_prompt,
                       uint32_t n_gen, uint32_t* out, int threads);

/* ---- GGUF load path (examples/llm/model/gguf.cpp, decode.cpp:60-229) ---- */
/* GGUFFile::dequantize (gguf.cpp:439-645) for F32, F16, BF16, Q4_0, Q4_1,
 * Q5_0, Q5_1, Q8_0, Q4_K, Q6_K; returns 0, or -1 for another type or a
 * partial block. */
int xo_dequantize(uint32_t type, const void* src, float* dst, uint64_t n);
/* The requantising packer (decode.cpp:97-229) over a whole matrix:
 * w[cols][rows] (row j = output column j), bf16 != 0 for best_bf16_scale and
 * the bf16 quad plane (uint16 sc[((b/4)*cols + j)*4 + b%4]), else fp32 scales
 * amax/7 as float sc[b*cols + j]. wq: the KM4 plane (rows*cols/8 words). */
void xo_pack_int4(const float* w, uint32_t rows, uint32_t cols, int bf16, uint32_t* wq,
                  void* sc);
/* quantise() (decode.cpp:97-104) and best_bf16_scale() (:127-151) alone. */
uint32_t xo_quantise(float v, float inv_scale);
float xo_best_bf16_scale(const float* blk32, float s0);

/* ---- prefill shapes (kernels/llm_sampling.cl:496-736) ---- */
void xo_softmax_rows_stats(float* stats, const float* x, uint32_t n_rows, uint32_t n_cols);
void xo_softmax_rows_apply(float* x, const float* stats, uint32_t n_rows, uint32_t n_cols);
void xo_attention_scores_prefill(float* scores, const float* q, const float* kcache,
                                 uint32_t n_heads, uint32_t kv_heads, uint32_t head_dim,
                                 uint32_t n_query, uint32_t seq_len, uint32_t q_offset,
                                 uint32_t window, float scale);
void xo_attention_apply_prefill(float* out, const float* probs, const float* vcache,
                                uint32_t n_heads, uint32_t kv_heads, uint32_t head_dim,
                                uint32_t n_query, uint32_t seq_len);
void xo_rmsnorm_rows_sumsq(float* rowss, const float* in, uint32_t n_rows, uint32_t n);
void xo_rmsnorm_rows_apply_gemma(float* out, const float* in, const float* w, const float* rowss,
                                 uint32_t n_rows, uint32_t n, float eps);
void xo_rmsnorm_heads_rows_gemma(float* out, const float* in, const float* w, uint32_t n_tokens,
                                 uint32_t n_heads, uint32_t head_dim, float eps);
void xo_rope_prefill(float* x, uint32_t n_tokens, uint32_t n_heads, uint32_t head_dim,
                     uint32_t pos0, float theta);
void xo_kv_append_rows(float* cache, const float* src, uint32_t n_tokens, uint32_t row,
                       uint32_t pos0);
void xo_embed_lookup_rows(float* out, const float* table, const uint32_t* tokens,
                          uint32_t n_tokens, uint32_t n);

/* ---- native-format repack (examples/llm/quant_repack.cpp) ---- */
/* repack() (:135-217) of rows x cols native blocks (type 8 Q8_0, 6 Q5_0,
 * 12 Q4_K, 14 Q6_K) into planes sized for rows padded to 64 (zeroed here);
 * high / bias unused (may be NULL) where the type has none. 0, or -1 where
 * repack() refuses. */
int xo_rq_repack(uint32_t type, const void* src, uint32_t rows, uint32_t cols, uint32_t* quant,
                 uint32_t* high, float* scale, float* bias);
/* reconstruct() (:219-239): element (r, k) of the repacked matrix. */
float xo_rq_reconstruct(uint32_t type, uint32_t nkb, const uint32_t* quant, const uint32_t* high,
                        const float* scale, const float* bias, uint32_t r, uint32_t k);

#ifdef __cplusplus
}
#endif
#endif
