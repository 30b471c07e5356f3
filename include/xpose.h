/*
 * xpose.h — C ABI of the MI355X (gfx950) Gemma-3 int4 decode hot path.
 *
 * Plain C: device pointers, sizes and an opaque stream handle; no C++ or torch
 * types cross this boundary. Every entry point returns 0 on success or a
 * negative XP_E* code; xp_last_error() then holds a message that names the
 * entry point and the offending argument (the reference throws
 * std::runtime_error with the kernel name, examples/llm/decode.cpp:46-56;
 * here the C++ wrapper in include/xpose.hpp turns the code back into that
 * exception).
 *
 * Threading: like the reference Context (agent-docs/vulkore-core.md:76) the
 * library is single-threaded per device. Scratch owned by the library (split-k
 * tickets, attention partials) is shared by every call on a device, so calls
 * that overlap on two streams of one device race.
 *
 * Packed weights (unchanged from the reference, examples/llm/decode.hpp:46-48,
 * :361-370):
 *   nibbles  KM4 plane: uint4 wq[(g*nblk + b)*64 + t], g = j/64, t = j%64,
 *            b = k/32; 32-bit component (k>>3)&3, nibble (k&7)*4;
 *            weight = nibble - 8.  `rows` = K (input length, multiple of 32),
 *            `cols` = N (outputs, multiple of 64).
 *   scales   one per (block, column), in one of three planes (xp_scale_fmt):
 *            XP_SCALE_F16_QUAD  uint16 sc[((b/4)*cols + j)*4 + (b%4)]  (fp16)
 *            XP_SCALE_BF16_QUAD same arrangement, bf16 payload — the reference
 *                               Km4Bf16 plane (decode.hpp:369-370)
 *            XP_SCALE_F32       float  sc[b*cols + j]  — the reference Km4
 *                               plane (llm_matvec.cl:187-200)
 *            The two quad planes need nblk % 4 == 0 (decode.cpp:997-1005).
 */
#ifndef XPOSE_H
#define XPOSE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define XP_OK            0
#define XP_E_ARG        -1   /* bad argument (shape, null pointer, range)   */
#define XP_E_HIP        -2   /* a HIP runtime call failed                    */
#define XP_E_NOMEM      -3   /* device or host allocation failed             */
#define XP_E_STATE      -4   /* call not valid in the current state          */
#define XP_E_DEVICE     -5   /* a kernel reported a device-side error        */
#define XP_E_FORMAT     -6   /* a model or cache file is malformed or unreadable */

typedef void* xp_stream;   /* a hipStream_t; NULL = the default stream */

enum xp_scale_fmt {
    XP_SCALE_F16_QUAD  = 0,
    XP_SCALE_BF16_QUAD = 1,
    XP_SCALE_F32       = 2
};

/* ---- library / device -------------------------------------------------- */
const char* xp_last_error(void);
const char* xp_version(void);
/* Selects device `dev` for this thread and sets up per-device scratch. */
int xp_init(int dev);
/* name (NUL-terminated, truncated to cap), CU count, HBM bytes, gcnArch. */
int xp_device_info(char* name, size_t cap, int* n_cu, size_t* hbm_bytes,
                   char* arch, size_t arch_cap);

/* ---- memory / streams / events (plumbing for hosts without a runtime) --- */
int xp_malloc(void** dptr, size_t bytes);
int xp_free(void* dptr);
int xp_memcpy_htod(void* dst, const void* src, size_t bytes);
int xp_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int xp_memcpy_dtod(void* dst, const void* src, size_t bytes);
int xp_memset(void* dst, int value, size_t bytes);
int xp_synchronize(void);
int xp_stream_create(xp_stream* s);
int xp_stream_destroy(xp_stream s);
int xp_stream_synchronize(xp_stream s);
typedef void* xp_event;
int xp_event_create(xp_event* e);
int xp_event_destroy(xp_event e);
int xp_event_record(xp_event e, xp_stream s);
int xp_event_elapsed_ms(xp_event start, xp_event stop, float* ms);

/* ---- kernel-level entry points (the named-kernel contract) -------------- */

/* int4 KM4 matvec: out[j] = sum_k in[k] * (nibble(k,j) - 8) * scale(k/32, j).
 * Replaces mv_km4 / mv_km4_bs (+ _split and mv_reduce)
 * (kernels/llm_matvec.cl:187-200, :339-356, :422-456, :128-135) and the COL
 * gold's semantics (kernels/llm.cl:488-573). `split` = number of k-chunks
 * (0 = choose); chunks are whole scale quads; split > 1 sums the chunks in
 * ascending order (deterministic). With split = 0 and quad scale planes, a
 * shape narrower than eight waves per CU instead runs one workgroup per
 * (column group, column slice of 64/S columns, S = 2 for >= 64 groups else
 * 4) over all of k when k <= 8192, or else one per (column group, k-chunk of
 * <= 16 quads, <= 8 chunks); the eight waves' partials are summed in wave
 * order, then the chunks in chunk order (deterministic). out must not alias
 * in. */
int xp_mv_int4(float* out, const float* in, const void* wq, const void* scales,
               int scale_fmt, uint32_t rows, uint32_t cols, uint32_t split,
               xp_stream stream);

/* xp_mv_int4 that allocates nothing. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Its
 * split-k / k-chunk partial sums and arrival tickets live in a fixed
 * per-GPU scratch (a device array of 1 MiB of partials + 4096 tickets, held
 * by each GPU the library runs on until the process ends, set up by xp_init
 * or by the first call on a device); the caller passes only inputs and
 * outputs. Same kernels, plans and results as xp_mv_int4; a plan that needs
 * more partials than the scratch holds first falls back from the k-chunk
 * plan to the split-k plan, and an explicit split whose partials do not fit
 * is rejected with XP_E_ARG. Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (different streams, threads)
 * race; calls ordered on one stream do not. */
int xp_mv_int4_noalloc(float* out, const float* in, const void* wq, const void* scales,
                       int scale_fmt, uint32_t rows, uint32_t cols, uint32_t split,
                       xp_stream stream);

/* Several int4 matvecs that share one input vector, in one launch
 * (Q/K/V, or gate/up). out_i has cols_i floats. n <= 4. */
int xp_mv_int4_multi(uint32_t n, float* const* outs, const float* in,
                     const void* const* wqs, const void* const* scales,
                     const uint32_t* cols, int scale_fmt, uint32_t rows,
                     xp_stream stream);

/* Measurement: `iters` back-to-back xp_mv_int4 launches on `stream`, cycling
 * through `ncopies` weight/scale planes (so each launch streams from HBM),
 * bracketed by HIP events; *ms = elapsed time of the whole loop. */
int xp_mv_int4_timed(float* out, const float* in, const void* const* wqs,
                     const void* const* scales, uint32_t ncopies, int scale_fmt,
                     uint32_t rows, uint32_t cols, uint32_t split, uint32_t iters,
                     xp_stream stream, float* ms);

/* Measurement as the reference's matvec bench takes it (one batch of `count`
 * dispatches recorded into one submission, best of R:
 * examples/llm/matvec_bench.cpp:326-353): `count` xp_mv_int4 launches
 * cycling through `ncopies` weight/scale planes are captured into one HIP
 * graph, which is replayed once untimed and then `reps` times on `stream`,
 * each replay between two events; *best_ms = the fastest replay (divide by
 * `count` for one launch). */
int xp_mv_int4_batch_timed(float* out, const float* in, const void* const* wqs,
                           const void* const* scales, uint32_t ncopies, int scale_fmt,
                           uint32_t rows, uint32_t cols, uint32_t split, uint32_t count,
                           uint32_t reps, xp_stream stream, float* best_ms);

/* Debug/unpack entry: expands a KM4 nibble plane to int8 weights w[k*cols+j]
 * = nibble - 8 (row-major [rows][cols]), for bit-exact unpack checks. */
int xp_unpack_km4(int8_t* out, const void* wq, uint32_t rows, uint32_t cols,
                  xp_stream stream);
/* Decodes n raw fp16 bit patterns to fp32 on the device (the reference's
 * fp16_decode sweep kernel, kernels/llm_quant.cl:79-87). */
int xp_fp16_decode(float* out, const uint16_t* src, uint32_t n, xp_stream stream);

/* Bandwidth probes. xp_stream_read_timed: `iters` launches that read `bytes`
 * with 16-byte loads and write nothing (the reference's stream4 probe,
 * kernels/llm_matvec.cl:357-378), bracketed by HIP events; *ms = their total
 * time. The measured ceiling the matvec and the token step are reported
 * against beside the spec peak. xp_copy: dst = src (16-byte aligned, bytes a
 * multiple of 16) — a transfer of known size for calibrating HBM byte
 * counters. */
int xp_stream_read_timed(const void* buf, size_t bytes, uint32_t iters, xp_stream stream,
                         float* ms);
/* The same probe over `nbufs` buffers of `bytes` each, launch i reading
 * buffer i % nbufs with `grid` workgroups of 512 threads (0 = one per CU),
 * each a contiguous chunk: the streaming ceiling at a given size when the
 * buffers together exceed the 256 MiB Infinity Cache. */
int xp_stream_read_rot_timed(const void* const* bufs, uint32_t nbufs, size_t bytes, uint32_t grid,
                             uint32_t iters, xp_stream stream, float* ms);
/* The same read in the batch form of xp_mv_int4_batch_timed: `count`
 * launches (launch i reads buffer i % nbufs) captured into one HIP graph,
 * best of `reps` replays. */
int xp_stream_read_rot_batch_timed(const void* const* bufs, uint32_t nbufs, size_t bytes, uint32_t grid,
                                   uint32_t count, uint32_t reps, xp_stream stream, float* best_ms);
int xp_copy(void* dst, const void* src, size_t bytes, xp_stream stream);
/* Exchange-latency probe (no reference counterpart: it measures the
 * cross-workgroup hand-off the persistent token kernel is built on, alone).
 * A chain of `stages` stages on a grid of one 512-thread workgroup per CU:
 * each of the `producers` roles of a stage publishes 64 tagged floats (32
 * 16-byte pairs), and every role of the next stage first waits until it has
 * read all of them. stride 1 spreads the roles over all XCDs, stride 8 keeps
 * them on one XCD; l2_local (stride 8 only) keeps the stores in that XCD's
 * L2 instead of writing them through to the device coherence point.
 * *ns_per_stage = (last publish - first publish) / (stages - 1), from the
 * workgroups' 100 MHz s_memrealtime stamps. XP_E_DEVICE if a wait timed out
 * (the grid was not resident at once). */
int xp_exchange_chain_timed(uint32_t producers, uint32_t stages, uint32_t stride, int l2_local,
                            xp_stream stream, float* ns_per_stage);
/* Hand-off probes (no reference counterpart), splitting one exchange of the
 * token kernel into its parts. xp_handoff_pingpong_timed: workgroup 0 stores
 * payload_pairs tagged 16-byte pairs (device-scope, or with l2_local kept in
 * its XCD's L2), the 512 threads of a workgroup on the same XCD (same_xcd)
 * or another poll them all, pass a barrier and answer with one pair;
 * *ns_round_trip is the mean round trip over `iters` rounds, *xcc_pair the
 * two workgroups' XCC ids (low byte ping). xp_load_latency: one lane's chain
 * of dependent 4-byte loads over `bytes` (nodes `stride` bytes apart, random
 * cyclic order), plain or device-scope: shader clocks per load. */
int xp_handoff_pingpong_timed(uint32_t same_xcd, uint32_t payload_pairs, int l2_local, uint32_t iters,
                              xp_stream stream, float* ns_round_trip, uint32_t* xcc_pair);
int xp_load_latency(uint32_t bytes, uint32_t stride, int device_scope, xp_stream stream, float* clk_per_load);

/* Two-pass Gemma RMSNorm in one launch: out = in * rsqrt(mean(in^2)+eps) *
 * (1 + w). Replaces rmsnorm_sumsq + rmsnorm_apply_gemma
 * (kernels/llm_transformer.cl:96-116). out may alias in. */
int xp_rmsnorm_gemma(float* out, const float* in, const float* w, uint32_t n,
                     float eps, xp_stream stream);

/* Per-head Gemma RMSNorm (QK-norm). Replaces rmsnorm_heads_gemma
 * (kernels/llm_transformer.cl:122-134). */
int xp_rmsnorm_heads_gemma(float* out, const float* in, const float* w,
                           uint32_t n_heads, uint32_t head_dim, float eps,
                           xp_stream stream);

/* In-place rotate-half RoPE. Replaces rope (kernels/llm_transformer.cl:158-179). */
int xp_rope(float* x, uint32_t n_heads, uint32_t head_dim, uint32_t pos,
            float theta, xp_stream stream);

/* QK-norm + RoPE on q and k, then append k and v at `pos` to fp16 caches
 * laid out [t][kv_heads][head_dim]. Fuses rmsnorm_heads_gemma x2, rope x2
 * and kv_append x2 (llm_transformer.cl:122-179, :590-595;
 * decode.cpp:1678-1683). q_out/k_out receive the normed, rotated vectors. */
int xp_qk_norm_rope_append(float* q_out, float* k_out, const float* q_raw,
                           const float* k_raw, const float* v,
                           const float* q_norm_w, const float* k_norm_w,
                           uint16_t* kcache, uint16_t* vcache,
                           uint32_t n_heads, uint32_t kv_heads, uint32_t head_dim,
                           uint32_t pos, float theta, float eps, xp_stream stream);

/* Decode attention over fp16 caches for keys [kv_start, kv_start+span):
 * out[h][d] = sum_j softmax_j(scale * q_h . k_j) * v_j[d], GQA head map
 * h / (n_heads/kv_heads). Replaces attention_scores(_mq4), softmax_rows(_*),
 * attention_apply(_mq4) + _reduce (llm_transformer.cl:287-557). */
int xp_attention_decode(float* out, const float* q, const uint16_t* kcache,
                        const uint16_t* vcache, uint32_t n_heads,
                        uint32_t kv_heads, uint32_t head_dim, uint32_t span,
                        uint32_t kv_start, float scale, xp_stream stream);

/* Measurement: `iters` back-to-back xp_attention_decode launches on `stream`,
 * cycling through `ncopies` K/V cache pairs (so each launch streams its span
 * from HBM), bracketed by HIP events; *ms = elapsed time of the whole loop. */
int xp_attention_decode_timed(float* out, const float* q, const uint16_t* const* kcaches,
                              const uint16_t* const* vcaches, uint32_t ncopies, uint32_t n_heads,
                              uint32_t kv_heads, uint32_t head_dim, uint32_t span,
                              uint32_t kv_start, float scale, uint32_t iters, xp_stream stream,
                              float* ms);

/* out = gelu_tanh(gate) * up. Replaces geglu (llm_transformer.cl:223-231). */
int xp_geglu(float* out, const float* gate, const float* up, uint32_t n,
             xp_stream stream);
/* x += y. Replaces add_residual (llm_transformer.cl:564-568). */
int xp_add_residual(float* x, const float* y, uint32_t n, xp_stream stream);
/* cache[pos*n + i] = fp16(src[i]). kv_append with an fp16 cache
 * (llm_transformer.cl:590-595). */
int xp_kv_append_f16(uint16_t* cache, const float* src, uint32_t n,
                     uint32_t pos, xp_stream stream);

/* Greedy argmax, lowest index on ties. out_val[0] = value, out_idx[0] = index.
 * Replaces argmax_partial/_reduce/_final (llm_sampling.cl:57-123). */
int xp_argmax(uint32_t* out_idx, float* out_val, const float* logits,
              uint32_t n, xp_stream stream);
/* Best 4 of each strided chain e = p (mod nparts), descending, sentinel
 * (-inf, 0xFFFFFFFF). Replaces topk4_partial (llm_sampling.cl:318-347). */
int xp_topk4_harvest(float* cval, uint32_t* cidx, const float* logits,
                     uint32_t n, uint32_t nparts, xp_stream stream);

/* ---- full-vocabulary sampling chain (llm_sampling.cl:130-225, 257-281,
 * 349-386, 399-488) ------------------------------------------------------
 * One entry per reference kernel, same argument meaning; strided chains are
 * e = p (mod nparts). Bit-identical to the reference's fp32 arithmetic on the
 * same inputs except exp (device libm) in xp_softmax_exp_partial. */
/* logits[i] *= inv_temp (apply_temperature, :130-134; T == 0 goes to argmax). */
int xp_apply_temperature(float* logits, float inv_temp, uint32_t n, xp_stream stream);
/* pmax[p] = max of chain p (reduce_max_partial, :156-163). */
int xp_reduce_max_partial(float* pmax, const float* x, uint32_t n, uint32_t nparts,
                          xp_stream stream);
/* stats[0] = max of pmax[0..nparts) (reduce_max_final, :165-172). */
int xp_reduce_max_final(float* stats, const float* pmax, uint32_t nparts, xp_stream stream);
/* out[k] = exp(x[k] - stats[0]), psum[p] = chain p's sum in chain order
 * (softmax_exp_partial, :175-191); out may alias x. */
int xp_softmax_exp_partial(float* out, float* psum, const float* x, const float* stats,
                           uint32_t n, uint32_t nparts, xp_stream stream);
/* out[p] = chain p's sum (reduce_sum_partial, :202-209). */
int xp_reduce_sum_partial(float* out, const float* in, uint32_t n, uint32_t nparts,
                          xp_stream stream);
/* stats[1] = serial sum of psum (reduce_sum_final, :211-218). */
int xp_reduce_sum_final(float* stats, const float* psum, uint32_t nparts, xp_stream stream);
/* out[i] /= stats[1] (softmax_normalize, :220-225). */
int xp_softmax_normalize(float* out, const float* stats, uint32_t n, xp_stream stream);
/* Chain p's best k (k <= 64), descending, strict '>', unfilled slots
 * (-inf, 0xFFFFFFFF), at cval/cidx[p*k ..] (topk_partial, :257-281). */
int xp_topk_partial(float* cval, uint32_t* cidx, const float* x, uint32_t n, uint32_t nparts,
                    uint32_t k, xp_stream stream);
/* oval/oidx[rank] for every filled candidate with rank < k, rank = number of
 * candidates beating it by (value desc, index asc) (topk_rank_select, :349-369). */
int xp_topk_rank_select(float* oval, uint32_t* oidx, const float* cval, const uint32_t* cidx,
                        uint32_t ncand, uint32_t k, xp_stream stream);
/* logits[i] = -inf where logits[i] < topk_val[k-1] (topk_mask, :380-386). */
int xp_topk_mask(float* logits, const float* topk_val, uint32_t k, uint32_t n, xp_stream stream);
/* Zeroes w[j] once the mass before j reaches p * total (topp_cutoff, :399-415). */
int xp_topp_cutoff(float* w, uint32_t k, float p, xp_stream stream);
/* CDF walk at u * total over w[0..k), ids idx; out = {id as float, weight},
 * idx_out[0] = id (multinomial_sample, :424-446). */
int xp_multinomial_sample(float* out, uint32_t* idx_out, const float* w, const uint32_t* idx,
                          uint32_t k, float u, xp_stream stream);
/* The same draw over the full vocabulary through the chain sums left by
 * xp_softmax_exp_partial / xp_reduce_sum_final (multinomial_strided, :462-488). */
int xp_multinomial_strided(float* out, uint32_t* idx_out, const float* w, const float* psum,
                           const float* stats, uint32_t n, uint32_t nparts, float u,
                           xp_stream stream);

/* ---- prefill shapes (kernels/llm_sampling.cl:496-736) ----------------------
 * Row-indexed twins of the decode kernels, one entry per reference kernel,
 * same arguments and layouts (row-major; q, scores and outputs
 * [head][query][...]; fp32 caches [t][kv_head][head_dim]). Row reductions
 * run one wave per row. */
/* softmax_rows_stats (:527-547): stats[2r] = row max, stats[2r+1] = sum of
 * exp(x - max); a row with no finite maximum gives (0, 1). */
int xp_softmax_rows_stats(float* stats, const float* x, uint32_t n_rows, uint32_t n_cols,
                          xp_stream stream);
/* softmax_rows_apply (:549-556): x = exp(x - max) / sum, in place. */
int xp_softmax_rows_apply(float* x, const float* stats, uint32_t n_rows, uint32_t n_cols,
                          xp_stream stream);
/* attention_scores_prefill (:574-600): scores[h][qi][t] = scale q.k, -inf
 * where t > q_offset + qi (causal) or, window != 0, t + window <= q_offset +
 * qi. q, kcache 16-byte aligned, head_dim % 4 == 0. */
int xp_attention_scores_prefill(float* scores, const float* q, const float* kcache, uint32_t n_heads,
                                uint32_t kv_heads, uint32_t head_dim, uint32_t n_query,
                                uint32_t seq_len, uint32_t q_offset, uint32_t window, float scale,
                                xp_stream stream);
/* attention_apply_prefill (:605-627): out[h][qi][d] = sum_t probs[h][qi][t]
 * v[t][kv_head(h)][d]. */
int xp_attention_apply_prefill(float* out, const float* probs, const float* vcache, uint32_t n_heads,
                               uint32_t kv_heads, uint32_t head_dim, uint32_t n_query,
                               uint32_t seq_len, xp_stream stream);
/* rmsnorm_rows_sumsq (:634-642) and rmsnorm_rows_apply_gemma (:645-656):
 * out = in rsqrt(rowss / n + eps) (1 + w), w shared across rows. */
int xp_rmsnorm_rows_sumsq(float* rowss, const float* in, uint32_t n_rows, uint32_t n,
                          xp_stream stream);
int xp_rmsnorm_rows_apply_gemma(float* out, const float* in, const float* w, const float* rowss,
                                uint32_t n_rows, uint32_t n, float eps, xp_stream stream);
/* rmsnorm_heads_rows_gemma (:659-672): per-head QK-norm over
 * [token][head][head_dim]; out must not alias in. */
int xp_rmsnorm_heads_rows_gemma(float* out, const float* in, const float* w, uint32_t n_tokens,
                                uint32_t n_heads, uint32_t head_dim, float eps, xp_stream stream);
/* rope_prefill (:687-708): rotate-half RoPE in place, token ti at position
 * pos0 + ti. */
int xp_rope_prefill(float* x, uint32_t n_tokens, uint32_t n_heads, uint32_t head_dim, uint32_t pos0,
                    float theta, xp_stream stream);
/* kv_append_rows (:714-721): cache[(pos0 + t) row + j] = src[t row + j]. */
int xp_kv_append_rows(float* cache, const float* src, uint32_t n_tokens, uint32_t row, uint32_t pos0,
                      xp_stream stream);
/* embed_lookup_rows (:728-736): out[t][j] = table[tokens[t]][j]; `vocab`
 * (an argument the reference does not take) bounds the ids: an id >= vocab
 * gives a zero row. */
int xp_embed_lookup_rows(float* out, const float* table, const uint32_t* tokens, uint32_t n_tokens,
                         uint32_t n, uint32_t vocab, xp_stream stream);

/* ---- synthetic inputs (host side, counter-based, any thread count) ------ */
/* Philox4x32-10 (Salmon et al., SC'11): out = philox(ctr, key). */
void xp_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* KM4 nibble plane for tensor `tensor_id`: uint4 i = philox((i,0,0,0),
 * (seed, tensor_id)); every nibble is uniform on [0,15]. */
int xp_synth_nibbles(uint32_t* wq, uint32_t rows, uint32_t cols, uint32_t seed,
                     uint32_t tensor_id);
/* fp16 scales fp16_rne(|N(0, sigma)|), logical index e = b*cols + j, written
 * in the plane `scale_fmt` (F16 quad or F32). */
int xp_synth_scales(void* sc, int scale_fmt, uint32_t rows, uint32_t cols,
                    float sigma, uint32_t seed, uint32_t tensor_id);
/* n floats ~ N(mean, sigma) (stream `tensor_id`). */
int xp_synth_normal(float* out, size_t n, float mean, float sigma, uint32_t seed,
                    uint32_t tensor_id);
/* n fp16 values fp16_rne(N(mean, sigma)). */
int xp_synth_normal_f16(uint16_t* out, size_t n, float mean, float sigma,
                        uint32_t seed, uint32_t tensor_id);
/* Round-to-nearest-even fp32 -> fp16 bits. */
uint16_t xp_f32_to_f16(float f);

/* ---- decode session (engine level) --------------------------------------
 * Mirrors DecodeSession (examples/llm/decode.hpp:605-676): construct = load,
 * prefill(ids), decode_step() -> token (sample first from the previous
 * pass's logits, then run the network on it, decode.cpp:1819-1866), reset(),
 * last_logits(), position(). Weights come from xp_session_upload (packed
 * KM4 planes, the reference's layout) or xp_session_synthesize (the seeded
 * synthetic model) or xp_session_load_gguf (a GGUF model, requantised). */
typedef struct xp_session xp_session;

typedef struct {
    uint32_t n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim, vocab, max_seq;
    uint32_t global_every;      /* layer l is global iff (l+1) % global_every == 0 */
    uint32_t sliding_window;    /* window of the local layers (decode.hpp:327-352) */
    float    rms_eps, rope_theta_global, rope_theta_local;
    float    embed_scale;       /* 0 => sqrt(hidden) */
    float    attn_scale;        /* 0 => 1/sqrt(head_dim) */
    int32_t  scale_fmt;         /* xp_scale_fmt of every int4 weight */
    /* Sampling (decode.hpp:158-202). mode 0 = greedy (device argmax),
     * 1 = temperature / top-k / top-p over the top-4-per-chain harvest. The
     * draw's uniform is Philox(key = (seed, seq_id), counter = step). */
    int32_t  sample_mode;
    float    temperature;
    uint32_t top_k;
    float    top_p;
    uint32_t seed;
    uint32_t seq_id;
    uint32_t topk_parts;
    /* How a token step executes: XP_EXEC_AUTO (the persistent token kernel
     * when the shape allows it, else the graph), XP_EXEC_GRAPH (one captured
     * graph of per-op kernels), XP_EXEC_LAUNCH (per-op kernels launched one
     * by one) or XP_EXEC_TOKEN (the persistent kernel; creation fails if the
     * shape or device does not allow it). */
    int32_t  exec_mode;
    /* How xp_session_prefill runs a prompt of n >= 3 tokens: XP_PREFILL_AUTO
     * (the first n - 1 tokens through the batched M = 16 step, 16 positions
     * per pass on the session's KV cache, then the last token on the
     * session's own path) or XP_PREFILL_TOKENS (one token step per token,
     * the reference's decode-shaped prefill, decode.cpp:1785-1815). */
    int32_t  prefill_mode;
    /* Where the persistent token kernel runs its exchanges: XP_PLACE_AUTO
     * (local layers keep attention, its chunk records and their combine on
     * one XCD, exchanging through that XCD's L2, when the session's probe
     * launch finds workgroup w on the XCD of w % 8; otherwise as
     * XP_PLACE_DEVICE) or XP_PLACE_DEVICE (every exchange through the device
     * coherence point, 32-key attention chunks). Results agree within
     * rounding; this build's own choice, no reference counterpart. */
    int32_t  placement;
} xp_config;

enum xp_prefill_mode { XP_PREFILL_AUTO = 0, XP_PREFILL_TOKENS = 1 };
enum xp_placement { XP_PLACE_AUTO = 0, XP_PLACE_DEVICE = 1 };

enum xp_exec_mode {
    XP_EXEC_AUTO = 0, XP_EXEC_GRAPH = 1, XP_EXEC_LAUNCH = 2, XP_EXEC_TOKEN = 3
};

/* Tensor ids for upload / synthesis. Matrices are (rows = input length,
 * cols = outputs): Q hidden->n_heads*hd, K/V hidden->kv_heads*hd,
 * O n_heads*hd->hidden, GATE/UP hidden->ffn, DOWN ffn->hidden, LM_HEAD
 * (tied embedding) hidden->vocab. OR a matrix id with XP_T_SCALES for its
 * scale plane. Norm weights are stored as multiplier - 1 (the kernels apply
 * 1 + w, decode.cpp:1490-1515). Per-layer ids take layer >= 0; LM_HEAD,
 * FINAL_NORM and EMBED take layer = -1. EMBED is optional: fp32
 * [vocab][hidden] embedding rows (a model loaded from GGUF embeds from its
 * original table, as decode.cpp:1618-1627 does); without it the embedding
 * is the dequantised LM_HEAD column. */
enum xp_tensor {
    XP_T_Q = 0, XP_T_K = 1, XP_T_V = 2, XP_T_O = 3, XP_T_GATE = 4, XP_T_UP = 5, XP_T_DOWN = 6,
    XP_T_ATTN_NORM = 16, XP_T_POST_ATTN_NORM = 17, XP_T_FFN_NORM = 18,
    XP_T_POST_FFN_NORM = 19, XP_T_Q_NORM = 20, XP_T_K_NORM = 21,
    XP_T_LM_HEAD = 32, XP_T_FINAL_NORM = 33, XP_T_EMBED = 34,
    XP_T_SCALES = 0x100
};

typedef struct {
    double   ms;            /* wall time of the last call */
    double   gpu_ms;        /* decode_step: launch + wait (host clock);
                               decode_steps: HIP events on the session stream
                               around the queued steps (device time) */
    double   sample_ms;     /* host draw (temperature mode) */
    double   tokens_per_sec;
    uint32_t position;
    uint32_t launches;      /* kernels per token step */
    int32_t  exec_mode;     /* the mode in use (XP_EXEC_*, never AUTO) */
} xp_metrics;

/* Gemma-3-1B shape and defaults (DecodeConfig::gemma3_1b, decode.hpp:204-356)
 * with fp16 quad scales and greedy sampling. */
void xp_config_gemma3_1b(xp_config* c);
int  xp_session_create(const xp_config* c, xp_session** out);
int  xp_session_destroy(xp_session* s);
int  xp_tensor_bytes(const xp_config* c, int layer, int tensor, size_t* bytes);
int  xp_session_upload(xp_session* s, int layer, int tensor, const void* host, size_t bytes);
/* Bytes [offset, offset + bytes) of a tensor, for streaming large ones. */
int  xp_session_upload_part(xp_session* s, int layer, int tensor, size_t offset,
                            const void* host, size_t bytes);
/* The synthetic model of the benchmark configs, bit-identical to what
 * xp_synth_tensor returns: nibbles uniform on [0,15], fp16 scales
 * |N(0, 0.02)|, norm multipliers N(1, 0.1) (stored minus 1). */
int  xp_synth_tensor(const xp_config* c, uint32_t seed, int layer, int tensor, void* host,
                     size_t bytes);
int  xp_session_synthesize(xp_session* s, uint32_t seed);
/* KV cache rows [pos0, pos0+n) of layer's K (which = 0) or V (1), fp16. */
int  xp_session_kv_upload(xp_session* s, int layer, int which, uint32_t pos0, uint32_t n,
                          const uint16_t* host);
int  xp_session_kv_download(xp_session* s, int layer, int which, uint32_t pos0, uint32_t n,
                            uint16_t* host);
/* Moves the position without running the network (the cache rows below
 * `pos` must already hold keys/values, e.g. from xp_session_kv_upload). */
int  xp_session_set_position(xp_session* s, uint32_t pos);
/* Poll rounds (each one device round trip, ~0.4-1 us) a cross-workgroup
 * wait takes before it gives up: the persistent token kernel's waits
 * (XP_EXEC_TOKEN) and, on the graph paths, the exchange-mode decode
 * attention's (chosen when all its splits fit the device at once). The step
 * then returns XP_E_DEVICE, its logits and appended KV rows are not valid,
 * and the session needs xp_session_set_position before the next step.
 * Default 2^18 (~0.1-0.25 s), at most 2^24; 0 fails every wait that its
 * first read does not satisfy (tests of the error path). No counterpart in
 * the reference, whose dispatches never wait on each other
 * (examples/llm/decode.cpp:1824-1826 errors, never hangs). */
int  xp_session_set_spin_limit(xp_session* s, uint32_t rounds);
int  xp_session_prefill(xp_session* s, const uint32_t* ids, uint32_t n);
int  xp_session_decode_step(xp_session* s, uint32_t* token);
/* n greedy steps queued back to back with one wait; tokens[i] is step i's id. */
int  xp_session_decode_steps(xp_session* s, uint32_t n, uint32_t* tokens);
int  xp_session_reset(xp_session* s);
int  xp_session_position(const xp_session* s, uint32_t* pos);
int  xp_session_last_logits(xp_session* s, float* host, uint32_t n);
/* Raw harvest of the last pass (temperature mode): 4*topk_parts pairs. */
int  xp_session_last_candidates(xp_session* s, float* val, uint32_t* idx, uint32_t n);
int  xp_session_last_metrics(const xp_session* s, xp_metrics* m);
int  xp_session_weight_bytes(const xp_session* s, size_t* bytes);
/* The execution the session uses (XP_EXEC_TOKEN, _GRAPH or _LAUNCH). */
int  xp_session_exec_mode(const xp_session* s, int32_t* mode);
int  xp_session_kv_bytes(const xp_session* s, size_t* bytes);
/* Stage timeline of the persistent token kernel (XP_EXEC_TOKEN only), for
 * profiling: once enabled, every launch records for event e and workgroup w
 * a timestamp at host[e * grid + w] in 100 MHz ticks (s_memrealtime), 0
 * where w had no work: e = 0 kernel start; e = 1 + 6 l + k the end of layer
 * l's stage k (QKV, attention, combine, O, gate/up, down); e = 6 L + 1 the
 * lm_head; e = 6 L + 2 the argmax; e = 6 L + 3 + 6 l + k the time w's
 * inputs of layer l's stage k had all arrived (its wait and the barrier
 * after it done). *grid receives the workgroup count. */
int  xp_session_trace(xp_session* s, int enable);
int  xp_session_last_trace(xp_session* s, uint64_t* host, size_t n, uint32_t* grid);
/* Host draw over (value, index) candidates, in place (decode.cpp:1873-1917),
 * with u in [0,1) standing in for the reference's mt19937_64 draw. */
/* ---- batched decode (up to 16 sequences per step) -------------------------
 * n_seq independent sequences decoded together on the weights of `weights`
 * (shared, not copied: the session must outlive the batch). Each sequence has
 * its own fp16 KV cache of max_seq positions, its position and its draw
 * counter; sequence i draws with Philox(key = (seed, seq_id + i), counter =
 * its step) using the session's temperature / top_k (<= 64) / top_p (greedy
 * when sample_mode is 0), over the reference's harvest (best 4 of 4096
 * strided chains) reduced to its exact best 64 on the device. The matvecs
 * are M = 16 MFMA GEMMs (int4 widened to bf16 in registers, fp32 activations
 * as two bf16 terms). No reference counterpart: the reference decodes one
 * sequence per DecodeSession (decode.hpp:605-676). */
typedef struct xp_batch xp_batch;
/* xp_batch_create2 with exec_mode XP_EXEC_AUTO. */
int xp_batch_create(const xp_session* weights, uint32_t n_seq, uint32_t max_seq, xp_batch** out);
/* exec_mode: XP_EXEC_GRAPH (and XP_EXEC_AUTO) runs each step as a captured
 * graph of one kernel per stage; XP_EXEC_TOKEN runs the layers as ONE
 * persistent kernel (one 512-thread workgroup per CU walking the stages,
 * per-tile flags between them; creation fails if the shape or the device's
 * free CUs do not allow it). EXPERIMENTAL: both give bit-identical results,
 * but the graph is the faster (1.2 vs 1.8 ms a config-5 step, measured:
 * each stage's flag hand-off costs 1.3-3.6 us where a kernel boundary inside
 * the graph costs next to nothing), so AUTO takes the graph; the persistent
 * kernel is kept as a measured alternative and for its stage timeline.
 * The persistent kernel's bounded waits turn a grid that is not resident
 * after all into XP_E_DEVICE from xp_batch_forward (that step's results and
 * the KV rows it appended are then not valid; positions are unchanged, so
 * the step can be run again). */
int xp_batch_create2(const xp_session* weights, uint32_t n_seq, uint32_t max_seq, int32_t exec_mode,
                     xp_batch** out);
/* The execution in use: XP_EXEC_TOKEN (persistent step kernel) or XP_EXEC_GRAPH. */
int xp_batch_exec_mode(const xp_batch* b, int32_t* mode);
/* Stage timeline of the step kernel (XP_EXEC_TOKEN only), for profiling:
 * while enabled each forward records, per workgroup w of the grid of G, the
 * 100 MHz realtime clock when its inputs of stage k (0 q|k|v, 1 attention,
 * 2 o, 3 staging, 4 gate|up, 5 down, 6 staging) of layer l were ready and
 * when its last tile of that stage ended: out[((l*7 + k)*2 + e)*G + w], e = 0
 * / 1 (0 where it had no tile), then its start at out[n_layers*14*G + w].
 * read with out == NULL sets *n_out to the entry count. */
int xp_batch_step_trace(xp_batch* b, int enable);
/* Poll rounds (each ~1 us) a wait takes before it gives up and the step
 * returns XP_E_DEVICE: the step kernel's waits (default 2^20) and, on the
 * graph path, the exchange-mode decode attention's (default 2^18); at most
 * 2^24. A small value forces that path (tests of the error handling). */
int xp_batch_set_spin_limit(xp_batch* b, uint32_t rounds);
int xp_batch_step_trace_read(xp_batch* b, unsigned long long* out, size_t n, size_t* n_out);
int xp_batch_destroy(xp_batch* b);
int xp_batch_kv_upload(xp_batch* b, uint32_t seq, int layer, int which, uint32_t start,
                       uint32_t count, const uint16_t* src);
int xp_batch_kv_download(xp_batch* b, uint32_t seq, int layer, int which, uint32_t start,
                         uint32_t count, uint16_t* dst);
int xp_batch_set_positions(xp_batch* b, const uint32_t* pos);
int xp_batch_positions(xp_batch* b, uint32_t* pos);
/* Runs the network on tokens[n_seq] at the current positions (their K / V
 * appended there), advances every position, keeps the logits and candidates. */
int xp_batch_forward(xp_batch* b, const uint32_t* tokens);
/* Sample-first step for every sequence (decode.cpp:1830-1850): draws
 * tokens_out from the last logits, then runs xp_batch_forward on them. */
int xp_batch_decode_step(xp_batch* b, uint32_t* tokens_out);
/* n sample-first steps, the same tokens as n calls of xp_batch_decode_step
 * (tokens_out[k * n_seq + i]: step k's token of sequence i): the first draw
 * on the host from the last candidates, the following ones by a kernel at
 * the end of each step's graph (the host draw's arithmetic: the candidates
 * in (value desc, index asc) order, exp in float, sums in double, the same
 * Philox uniforms), so the steps are queued back to back with no host round
 * trip between them (the reference's loop draws on the host between steps,
 * decode.cpp:1830-1861). Falls back to n xp_batch_decode_step calls for the
 * persistent step kernel. */
int xp_batch_decode_steps(xp_batch* b, uint32_t n, uint32_t* tokens_out);
int xp_batch_last_logits(xp_batch* b, uint32_t seq, float* out, uint32_t n);
/* The best n <= 64 candidates of sequence seq, (value desc, index asc). */
int xp_batch_last_candidates(xp_batch* b, uint32_t seq, float* val, uint32_t* idx, uint32_t n);
/* Device time of the last forward (HIP events around the graph). */
int xp_batch_last_ms(xp_batch* b, float* ms);

uint32_t xp_draw(float* val, uint32_t* idx, uint32_t n, float temperature, uint32_t top_k,
                 float top_p, double u);
double xp_philox_uniform(uint32_t seed, uint32_t seq, uint32_t step);

/* ---- GGUF load path -------------------------------------------------------
 * Host side, no GPU (except xp_session_load_gguf's uploads). Replaces GGUFFile
 * (examples/llm/model/gguf.hpp:173-215, gguf.cpp:234-645), the requantising
 * packer (decode.cpp:60-229: symmetric int4, q = round(v / s) + 8 clamped to
 * [0, 15], s = amax / 7 rounded to whichever neighbouring bf16 value has the
 * smaller block error; KM4 nibble plane + bf16 quad scale plane) and the
 * load path with its packed-weight cache (decode.cpp:710-1328). The cache is
 * this library's own format: a header stamped with the model file's size,
 * mtime and a digest of its first and last 64 KiB, the scale format and the
 * packer revision; a table of (name, shape, byte counts, digest) per tensor;
 * written to "<path>.tmp" and renamed into place. Any mismatch repacks. */
typedef struct xp_gguf xp_gguf;
enum xp_ggml_type {
    XP_GGML_F32 = 0, XP_GGML_F16 = 1, XP_GGML_Q4_0 = 2, XP_GGML_Q4_1 = 3, XP_GGML_Q5_0 = 6,
    XP_GGML_Q5_1 = 7, XP_GGML_Q8_0 = 8, XP_GGML_Q4_K = 12, XP_GGML_Q6_K = 14, XP_GGML_BF16 = 30
};
typedef struct {
    uint32_t version;
    uint64_t n_tensors, n_meta, alignment, data_offset, file_size;
} xp_gguf_info;
/* ModelConfig (gguf.hpp:144-165): the "<arch>." keys. */
typedef struct {
    char     arch[32];
    uint32_t n_layers, n_heads, n_kv_heads, hidden, ffn, context_length;
    uint32_t key_length, value_length, vocab, sliding_window, head_dim;
    float    rope_freq_base, rms_eps;
} xp_gguf_model;
typedef struct {
    double   total_ms, pack_ms, cache_ms, upload_ms;
    uint64_t packed_bytes;      /* int4 planes + scale planes */
    int32_t  from_cache;        /* 1: the cache was valid and used */
    int32_t  cache_written;     /* 1: a new cache file was written */
    uint32_t threads;
    uint32_t n_tensors;
} xp_load_stats;
enum xp_load_flags {
    XP_LOAD_REPACK = 1,         /* ignore a valid cache (still rewrite it) */
    XP_LOAD_NORM_RAW = 2,       /* the file's norms are w, not 1 + w: no "- 1" */
    XP_LOAD_NO_EMBED = 4        /* embed from the int4 LM_HEAD instead of the file's table */
};
int xp_gguf_open(const char* path, xp_gguf** out);
int xp_gguf_close(xp_gguf* g);
int xp_gguf_get_info(xp_gguf* g, xp_gguf_info* info);
int xp_gguf_get_model(xp_gguf* g, xp_gguf_model* m);
int xp_gguf_tensor_count(xp_gguf* g, uint64_t* n);
int xp_gguf_tensor_at(xp_gguf* g, uint64_t i, char* name, size_t cap);
/* dims[4] (dims[0] fastest); unused dims are 1. */
int xp_gguf_tensor_info(xp_gguf* g, const char* name, uint32_t* type, uint32_t* n_dims,
                        uint64_t* dims, uint64_t* nbytes);
int xp_gguf_meta_number(xp_gguf* g, const char* key, double* value);
int xp_gguf_meta_string(xp_gguf* g, const char* key, char* out, size_t cap, size_t* len);
int xp_gguf_meta_array_length(xp_gguf* g, const char* key, uint64_t* n);
/* GGUFFile::dequantize (gguf.cpp:439-645): n elements (whole blocks). */
int xp_dequantize(uint32_t type, const void* src, float* out, uint64_t n);
/* Rows [row0, row0 + nrows) of a 2-D tensor, fp32 [nrows][dims[0]]
 * (RowReader, decode.cpp:60-96). */
int xp_gguf_dequantize_rows(xp_gguf* g, const char* name, uint64_t row0, uint64_t nrows,
                            float* out);
/* Shapes from the file onto c (DecodeConfig::from_model, decode.cpp:258-275);
 * c's policy fields (max_seq, sampling, global_every, scale_fmt, ...) stay,
 * and so does a sliding_window other than the default 512 (the merge of
 * decode.cpp:1422-1434); otherwise the file's window extent is taken. */
int xp_config_from_gguf(xp_gguf* g, xp_config* c);
/* Requantises w[cols][rows] (GGUF row order: row j of length `rows` is
 * output column j) to the KM4 plane wq (rows * cols / 2 bytes) and the scale
 * plane sc (XP_SCALE_BF16_QUAD: rows / 32 * cols * 2 bytes; XP_SCALE_F32:
 * rows / 32 * cols * 4 bytes, s = amax / 7 unrounded). threads 0 = all cores. */
int xp_pack_int4(const float* w, uint32_t rows, uint32_t cols, int scale_fmt, uint32_t threads,
                 void* wq, void* sc);
/* Packs every matrix of the model for config c (7 per layer, then the
 * output head: output.weight, or token_embd.weight when tied) into the cache
 * at cache_path, no GPU. */
int xp_gguf_pack_model(xp_gguf* g, const xp_config* c, const char* cache_path, uint32_t threads,
                       xp_load_stats* st);
/* --verify-cache (decode.cpp:2580-2661): repacks every matrix and compares
 * the cache payload byte for byte; *mismatches = tensors that differ (0 =
 * identical). XP_E_FORMAT if there is no valid cache. */
int xp_gguf_verify_cache(xp_gguf* g, const xp_config* c, const char* cache_path,
                         uint32_t threads, uint32_t* mismatches);
/* Loads the model into a session created with shapes from the same file:
 * matrices from a valid cache (digests checked) or packed afresh (and
 * cached when cache_path is given), norms minus 1, and the fp32 embedding
 * table (XP_T_EMBED) from token_embd.weight. */
int xp_session_load_gguf(xp_session* s, xp_gguf* g, const char* cache_path, uint32_t flags,
                         uint32_t threads, xp_load_stats* st);

/* ---- native-format weights ------------------------------------------------
 * GGUF's own Q8_0 / Q5_0 / Q4_K / Q6_K blocks, used without requantising
 * (kernels/llm_quant.cl:83-615, examples/llm/quant_repack.{hpp,cpp}). Matrix
 * convention of that code: `rows` outputs, each a GGUF row of `cols`
 * reduction elements (cols = dims[0], a multiple of 32, of 256 for Q4_K /
 * Q6_K); out[r] = sum_k w[r][k] in[k].
 *
 * Native layout, straight from the file: xp_dequant_native replaces
 * dequant_q8_0 / _q5_0 / _q4_k / _q6_k (llm_quant.cl:92-99, 144-149,
 * 200-219, 284-291) and is bit-identical to xp_dequantize; xp_mv_native
 * replaces matvec_q8_0 / _q5_0 / _q4_k / _q6_k (llm_quant.cl:101-121,
 * 151-170, 221-272, 293-322). `src` must be 2-byte aligned.
 *
 * Repacked layout (RepackedTensor, quant_repack.hpp:13-67), made once at
 * load: output row r = 64 g + t, k-block kb = k / 32, j = k % 32, slot
 * idx = (g nkb + kb) 64 + t with nkb = cols / 32, rows padded to a multiple
 * of 64 with zero planes.
 *   quant  Q4_K / Q5_0 / Q6_K: words 4 idx .. 4 idx + 3, the low nibble of
 *          quant j at bits 4 (j % 8) of word j / 8 (the int4 plane's shape);
 *          Q8_0: words 8 idx .. 8 idx + 7, the int8 of j at bits 8 (j % 4)
 *          of word j / 4.
 *   high   Q5_0: word idx, bit j = bit 4 of quant j; Q6_K: words 2 idx +
 *          j / 16, bits 2 (j % 16) = bits 4-5 of quant j; else absent.
 *   scale  fp32 per slot (Q6_K: two, 2 idx + j / 16): d for Q8_0 / Q5_0,
 *          d * sub-scale for Q4_K / Q6_K.
 *   bias   fp32 per slot, Q4_K only: dmin * sub-min.
 * Weight (r, k) = scale * q (Q8_0), scale * (q - 16) (Q5_0), scale * (q - 32)
 * (Q6_K), scale * q - bias (Q4_K): the same fp32 operations the dequantiser
 * performs, so xp_rq_reconstruct == xp_dequantize bit for bit. */
typedef struct {
    uint32_t type;          /* XP_GGML_Q8_0, _Q5_0, _Q4_K or _Q6_K */
    uint32_t rows;          /* outputs */
    uint32_t padded_rows;   /* rows rounded up to a multiple of 64 */
    uint32_t cols;          /* reduction length */
    uint32_t nkb;           /* cols / 32 */
    uint32_t reserved;
    uint64_t quant_bytes, high_bytes, scale_bytes, bias_bytes;   /* 0 = plane absent */
    uint64_t native_bytes;  /* the GGUF blocks of the same matrix (native_bytes()) */
} xp_rq_layout;

/* Device planes of one repacked matrix, as xp_rq_layout describes them. */
typedef struct {
    uint32_t        type, rows, cols, reserved;
    const void*     quant;  /* 16-byte aligned */
    const uint32_t* high;   /* Q5_0 / Q6_K, else NULL */
    const float*    scale;
    const float*    bias;   /* Q4_K, else NULL */
} xp_rq_tensor;

/* Plane sizes for a matrix; XP_E_ARG for another type, cols % 32 != 0 or
 * (Q4_K / Q6_K) cols % 256 != 0, as repack() refuses. */
int xp_rq_layout_of(uint32_t type, uint32_t rows, uint32_t cols, xp_rq_layout* out);
/* repack() (quant_repack.cpp:135-217): rows x cols native blocks at src
 * (rows * native_bytes / rows contiguous) into host planes of the layout's
 * sizes (high / bias may be NULL when absent); rows are packed on `threads`
 * host threads (0 = all). */
int xp_rq_repack(const xp_rq_layout* l, const void* src, uint32_t threads, void* quant,
                 uint32_t* high, float* scale, float* bias);
/* reconstruct() over the whole matrix (quant_repack.cpp:219-239):
 * out[r * cols + k], host planes. */
int xp_rq_reconstruct(const xp_rq_layout* l, const void* quant, const uint32_t* high,
                      const float* scale, const float* bias, float* out);
/* matvec_rq4_k / _rq5_0 / _rq6_k / _rq8_0 (llm_quant.cl:515-549) for
 * split == 1, their _split forms + mv_reduce (llm_quant.cl:574-615) for
 * split > 1 (here one launch: the last k-chunk of a row group to finish sums
 * the partials in chunk order), split == 0 picks one: for shapes narrower
 * than eight waves per CU, one workgroup per (row group, k-chunk of <= 40
 * blocks, <= 8 chunks) whose waves split the chunk (deterministic: wave
 * order, then chunk order). `in` is fp32 [cols],
 * 16-byte aligned; out [rows]. Within 1e-5 of max|out| of the float64
 * product (activations are staged as 20-bit block fixed point; every block
 * product is an exact integer). */
int xp_mv_rq(float* out, const float* in, const xp_rq_tensor* w, uint32_t split,
             xp_stream stream);
/* `iters` calls of xp_mv_rq rotating over `ncopies` weight copies; *ms is
 * the total elapsed time on the stream (HIP events). */
int xp_mv_rq_timed(float* out, const float* in, const xp_rq_tensor* ws, uint32_t ncopies,
                   uint32_t split, uint32_t iters, xp_stream stream, float* ms);
int xp_dequant_native(float* out, const void* src, uint32_t type, uint64_t n, xp_stream stream);
int xp_mv_native(float* out, const float* in, const void* src, uint32_t type, uint32_t rows,
                 uint32_t cols, xp_stream stream);

/* ---- tokenizer ------------------------------------------------------------
 * SentencePiece from the GGUF vocabulary (Tokenizer, model/tokenizer.hpp:46-94,
 * tokenizer.cpp:70-374): control / unknown tokens cut out first (longest
 * spelling), fragments normalised (space -> U+2581, one leading U+2581 when
 * add_space_prefix), best-score adjacent merges (leftmost on a tie), byte
 * fallback to "<0xAB>" tokens. The handle borrows the xp_gguf's strings:
 * destroy it before closing the file. */
typedef struct xp_tokenizer xp_tokenizer;
typedef struct {
    uint32_t vocab;
    int32_t  bos, eos, unk, pad;        /* -1 when the file names none */
    int32_t  add_bos, add_eos, add_space_prefix;
} xp_tokenizer_ids;
int xp_tokenizer_create(xp_gguf* g, xp_tokenizer** out);
int xp_tokenizer_destroy(xp_tokenizer* t);
int xp_tokenizer_info(xp_tokenizer* t, xp_tokenizer_ids* info);
/* encode: *n = number of ids; ids may be NULL to size the output first. */
int xp_tokenize(xp_tokenizer* t, const char* text, size_t len, int add_bos, int add_eos,
                int32_t* ids, size_t cap, size_t* n);
/* decode (skip_special drops control / unknown tokens); *len = bytes, the
 * output is NUL-terminated within cap. */
int xp_detokenize(xp_tokenizer* t, const int32_t* ids, size_t n, int skip_special, char* out,
                  size_t cap, size_t* len);
/* One token's text: piece = as decoded (byte resolved, U+2581 -> ' '),
 * text = the raw vocabulary spelling. */
int xp_token_piece(xp_tokenizer* t, int32_t id, char* out, size_t cap, size_t* len);
int xp_token_text(xp_tokenizer* t, int32_t id, char* out, size_t cap, size_t* len);
/* The id of an exact spelling (the lowest id on duplicates), -1 if none. */
int xp_token_find(xp_tokenizer* t, const char* spelling, size_t len, int32_t* id);
/* token_type (0 when out of range) and score. */
int xp_token_kind(xp_tokenizer* t, int32_t id, int32_t* kind, float* score);

#ifdef __cplusplus
}
#endif
#endif /* XPOSE_H */
