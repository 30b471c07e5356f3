// Internal launchers shared by the C-ABI entry points and the decode
// session. The session passes its own scratch buffers so that nothing inside
// a captured token step allocates.
#pragma once

#include <cmath>

#include "xp_internal.hpp"

namespace xp {

constexpr int kMvMaxMats = 4;
constexpr int kMaxHeadDim = 512;

// RoPE inverse frequencies theta^(-2d / head_dim), formed on the host
// (exp2(-log2(theta) 2d / head_dim), llm_transformer.cl:158-179) and passed
// by value, so every RoPE kernel rotates by the same angles.
struct RopeFreq {
    float inv[kMaxHeadDim / 2];
};
inline void rope_freq(RopeFreq& f, uint32_t head_dim, float theta) {
    for (uint32_t d = 0; d < head_dim / 2; ++d) {
        const float frac = float(2u * d) / float(head_dim);
        f.inv[d] = std::exp2f(-std::log2f(theta) * frac);
    }
}

// ---- int4 matvec ----
struct MvMatDesc {
    float*      out;
    const void* wq;
    const void* sc;
    uint32_t    cols;
};
// Partial floats a call with these shapes needs for a given split (0 = auto).
size_t mv_partial_floats(uint32_t rows, uint32_t total_cols, uint32_t split, int n_cu);
// An operation the column-slice matvec applies to its input while staging
// it, so that the elementwise launch before the matvec is not needed (the
// graph path's GeGLU and residual + RMSNorm):
//   kMvInGeglu  the input is gelu(x) * up (the tanh form on the hardware
//               exponential and reciprocal, as the token kernel's tiles);
//   kMvInNorm   x_new = x + rmsnorm(y) (1 + w_post); the input is
//               rmsnorm(x_new) (1 + w_pre), with the scalar of that norm
//               applied to the outputs (the staged block fixed point does
//               not depend on a common scale); workgroup 0 writes x_new to
//               x_out (which must not alias x, y or the outputs).
// geglu_out (with kMvInPlain or kMvInNorm): the call's two matrices are a
// gate and an up projection of equal width, and the output, into the first
// matrix's `out`, is gelu(gate) * up (each workgroup takes the same 32
// columns of both; the second matrix's `out` is not written).
enum : int { kMvInPlain = 0, kMvInGeglu = 1, kMvInNorm = 2 };
struct MvIn {
    int mode = kMvInPlain;
    const float* up = nullptr;
    const float* y = nullptr;
    const float* w_post = nullptr;
    const float* w_pre = nullptr;
    float* x_out = nullptr;
    float eps = 0.0f;
    bool geglu_out = false;
};
// Whether launch_mv takes the column-slice plan for these shapes (the only
// plan that accepts an MvIn other than kMvInPlain), and whether it can
// produce a gate / up pair's GeGLU (geglu_out) for rows x cols matrices.
bool mv_slice_plan(uint32_t rows, uint32_t total_cols, int fmt, int n_cu);
bool mv_geglu_plan(uint32_t rows, uint32_t cols, int fmt, int n_cu);
// With caller-provided partial and ticket buffers, n_cu is the CU count the
// plan is made for (0: 256); without them the library's scratch is used.
int launch_mv(const MvMatDesc* mats, uint32_t n, const float* x, int fmt, uint32_t rows,
              uint32_t split, float* partial, size_t partial_cap, uint32_t* tickets,
              size_t tickets_cap, hipStream_t st, const char* who, int n_cu = 0,
              const MvIn* in = nullptr);
// Set-up of the allocation-free matvec entry point on the current device:
// the device address of its fixed scratch (partial sums, then tickets), its
// tickets cleared once by a fill kernel on `st` (synchronised when `sync`).
struct MvNoAlloc {
    float*    partial;
    size_t    partial_floats;
    uint32_t* tickets;
    size_t    n_tickets;
    int       n_cu;
};
int mv_noalloc_setup(hipStream_t st, bool sync, MvNoAlloc* out);

// ---- repacked native-format matvec (xp_mv_rq) ----
int launch_mv_rq(float* out, const float* x, const xp_rq_tensor& w, uint32_t split,
                 hipStream_t st, const char* who);

// ---- QK-norm + RoPE + KV append ----
struct QkArgs {
    float* q_out;
    float* k_out;
    const float* q_raw;
    const float* k_raw;
    const float* v;
    const float* qw;
    const float* kw;
    uint16_t* kcache;
    uint16_t* vcache;
    uint32_t n_heads, kv_heads, head_dim;
    float eps;
    const uint32_t* pos_dev;   // when non-null, the position is read here (pos_dev[b])
    uint32_t pos;
    // Batched sequences (grid.y = batch): element strides between sequence b
    // and b + 1 of q_raw / q_out, of k_raw / v / k_out, and of the caches.
    uint32_t batch = 1;
    uint32_t bq = 0, bkv = 0;
    size_t bcache = 0;
};
int launch_qk(const QkArgs& a, float theta, hipStream_t st);

// ---- decode attention ----
struct AttnArgs {
    float* out;
    const float* q;
    const uint16_t* kc;
    const uint16_t* vc;
    uint32_t n_heads, kv_heads, head_dim, group;
    uint32_t span, kv_start;
    const uint32_t* pos_dev;   // when non-null: span / kv_start derive from it
    uint32_t window;           // 0 = global (with pos_dev)
    float scale;
    uint32_t nsplit;
    float* part;               // [kv_heads][256 + 16][8 + group * head_dim]
    uint32_t* tickets;         // [kv_heads][kAttnTicketsPerHead], zero at rest (epoch words aside)
    // Batched sequences (grid.z = batch): sequence b reads q + b bq, the caches
    // at + b bcache, position pos_dev[b], and writes out + b bq, its own partials
    // (+ b bpart) and tickets (+ b kv_heads kAttnTicketsPerHead).
    uint32_t batch = 1;
    uint32_t bq = 0;
    size_t bcache = 0, bpart = 0;
    // Fused QK-norm + RoPE + KV append (decode with pos_dev, every sequence
    // its own cache rows): with q_raw set, each workgroup forms the normed,
    // rotated q of its kv head's query heads and the current key / value
    // from q_raw, k_raw and v_raw (sequence b at + b bq, + b bkv) itself, uses
    // the current key / value from LDS, and the split holding the current
    // position appends them to the caches; q is not read. Not for prefill
    // rows that share one cache (a row's span includes rows the same launch
    // appends).
    const float* q_raw = nullptr;
    const float* k_raw = nullptr;
    const float* v_raw = nullptr;
    const float* qw = nullptr;   // QK-norm weights of the query heads / the key
    const float* kw = nullptr;
    float eps = 0.0f;
    float theta = 0.0f;          // RoPE base of the layer
    uint32_t bkv = 0;
    // Set by launch_attention: the splits combine through tagged records
    // (every workgroup of the launch resident at once) instead of tickets.
    uint32_t xchg = 0;
    // Exchange mode: poll rounds before a wait gives up (it then writes NaN
    // into its slice of the output and sets the head's error word; when
    // `status` is set, bit 0 of *status too, the batched step kernel's word).
    uint32_t spin_limit = 1u << 18;
    uint32_t* status = nullptr;
};
// Arrival tickets per (sequence, kv head) of the decode attention: one for
// the final combine, one per group of 16 splits (at most 256 splits); then
// the exchange mode's epoch (the last launch's record tag) and its timeout
// flag.
constexpr uint32_t kAttnTicketsPerHead = 19;
// Words of a head's tickets: the exchange mode's epoch (the last completed
// launch's record tag) and its error word (non-zero after a wait timed out:
// the launch's output holds NaN and the head's records and epoch are stale;
// the owner of the tickets reports it and zeroes the records and tickets).
constexpr uint32_t kAttnEpochWord = 17;
constexpr uint32_t kAttnXErrWord = 18;
// Splits per (sequence, kv head) for a launch over `batch` sequences whose
// spans are at most max_span; the partials one sequence needs (any span).
uint32_t attn_splits(uint32_t max_span, uint32_t batch, uint32_t kv_heads);
size_t attn_partial_floats(uint32_t kv_heads, uint32_t n_heads, uint32_t head_dim);
// allow_xchg false keeps the ticket chain whatever the span: callers that
// cannot check the exchange mode's error word afterwards (an asynchronous
// kernel-level call on the library's own records) use it.
int launch_attention(AttnArgs a, uint32_t max_span, hipStream_t st, bool allow_xchg = true);
// launch_attention's plan without the launch: fills group, nsplit, xchg (only
// with allow_xchg), a fallback part / tickets, and returns the keys per lane
// per pass (U) and the layer's RoPE frequencies.
int plan_attention(AttnArgs& a, uint32_t max_span, bool allow_xchg, int* U_out, RopeFreq* f_out);

// ---- sampling ----
constexpr int kAmMaxWg = 256;
// advance: when set, the launch also adds 1 to *advance once its result is
// written (the session's position, saving the step a launch of its own).
int launch_argmax(uint32_t* out_idx, float* out_val, const float* logits, uint32_t n,
                  float* pval, uint32_t* pidx, uint32_t* ticket, hipStream_t st,
                  uint32_t* advance = nullptr);
int launch_topk4(float* cval, uint32_t* cidx, const float* x, uint32_t n, uint32_t nparts,
                 hipStream_t st, uint32_t rows = 1);
// The best k (<= 64) of each of `rows` candidate lists (row r at cval / cidx +
// r ncand), sorted by (value desc, index asc), into oval / oidx [rows][k];
// exact. Unfilled list slots carry index 0xFFFFFFFF and are skipped. With
// pos_inc, row r's workgroup also adds 1 to pos_inc[r] (the batched step's
// position advance, which nothing in the select reads).
// The batched step's sample-first draw on the device (one wave per row, the
// host draw's arithmetic): token of row r to tok[r] and to
// hist[(steps[r] % hist_cap) * rows + r]; steps[r] advances (sampling only).
int launch_draw_rows(const float* val, const uint32_t* idx, uint32_t k, uint32_t rows, int mode,
                     float temperature, uint32_t top_k, float top_p, uint32_t seed, uint32_t seq0,
                     uint32_t* steps, uint32_t* tok, uint32_t* hist, uint32_t hist_cap, hipStream_t st);
int launch_select_rows(float* oval, uint32_t* oidx, const float* cval, const uint32_t* cidx,
                       uint32_t ncand, uint32_t k, uint32_t rows, hipStream_t st,
                       uint32_t* pos_inc = nullptr);


// ---- batched decode (batch_kernels.hip) ----
// Staging of one sequence row per workgroup into the M = 16 MFMA operand
// (see bprep_kernel for the modes).
struct BprepArgs {
    int mode;
    float* x;                  // [batch][K] residual stream (modes 0, 1)
    const float* y;            // [batch][K] sublayer output / input / gate
    const float* u;            // [batch][K] up (mode 3)
    const float* w_post;
    const float* w_pre;
    void* a;                   // [K/32][2][64] 16-byte staged hi / lo operand
    float* asum;               // [K/32][16]
    uint32_t K;
    float eps;
    float* x_out = nullptr;    // modes 0, 1: the updated x goes here instead of x (same layout)
    // mode 0 with tok: row b of x is first set to the embedding of token
    // tok[b] (a column of the tied int4 table ewq / esc in format efmt, or
    // row tok[b] of the fp32 table etable) times escale, and stored to x
    const uint32_t* tok = nullptr;
    const void* ewq = nullptr;
    const void* esc = nullptr;
    const float* etable = nullptr;
    uint32_t vocab = 0;
    int efmt = 0;
    float escale = 1.0f;
};
int launch_bprep(const BprepArgs& a, uint32_t batch, hipStream_t st);
// y[m][row][col] = sum_k A[row][k] W_m[k][col] for the staged A (rows = sequences).
struct BmmArgs {
    const void* a;             // staged operand (BprepArgs::a)
    const float* asum;
    // Or the operand's fp32 rows ([rows][lda]), converted in the GEMM:
    // amode 2 stages xa as is (bprep mode 2), 3 stages gelu_tanh(xa) * xu
    // (bprep mode 3); 0 reads a / asum.
    const float* xa;
    const float* xu;
    uint32_t amode;
    uint32_t lda;
    // GeGLU epilogue (two matrices of equal width, gate then up, k in one
    // split): workgroup c takes columns 32 c .. 32 c + 31 of both and writes
    // gelu_tanh(gate) * up of its 16 rows x 32 columns as the staged operand
    // block c of a following GEMM (a / asum, bprep_kernel's layout) instead of
    // the two outputs. a_out / asum_out must not alias a / asum.
    uint32_t geglu;
    void* a_out;
    float* asum_out;
    MvMatDesc mats[4];         // out is [rows][cols] row-major
    uint32_t n_mats;
    uint32_t groups[5];        // set by launch_bmm
    uint32_t nblk;             // k / 32
    uint32_t rows;             // sequences (<= 16)
    uint32_t kc, nsplit, n_colwg;   // set by launch_bmm
    float* part;
    size_t part_cap;
    uint32_t* tickets;
    uint32_t tickets_cap;
};
uint32_t bmm_split(uint32_t total_cols, uint32_t nblk, int n_cu);
size_t bmm_partial_floats(uint32_t total_cols, uint32_t nblk, int n_cu);
int launch_bmm(BmmArgs a, int fmt, int n_cu, hipStream_t st, const char* who);
// launch_bmm's plan for the tiled kernel (not the streamed one): fills
// groups, n_colwg, nsplit and kc, and returns the column blocks and whether
// they are quarter groups (one MFMA tile) or whole groups (four).
int plan_bmm(BmmArgs& a, int fmt, int n_cu, const char* who, uint32_t* n_blocks, bool* quarter);

// ---- persistent batched decode step (batch_step.hip; experimental, opt-in) ----
// One launch runs every layer of a batched decode step: one 512-thread
// workgroup per CU walks the stages of each layer (q|k|v GEMM, attention,
// o GEMM, staging, gate|up GEMM, down GEMM, staging) and takes the tiles of
// each stage the per-op kernels would run as workgroups. A stage's outputs
// are written with device-scope stores, then each tile stores the launch's
// tag in its own flag word; a stage's first tile on a workgroup waits
// (bounded) for every flag of the stage before. Per-layer argument blocks come from the per-op path's plans.
constexpr uint32_t kBsStages = 7;   // qkv, attention, o, staging, gate|up, down, staging
constexpr uint32_t kBsMaxTiles = 512;   // tiles of one stage (one flag per waiting thread)
struct BstepLayer {
    BmmArgs qkv, o, gu, dn;      // planned by plan_bmm (qkv, o, dn quarter blocks)
    AttnArgs att;                // planned by plan_attention
    BprepArgs prep1, prep2;      // mode 1, x_out set
    uint32_t att_u;              // keys per lane per pass (2, 4 or 8)
    uint32_t att_rope;           // index of the layer's RoPE frequencies
    uint32_t n_att;              // attention tiles (nsplit x kv heads x batch)
};
struct BstepArgs {
    const BstepLayer* layers;    // [n_layers], device memory, read-only while the kernel runs
    const RopeFreq* rope;        // [2] local, global
    uint32_t n_layers, batch;
    uint32_t ncb_qkv, ncb_o, ncb_dn, ns_dn, n_gu;   // column blocks; the down GEMM's k splits; gate|up tiles
    uint32_t* flags;             // [n_layers][kBsStages][kBsMaxTiles] tile flags (last launch's tag)
    uint32_t* epoch;             // the last launch's tag
    uint32_t* exit_cnt;          // workgroups that finished this launch (zero at rest)
    uint32_t* status;            // set when a wait ran past spin_limit
    uint32_t spin_limit;
    // Stage timeline (null: off): s_memrealtime (100 MHz) of each workgroup
    // at [((l kBsStages + k) 2 + e) grid + wg], e = 0 when its inputs of
    // stage k were ready, 1 when its last tile of the stage ended (0 when it
    // had none); then its start at [n_layers kBsStages 2 grid + wg].
    unsigned long long* trace;
};
int launch_bstep(const BstepArgs& a, int fmt, uint32_t grid, hipStream_t st);
int bstep_occupancy(int fmt, int* blocks_per_cu);

// ---- a decode session's device weights, for the batch (session.cpp) ----
constexpr int kMaxSessionLayers = 64;
struct SessionWeights {
    xp_config cfg;
    int n_cu;
    float embed_scale, attn_scale;
    struct Layer {
        const void* w[7];       // Q K V O GATE UP DOWN
        const void* s[7];
        const float* norm[6];   // attn, post_attn, ffn, post_ffw, q_norm, k_norm
        uint16_t* kc;           // the session's KV cache of the layer
        uint16_t* vc;
        bool global;
    } layer[kMaxSessionLayers];
    const void* lm_w;
    const void* lm_s;
    const float* final_norm;
    const float* embed;         // optional fp32 [vocab][hidden] embedding rows
};
int session_weights(const xp_session* h, SessionWeights* out);
// Batched prefill of a session (batch.cpp): tokens ids[0..n) at positions
// pos0 .. pos0 + n - 1 through the batched step, 16 positions per pass, rows
// sharing the session's KV cache; writes the KV rows, no logits. create
// returns nullptr (error set) when the shape does not fit the batched step.
struct PrefillBatch;
PrefillBatch* prefill_batch_create(const xp_session* s);
int prefill_batch_run(PrefillBatch* p, const uint32_t* ids, uint32_t n, uint32_t pos0);
void prefill_batch_destroy(PrefillBatch* p);
// The session's host draw and Philox uniform (decode.cpp:1873-1917).
uint32_t draw(float* val, uint32_t* idx, uint32_t n, float temperature, uint32_t top_k,
              float top_p, double u);
double philox_uniform(uint32_t seed, uint32_t seq, uint32_t step);

// ---- persistent token step (token_kernel.hip) ----
// Per-layer pointers, kept in device memory and read with uniform loads.
struct TokLayer {
    const void*  w[7];      // Q K V O GATE UP DOWN nibble planes (KM4)
    const void*  s[7];      // their scale planes (fp16 / bf16 quads)
    const float* norm[6];   // attn, post_attn, ffn, post_ffw, q_norm, k_norm (stored w - 1)
    uint16_t*    kc;        // fp16 caches [t][head_dim] (one kv head)
    uint16_t*    vc;
    uint32_t     global;    // 1: full-context layer, 0: sliding window
    uint32_t     pad;
};

struct TokArgs {
    const TokLayer* layers;
    uint32_t n_layers, hidden, ffn, n_heads, vocab, window;
    float eps, embed_scale, attn_scale;
    int fmt;                              // XP_SCALE_F16_QUAD or XP_SCALE_BF16_QUAD
    const void* lm_w;
    const void* lm_s;
    const float* final_norm;
    const float* embed_f32;               // optional fp32 [vocab][hidden] embedding rows
    const float* freq_local;              // [head_dim/2] theta^(-2d/head_dim)
    const float* freq_global;
    // Exchange slots: 8 bytes = (launch tag << 32) | fp32 bits, written with
    // one device-coherent store and read until the tag matches. Per layer
    // (stride ll_layer): xa[hidden] | xb[hidden] | qkv[split][q_dim + 2 hd] |
    // attp[grid][n_heads][2 + hd] | atto[q_dim] | o[split][hidden] | gu[ffn] (GeGLU output) |
    // dnp[down chunks][hidden]; then am[2 grid] once.
    unsigned long long* ll;
    size_t ll_layer;
    float* logits;                        // [vocab]
    uint32_t* state;                      // [0] position, [1] token, [2] status bits:
                                          // 1 a wait ran past its spin limit,
                                          // 2 the XCD placement changed
    uint32_t* hist;                       // [max_seq] token run at each position
    unsigned long long* trace;            // optional: [stage event][grid] timestamps
    uint32_t tag;                         // this launch's tag (never 0)
    uint32_t want_logits;                 // 0: prefill pass without the lm_head
    uint32_t greedy;                      // 1: the argmax becomes the next token
    // Non-zero when the probe found the grid dealt to eight distinct XCDs in
    // turn; nibble r of xcd_ids is the hardware XCC id of residue r. Each
    // workgroup then takes the role id whose residue is its own XCD's (the
    // starting XCD of a launch varies), and a local layer's attention and
    // combine run on one XCD (roles grid - 1 - 8 s) and exchange through its
    // L2 instead of the device coherence point.
    uint32_t xcd_local;
    uint32_t xcd_ids;
    // Poll rounds a wait takes before it records status bit 1 and gives up
    // (each round one device round trip, ~0.4-1 us).
    uint32_t spin_limit;
};
// Default spin limit of the token kernel's waits: ~0.1-0.25 s of poll rounds,
// far beyond any wait of a resident grid (the longest, the lm_head's final
// argmax poll, is ~30 us), so a grid that is not resident after all reports
// XP_E_DEVICE within a fraction of a second.
constexpr uint32_t kTokSpinLimit = 1u << 18;

// The token kernel's down projection is split along k into chunks of this
// many quads (128 k each); the next layer adds the chunks' partial sums. The
// q|k|v and o projections are split along k into this many halves likewise.
// Build-time knobs (-D) for sweeps; the whole library must be built with the
// same values, since the session sizes the exchange slots from them.
#ifndef XP_TOK_DOWN_QUADS
#define XP_TOK_DOWN_QUADS 14
#endif
#ifndef XP_TOK_QKV_SPLIT
#define XP_TOK_QKV_SPLIT 1
#endif
#ifndef XP_TOK_O_SPLIT
#define XP_TOK_O_SPLIT 1
#endif
constexpr uint32_t kTokDownQuads = XP_TOK_DOWN_QUADS;
constexpr uint32_t kTokQkvSplit = XP_TOK_QKV_SPLIT;
constexpr uint32_t kTokOSplit = XP_TOK_O_SPLIT;
__host__ __device__ constexpr uint32_t tok_down_chunks(uint32_t ffn) {
    return (ffn / 128u + kTokDownQuads - 1u) / kTokDownQuads;
}

// Exchange-slot offsets within one layer's block (in slots).
struct TokLL {
    size_t xa, xb, qkv, attp, atto, o, gu, dnp, layer;
};
__host__ __device__ inline TokLL tok_ll_layout(uint32_t hidden, uint32_t ffn, uint32_t n_heads, uint32_t head_dim,
                           uint32_t grid) {
    TokLL t{};
    const size_t qd = size_t(n_heads) * head_dim;
    t.xa = 0;
    t.xb = t.xa + hidden;
    t.qkv = t.xb + hidden;
    t.attp = t.qkv + kTokQkvSplit * (qd + 2 * head_dim);
    t.atto = t.attp + size_t(grid) * n_heads * (2 + head_dim);
    t.o = t.atto + qd;
    t.gu = t.o + kTokOSplit * size_t(hidden);
    t.dnp = t.gu + size_t(ffn);
    t.layer = t.dnp + size_t(tok_down_chunks(ffn)) * hidden;
    t.layer = (t.layer + 31) & ~size_t(31);
    return t;
}

constexpr int kTokThreads = 512;
// Trace events per launch, one timestamp per workgroup each: kernel start,
// then per layer the completion of QKV, attention, combine, O, gate/up and
// down (zero where the workgroup had no work), then lm_head and argmax.
inline uint32_t tok_trace_events(uint32_t n_layers) { return 12u * n_layers + 3u; }
// Dynamic LDS the token kernel asks for; larger than half a CU's LDS so that
// no CU holds two of the grid's workgroups.
size_t tok_lds_bytes();
// Checks the kernel can run this shape on the current device (grid = CUs).
int tok_supported(uint32_t n_layers, uint32_t hidden, uint32_t ffn, uint32_t n_heads,
                  uint32_t n_kv_heads, uint32_t head_dim, uint32_t vocab, uint32_t max_seq,
                  int fmt, int n_cu);
int launch_token(const TokArgs& a, uint32_t grid, hipStream_t st);
// Workgroups of the token kernel one CU can hold at once.
int tok_occupancy(uint32_t hidden, uint32_t ffn, uint32_t n_heads, int fmt, int* blocks_per_cu);
// For every workgroup of a token-kernel-shaped launch of `grid` workgroups
// (out: grid entries, host memory): its XCC id, | 0x100 when it saw the
// whole grid resident at once.
int probe_token_grid(uint32_t grid, hipStream_t st, uint32_t* out);

}  // namespace xp
