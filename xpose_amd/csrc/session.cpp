// Decode session: the token step of DecodeSession (examples/llm/decode.cpp:
// 1634-1866) on gfx950.
//
// One token step is recorded once into a HIP graph and replayed for every
// token. Everything that changes per token lives in device memory: the
// position and the token id (`state`), the KV cache, and the sampled ids
// (`hist`). Attention derives its window and span from the device position,
// so the graph never needs re-recording — the reference rejected static
// re-recording for exactly this reason (agent-docs/llm-inference.md:319-330)
// and instead re-records 838 dispatches per token on the host.
//
// Greedy decoding keeps the sampled token on the device: the argmax of pass t
// is the token pass t+1 embeds, which is the reference's sample-first order
// (decode.cpp:1830-1861) without a host round trip, so decode_steps(n) can
// queue n replays behind one wait.
#include "xp_internal.hpp"
#include "xp_launch.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

namespace xp {

int launch_norm_res_norm(float* x, const float* y, const float* w_post, const float* w_pre,
                         float* out, uint32_t n, float eps, hipStream_t st);
int launch_embed_norm(float* x, float* xn, const float* w_pre, float eps, const void* wq, const void* sc,
                      int fmt, uint32_t hidden, uint32_t vocab, float embed_scale, const uint32_t* state,
                      uint32_t* hist, const float* table, hipStream_t st);
int launch_advance(uint32_t* state, hipStream_t st);
uint16_t f32_to_f16(float f);

namespace {

double now_ms() {
    using namespace std::chrono;
    return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

constexpr int kNMat = 7;
constexpr int kNNorm = 6;
constexpr size_t kAlign = 256;
// Ticket regions: matvec split-k, decode attention (kAttnTicketsPerHead per
// kv head, at most 53 kv heads), argmax.
constexpr uint32_t kTicketMv = 0, kTicketAttn = 8192, kTicketAm = 8192 + 1024, kTickets = 8192 + 1088;
constexpr uint32_t kMaxKvHeads = (kTicketAm - kTicketAttn) / kAttnTicketsPerHead;

size_t align_up(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }

bool mat_dims(const xp_config& c, int m, uint32_t& rows, uint32_t& cols) {
    const uint32_t qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    switch (m) {
        case XP_T_Q: rows = c.hidden; cols = qd; return true;
        case XP_T_K:
        case XP_T_V: rows = c.hidden; cols = kvd; return true;
        case XP_T_O: rows = qd; cols = c.hidden; return true;
        case XP_T_GATE:
        case XP_T_UP: rows = c.hidden; cols = c.ffn; return true;
        case XP_T_DOWN: rows = c.ffn; cols = c.hidden; return true;
        case XP_T_LM_HEAD: rows = c.hidden; cols = c.vocab; return true;
        default: return false;
    }
}

size_t scale_bytes(const xp_config& c, uint32_t rows, uint32_t cols) {
    const size_t n = size_t(rows / 32) * cols;
    return c.scale_fmt == XP_SCALE_F32 ? n * 4 : n * 2;
}

// Bytes of a tensor, or 0 if the (layer, tensor) pair is not valid.
size_t tensor_bytes(const xp_config& c, int layer, int tensor) {
    const bool scales = (tensor & XP_T_SCALES) != 0;
    const int t = tensor & ~XP_T_SCALES;
    uint32_t rows = 0, cols = 0;
    if (t == XP_T_LM_HEAD) {
        if (layer != -1 || !mat_dims(c, t, rows, cols)) return 0;
    } else if (t <= XP_T_DOWN) {
        if (layer < 0 || uint32_t(layer) >= c.n_layers || !mat_dims(c, t, rows, cols)) return 0;
    } else if (scales) {
        return 0;
    } else if (t == XP_T_FINAL_NORM) {
        return layer == -1 ? size_t(c.hidden) * 4 : 0;
    } else if (t == XP_T_EMBED) {
        return layer == -1 ? size_t(c.vocab) * c.hidden * 4 : 0;
    } else if (t >= XP_T_ATTN_NORM && t <= XP_T_K_NORM) {
        if (layer < 0 || uint32_t(layer) >= c.n_layers) return 0;
        return (t >= XP_T_Q_NORM ? size_t(c.head_dim) : size_t(c.hidden)) * 4;
    } else {
        return 0;
    }
    return scales ? scale_bytes(c, rows, cols) : size_t(rows) * cols / 2;
}

// Synthetic tensor stream id: unique per (layer, tensor).
uint32_t synth_id(int layer, int tensor) {
    return uint32_t(layer + 1) * 1024u + uint32_t(tensor & 0x3FF) * 2u +
           ((tensor & XP_T_SCALES) ? 1u : 0u);
}

int check_config(const xp_config& c) {
    if (!c.n_layers || !c.hidden || !c.ffn || !c.n_heads || !c.n_kv_heads || !c.head_dim ||
        !c.vocab || !c.max_seq)
        return set_error(XP_E_ARG, "config: every shape field must be positive");
    if (c.hidden % 128 || c.ffn % 128 || (c.n_heads * c.head_dim) % 128)
        return set_error(XP_E_ARG, "config: matvec inputs (hidden=%u, ffn=%u, q_dim=%u) must be "
                         "multiples of 128", c.hidden, c.ffn, c.n_heads * c.head_dim);
    if (c.vocab % 64 || (c.n_kv_heads * c.head_dim) % 64)
        return set_error(XP_E_ARG, "config: vocab and kv_dim must be multiples of 64");
    const uint32_t grp = c.n_heads % c.n_kv_heads ? 0 : c.n_heads / c.n_kv_heads;
    if (c.head_dim != 256 || (grp != 1 && grp != 2 && grp != 4))
        return set_error(XP_E_ARG, "config: head_dim=%u (must be 256), heads %u over %u kv "
                         "heads (1, 2 or 4 per kv head)", c.head_dim, c.n_heads, c.n_kv_heads);
    if (c.max_seq > 8192)
        return set_error(XP_E_ARG, "config: max_seq=%u > 8192 (the reference's context limit)",
                         c.max_seq);
    if (c.n_kv_heads > kMaxKvHeads)
        return set_error(XP_E_ARG, "config: n_kv_heads=%u > %u", c.n_kv_heads, kMaxKvHeads);
    if (c.hidden > 8192)
        return set_error(XP_E_ARG, "config: hidden=%u > 8192", c.hidden);
    if (c.scale_fmt != XP_SCALE_F16_QUAD && c.scale_fmt != XP_SCALE_BF16_QUAD &&
        c.scale_fmt != XP_SCALE_F32)
        return set_error(XP_E_ARG, "config: unknown scale_fmt %d", c.scale_fmt);
    if (c.sample_mode != 0 && c.sample_mode != 1)
        return set_error(XP_E_ARG, "config: sample_mode %d (0 greedy, 1 temperature)",
                         c.sample_mode);
    if (c.sample_mode == 1 && (c.topk_parts == 0 || c.topk_parts > c.vocab))
        return set_error(XP_E_ARG, "config: topk_parts=%u must be in [1, vocab]", c.topk_parts);
    return XP_OK;
}

}  // namespace

struct Session {
    xp_config cfg{};
    hipStream_t st = nullptr;
    int n_cu = 256;
    char* warena = nullptr;
    size_t wbytes = 0;
    char* kvarena = nullptr;
    size_t kvbytes = 0;
    char* aarena = nullptr;
    char* tarena = nullptr;      // persistent-kernel tables and exchange buffers
    struct Layer {
        void* w[kNMat];
        void* s[kNMat];
        float* norm[kNNorm];
        uint16_t* kc;
        uint16_t* vc;
    };
    std::vector<Layer> L;
    void* lm_w = nullptr;
    void* lm_s = nullptr;
    float* final_norm = nullptr;
    float* embed = nullptr;      // optional fp32 [vocab][hidden] embedding rows
    PrefillBatch* pre = nullptr; // batched prefill (created on first use)
    bool pre_unavailable = false;
    float *x, *xb, *xb2, *q_raw, *k_raw, *v, *q, *k, *att, *gate, *up, *hb, *logits;
    float* mv_partial = nullptr;
    size_t mv_partial_cap = 0;
    float* attn_part = nullptr;
    uint32_t* tickets = nullptr;
    float* am_val = nullptr;
    uint32_t* am_idx = nullptr;
    float* am_out = nullptr;
    float* cand_val = nullptr;
    uint32_t* cand_idx = nullptr;
    uint32_t* state = nullptr;   // [0] position, [1] token
    uint32_t* hist = nullptr;    // [max_seq] token run at each position
    uint32_t* h_ids = nullptr;   // pinned staging for host-chosen token ids
    uint32_t* h_stat = nullptr;  // pinned: [0] device status word after a step
    uint32_t* h_attn = nullptr;  // pinned: the attention tickets after a step (graph paths)
    uint32_t attn_spin = 1u << 18;   // exchange-mode attention's spin limit (graph paths)
    size_t attn_floats = 0;      // attn_part's size
    hipGraphExec_t graph[3] = {nullptr, nullptr, nullptr};   // prefill, greedy, harvest
    uint32_t launches[3] = {0, 0, 0};
    int mode = XP_EXEC_GRAPH;    // XP_EXEC_TOKEN (persistent kernel), _GRAPH or _LAUNCH
    // Persistent token kernel: layer table, exchange buffers, barrier flags.
    TokLayer* d_layers = nullptr;
    TokArgs ta{};
    uint32_t tok_grid = 0;
    uint32_t tag = 0;            // tag of the last queued launch (exchange slots)
    unsigned long long* trace_buf = nullptr;
    hipEvent_t ev[2] = {nullptr, nullptr};   // decode_steps: device time of the queued steps
    uint32_t pos = 0;
    uint32_t step = 0;           // draws made (Philox counter)
    bool logits_valid = false;
    xp_metrics met{};
    std::vector<float> cv;
    std::vector<uint32_t> ci;

    float embed_scale() const {
        return cfg.embed_scale > 0.0f ? cfg.embed_scale : std::sqrt(float(cfg.hidden));
    }
    float attn_scale() const {
        return cfg.attn_scale > 0.0f ? cfg.attn_scale : 1.0f / std::sqrt(float(cfg.head_dim));
    }
    bool is_global(uint32_t l) const {
        return cfg.global_every == 0 || (l + 1) % cfg.global_every == 0;
    }

    int record(int variant, uint32_t& n);
    int run_token(int variant);
    int graph_for(int variant);
    int run(int variant);
};

int Session::record(int variant, uint32_t& n) {
    const xp_config& c = cfg;
    const uint32_t H = c.hidden, qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    const int fmt = c.scale_fmt;
    const float eps = c.rms_eps;
    int rc;
    n = 0;
#define XP_STEP(call)                \
    do {                             \
        if ((rc = (call)) != XP_OK) return rc; \
        ++n;                         \
    } while (0)
    // the embedding row and the first input norm (one launch)
    XP_STEP(launch_embed_norm(x, xb, L[0].norm[0], eps, lm_w, lm_s, fmt, H, c.vocab, embed_scale(), state,
                              hist, embed, st));
    // Where the column-slice matvec takes the shape, the residual add and
    // the two RMSNorms before the q|k|v and gate/up matvecs, and the GeGLU
    // before the down matvec, run inside those matvecs' staging instead of
    // as launches of their own (3 launches fewer a layer). The fused norm
    // writes the new residual to the other of two buffers, x and xb (xb is
    // free once layer 0's q|k|v has read its normed input).
    const bool fuse_norm = mv_slice_plan(H, qd + 2 * kvd, fmt, n_cu) && mv_slice_plan(H, 2 * c.ffn, fmt, n_cu);
    // the GeGLU as the gate/up matvec's output (each workgroup pairs the
    // same 32 columns of both), else staged by the down matvec
    const bool geglu_out = fuse_norm && mv_geglu_plan(H, c.ffn, fmt, n_cu);
    const bool fuse_geglu = !geglu_out && mv_slice_plan(c.ffn, H, fmt, n_cu);
    float* xr = x;                        // the residual stream
    float* xo = fuse_norm ? xb : nullptr;  // the other buffer (fused norms)
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        Layer& w = L[l];
        const bool glob = is_global(l);
        const float theta = glob ? c.rope_theta_global : c.rope_theta_local;
        const MvMatDesc qkv[3] = {{q_raw, w.w[XP_T_Q], w.s[XP_T_Q], qd},
                                  {k_raw, w.w[XP_T_K], w.s[XP_T_K], kvd},
                                  {v, w.w[XP_T_V], w.s[XP_T_V], kvd}};
        if (fuse_norm && l > 0) {
            MvIn in;
            in.mode = kMvInNorm;
            in.y = xb2;                       // the previous layer's down projection
            in.w_post = L[l - 1].norm[3];
            in.w_pre = w.norm[0];
            in.x_out = xo;
            in.eps = eps;
            XP_STEP(launch_mv(qkv, 3, xr, fmt, H, 0, mv_partial, mv_partial_cap, tickets + kTicketMv,
                              8192, st, "session qkv", n_cu, &in));
            std::swap(xr, xo);
        } else {
            XP_STEP(launch_mv(qkv, 3, xb, fmt, H, 0, mv_partial, mv_partial_cap, tickets + kTicketMv,
                              8192, st, "session qkv", n_cu));
        }
        // QK-norm, RoPE and the KV append run inside the attention launch
        AttnArgs aa{};
        aa.out = att; aa.kc = w.kc; aa.vc = w.vc;
        aa.q_raw = q_raw; aa.k_raw = k_raw; aa.v_raw = v;
        aa.qw = w.norm[4]; aa.kw = w.norm[5];
        aa.eps = eps;
        aa.theta = theta;
        aa.n_heads = c.n_heads; aa.kv_heads = c.n_kv_heads; aa.head_dim = c.head_dim;
        aa.pos_dev = state;
        aa.window = glob ? 0u : c.sliding_window;
        aa.scale = attn_scale();
        aa.part = attn_part;
        aa.tickets = tickets + kTicketAttn;
        aa.spin_limit = attn_spin;
        const uint32_t max_span = glob || c.sliding_window == 0
                                      ? c.max_seq : std::min(c.sliding_window, c.max_seq);
        XP_STEP(launch_attention(aa, max_span, st));
        const MvMatDesc o{xb2, w.w[XP_T_O], w.s[XP_T_O], H};
        XP_STEP(launch_mv(&o, 1, att, fmt, qd, 0, mv_partial, mv_partial_cap, tickets + kTicketMv,
                          8192, st, "session o_proj", n_cu));
        const MvMatDesc gu[2] = {{gate, w.w[XP_T_GATE], w.s[XP_T_GATE], c.ffn},
                                 {up, w.w[XP_T_UP], w.s[XP_T_UP], c.ffn}};
        if (fuse_norm) {
            MvIn in;
            in.mode = kMvInNorm;
            in.y = xb2;                       // the o projection
            in.w_post = w.norm[1];
            in.w_pre = w.norm[2];
            in.x_out = xo;
            in.eps = eps;
            in.geglu_out = geglu_out;
            const MvMatDesc guh[2] = {{hb, w.w[XP_T_GATE], w.s[XP_T_GATE], c.ffn},
                                      {up, w.w[XP_T_UP], w.s[XP_T_UP], c.ffn}};
            XP_STEP(launch_mv(geglu_out ? guh : gu, 2, xr, fmt, H, 0, mv_partial, mv_partial_cap,
                              tickets + kTicketMv, 8192, st, "session gate/up", n_cu, &in));
            std::swap(xr, xo);
        } else {
            XP_STEP(launch_norm_res_norm(x, xb2, w.norm[1], w.norm[2], xb, H, eps, st));
            XP_STEP(launch_mv(gu, 2, xb, fmt, H, 0, mv_partial, mv_partial_cap, tickets + kTicketMv,
                              8192, st, "session gate/up", n_cu));
        }
        const MvMatDesc d{xb2, w.w[XP_T_DOWN], w.s[XP_T_DOWN], H};
        if (geglu_out) {
            XP_STEP(launch_mv(&d, 1, hb, fmt, c.ffn, 0, mv_partial, mv_partial_cap,
                              tickets + kTicketMv, 8192, st, "session down", n_cu));
        } else if (fuse_geglu) {
            MvIn in;
            in.mode = kMvInGeglu;
            in.up = up;
            XP_STEP(launch_mv(&d, 1, gate, fmt, c.ffn, 0, mv_partial, mv_partial_cap,
                              tickets + kTicketMv, 8192, st, "session down", n_cu, &in));
        } else {
            XP_STEP(xp_geglu(hb, gate, up, c.ffn, st));
            XP_STEP(launch_mv(&d, 1, hb, fmt, c.ffn, 0, mv_partial, mv_partial_cap,
                              tickets + kTicketMv, 8192, st, "session down", n_cu));
        }
        if (!fuse_norm) {
            const float* next = (l + 1 < c.n_layers) ? L[l + 1].norm[0] : final_norm;
            XP_STEP(launch_norm_res_norm(x, xb2, w.norm[3], next, xb, H, eps, st));
        } else if (l + 1 == c.n_layers) {
            // the final norm, into the other buffer (the lm_head's input)
            XP_STEP(launch_norm_res_norm(xr, xb2, w.norm[3], final_norm, xo, H, eps, st));
        }
    }
    const float* lm_in = fuse_norm ? xo : xb;
    if (variant >= 1) {
        const MvMatDesc lm{logits, lm_w, lm_s, c.vocab};
        XP_STEP(launch_mv(&lm, 1, lm_in, fmt, H, 0, mv_partial, mv_partial_cap, tickets + kTicketMv,
                          8192, st, "session lm_head", n_cu));
        if (variant == 1)   // the greedy argmax also advances the position
            XP_STEP(launch_argmax(state + 1, am_out, logits, c.vocab, am_val, am_idx,
                                  tickets + kTicketAm, st, state));
        else
            XP_STEP(launch_topk4(cand_val, cand_idx, logits, c.vocab, c.topk_parts, st));
    }
    if (variant != 1) XP_STEP(launch_advance(state, st));
#undef XP_STEP
    return XP_OK;
}

int Session::graph_for(int variant) {
    if (graph[variant]) return XP_OK;
    hipGraph_t g = nullptr;
    XP_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    uint32_t n = 0;
    const int rc = record(variant, n);
    const hipError_t e = hipStreamEndCapture(st, &g);
    if (rc != XP_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess)
        return set_error(XP_E_HIP, "session: stream capture failed: %s", hipGetErrorString(e));
    const hipError_t ie = hipGraphInstantiate(&graph[variant], g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ie != hipSuccess) {
        graph[variant] = nullptr;
        return set_error(XP_E_HIP, "session: hipGraphInstantiate: %s", hipGetErrorString(ie));
    }
    launches[variant] = n;
    return XP_OK;
}

int Session::run_token(int variant) {
    ta.want_logits = variant >= 1 ? 1u : 0u;
    ta.greedy = variant == 1 ? 1u : 0u;
    if (++tag == 0) ++tag;       // slots start at tag 0; a launch never uses it
    ta.tag = tag;
    int rc = launch_token(ta, tok_grid, st);
    if (rc != XP_OK) return rc;
    launches[variant] = variant == 2 ? 2u : 1u;
    if (variant == 2) return launch_topk4(cand_val, cand_idx, logits, cfg.vocab, cfg.topk_parts, st);
    return XP_OK;
}

int Session::run(int variant) {
    if (mode == XP_EXEC_TOKEN) return run_token(variant);
    if (mode == XP_EXEC_LAUNCH) {
        uint32_t n = 0;
        const int r = record(variant, n);
        launches[variant] = n;
        return r;
    }
    int rc = graph_for(variant);
    if (rc != XP_OK) return rc;
    XP_HIP(hipGraphLaunch(graph[variant], st));
    return XP_OK;
}

// Host draw, examples/llm/decode.cpp:1873-1917: candidates ordered by (value
// desc, index asc) and cut to top_k; c = exp((v - max) / T) in float, sums in
// double; top-p keeps through the first candidate whose running mass reaches
// p * sum; r = u * sum walked down the list. The kept candidates are walked in
// sorted order (the reference walks nth_element's unspecified order unless
// top-p sorts them).
uint32_t draw(float* val, uint32_t* idx, uint32_t n, float temperature, uint32_t top_k,
              float top_p, double u) {
    if (n == 0) return 0;
    const float t = temperature > 0.0f ? temperature : 1.0f;
    std::vector<uint32_t> ord(n);
    for (uint32_t i = 0; i < n; ++i) ord[i] = i;
    std::sort(ord.begin(), ord.end(), [&](uint32_t a, uint32_t b) {
        return val[a] > val[b] || (val[a] == val[b] && idx[a] < idx[b]);
    });
    std::vector<float> v(n);
    std::vector<uint32_t> id(n);
    for (uint32_t i = 0; i < n; ++i) { v[i] = val[ord[i]]; id[i] = idx[ord[i]]; }
    const uint32_t k = top_k ? std::min(top_k, n) : n;
    n = k;
    float maxl = -INFINITY;
    for (uint32_t i = 0; i < n; ++i) maxl = std::max(maxl, v[i]);
    double sum = 0;
    for (uint32_t i = 0; i < n; ++i) {
        v[i] = std::exp((v[i] - maxl) / t);
        sum += v[i];
    }
    if (top_p > 0.0f && top_p < 1.0f && sum > 0) {
        double acc = 0, cut = top_p * sum;
        uint32_t keep = 0;
        for (; keep < n; ++keep) {
            acc += v[keep];
            if (acc >= cut) break;
        }
        n = std::min(n, keep + 1);
        sum = 0;
        for (uint32_t i = 0; i < n; ++i) sum += v[i];
    }
    for (uint32_t i = 0; i < n; ++i) { val[i] = v[i]; idx[i] = id[i]; }
    double r = u * sum;
    for (uint32_t i = 0; i < n; ++i) {
        r -= v[i];
        if (r <= 0) return id[i];
    }
    return id[n - 1];
}

double philox_uniform(uint32_t seed, uint32_t seq, uint32_t step) {
    const uint32_t c[4] = {step, 0u, 0u, 0u}, k[2] = {seed, seq};
    uint32_t o[4];
    xp_philox4x32_10(c, k, o);
    const uint64_t m = (uint64_t(o[0]) << 21) | (o[1] >> 11);
    return double(m) * (1.0 / 9007199254740992.0);
}

}  // namespace xp

using namespace xp;

struct xp_session {
    Session s;
};

namespace xp {
int session_weights(const xp_session* h, SessionWeights* out) {
    XP_REQUIRE(h && out, "null pointer");
    const Session& s = h->s;
    XP_REQUIRE(s.cfg.n_layers <= uint32_t(kMaxSessionLayers), "at most %d layers", kMaxSessionLayers);
    out->cfg = s.cfg;
    out->n_cu = s.n_cu;
    out->embed_scale = s.embed_scale();
    out->attn_scale = s.attn_scale();
    for (uint32_t l = 0; l < s.cfg.n_layers; ++l) {
        for (int m = 0; m < kNMat; ++m) {
            out->layer[l].w[m] = s.L[l].w[m];
            out->layer[l].s[m] = s.L[l].s[m];
        }
        for (int n = 0; n < kNNorm; ++n) out->layer[l].norm[n] = s.L[l].norm[n];
        out->layer[l].kc = s.L[l].kc;
        out->layer[l].vc = s.L[l].vc;
        out->layer[l].global = s.is_global(l);
    }
    out->lm_w = s.lm_w;
    out->lm_s = s.lm_s;
    out->final_norm = s.final_norm;
    out->embed = s.embed;
    return XP_OK;
}
}  // namespace xp

namespace {

int destroy(xp_session* h) {
    if (!h) return XP_OK;
    Session& s = h->s;
    if (s.pre) prefill_batch_destroy(s.pre);
    for (auto& g : s.graph)
        if (g) (void)hipGraphExecDestroy(g);
    for (auto& e : s.ev)
        if (e) (void)hipEventDestroy(e);
    if (s.st) (void)hipStreamSynchronize(s.st);
    if (s.warena) (void)hipFree(s.warena);
    if (s.kvarena) (void)hipFree(s.kvarena);
    if (s.aarena) (void)hipFree(s.aarena);
    if (s.tarena) (void)hipFree(s.tarena);
    if (s.embed) (void)hipFree(s.embed);
    if (s.trace_buf) (void)hipFree(s.trace_buf);
    if (s.h_ids) (void)hipHostFree(s.h_ids);
    if (s.h_stat) (void)hipHostFree(s.h_stat);
    if (s.h_attn) (void)hipHostFree(s.h_attn);
    if (s.st) (void)hipStreamDestroy(s.st);
    delete h;
    return XP_OK;
}

// Draws the next token from the last harvest (temperature mode).
int sample_from_candidates(Session& s, uint32_t& token) {
    const uint32_t nc = 4 * s.cfg.topk_parts;
    s.cv.resize(nc);
    s.ci.resize(nc);
    XP_HIP(hipMemcpy(s.cv.data(), s.cand_val, nc * 4, hipMemcpyDeviceToHost));
    XP_HIP(hipMemcpy(s.ci.data(), s.cand_idx, nc * 4, hipMemcpyDeviceToHost));
    uint32_t m = 0;
    for (uint32_t i = 0; i < nc; ++i)
        if (s.ci[i] != 0xFFFFFFFFu) { s.cv[m] = s.cv[i]; s.ci[m] = s.ci[i]; ++m; }
    const double u = philox_uniform(s.cfg.seed, s.cfg.seq_id, s.step++);
    token = draw(s.cv.data(), s.ci.data(), m, s.cfg.temperature, s.cfg.top_k, s.cfg.top_p, u);
    return XP_OK;
}

// Layer table, RoPE tables and exchange buffers of the persistent token
// kernel (token_kernel.hip); switches the session to it. Fails (and leaves
// the session on its graph path) when the device cannot hold the kernel's
// grid of one workgroup per CU resident at once: the occupancy query, then a
// probe launch of the same shape whose workgroups wait (bounded) for each
// other.
int setup_token(Session& s) {
    const xp_config& c = s.cfg;
    const uint32_t grid = uint32_t(s.n_cu);
    int per_cu = 0;
    if (int rc = tok_occupancy(c.hidden, c.ffn, c.n_heads, c.scale_fmt, &per_cu); rc != XP_OK)
        return rc;
    if (per_cu < 1)
        return set_error(XP_E_HIP, "token kernel: a CU cannot hold one 512-thread workgroup with "
                         "%zu B of LDS", tok_lds_bytes());
    std::vector<uint32_t> probe(grid);
    if (int rc = probe_token_grid(grid, s.st, probe.data()); rc != XP_OK) return rc;
    uint32_t resident = 0;
    for (uint32_t w = 0; w < grid; ++w) resident += (probe[w] >> 8) & 1u;
    if (resident != grid)
        return set_error(XP_E_DEVICE, "token kernel: %u of %u workgroups saw the whole grid "
                         "resident (another kernel holds CUs of this GPU)", resident, grid);
    const TokLL lay = tok_ll_layout(c.hidden, c.ffn, c.n_heads, c.head_dim, grid);
    const size_t sizes[] = {
        size_t(c.n_layers) * sizeof(TokLayer),                   // layer table
        size_t(c.head_dim / 2) * 4, size_t(c.head_dim / 2) * 4,  // freq local / global
        (size_t(c.n_layers) * lay.layer + 2 * size_t(grid)) * 8}; // exchange slots
    size_t tb = 0;
    for (size_t z : sizes) tb += align_up(z);
    if (hipMalloc(&s.tarena, tb) != hipSuccess)
        return set_error(XP_E_NOMEM, "xp_session_create: %zu token-kernel bytes", tb);
    if (hipMemset(s.tarena, 0, tb) != hipSuccess)
        return set_error(XP_E_HIP, "xp_session_create: clearing token-kernel buffers failed");
    char* p = s.tarena;
    size_t si = 0;
    auto nxt = [&]() { char* r = p; p += align_up(sizes[si++]); return r; };
    s.d_layers = reinterpret_cast<TokLayer*>(nxt());
    float* fl = reinterpret_cast<float*>(nxt());
    float* fg = reinterpret_cast<float*>(nxt());
    TokArgs& a = s.ta;
    a.ll = reinterpret_cast<unsigned long long*>(nxt());
    a.ll_layer = lay.layer;
    std::vector<TokLayer> tl(c.n_layers);
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        for (int m = 0; m < kNMat; ++m) { tl[l].w[m] = s.L[l].w[m]; tl[l].s[m] = s.L[l].s[m]; }
        for (int n = 0; n < kNNorm; ++n) tl[l].norm[n] = s.L[l].norm[n];
        tl[l].kc = s.L[l].kc;
        tl[l].vc = s.L[l].vc;
        tl[l].global = s.is_global(l) ? 1u : 0u;
        tl[l].pad = 0;
    }
    std::vector<float> f(c.head_dim / 2);
    auto freq = [&](float theta) {
        for (uint32_t d = 0; d < c.head_dim / 2; ++d)
            f[d] = std::exp2f(-std::log2f(theta) * (float(2u * d) / float(c.head_dim)));
    };
    XP_HIP(hipMemcpy(s.d_layers, tl.data(), tl.size() * sizeof(TokLayer), hipMemcpyHostToDevice));
    freq(c.rope_theta_local);
    XP_HIP(hipMemcpy(fl, f.data(), f.size() * 4, hipMemcpyHostToDevice));
    freq(c.rope_theta_global);
    XP_HIP(hipMemcpy(fg, f.data(), f.size() * 4, hipMemcpyHostToDevice));
    a.layers = s.d_layers;
    a.n_layers = c.n_layers;
    a.hidden = c.hidden;
    a.ffn = c.ffn;
    a.n_heads = c.n_heads;
    a.vocab = c.vocab;
    a.window = c.sliding_window;
    a.eps = c.rms_eps;
    a.embed_scale = s.embed_scale();
    a.attn_scale = s.attn_scale();
    a.fmt = c.scale_fmt;
    a.lm_w = s.lm_w;
    a.lm_s = s.lm_s;
    a.final_norm = s.final_norm;
    a.embed_f32 = s.embed;
    a.freq_local = fl;
    a.freq_global = fg;
    a.logits = s.logits;
    a.state = s.state;
    a.hist = s.hist;
    // Workgroup placement: the kernel groups producers and consumers by XCD
    // when the probe found the grid dealt to eight distinct XCDs in turn
    // (workgroup w on the XCD of w % 8); the kernel then takes each
    // workgroup's role from the XCD it runs on, since a launch's starting XCD
    // varies. Anything else (XP_PLACE_DEVICE, another layout) keeps every
    // exchange device-coherent.
    a.xcd_local = 0;
    a.xcd_ids = 0;
    a.spin_limit = kTokSpinLimit;
    if (c.placement == XP_PLACE_AUTO && grid >= 8 && grid % 8 == 0) {
        auto xcc = [&](uint32_t w) { return probe[w] & 0xFFu; };
        bool periodic = true;
        for (uint32_t w = 0; w < grid; ++w) periodic &= xcc(w) == xcc(w % 8);
        for (uint32_t i = 0; i < 8; ++i)
            for (uint32_t j = 0; j < i; ++j) periodic &= xcc(i) != xcc(j);
        if (periodic) {
            a.xcd_local = 1;
            for (uint32_t r = 0; r < 8; ++r) a.xcd_ids |= (xcc(r) & 15u) << (4 * r);
        }
    }
    s.tok_grid = grid;
    s.tag = 0;
    s.mode = XP_EXEC_TOKEN;
    return XP_OK;
}

// Device status word of the persistent kernel (state[2]): non-zero after a
// wait for another workgroup's data ran past its spin limit. queue_status
// copies it to pinned memory behind the queued work; check_status reads that
// copy after the stream has been synchronised.
// On the graph paths it copies the decode attention's tickets instead: an
// exchange-mode wait that timed out (its splits were not resident at once)
// leaves its head's error word set.
int queue_status(Session& s) {
    if (s.mode != XP_EXEC_TOKEN) {
        const size_t words = size_t(s.cfg.n_kv_heads) * kAttnTicketsPerHead;
        XP_HIP(hipMemcpyAsync(s.h_attn, s.tickets + kTicketAttn, words * 4, hipMemcpyDeviceToHost,
                              s.st));
        return XP_OK;
    }
    XP_HIP(hipMemcpyAsync(s.h_stat, s.state + 2, 4, hipMemcpyDeviceToHost, s.st));
    return XP_OK;
}
// Either error leaves the session's logits and the KV rows of the failed
// step invalid until the caller sets a position (xp_session_set_position or
// xp_session_reset), which also clears the status word.
int check_status(Session& s) {
    if (s.mode != XP_EXEC_TOKEN) {
        uint32_t err = 0;
        for (uint32_t g = 0; g < s.cfg.n_kv_heads; ++g)
            err |= s.h_attn[size_t(g) * kAttnTicketsPerHead + kAttnXErrWord];
        if (!err) return XP_OK;
        // the attention's records and tickets start over from zero
        XP_HIP(hipMemsetAsync(s.attn_part, 0, s.attn_floats * 4, s.st));
        XP_HIP(hipMemsetAsync(s.tickets + kTicketAttn, 0,
                              size_t(s.cfg.n_kv_heads) * kAttnTicketsPerHead * 4, s.st));
        XP_HIP(hipStreamSynchronize(s.st));
        s.logits_valid = false;
        return set_error(XP_E_DEVICE, "decode attention: an exchange-mode wait ran past its spin "
                         "limit (another kernel held CUs of this GPU); the step's results and KV "
                         "rows are invalid: set a position to go on");
    }
    const uint32_t st = s.h_stat[0];
    if (st & 2u) {
        // Later launches exchange every value through the device coherence
        // point (as XP_PLACE_DEVICE does).
        s.ta.xcd_local = 0;
        return set_error(XP_E_DEVICE, "token kernel: a workgroup ran on an XCD the session's "
                         "probe never saw (status %u); XCD-local exchange is now off. The step's "
                         "results and KV rows are invalid: set a position to go on", st);
    }
    if (st != 0)
        return set_error(XP_E_DEVICE, "token kernel: a wait for another workgroup's data ran "
                         "past its spin limit (status %u); the step's results and KV rows are "
                         "invalid: set a position to go on", st);
    return XP_OK;
}

}  // namespace

extern "C" {

int xp_session_trace(xp_session* h, int enable) {
    XP_REQUIRE(h, "null session");
    Session& s = h->s;
    XP_REQUIRE(s.mode == XP_EXEC_TOKEN, "barrier traces exist for the persistent token kernel only");
    XP_HIP(hipStreamSynchronize(s.st));
    if (!enable) {
        s.ta.trace = nullptr;
        return XP_OK;
    }
    if (!s.trace_buf) {
        const size_t n = size_t(tok_trace_events(s.cfg.n_layers)) * s.tok_grid;
        XP_HIP(hipMalloc(&s.trace_buf, n * 8));
        XP_HIP(hipMemset(s.trace_buf, 0, n * 8));
    }
    s.ta.trace = s.trace_buf;
    return XP_OK;
}

int xp_session_last_trace(xp_session* h, uint64_t* host, size_t n, uint32_t* grid) {
    XP_REQUIRE(h && host && grid, "null pointer");
    Session& s = h->s;
    XP_REQUIRE(s.trace_buf != nullptr, "tracing was never enabled");
    const size_t cap = size_t(tok_trace_events(s.cfg.n_layers)) * s.tok_grid;
    XP_REQUIRE(n <= cap, "n=%zu > %zu trace slots", n, cap);
    XP_HIP(hipStreamSynchronize(s.st));
    XP_HIP(hipMemcpy(host, s.trace_buf, n * 8, hipMemcpyDeviceToHost));
    *grid = s.tok_grid;
    return XP_OK;
}

void xp_config_gemma3_1b(xp_config* c) {
    if (!c) return;
    std::memset(c, 0, sizeof *c);
    c->n_layers = 26; c->hidden = 1152; c->ffn = 6912; c->n_heads = 4; c->n_kv_heads = 1;
    c->head_dim = 256; c->vocab = 262144; c->max_seq = 8192;
    c->global_every = 6; c->sliding_window = 512;
    c->rms_eps = 1e-6f; c->rope_theta_global = 1e6f; c->rope_theta_local = 1e4f;
    c->embed_scale = 0.0f; c->attn_scale = 0.0f;
    c->scale_fmt = XP_SCALE_F16_QUAD;
    c->sample_mode = 0; c->temperature = 1.0f; c->top_k = 0; c->top_p = 1.0f;
    c->seed = 1234; c->seq_id = 0; c->topk_parts = 1024;
}

int xp_tensor_bytes(const xp_config* c, int layer, int tensor, size_t* bytes) {
    XP_REQUIRE(c && bytes, "null pointer");
    const size_t b = tensor_bytes(*c, layer, tensor);
    XP_REQUIRE(b > 0, "no tensor %d at layer %d", tensor, layer);
    *bytes = b;
    return XP_OK;
}

int xp_synth_tensor(const xp_config* c, uint32_t seed, int layer, int tensor, void* host,
                    size_t bytes) {
    XP_REQUIRE(c && host, "null pointer");
    const size_t need = tensor_bytes(*c, layer, tensor);
    XP_REQUIRE(need > 0, "no tensor %d at layer %d", tensor, layer);
    XP_REQUIRE(bytes == need, "tensor %d at layer %d is %zu bytes, got %zu", tensor, layer, need,
               bytes);
    const int t = tensor & ~XP_T_SCALES;
    const uint32_t id = synth_id(layer, tensor);
    uint32_t rows = 0, cols = 0;
    if (mat_dims(*c, t, rows, cols)) {
        if (tensor & XP_T_SCALES) {
            XP_REQUIRE(c->scale_fmt != XP_SCALE_BF16_QUAD,
                       "synthetic scales are fp16 (F16 quad or F32 planes)");
            return xp_synth_scales(host, c->scale_fmt, rows, cols, 0.02f, seed, id);
        }
        return xp_synth_nibbles(static_cast<uint32_t*>(host), rows, cols, seed, id);
    }
    // Norm weight: multiplier m ~ N(1, 0.1) stored as m - 1.
    const size_t n = bytes / 4;
    float* f = static_cast<float*>(host);
    int rc = xp_synth_normal(f, n, 1.0f, 0.1f, seed, id);
    if (rc != XP_OK) return rc;
    for (size_t i = 0; i < n; ++i) f[i] = f[i] - 1.0f;
    return XP_OK;
}

int xp_session_create(const xp_config* cfg, xp_session** out) {
    XP_REQUIRE(cfg && out, "null pointer");
    *out = nullptr;
    int rc = check_config(*cfg);
    if (rc != XP_OK) return rc;
    xp_session* h = new (std::nothrow) xp_session;
    if (!h) return set_error(XP_E_NOMEM, "xp_session_create: out of host memory");
    Session& s = h->s;
    s.cfg = *cfg;
    const xp_config& c = s.cfg;
    if (c.exec_mode < XP_EXEC_AUTO || c.exec_mode > XP_EXEC_TOKEN) {
        delete h;
        return set_error(XP_E_ARG, "config: unknown exec_mode %d", c.exec_mode);
    }
    if (c.placement != XP_PLACE_AUTO && c.placement != XP_PLACE_DEVICE) {
        delete h;
        return set_error(XP_E_ARG, "config: unknown placement %d", c.placement);
    }
    try {
        int dev = 0;
        hipDeviceProp_t p;
        if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) {
            destroy(h);
            return set_error(XP_E_HIP, "xp_session_create: no HIP device");
        }
        s.n_cu = p.multiProcessorCount;
        if (hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking) != hipSuccess) {
            destroy(h);
            return set_error(XP_E_HIP, "xp_session_create: hipStreamCreate failed");
        }
        // ---- weights: one arena, every tensor 256-byte aligned
        size_t wb = 0;
        for (uint32_t l = 0; l < c.n_layers; ++l) {
            for (int m = 0; m < kNMat; ++m)
                wb += align_up(tensor_bytes(c, l, m)) + align_up(tensor_bytes(c, l, m | XP_T_SCALES));
            for (int nn = 0; nn < kNNorm; ++nn) wb += align_up(tensor_bytes(c, l, XP_T_ATTN_NORM + nn));
        }
        wb += align_up(tensor_bytes(c, -1, XP_T_LM_HEAD)) +
              align_up(tensor_bytes(c, -1, XP_T_LM_HEAD | XP_T_SCALES)) +
              align_up(tensor_bytes(c, -1, XP_T_FINAL_NORM));
        if (hipMalloc(&s.warena, wb) != hipSuccess) {
            destroy(h);
            return set_error(XP_E_NOMEM, "xp_session_create: %zu weight bytes", wb);
        }
        s.wbytes = wb;
        char* p8 = s.warena;
        auto take = [&](size_t b) { char* r = p8; p8 += align_up(b); return r; };
        s.L.resize(c.n_layers);
        for (uint32_t l = 0; l < c.n_layers; ++l) {
            for (int m = 0; m < kNMat; ++m) {
                s.L[l].w[m] = take(tensor_bytes(c, l, m));
                s.L[l].s[m] = take(tensor_bytes(c, l, m | XP_T_SCALES));
            }
            for (int nn = 0; nn < kNNorm; ++nn)
                s.L[l].norm[nn] = reinterpret_cast<float*>(take(tensor_bytes(c, l, XP_T_ATTN_NORM + nn)));
        }
        s.lm_w = take(tensor_bytes(c, -1, XP_T_LM_HEAD));
        s.lm_s = take(tensor_bytes(c, -1, XP_T_LM_HEAD | XP_T_SCALES));
        s.final_norm = reinterpret_cast<float*>(take(tensor_bytes(c, -1, XP_T_FINAL_NORM)));
        // ---- KV cache: [t][kv_heads][head_dim] fp16 per layer, K and V
        const size_t kvrow = size_t(c.n_kv_heads) * c.head_dim;
        const size_t per = align_up(size_t(c.max_seq) * kvrow * 2);
        s.kvbytes = per * 2 * c.n_layers;
        if (hipMalloc(&s.kvarena, s.kvbytes) != hipSuccess) {
            destroy(h);
            return set_error(XP_E_NOMEM, "xp_session_create: %zu KV bytes", s.kvbytes);
        }
        (void)hipMemset(s.kvarena, 0, s.kvbytes);
        for (uint32_t l = 0; l < c.n_layers; ++l) {
            s.L[l].kc = reinterpret_cast<uint16_t*>(s.kvarena + per * (2 * l));
            s.L[l].vc = reinterpret_cast<uint16_t*>(s.kvarena + per * (2 * l + 1));
        }
        // ---- activations and scratch
        const uint32_t H = c.hidden, qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
        size_t mvp = 0;
        mvp = std::max(mvp, mv_partial_floats(H, qd + 2 * kvd, 0, s.n_cu));
        mvp = std::max(mvp, mv_partial_floats(qd, H, 0, s.n_cu));
        mvp = std::max(mvp, mv_partial_floats(H, 2 * c.ffn, 0, s.n_cu));
        mvp = std::max(mvp, mv_partial_floats(c.ffn, H, 0, s.n_cu));
        mvp = std::max(mvp, mv_partial_floats(H, c.vocab, 0, s.n_cu));
        s.mv_partial_cap = std::max<size_t>(mvp, 64);
        const size_t attnp = attn_partial_floats(c.n_kv_heads, c.n_heads, c.head_dim);
        s.attn_floats = attnp;
        const uint32_t nc = c.sample_mode == 1 ? 4 * c.topk_parts : 4;
        const size_t sizes[] = {
            H * 4, std::max(H, qd) * 4, H * 4, qd * 4, kvd * 4, kvd * 4, qd * 4, kvd * 4, qd * 4,
            c.ffn * 4ull, c.ffn * 4ull, c.ffn * 4ull, c.vocab * 4ull,
            s.mv_partial_cap * 4, attnp * 4, kTickets * 4ull, kAmMaxWg * 4ull, kAmMaxWg * 4ull, 16,
            nc * 4ull, nc * 4ull, 64, c.max_seq * 4ull};
        size_t ab = 0;
        for (size_t z : sizes) ab += align_up(z);
        if (hipMalloc(&s.aarena, ab) != hipSuccess) {
            destroy(h);
            return set_error(XP_E_NOMEM, "xp_session_create: %zu activation bytes", ab);
        }
        (void)hipMemset(s.aarena, 0, ab);
        p8 = s.aarena;
        size_t si = 0;
        auto nxt = [&]() { return take(sizes[si++]); };
        s.x = (float*)nxt(); s.xb = (float*)nxt(); s.xb2 = (float*)nxt(); s.q_raw = (float*)nxt();
        s.k_raw = (float*)nxt(); s.v = (float*)nxt(); s.q = (float*)nxt(); s.k = (float*)nxt();
        s.att = (float*)nxt(); s.gate = (float*)nxt(); s.up = (float*)nxt(); s.hb = (float*)nxt();
        s.logits = (float*)nxt(); s.mv_partial = (float*)nxt(); s.attn_part = (float*)nxt();
        s.tickets = (uint32_t*)nxt(); s.am_val = (float*)nxt(); s.am_idx = (uint32_t*)nxt();
        s.am_out = (float*)nxt(); s.cand_val = (float*)nxt(); s.cand_idx = (uint32_t*)nxt();
        s.state = (uint32_t*)nxt(); s.hist = (uint32_t*)nxt();
        if (hipHostMalloc(reinterpret_cast<void**>(&s.h_ids), size_t(c.max_seq) * 4) !=
                hipSuccess ||
            hipHostMalloc(reinterpret_cast<void**>(&s.h_stat), 16) != hipSuccess ||
            hipHostMalloc(reinterpret_cast<void**>(&s.h_attn),
                          size_t(kMaxKvHeads) * kAttnTicketsPerHead * 4) != hipSuccess) {
            destroy(h);
            return set_error(XP_E_NOMEM, "xp_session_create: pinned staging");
        }
        // ---- execution mode
        s.mode = c.exec_mode == XP_EXEC_LAUNCH ? XP_EXEC_LAUNCH : XP_EXEC_GRAPH;
        const int tok_ok = (c.exec_mode == XP_EXEC_AUTO || c.exec_mode == XP_EXEC_TOKEN)
                               ? tok_supported(c.n_layers, c.hidden, c.ffn, c.n_heads,
                                               c.n_kv_heads, c.head_dim, c.vocab, c.max_seq,
                                               c.scale_fmt, s.n_cu)
                               : XP_E_ARG;
        if (c.exec_mode == XP_EXEC_TOKEN && tok_ok != XP_OK) {
            destroy(h);
            return tok_ok;
        }
        if (tok_ok == XP_OK) {
            int rc = setup_token(s);
            if (rc != XP_OK && c.exec_mode == XP_EXEC_TOKEN) {
                destroy(h);
                return rc;
            }
            // XP_EXEC_AUTO: a device that cannot run the token kernel keeps
            // the graph path chosen above
        }
        clear_error();
        if (hipDeviceSynchronize() != hipSuccess) {
            destroy(h);
            return set_error(XP_E_HIP, "xp_session_create: initialisation failed");
        }
    } catch (const std::bad_alloc&) {
        destroy(h);
        return set_error(XP_E_NOMEM, "xp_session_create: out of host memory");
    }
    *out = h;
    return XP_OK;
}

int xp_session_destroy(xp_session* h) { return destroy(h); }

int xp_session_upload(xp_session* h, int layer, int tensor, const void* host, size_t bytes) {
    XP_REQUIRE(h && host, "null pointer");
    const size_t need = tensor_bytes(h->s.cfg, layer, tensor);
    XP_REQUIRE(need > 0, "no tensor %d at layer %d", tensor, layer);
    XP_REQUIRE(bytes == need, "tensor %d at layer %d is %zu bytes, got %zu", tensor, layer, need,
               bytes);
    return xp_session_upload_part(h, layer, tensor, 0, host, bytes);
}

int xp_session_upload_part(xp_session* h, int layer, int tensor, size_t offset, const void* host,
                           size_t bytes) {
    XP_REQUIRE(h && host, "null pointer");
    Session& s = h->s;
    const size_t need = tensor_bytes(s.cfg, layer, tensor);
    XP_REQUIRE(need > 0, "no tensor %d at layer %d", tensor, layer);
    XP_REQUIRE(offset <= need && bytes <= need - offset,
               "bytes [%zu, +%zu) outside tensor %d at layer %d (%zu bytes)", offset, bytes, tensor,
               layer, need);
    const bool sc = (tensor & XP_T_SCALES) != 0;
    const int t = tensor & ~XP_T_SCALES;
    void* dst = nullptr;
    if (t == XP_T_EMBED) {
        if (!s.embed) {
            // First use: allocate the table and drop recorded graphs, whose
            // embedding step was recorded without it.
            XP_HIP(hipStreamSynchronize(s.st));
            if (hipMalloc(&s.embed, need) != hipSuccess) {
                s.embed = nullptr;
                return set_error(XP_E_NOMEM, "xp_session_upload_part: %zu embedding bytes", need);
            }
            for (auto& g : s.graph)
                if (g) {
                    (void)hipGraphExecDestroy(g);
                    g = nullptr;
                }
            s.ta.embed_f32 = s.embed;
        }
        dst = s.embed;
    } else if (t == XP_T_LM_HEAD) dst = sc ? s.lm_s : s.lm_w;
    else if (t == XP_T_FINAL_NORM) dst = s.final_norm;
    else if (t <= XP_T_DOWN) dst = sc ? s.L[layer].s[t] : s.L[layer].w[t];
    else dst = s.L[layer].norm[t - XP_T_ATTN_NORM];
    XP_HIP(hipMemcpy(static_cast<char*>(dst) + offset, host, bytes, hipMemcpyHostToDevice));
    return XP_OK;
}

int xp_session_synthesize(xp_session* h, uint32_t seed) {
    XP_REQUIRE(h, "null session");
    Session& s = h->s;
    std::vector<char> buf;
    auto one = [&](int layer, int tensor) -> int {
        const size_t b = tensor_bytes(s.cfg, layer, tensor);
        buf.resize(b);
        int rc = xp_synth_tensor(&s.cfg, seed, layer, tensor, buf.data(), b);
        if (rc == XP_OK) rc = xp_session_upload(h, layer, tensor, buf.data(), b);
        return rc;
    };
    try {
        int rc;
        for (uint32_t l = 0; l < s.cfg.n_layers; ++l) {
            for (int m = 0; m < kNMat; ++m) {
                if ((rc = one(int(l), m)) != XP_OK) return rc;
                if ((rc = one(int(l), m | XP_T_SCALES)) != XP_OK) return rc;
            }
            for (int nn = 0; nn < kNNorm; ++nn)
                if ((rc = one(int(l), XP_T_ATTN_NORM + nn)) != XP_OK) return rc;
        }
        if ((rc = one(-1, XP_T_LM_HEAD)) != XP_OK) return rc;
        if ((rc = one(-1, XP_T_LM_HEAD | XP_T_SCALES)) != XP_OK) return rc;
        return one(-1, XP_T_FINAL_NORM);
    } catch (const std::bad_alloc&) {
        return set_error(XP_E_NOMEM, "xp_session_synthesize: out of host memory");
    }
}

int xp_session_kv_upload(xp_session* h, int layer, int which, uint32_t pos0, uint32_t n,
                         const uint16_t* host) {
    XP_REQUIRE(h && host, "null pointer");
    Session& s = h->s;
    XP_REQUIRE(layer >= 0 && uint32_t(layer) < s.cfg.n_layers && (which == 0 || which == 1),
               "layer %d / which %d out of range", layer, which);
    XP_REQUIRE(uint64_t(pos0) + n <= s.cfg.max_seq, "rows [%u, %u) exceed max_seq %u", pos0,
               pos0 + n, s.cfg.max_seq);
    const size_t row = size_t(s.cfg.n_kv_heads) * s.cfg.head_dim;
    uint16_t* base = which ? s.L[layer].vc : s.L[layer].kc;
    XP_HIP(hipMemcpy(base + row * pos0, host, row * n * 2, hipMemcpyHostToDevice));
    return XP_OK;
}

int xp_session_kv_download(xp_session* h, int layer, int which, uint32_t pos0, uint32_t n,
                           uint16_t* host) {
    XP_REQUIRE(h && host, "null pointer");
    Session& s = h->s;
    XP_REQUIRE(layer >= 0 && uint32_t(layer) < s.cfg.n_layers && (which == 0 || which == 1),
               "layer %d / which %d out of range", layer, which);
    XP_REQUIRE(uint64_t(pos0) + n <= s.cfg.max_seq, "rows [%u, %u) exceed max_seq %u", pos0,
               pos0 + n, s.cfg.max_seq);
    const size_t row = size_t(s.cfg.n_kv_heads) * s.cfg.head_dim;
    const uint16_t* base = which ? s.L[layer].vc : s.L[layer].kc;
    XP_HIP(hipStreamSynchronize(s.st));
    XP_HIP(hipMemcpy(host, base + row * pos0, row * n * 2, hipMemcpyDeviceToHost));
    return XP_OK;
}

int xp_session_set_position(xp_session* h, uint32_t pos) {
    XP_REQUIRE(h, "null session");
    Session& s = h->s;
    XP_REQUIRE(pos <= s.cfg.max_seq, "position %u > max_seq %u", pos, s.cfg.max_seq);
    XP_HIP(hipStreamSynchronize(s.st));
    s.pos = pos;
    s.logits_valid = false;
    // position, then the token kernel's status word: a failed step's error
    // does not outlive the context the caller rebuilds from here
    const uint32_t st[3] = {pos, 0u, 0u};
    XP_HIP(hipMemcpy(s.state, &st[0], 4, hipMemcpyHostToDevice));
    XP_HIP(hipMemcpy(s.state + 2, &st[2], 4, hipMemcpyHostToDevice));
    s.h_stat[0] = 0;
    return XP_OK;
}

int xp_session_reset(xp_session* h) { return xp_session_set_position(h, 0); }

int xp_session_set_spin_limit(xp_session* h, uint32_t rounds) {
    XP_REQUIRE(h, "null session");
    Session& s = h->s;
    XP_REQUIRE(rounds <= (1u << 24), "xp_session_set_spin_limit: rounds=%u > 2^24", rounds);
    XP_HIP(hipStreamSynchronize(s.st));
    s.ta.spin_limit = rounds;   // passed by value at each token-kernel launch
    if (s.attn_spin != rounds) {
        s.attn_spin = rounds;   // the graphs hold it: recaptured at their next use
        for (auto& g : s.graph) {
            if (g) (void)hipGraphExecDestroy(g);
            g = nullptr;
        }
    }
    return XP_OK;
}

int xp_session_prefill(xp_session* h, const uint32_t* ids, uint32_t n) {
    XP_REQUIRE(h, "null session");
    if (n == 0) return XP_OK;
    XP_REQUIRE(ids, "ids is null");
    Session& s = h->s;
    XP_REQUIRE(uint64_t(s.pos) + n <= s.cfg.max_seq, "prompt exceeds max_seq (%u)",
               s.cfg.max_seq);
    for (uint32_t i = 0; i < n; ++i)
        XP_REQUIRE(ids[i] < s.cfg.vocab, "token id %u is outside the vocabulary", ids[i]);
    const double t0 = now_ms();
    XP_HIP(hipStreamSynchronize(s.st));
    std::memcpy(s.h_ids, ids, size_t(n) * 4);
    const int last = s.cfg.sample_mode == 0 ? 1 : 2;
    uint32_t first = 0;
    if (n >= 3 && s.cfg.prefill_mode == XP_PREFILL_AUTO && !s.pre_unavailable) {
        if (!s.pre && !(s.pre = prefill_batch_create(h))) {
            s.pre_unavailable = true;   // the shape does not fit: token by token
            clear_error();
        }
        if (s.pre) {
            // positions pos .. pos + n - 2 through the batched step, then the
            // last token on the session's own path
            int rc = prefill_batch_run(s.pre, ids, n - 1, s.pos);
            if (rc != XP_OK) return rc;
            first = n - 1;
            s.h_stat[3] = s.pos + first;
            XP_HIP(hipMemcpyAsync(s.state, s.h_stat + 3, 4, hipMemcpyHostToDevice, s.st));
            XP_HIP(hipMemcpyAsync(s.hist + s.pos, s.h_ids, size_t(first) * 4,
                                  hipMemcpyHostToDevice, s.st));
        }
    }
    for (uint32_t i = first; i < n; ++i) {
        XP_HIP(hipMemcpyAsync(s.state + 1, s.h_ids + i, 4, hipMemcpyHostToDevice, s.st));
        int rc = s.run(i + 1 == n ? last : 0);
        if (rc != XP_OK) return rc;
    }
    if (int rc = queue_status(s); rc != XP_OK) return rc;
    XP_HIP(hipStreamSynchronize(s.st));
    if (int rc = check_status(s); rc != XP_OK) return rc;
    s.pos += n;
    s.logits_valid = true;
    const double ms = now_ms() - t0;
    s.met = xp_metrics{ms, ms, 0.0, ms > 0 ? n * 1000.0 / ms : 0.0, s.pos, s.launches[0], s.mode};
    return XP_OK;
}

int xp_session_decode_step(xp_session* h, uint32_t* token) {
    XP_REQUIRE(h && token, "null pointer");
    Session& s = h->s;
    if (s.pos == 0 || !s.logits_valid)
        return set_error(XP_E_STATE, "decode_step() before prefill() - there is no context to "
                         "condition on");
    if (s.pos >= s.cfg.max_seq)
        return set_error(XP_E_STATE, "KV cache is full (max_seq %u)", s.cfg.max_seq);
    const double t0 = now_ms();
    double ts = 0;
    int variant = 1;
    if (s.cfg.sample_mode == 1) {
        variant = 2;
        uint32_t tok = 0;
        int rc = sample_from_candidates(s, tok);
        if (rc != XP_OK) return rc;
        s.h_ids[0] = tok;
        XP_HIP(hipMemcpyAsync(s.state + 1, s.h_ids, 4, hipMemcpyHostToDevice, s.st));
        ts = now_ms() - t0;
    }
    const double t1 = now_ms();
    int rc = s.run(variant);
    if (rc != XP_OK) return rc;
    XP_HIP(hipMemcpyAsync(s.h_ids + 1, s.hist + s.pos, 4, hipMemcpyDeviceToHost, s.st));
    if (int rc2 = queue_status(s); rc2 != XP_OK) return rc2;
    XP_HIP(hipStreamSynchronize(s.st));
    if (int rc2 = check_status(s); rc2 != XP_OK) return rc2;
    *token = s.h_ids[1];
    const double t2 = now_ms();
    ++s.pos;
    s.met = xp_metrics{t2 - t0, t2 - t1, ts, (t2 - t0) > 0 ? 1000.0 / (t2 - t0) : 0.0, s.pos,
                       s.launches[variant], s.mode};
    return XP_OK;
}

int xp_session_decode_steps(xp_session* h, uint32_t n, uint32_t* tokens) {
    XP_REQUIRE(h, "null session");
    if (n == 0) return XP_OK;
    Session& s = h->s;
    XP_REQUIRE(s.cfg.sample_mode == 0, "decode_steps queues greedy steps only");
    if (s.pos == 0 || !s.logits_valid)
        return set_error(XP_E_STATE, "decode_steps() before prefill()");
    if (uint64_t(s.pos) + n > s.cfg.max_seq)
        return set_error(XP_E_STATE, "KV cache is full (max_seq %u)", s.cfg.max_seq);
    if (!s.ev[0]) {
        XP_HIP(hipEventCreate(&s.ev[0]));
        XP_HIP(hipEventCreate(&s.ev[1]));
    }
    const double t0 = now_ms();
    XP_HIP(hipEventRecord(s.ev[0], s.st));
    for (uint32_t i = 0; i < n; ++i) {
        int rc = s.run(1);
        if (rc != XP_OK) return rc;
    }
    XP_HIP(hipEventRecord(s.ev[1], s.st));
    if (int rc = queue_status(s); rc != XP_OK) return rc;
    XP_HIP(hipStreamSynchronize(s.st));
    const double t1 = now_ms();
    float dev_ms = 0.0f;
    XP_HIP(hipEventElapsedTime(&dev_ms, s.ev[0], s.ev[1]));
    if (int rc = check_status(s); rc != XP_OK) return rc;
    if (tokens) XP_HIP(hipMemcpy(tokens, s.hist + s.pos, size_t(n) * 4, hipMemcpyDeviceToHost));
    s.pos += n;
    s.met = xp_metrics{t1 - t0, double(dev_ms), 0.0, (t1 - t0) > 0 ? n * 1000.0 / (t1 - t0) : 0.0,
                       s.pos, s.launches[1], s.mode};
    return XP_OK;
}

int xp_session_position(const xp_session* h, uint32_t* pos) {
    XP_REQUIRE(h && pos, "null pointer");
    *pos = h->s.pos;
    return XP_OK;
}

int xp_session_last_logits(xp_session* h, float* host, uint32_t n) {
    XP_REQUIRE(h && host, "null pointer");
    Session& s = h->s;
    XP_REQUIRE(n <= s.cfg.vocab, "n=%u > vocab %u", n, s.cfg.vocab);
    XP_HIP(hipStreamSynchronize(s.st));
    XP_HIP(hipMemcpy(host, s.logits, size_t(n) * 4, hipMemcpyDeviceToHost));
    return XP_OK;
}

int xp_session_last_candidates(xp_session* h, float* val, uint32_t* idx, uint32_t n) {
    XP_REQUIRE(h && val && idx, "null pointer");
    Session& s = h->s;
    XP_REQUIRE(s.cfg.sample_mode == 1, "the harvest runs in temperature mode only");
    XP_REQUIRE(n <= 4 * s.cfg.topk_parts, "n=%u > %u candidates", n, 4 * s.cfg.topk_parts);
    XP_HIP(hipStreamSynchronize(s.st));
    XP_HIP(hipMemcpy(val, s.cand_val, size_t(n) * 4, hipMemcpyDeviceToHost));
    XP_HIP(hipMemcpy(idx, s.cand_idx, size_t(n) * 4, hipMemcpyDeviceToHost));
    return XP_OK;
}

int xp_session_last_metrics(const xp_session* h, xp_metrics* m) {
    XP_REQUIRE(h && m, "null pointer");
    *m = h->s.met;
    return XP_OK;
}

int xp_session_weight_bytes(const xp_session* h, size_t* bytes) {
    XP_REQUIRE(h && bytes, "null pointer");
    *bytes = h->s.wbytes;
    return XP_OK;
}

int xp_session_exec_mode(const xp_session* h, int32_t* mode) {
    XP_REQUIRE(h && mode, "null pointer");
    *mode = h->s.mode;
    return XP_OK;
}

int xp_session_kv_bytes(const xp_session* h, size_t* bytes) {
    XP_REQUIRE(h && bytes, "null pointer");
    *bytes = h->s.kvbytes;
    return XP_OK;
}

uint32_t xp_draw(float* val, uint32_t* idx, uint32_t n, float temperature, uint32_t top_k,
                 float top_p, double u) {
    if (!val || !idx) return 0;
    return draw(val, idx, n, temperature, top_k, top_p, u);
}

double xp_philox_uniform(uint32_t seed, uint32_t seq, uint32_t step) {
    return philox_uniform(seed, seq, step);
}

}  // extern "C"
