// Batched decode: up to 16 independent sequences per step on one session's
// weights (benchmark config 5). The reference decodes one sequence per
// DecodeSession (examples/llm/decode.cpp:1634-1866); a batch runs the same
// token step for every sequence at once, so the 0.56 GB of int4 weights are
// read once per step instead of once per sequence and the matvecs become
// M = 16 GEMMs on the matrix cores (batch_kernels.hip).
//
// Each sequence keeps the single-sequence semantics: its own fp16 KV cache,
// position and sample-first order (decode.cpp:1830-1850) — draw from the last
// logits, then run the network on the drawn token. Sequence i draws with
// Philox(key = (seed, seq_id + i), counter = its own draw count), so a
// sequence's stream does not depend on the batch it runs in. The draw is the
// session's host draw (decode.cpp:1873-1917) over the exact top-64 candidates
// of the sequence's logits, computed on the device.
//
// The step is recorded once into a HIP graph: positions and tokens live in
// device arrays, so every replay is the same graph.
#include "xp_internal.hpp"
#include "xp_launch.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

namespace xp {
namespace {

constexpr uint32_t kBatchMax = 16;
constexpr uint32_t kBlkB = 32;           // quantisation block along k
constexpr uint32_t kGrpB = 64;           // KM4 column group
constexpr uint32_t kCand = 64;           // candidates per sequence (top-k <= 64)
// The candidates are the reference's harvest, the best 4 of each of 4096
// strided chains (topk4_partial, llm_sampling.cl:318-347); the 64 best of
// those are selected exactly on the device.
constexpr uint32_t kHarvestParts = 4096;
constexpr uint32_t kHarvest = 4 * kHarvestParts;
constexpr size_t kAlignB = 256;

size_t al(size_t v) { return (v + kAlignB - 1) & ~(kAlignB - 1); }

struct Batch {
    SessionWeights w{};
    uint32_t B = 0, S = 0;
    hipStream_t st = nullptr;
    char* arena = nullptr;
    uint16_t* kc[kMaxSessionLayers] = {};
    uint16_t* vc[kMaxSessionLayers] = {};
    float *x, *q_raw, *k_raw, *v, *q, *k, *att, *o, *dn, *logits;
    void* a = nullptr;
    float* asum = nullptr;
    // the down projection's operand, staged by the gate|up GEMM's GeGLU epilogue
    void* a2 = nullptr;
    float* asum2 = nullptr;
    float* part = nullptr;
    size_t part_cap = 0;
    uint32_t* tickets = nullptr;
    uint32_t tickets_cap = 0;
    float* attn_part = nullptr;
    size_t attn_part_seq = 0;
    uint32_t* attn_tickets = nullptr;
    float *cval, *oval;
    uint32_t *cidx, *oidx, *d_tok, *d_pos;
    uint32_t* h_tok = nullptr;           // pinned
    float* h_val = nullptr;              // pinned [B][64]
    uint32_t* h_idx = nullptr;
    hipGraphExec_t graph = nullptr;
    hipEvent_t ev[2] = {nullptr, nullptr};
    std::vector<uint32_t> pos, steps;
    bool logits_valid = false;
    float last_ms = 0.0f;
    // Prefill mode: the rows are consecutive positions of one sequence and
    // share the session's KV cache; the step ends after the last layer.
    bool prefill = false;

    int record();
    int forward(const uint32_t* tokens);
};

int Batch::record() {
    const xp_config& c = w.cfg;
    const uint32_t H = c.hidden, qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    const int fmt = c.scale_fmt;
    const float eps = c.rms_eps;
    int rc;
#define XB(call) do { if ((rc = (call)) != XP_OK) return rc; } while (0)
    auto prep = [&](int mode, float* x_, const float* y_, const float* u_, const float* wpost,
                    const float* wpre, uint32_t K) {
        BprepArgs p{mode, x_, y_, u_, wpost, wpre, a, asum, K, eps};
        return launch_bprep(p, B, st);
    };
    // amode 2 / 3: the GEMM stages its operand from fp32 rows xa (and xu)
    // itself, in place of a bprep mode 2 / 3 launch
    // geglu: the GEMM's epilogue stages gelu(gate) * up into a2 / asum2; op2:
    // the GEMM reads its operand from a2 / asum2
    auto gemm = [&](const MvMatDesc* m, uint32_t n, uint32_t K, const char* who,
                    uint32_t amode = 0, const float* xa = nullptr, const float* xu = nullptr,
                    bool geglu = false, bool op2 = false) {
        BmmArgs g{};
        g.a = op2 ? a2 : a;
        g.asum = op2 ? asum2 : asum;
        g.geglu = geglu ? 1u : 0u;
        g.a_out = geglu ? a2 : nullptr;
        g.asum_out = geglu ? asum2 : nullptr;
        g.amode = amode;
        g.xa = xa;
        g.xu = xu;
        g.lda = K;
        for (uint32_t i = 0; i < n; ++i) g.mats[i] = m[i];
        g.n_mats = n;
        g.nblk = K / kBlkB;
        g.rows = B;
        g.part = part;
        g.part_cap = part_cap;
        g.tickets = tickets;
        g.tickets_cap = tickets_cap;
        return launch_bmm(g, fmt, w.n_cu, st, who);
    };
    XB(launch_bembed(x, w.lm_w, w.lm_s, fmt, H, c.vocab, w.embed_scale, d_tok, B, w.embed, st));
    XB(prep(0, x, nullptr, nullptr, nullptr, w.layer[0].norm[0], H));
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const SessionWeights::Layer& L = w.layer[l];
        const bool glob = L.global;
        const MvMatDesc qkv[3] = {{q_raw, L.w[XP_T_Q], L.s[XP_T_Q], qd},
                                  {k_raw, L.w[XP_T_K], L.s[XP_T_K], kvd},
                                  {v, L.w[XP_T_V], L.s[XP_T_V], kvd}};
        XB(gemm(qkv, 3, H, "batch qkv"));
        const float theta = glob ? c.rope_theta_global : c.rope_theta_local;
        if (prefill) {
            // prefill rows share one cache: every row's key / value is
            // appended before any row attends (a row's span includes the
            // rows before it)
            QkArgs qa{q, k, q_raw, k_raw, v, L.norm[4], L.norm[5], kc[l], vc[l],
                      c.n_heads, c.n_kv_heads, c.head_dim, eps, d_pos, 0};
            qa.batch = B;
            qa.bq = qd;
            qa.bkv = kvd;
            qa.bcache = 0;
            XB(launch_qk(qa, theta, st));
            // the last layer's K/V rows are the last thing the step must produce
            if (l + 1 == c.n_layers) break;
        }
        AttnArgs aa{};
        aa.out = att; aa.q = q; aa.kc = kc[l]; aa.vc = vc[l];
        if (!prefill) {
            // decode: QK-norm, RoPE and the KV append inside the attention launch
            aa.q_raw = q_raw; aa.k_raw = k_raw; aa.v_raw = v;
            aa.qw = L.norm[4]; aa.kw = L.norm[5];
            aa.eps = eps;
            aa.theta = theta;
            aa.bkv = kvd;
        }
        aa.n_heads = c.n_heads; aa.kv_heads = c.n_kv_heads; aa.head_dim = c.head_dim;
        aa.pos_dev = d_pos;
        aa.window = glob ? 0u : c.sliding_window;
        aa.scale = w.attn_scale;
        aa.part = attn_part;
        aa.tickets = attn_tickets;
        aa.batch = B;
        aa.bq = qd;
        aa.bcache = prefill ? 0 : size_t(S) * kvd;
        aa.bpart = attn_part_seq;
        const uint32_t max_span = glob || c.sliding_window == 0 ? S : std::min(c.sliding_window, S);
        XB(launch_attention(aa, max_span, st));
        const MvMatDesc om{o, L.w[XP_T_O], L.s[XP_T_O], H};
        XB(gemm(&om, 1, qd, "batch o_proj", 2, att));
        XB(prep(1, x, o, nullptr, L.norm[1], L.norm[2], H));
        // gate and up of the same 32 columns per workgroup; its epilogue
        // stages gelu(gate) * up as the down projection's operand block
        // (no fp32 gate / up rows, no staging launch)
        const MvMatDesc gu[2] = {{nullptr, L.w[XP_T_GATE], L.s[XP_T_GATE], c.ffn},
                                 {nullptr, L.w[XP_T_UP], L.s[XP_T_UP], c.ffn}};
        XB(gemm(gu, 2, H, "batch gate/up", 0, nullptr, nullptr, true));
        const MvMatDesc dm{dn, L.w[XP_T_DOWN], L.s[XP_T_DOWN], H};
        XB(gemm(&dm, 1, c.ffn, "batch down", 0, nullptr, nullptr, false, true));
        const float* next = l + 1 < c.n_layers ? w.layer[l + 1].norm[0] : w.final_norm;
        XB(prep(1, x, dn, nullptr, L.norm[3], next, H));
    }
    if (!prefill) {
        const MvMatDesc lm{logits, w.lm_w, w.lm_s, c.vocab};
        XB(gemm(&lm, 1, H, "batch lm_head"));
        XB(launch_topk4(cval, cidx, logits, c.vocab, kHarvestParts, st, B));
        XB(launch_select_rows(oval, oidx, cval, cidx, kHarvest, kCand, B, st));
        XB(launch_badvance(d_pos, B, st));
    }
#undef XB
    return XP_OK;
}

int Batch::forward(const uint32_t* tokens) {
    for (uint32_t i = 0; i < B; ++i) {
        XP_REQUIRE(pos[i] < S, "xp_batch_forward: sequence %u is at position %u of max_seq %u", i,
                   pos[i], S);
        XP_REQUIRE(tokens[i] < w.cfg.vocab, "xp_batch_forward: token %u of sequence %u >= vocab",
                   tokens[i], i);
    }
    if (!graph) {
        hipGraph_t g = nullptr;
        XP_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        const int rc = record();
        const hipError_t e = hipStreamEndCapture(st, &g);
        if (rc != XP_OK) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess)
            return set_error(XP_E_HIP, "xp_batch_forward: capture failed: %s", hipGetErrorString(e));
        const hipError_t ie = hipGraphInstantiate(&graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (ie != hipSuccess) {
            graph = nullptr;
            return set_error(XP_E_HIP, "xp_batch_forward: instantiate: %s", hipGetErrorString(ie));
        }
    }
    std::memcpy(h_tok, tokens, B * 4);
    XP_HIP(hipMemcpyAsync(d_tok, h_tok, B * 4, hipMemcpyHostToDevice, st));
    XP_HIP(hipEventRecord(ev[0], st));
    XP_HIP(hipGraphLaunch(graph, st));
    XP_HIP(hipEventRecord(ev[1], st));
    if (!prefill) {
        XP_HIP(hipMemcpyAsync(h_val, oval, size_t(B) * kCand * 4, hipMemcpyDeviceToHost, st));
        XP_HIP(hipMemcpyAsync(h_idx, oidx, size_t(B) * kCand * 4, hipMemcpyDeviceToHost, st));
    }
    XP_HIP(hipStreamSynchronize(st));
    (void)hipEventElapsedTime(&last_ms, ev[0], ev[1]);
    for (uint32_t i = 0; i < B; ++i) ++pos[i];
    logits_valid = true;
    return XP_OK;
}

// Releases a batch's resources (the object itself is freed by its owner).
void release(Batch* b) {
    if (!b) return;
    if (b->st) (void)hipStreamSynchronize(b->st);
    if (b->graph) (void)hipGraphExecDestroy(b->graph);
    for (auto& e : b->ev)
        if (e) (void)hipEventDestroy(e);
    if (b->arena) (void)hipFree(b->arena);
    if (b->h_tok) (void)hipHostFree(b->h_tok);
    if (b->h_val) (void)hipHostFree(b->h_val);
    if (b->h_idx) (void)hipHostFree(b->h_idx);
    if (b->st) (void)hipStreamDestroy(b->st);
}

}  // namespace
}  // namespace xp

using namespace xp;

struct xp_batch {
    Batch b;
};

namespace {

// A batch of n_seq rows over the session's weights. prefill: the rows are
// positions of one sequence on the session's own KV cache (no caches of its
// own, no lm_head or sampling).
int make_batch(const xp_session* weights, uint32_t n_seq, uint32_t max_seq, bool prefill,
               xp_batch** out) {
    XP_REQUIRE(weights && out, "null pointer");
    *out = nullptr;
    XP_REQUIRE(n_seq >= 1 && n_seq <= kBatchMax, "n_seq=%u must be in [1, %u]", n_seq, kBatchMax);
    xp_batch* h = new (std::nothrow) xp_batch;
    if (!h) return set_error(XP_E_NOMEM, "xp_batch_create: out of host memory");
    Batch& b = h->b;
    int rc = session_weights(weights, &b.w);
    if (rc != XP_OK) {
        delete h;
        return rc;
    }
    const xp_config& c = b.w.cfg;
    auto fail = [&](int code, const char* msg) {
        release(&h->b);
        delete h;
        return set_error(code, "xp_batch_create: %s", msg);
    };
    if (c.scale_fmt != XP_SCALE_F16_QUAD && c.scale_fmt != XP_SCALE_BF16_QUAD) {
        delete h;
        return set_error(XP_E_ARG, "xp_batch_create: the batched GEMM takes fp16 or bf16 quad scales");
    }
    if (c.sample_mode == 1 && (c.top_k == 0 || c.top_k > kCand)) {
        delete h;
        return set_error(XP_E_ARG, "xp_batch_create: top_k=%u must be in [1, %u]", c.top_k, kCand);
    }
    if (max_seq == 0 || max_seq > 8192) {
        delete h;
        return set_error(XP_E_ARG, "xp_batch_create: max_seq=%u must be in [1, 8192]", max_seq);
    }
    if (c.vocab < kCand) {
        delete h;
        return set_error(XP_E_ARG, "xp_batch_create: vocab %u < %u candidates", c.vocab, kCand);
    }
    b.B = n_seq;
    b.S = max_seq;
    b.prefill = prefill;
    b.pos.assign(n_seq, 0);
    b.steps.assign(n_seq, 0);
    const uint32_t B = n_seq, H = c.hidden, qd = c.n_heads * c.head_dim,
                   kvd = c.n_kv_heads * c.head_dim, F = c.ffn;
    const uint32_t kmax = std::max(H, qd);   // widest k staged into a (the down operand goes to a2)
    size_t part_cap = 0;
    uint32_t tick = 1;
    auto gemm_need = [&](uint32_t cols, uint32_t K) {
        part_cap = std::max(part_cap, bmm_partial_floats(cols, K / kBlkB, b.w.n_cu));
        tick = std::max(tick, cols / kGrpB);
    };
    gemm_need(qd + 2 * kvd, H);
    gemm_need(H, qd);
    gemm_need(2 * F, H);
    gemm_need(H, F);
    gemm_need(c.vocab, H);
    b.part_cap = part_cap;
    b.tickets_cap = tick;
    b.attn_part_seq = attn_partial_floats(c.n_kv_heads, c.n_heads, c.head_dim);
    const size_t kvseq = size_t(max_seq) * kvd;                 // fp16 elements per (layer, K/V, seq)
    std::vector<size_t> sz = {
        prefill ? 0 : size_t(c.n_layers) * 2 * B * kvseq * 2,   // KV caches
        size_t(B) * H * 4, size_t(B) * qd * 4, size_t(B) * kvd * 4, size_t(B) * kvd * 4,
        size_t(B) * qd * 4, size_t(B) * kvd * 4, size_t(B) * qd * 4, size_t(B) * H * 4,
        size_t(F / kBlkB) * 2 * 64 * 16,                         // staged down operand
        size_t(F / kBlkB) * 16 * 4,                              // its block sums
        size_t(B) * H * 4, size_t(B) * c.vocab * 4,
        size_t(kmax / kBlkB) * 2 * 64 * 16,                      // staged operand
        size_t(kmax / kBlkB) * 16 * 4,                           // block sums
        std::max<size_t>(part_cap, 1) * 4, size_t(tick) * 4,
        size_t(B) * b.attn_part_seq * 4 + 4, size_t(B) * c.n_kv_heads * kAttnTicketsPerHead * 4,
        size_t(B) * kHarvest * 4, size_t(B) * kHarvest * 4,
        size_t(B) * kCand * 4, size_t(B) * kCand * 4, size_t(B) * 4, size_t(B) * 4};
    size_t total = 0;
    for (size_t z : sz) total += al(z);
    if (hipStreamCreateWithFlags(&b.st, hipStreamNonBlocking) != hipSuccess)
        return fail(XP_E_HIP, "hipStreamCreate failed");
    if (hipMalloc(&b.arena, total) != hipSuccess) return fail(XP_E_NOMEM, "device memory");
    if (hipMemset(b.arena, 0, total) != hipSuccess) return fail(XP_E_HIP, "clearing device memory");
    char* p = b.arena;
    size_t si = 0;
    auto nxt = [&]() { char* r = p; p += al(sz[si++]); return r; };
    uint16_t* kv = reinterpret_cast<uint16_t*>(nxt());
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        b.kc[l] = prefill ? b.w.layer[l].kc : kv + (size_t(l) * 2 + 0) * B * kvseq;
        b.vc[l] = prefill ? b.w.layer[l].vc : kv + (size_t(l) * 2 + 1) * B * kvseq;
    }
    b.x = reinterpret_cast<float*>(nxt());
    b.q_raw = reinterpret_cast<float*>(nxt());
    b.k_raw = reinterpret_cast<float*>(nxt());
    b.v = reinterpret_cast<float*>(nxt());
    b.q = reinterpret_cast<float*>(nxt());
    b.k = reinterpret_cast<float*>(nxt());
    b.att = reinterpret_cast<float*>(nxt());
    b.o = reinterpret_cast<float*>(nxt());
    b.a2 = nxt();
    b.asum2 = reinterpret_cast<float*>(nxt());
    b.dn = reinterpret_cast<float*>(nxt());
    b.logits = reinterpret_cast<float*>(nxt());
    b.a = nxt();
    b.asum = reinterpret_cast<float*>(nxt());
    b.part = reinterpret_cast<float*>(nxt());
    b.tickets = reinterpret_cast<uint32_t*>(nxt());
    b.attn_part = reinterpret_cast<float*>(nxt());
    b.attn_tickets = reinterpret_cast<uint32_t*>(nxt());
    b.cval = reinterpret_cast<float*>(nxt());
    b.cidx = reinterpret_cast<uint32_t*>(nxt());
    b.oval = reinterpret_cast<float*>(nxt());
    b.oidx = reinterpret_cast<uint32_t*>(nxt());
    b.d_tok = reinterpret_cast<uint32_t*>(nxt());
    b.d_pos = reinterpret_cast<uint32_t*>(nxt());
    if (hipHostMalloc(reinterpret_cast<void**>(&b.h_tok), B * 4) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&b.h_val), size_t(B) * kCand * 4) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&b.h_idx), size_t(B) * kCand * 4) != hipSuccess)
        return fail(XP_E_NOMEM, "pinned host memory");
    if (hipEventCreate(&b.ev[0]) != hipSuccess || hipEventCreate(&b.ev[1]) != hipSuccess)
        return fail(XP_E_HIP, "hipEventCreate failed");
    *out = h;
    return XP_OK;
}

}  // namespace

namespace xp {

struct PrefillBatch {
    xp_batch* b = nullptr;
};

PrefillBatch* prefill_batch_create(const xp_session* s) {
    xp_batch* b = nullptr;
    SessionWeights w;
    if (session_weights(s, &w) != XP_OK) return nullptr;
    if (make_batch(s, kBatchMax, w.cfg.max_seq, true, &b) != XP_OK) return nullptr;
    PrefillBatch* p = new (std::nothrow) PrefillBatch;
    if (!p) {
        release(&b->b);
        delete b;
        set_error(XP_E_NOMEM, "prefill: out of host memory");
        return nullptr;
    }
    p->b = b;
    return p;
}

int prefill_batch_run(PrefillBatch* p, const uint32_t* ids, uint32_t n, uint32_t pos0) {
    Batch& b = p->b->b;
    uint32_t pos[kBatchMax], tok[kBatchMax];
    for (uint32_t c0 = 0; c0 < n; c0 += kBatchMax) {
        const uint32_t m = std::min(kBatchMax, n - c0);
        // rows past the prompt repeat its last token at its position: they
        // write the same K/V row with the same values
        for (uint32_t r = 0; r < kBatchMax; ++r) {
            const uint32_t i = c0 + std::min(r, m - 1);
            pos[r] = pos0 + i;
            tok[r] = ids[i];
        }
        XP_HIP(hipMemcpyAsync(b.d_pos, pos, sizeof pos, hipMemcpyHostToDevice, b.st));
        b.pos.assign(pos, pos + kBatchMax);
        int rc = b.forward(tok);
        if (rc != XP_OK) return rc;
    }
    return XP_OK;
}

void prefill_batch_destroy(PrefillBatch* p) {
    if (!p) return;
    if (p->b) {
        release(&p->b->b);
        delete p->b;
    }
    delete p;
}

}  // namespace xp

extern "C" {

int xp_batch_create(const xp_session* weights, uint32_t n_seq, uint32_t max_seq, xp_batch** out) {
    return make_batch(weights, n_seq, max_seq, false, out);
}

int xp_batch_destroy(xp_batch* h) {
    if (h) {
        release(&h->b);
        delete h;
    }
    return XP_OK;
}

int xp_batch_kv_upload(xp_batch* h, uint32_t seq, int layer, int which, uint32_t start,
                       uint32_t count, const uint16_t* src) {
    XP_REQUIRE(h && src, "null pointer");
    Batch& b = h->b;
    const xp_config& c = b.w.cfg;
    XP_REQUIRE(seq < b.B, "seq %u >= n_seq %u", seq, b.B);
    XP_REQUIRE(layer >= 0 && uint32_t(layer) < c.n_layers, "layer %d out of range", layer);
    XP_REQUIRE(which == 0 || which == 1, "which must be 0 (K) or 1 (V)");
    XP_REQUIRE(uint64_t(start) + count <= b.S, "rows [%u, %u) exceed max_seq %u", start, start + count,
               b.S);
    const size_t kvd = size_t(c.n_kv_heads) * c.head_dim;
    uint16_t* dst = (which ? b.vc[layer] : b.kc[layer]) + (size_t(seq) * b.S + start) * kvd;
    XP_HIP(hipMemcpy(dst, src, size_t(count) * kvd * 2, hipMemcpyHostToDevice));
    return XP_OK;
}

int xp_batch_kv_download(xp_batch* h, uint32_t seq, int layer, int which, uint32_t start,
                         uint32_t count, uint16_t* dst) {
    XP_REQUIRE(h && dst, "null pointer");
    Batch& b = h->b;
    const xp_config& c = b.w.cfg;
    XP_REQUIRE(seq < b.B, "seq %u >= n_seq %u", seq, b.B);
    XP_REQUIRE(layer >= 0 && uint32_t(layer) < c.n_layers, "layer %d out of range", layer);
    XP_REQUIRE(which == 0 || which == 1, "which must be 0 (K) or 1 (V)");
    XP_REQUIRE(uint64_t(start) + count <= b.S, "rows exceed max_seq %u", b.S);
    const size_t kvd = size_t(c.n_kv_heads) * c.head_dim;
    const uint16_t* src = (which ? b.vc[layer] : b.kc[layer]) + (size_t(seq) * b.S + start) * kvd;
    XP_HIP(hipStreamSynchronize(b.st));
    XP_HIP(hipMemcpy(dst, src, size_t(count) * kvd * 2, hipMemcpyDeviceToHost));
    return XP_OK;
}

int xp_batch_set_positions(xp_batch* h, const uint32_t* pos) {
    XP_REQUIRE(h && pos, "null pointer");
    Batch& b = h->b;
    for (uint32_t i = 0; i < b.B; ++i)
        XP_REQUIRE(pos[i] < b.S, "position %u of sequence %u >= max_seq %u", pos[i], i, b.S);
    XP_HIP(hipStreamSynchronize(b.st));
    XP_HIP(hipMemcpy(b.d_pos, pos, b.B * 4, hipMemcpyHostToDevice));
    b.pos.assign(pos, pos + b.B);
    b.logits_valid = false;
    return XP_OK;
}

int xp_batch_positions(xp_batch* h, uint32_t* pos) {
    XP_REQUIRE(h && pos, "null pointer");
    std::copy(h->b.pos.begin(), h->b.pos.end(), pos);
    return XP_OK;
}

int xp_batch_forward(xp_batch* h, const uint32_t* tokens) {
    XP_REQUIRE(h && tokens, "null pointer");
    return h->b.forward(tokens);
}

int xp_batch_decode_step(xp_batch* h, uint32_t* tokens_out) {
    XP_REQUIRE(h && tokens_out, "null pointer");
    Batch& b = h->b;
    XP_REQUIRE(b.logits_valid, "xp_batch_decode_step: no logits yet (run xp_batch_forward first)");
    const xp_config& c = b.w.cfg;
    std::vector<float> val(kCand);
    std::vector<uint32_t> idx(kCand);
    for (uint32_t i = 0; i < b.B; ++i) {
        const float* cv = b.h_val + size_t(i) * kCand;
        const uint32_t* ci = b.h_idx + size_t(i) * kCand;
        if (c.sample_mode == 0) {
            tokens_out[i] = ci[0];    // the maximum, lowest index on ties
            continue;
        }
        uint32_t n = 0;
        for (uint32_t j = 0; j < kCand; ++j)
            if (ci[j] != 0xFFFFFFFFu) { val[n] = cv[j]; idx[n] = ci[j]; ++n; }
        const double u = philox_uniform(c.seed, c.seq_id + i, b.steps[i]++);
        tokens_out[i] = draw(val.data(), idx.data(), n, c.temperature, c.top_k, c.top_p, u);
    }
    return b.forward(tokens_out);
}

int xp_batch_last_logits(xp_batch* h, uint32_t seq, float* out, uint32_t n) {
    XP_REQUIRE(h && out, "null pointer");
    Batch& b = h->b;
    XP_REQUIRE(b.logits_valid, "no logits yet");
    XP_REQUIRE(seq < b.B && n <= b.w.cfg.vocab, "seq %u / n %u out of range", seq, n);
    XP_HIP(hipStreamSynchronize(b.st));
    XP_HIP(hipMemcpy(out, b.logits + size_t(seq) * b.w.cfg.vocab, size_t(n) * 4, hipMemcpyDeviceToHost));
    return XP_OK;
}

int xp_batch_last_candidates(xp_batch* h, uint32_t seq, float* val, uint32_t* idx, uint32_t n) {
    XP_REQUIRE(h && val && idx, "null pointer");
    Batch& b = h->b;
    XP_REQUIRE(b.logits_valid, "no logits yet");
    XP_REQUIRE(seq < b.B && n <= kCand, "seq %u / n %u out of range", seq, n);
    std::copy(b.h_val + size_t(seq) * kCand, b.h_val + size_t(seq) * kCand + n, val);
    std::copy(b.h_idx + size_t(seq) * kCand, b.h_idx + size_t(seq) * kCand + n, idx);
    return XP_OK;
}

int xp_batch_last_ms(xp_batch* h, float* ms) {
    XP_REQUIRE(h && ms, "null pointer");
    *ms = h->b.last_ms;
    return XP_OK;
}

}  // extern "C"
