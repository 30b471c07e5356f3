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
#include <string>
#include <vector>

namespace xp {
namespace {

constexpr uint32_t kBatchMax = 16;
constexpr uint32_t kBlkB = 32;           // quantisation block along k
constexpr uint32_t kGrpB = 64;           // KM4 column group
constexpr uint32_t kCand = 64;           // candidates per sequence (top-k <= 64)
constexpr uint32_t kHistCap = 256;       // steps a chained decode records between host reads
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
    float* cval;
    uint32_t *cidx, *d_pos;
    // Pinned, coherent host memory the device reads and writes in place
    // (mapped, not cached on the device): the step's tokens, read by the
    // embedding gather, and the 64 candidates of each sequence, written by
    // the select, so a step needs no copy either way; m_* are their device
    // addresses.
    uint32_t* h_tok = nullptr;           // [B]
    float* h_val = nullptr;              // [B][64]
    uint32_t* h_idx = nullptr;
    uint32_t* m_tok = nullptr;
    float* m_val = nullptr;
    uint32_t* m_idx = nullptr;
    // any layer's attention in exchange mode (whose error words the host
    // reads after each step)
    bool any_xchg = false;
    hipGraphExec_t graph = nullptr;
    // Chained decode (xp_batch_decode_steps): the step's graph with the
    // draw on the device appended, reading its tokens from d_tok and writing
    // the candidates to d_val / d_idx, the drawn tokens to d_tok and d_hist
    // ([kHistCap][B], slot = Philox step % kHistCap); d_steps the sequences'
    // Philox step counters.
    hipGraphExec_t graph_fd = nullptr;
    float* d_val = nullptr;
    uint32_t *d_idx = nullptr, *d_tok = nullptr, *d_steps = nullptr, *d_hist = nullptr;
    hipEvent_t ev[2] = {nullptr, nullptr};
    std::vector<uint32_t> pos, steps;
    bool logits_valid = false;
    float last_ms = 0.0f;
    // Prefill mode: the rows are consecutive positions of one sequence and
    // share the session's KV cache; the step ends after the last layer.
    bool prefill = false;
    // Decode through the persistent step kernel (batch_step.hip) instead of
    // a graph of per-op kernels: its per-layer stage buffers and argument
    // table (step_arena), the operand the first layer reads (a0 / asum0) and
    // the one the lm_head reads (af / asumf), counters and status word.
    bool step_kernel = false;
    char* step_arena = nullptr;
    BstepArgs bs{};
    void* a0 = nullptr;
    float* asum0 = nullptr;
    void* af = nullptr;
    float* asumf = nullptr;
    uint32_t* h_status = nullptr;        // pinned
    uint32_t* h_attn = nullptr;          // pinned: the attention tickets after a graph step
    uint32_t attn_spin = 1u << 18;       // exchange-mode attention's spin limit (graph path)
    unsigned long long* d_trace = nullptr;   // the step kernel's stage timeline, when on
    size_t trace_n = 0;

    int record(bool chain = false);
    int setup_step(int exec);
    int forward(const uint32_t* tokens);
    int decode_steps(uint32_t n, uint32_t* tokens_out);
    int capture(bool chain, hipGraphExec_t* out);
    int attn_error_check();
    void host_draw(uint32_t* tokens_out);
};

int Batch::record(bool chain) {
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
    // the embedding rows of the step's tokens and layer 0's operand in one
    // staging launch
    auto embed_prep = [&](void* a_, float* asum_) {
        BprepArgs p0{0, x, nullptr, nullptr, nullptr, w.layer[0].norm[0], a_, asum_, H, eps};
        p0.tok = chain ? d_tok : m_tok;
        p0.ewq = w.lm_w;
        p0.esc = w.lm_s;
        p0.etable = w.embed;
        p0.vocab = c.vocab;
        p0.efmt = fmt;
        p0.escale = w.embed_scale;
        return launch_bprep(p0, B, st);
    };
    if (step_kernel) {
        // layer 0's operand, then every layer in one launch, then the lm_head
        // on the operand its last stage staged
        XB(embed_prep(a0, asum0));
        XB(launch_bstep(bs, fmt, uint32_t(w.n_cu), st));
        BmmArgs g{};
        g.a = af;
        g.asum = asumf;
        g.lda = H;
        g.mats[0] = {logits, w.lm_w, w.lm_s, c.vocab};
        g.n_mats = 1;
        g.nblk = H / kBlkB;
        g.rows = B;
        g.part = part;
        g.part_cap = part_cap;
        g.tickets = tickets;
        g.tickets_cap = tickets_cap;
        XB(launch_bmm(g, fmt, w.n_cu, st, "batch lm_head"));
        XB(launch_topk4(cval, cidx, logits, c.vocab, kHarvestParts, st, B));
        XB(launch_select_rows(m_val, m_idx, cval, cidx, kHarvest, kCand, B, st, d_pos));
        return XP_OK;
    }
    XB(embed_prep(a, asum));
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
        aa.spin_limit = attn_spin;
        aa.batch = B;
        aa.bq = qd;
        aa.bcache = prefill ? 0 : size_t(S) * kvd;
        aa.bpart = attn_part_seq;
        const uint32_t max_span = glob || c.sliding_window == 0 ? S : std::min(c.sliding_window, S);
        {
            AttnArgs pa = aa;
            int pu = 0;
            RopeFreq pf{};
            if (plan_attention(pa, max_span, true, &pu, &pf) == XP_OK && pa.xchg) any_xchg = true;
        }
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
        XB(launch_select_rows(chain ? d_val : m_val, chain ? d_idx : m_idx, cval, cidx, kHarvest, kCand, B, st,
                              d_pos));
        if (chain)
            XB(launch_draw_rows(d_val, d_idx, kCand, B, c.sample_mode, c.temperature, c.top_k, c.top_p, c.seed,
                                c.seq_id, d_steps, d_tok, d_hist, kHistCap, st));
    }
#undef XB
    return XP_OK;
}

// Decode through the persistent step kernel: per-layer stage buffers (each
// stage's output its own per layer, so no consumer reads a line it read
// before in the same launch), the layer table built with the per-op path's
// own plans (plan_bmm, plan_attention: results are bit-identical), and the
// residency checks the token kernel uses (one 512-thread workgroup per CU).
// Opt-in (XP_EXEC_TOKEN): measured slower than the graph of per-op kernels
// (1.93 vs 1.41 ms a config-5 step), whose kernel boundaries cost less than
// the kernel's flag hand-offs.
int Batch::setup_step(int exec) {
    const xp_config& c = w.cfg;
    const uint32_t H = c.hidden, qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim, F = c.ffn;
    const int fmt = c.scale_fmt;
    const float eps = c.rms_eps;
    step_kernel = false;
    auto refuse = [&](const char* why) -> int {
        if (exec == XP_EXEC_TOKEN)
            return set_error(XP_E_ARG, "xp_batch_create: the step kernel %s", why);
        clear_error();
        return XP_OK;
    };
    (void)exec;
    if (c.n_kv_heads == 0 || c.n_heads != 4u * c.n_kv_heads || c.head_dim != 256u)
        return refuse("takes 4 query heads of 256 dims per kv head");
    if (w.n_cu <= 0 || H / 8u > 512u) return refuse("needs a known CU count and hidden <= 4096");
    int per_cu = 0;
    if (bstep_occupancy(fmt, &per_cu) != XP_OK || per_cu < 1) return refuse("does not fit a CU");
    // per-layer stage buffers: layer l at step_arena + l * per (layer
    // n_layers holds only the lm_head's operand)
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off += al(bytes); return o; };
    const size_t o_q = take(size_t(B) * qd * 4), o_k = take(size_t(B) * kvd * 4),
                 o_v = take(size_t(B) * kvd * 4), o_att = take(size_t(B) * qd * 4),
                 o_o = take(size_t(B) * H * 4), o_xa = take(size_t(B) * H * 4), o_xb = take(size_t(B) * H * 4),
                 o_a0 = take(size_t(H / kBlkB) * 2 * 64 * 16), o_s0 = take(size_t(H / kBlkB) * 16 * 4),
                 o_a1 = take(size_t(H / kBlkB) * 2 * 64 * 16), o_s1 = take(size_t(H / kBlkB) * 16 * 4),
                 o_a2 = take(size_t(F / kBlkB) * 2 * 64 * 16), o_s2 = take(size_t(F / kBlkB) * 16 * 4),
                 o_dn = take(size_t(B) * H * 4);
    const size_t per = off;
    const size_t tab = al(size_t(per) * (c.n_layers + 1));
    const size_t rope_off = tab + al(sizeof(BstepLayer) * c.n_layers);
    const size_t cnt_off = rope_off + al(sizeof(RopeFreq) * 2);
    const size_t total = cnt_off + al((size_t(c.n_layers) * kBsStages * kBsMaxTiles + 3) * 4);
    if (hipMalloc(&step_arena, total) != hipSuccess) return set_error(XP_E_NOMEM, "xp_batch_create: device memory");
    XP_HIP(hipMemset(step_arena, 0, total));
    auto at = [&](uint32_t l, size_t o) { return step_arena + size_t(l) * per + o; };
    std::vector<BstepLayer> T(c.n_layers);
    RopeFreq rf[2]{};
    uint32_t ncb_q = 0, ncb_o = 0, ncb_d = 0, ns_d = 0, n_gu = 0;
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const SessionWeights::Layer& L = w.layer[l];
        BstepLayer& t = T[l];
        t = BstepLayer{};
        float* q_raw = reinterpret_cast<float*>(at(l, o_q));
        float* k_raw = reinterpret_cast<float*>(at(l, o_k));
        float* v_raw = reinterpret_cast<float*>(at(l, o_v));
        float* att_l = reinterpret_cast<float*>(at(l, o_att));
        float* o_l = reinterpret_cast<float*>(at(l, o_o));
        float* xa = reinterpret_cast<float*>(at(l, o_xa));
        float* xb = reinterpret_cast<float*>(at(l, o_xb));
        float* dn_l = reinterpret_cast<float*>(at(l, o_dn));
        auto gemm = [&](BmmArgs& g, uint32_t nblk, const char* who, uint32_t* ncb, bool want_quarter) {
            g.nblk = nblk;
            g.rows = B;
            g.part = part;
            g.part_cap = part_cap;
            g.tickets = tickets;
            g.tickets_cap = tickets_cap;
            uint32_t nb = 0;
            bool quarter = false;
            if (int rc = plan_bmm(g, fmt, w.n_cu, who, &nb, &quarter); rc != XP_OK) return rc;
            if (quarter != want_quarter) return set_error(XP_E_ARG, "%s: plan shape", who);
            if (*ncb != 0 && *ncb != nb) return set_error(XP_E_ARG, "%s: plan differs between layers", who);
            *ncb = nb;
            return XP_OK;
        };
        t.qkv.a = at(l, o_a0);
        t.qkv.asum = reinterpret_cast<float*>(at(l, o_s0));
        t.qkv.lda = H;
        t.qkv.mats[0] = {q_raw, L.w[XP_T_Q], L.s[XP_T_Q], qd};
        t.qkv.mats[1] = {k_raw, L.w[XP_T_K], L.s[XP_T_K], kvd};
        t.qkv.mats[2] = {v_raw, L.w[XP_T_V], L.s[XP_T_V], kvd};
        t.qkv.n_mats = 3;
        t.o.amode = 2;
        t.o.xa = att_l;
        t.o.lda = qd;
        t.o.mats[0] = {o_l, L.w[XP_T_O], L.s[XP_T_O], H};
        t.o.n_mats = 1;
        t.gu.a = at(l, o_a1);
        t.gu.asum = reinterpret_cast<float*>(at(l, o_s1));
        t.gu.lda = H;
        t.gu.geglu = 1;
        t.gu.a_out = at(l, o_a2);
        t.gu.asum_out = reinterpret_cast<float*>(at(l, o_s2));
        t.gu.mats[0] = {nullptr, L.w[XP_T_GATE], L.s[XP_T_GATE], F};
        t.gu.mats[1] = {nullptr, L.w[XP_T_UP], L.s[XP_T_UP], F};
        t.gu.n_mats = 2;
        t.dn.a = at(l, o_a2);
        t.dn.asum = reinterpret_cast<float*>(at(l, o_s2));
        t.dn.lda = F;
        t.dn.mats[0] = {dn_l, L.w[XP_T_DOWN], L.s[XP_T_DOWN], H};
        t.dn.n_mats = 1;
        if (gemm(t.qkv, H / kBlkB, "batch step q|k|v", &ncb_q, true) != XP_OK || t.qkv.nsplit != 1 ||
            gemm(t.o, qd / kBlkB, "batch step o_proj", &ncb_o, true) != XP_OK || t.o.nsplit != 1 ||
            gemm(t.gu, H / kBlkB, "batch step gate/up", &n_gu, false) != XP_OK ||
            gemm(t.dn, F / kBlkB, "batch step down", &ncb_d, true) != XP_OK)
            return refuse("needs the per-op path's GEMM plans (quarter column blocks, one k split)");
        if (ns_d != 0 && ns_d != t.dn.nsplit) return refuse("needs one down plan for every layer");
        ns_d = t.dn.nsplit;
        // attention as the per-op path plans it (record())
        const bool glob = L.global;
        AttnArgs& aa = t.att;
        aa.out = att_l;
        aa.q = q_raw;
        aa.kc = kc[l];
        aa.vc = vc[l];
        aa.q_raw = q_raw;
        aa.k_raw = k_raw;
        aa.v_raw = v_raw;
        aa.qw = L.norm[4];
        aa.kw = L.norm[5];
        aa.eps = eps;
        aa.theta = glob ? c.rope_theta_global : c.rope_theta_local;
        aa.bkv = kvd;
        aa.n_heads = c.n_heads;
        aa.kv_heads = c.n_kv_heads;
        aa.head_dim = c.head_dim;
        aa.pos_dev = d_pos;
        aa.window = glob ? 0u : c.sliding_window;
        aa.scale = w.attn_scale;
        aa.part = attn_part;
        aa.tickets = attn_tickets;
        // an exchange-mode wait that times out sets the step's status word (bs.status)
        aa.status = reinterpret_cast<uint32_t*>(step_arena + cnt_off) +
                    size_t(c.n_layers) * kBsStages * kBsMaxTiles + 1;
        aa.batch = B;
        aa.bq = qd;
        aa.bcache = size_t(S) * kvd;
        aa.bpart = attn_part_seq;
        const uint32_t max_span = glob || c.sliding_window == 0 ? S : std::min(c.sliding_window, S);
        int U = 0;
        RopeFreq f{};
        if (plan_attention(aa, max_span, true, &U, &f) != XP_OK || aa.group != 4u)
            return refuse("needs the per-op path's attention plan");
        t.att_u = uint32_t(U);
        t.att_rope = glob ? 1u : 0u;
        rf[t.att_rope] = f;
        t.n_att = aa.nsplit * aa.kv_heads * B;
        if (t.n_att > kBsMaxTiles) return refuse("takes at most 512 attention tiles");
        const float* next = l + 1 < c.n_layers ? w.layer[l + 1].norm[0] : w.final_norm;
        t.prep1 = BprepArgs{1, l == 0 ? x : reinterpret_cast<float*>(at(l - 1, o_xb)), o_l, nullptr,
                            L.norm[1], L.norm[2], at(l, o_a1), reinterpret_cast<float*>(at(l, o_s1)), H, eps};
        t.prep1.x_out = xa;
        t.prep2 = BprepArgs{1, xa, dn_l, nullptr, L.norm[3], next, at(l + 1, o_a0),
                            reinterpret_cast<float*>(at(l + 1, o_s0)), H, eps};
        t.prep2.x_out = xb;
    }
    a0 = at(0, o_a0);
    asum0 = reinterpret_cast<float*>(at(0, o_s0));
    af = at(c.n_layers, o_a0);
    asumf = reinterpret_cast<float*>(at(c.n_layers, o_s0));
    XP_HIP(hipMemcpy(step_arena + tab, T.data(), sizeof(BstepLayer) * c.n_layers, hipMemcpyHostToDevice));
    XP_HIP(hipMemcpy(step_arena + rope_off, rf, sizeof(rf), hipMemcpyHostToDevice));
    bs = BstepArgs{};
    bs.layers = reinterpret_cast<const BstepLayer*>(step_arena + tab);
    bs.rope = reinterpret_cast<const RopeFreq*>(step_arena + rope_off);
    bs.n_layers = c.n_layers;
    bs.batch = B;
    bs.ncb_qkv = ncb_q;
    bs.ncb_o = ncb_o;
    bs.ncb_dn = ncb_d;
    bs.ns_dn = ns_d;
    bs.n_gu = n_gu;
    bs.flags = reinterpret_cast<uint32_t*>(step_arena + cnt_off);
    bs.epoch = bs.flags + size_t(c.n_layers) * kBsStages * kBsMaxTiles;
    bs.status = bs.epoch + 1;   // the attention tiles' AttnArgs::status points here too
    bs.exit_cnt = bs.epoch + 2;
    if (ncb_q > kBsMaxTiles || ncb_o > kBsMaxTiles || n_gu > kBsMaxTiles || ncb_d * ns_d > kBsMaxTiles ||
        B > kBsMaxTiles)
        return refuse("takes at most 512 tiles a stage");
    bs.spin_limit = 1u << 20;
    if (hipHostMalloc(reinterpret_cast<void**>(&h_status), 16) != hipSuccess)
        return set_error(XP_E_NOMEM, "xp_batch_create: pinned host memory");
    h_status[0] = 0u;
    // the grid of one workgroup per CU resident at once (the token kernel's probe)
    std::vector<uint32_t> probe(uint32_t(w.n_cu));
    if (probe_token_grid(uint32_t(w.n_cu), st, probe.data()) != XP_OK) return refuse("probe launch failed");
    for (uint32_t v : probe)
        if (!((v >> 8) & 1u)) return refuse("grid is not resident at once (another kernel holds CUs)");
    step_kernel = true;
    return XP_OK;
}

// Captures the step (with the device draw appended when `chain`) into *out.
int Batch::capture(bool chain, hipGraphExec_t* out) {
    hipGraph_t g = nullptr;
    XP_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    const int rc = record(chain);
    const hipError_t e = hipStreamEndCapture(st, &g);
    if (rc != XP_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess)
        return set_error(XP_E_HIP, "xp_batch_forward: capture failed: %s", hipGetErrorString(e));
    const hipError_t ie = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ie != hipSuccess) {
        *out = nullptr;
        return set_error(XP_E_HIP, "xp_batch_forward: instantiate: %s", hipGetErrorString(ie));
    }
    return XP_OK;
}

// After a synchronised graph step: the exchange-mode attention's error words
// (copied to h_attn by the step).
int Batch::attn_error_check() {
    if (!any_xchg) return XP_OK;
    const size_t attn_words = size_t(B) * w.cfg.n_kv_heads * kAttnTicketsPerHead;
    uint32_t err = 0;
    for (size_t i = kAttnXErrWord; i < attn_words; i += kAttnTicketsPerHead) err |= h_attn[i];
    if (!err) return XP_OK;
    // an exchange-mode attention wait timed out (its splits were not
    // resident at once): outputs hold NaN; the records and tickets start
    // over from zero, positions stay where they were
    XP_HIP(hipMemcpy(d_pos, pos.data(), B * 4, hipMemcpyHostToDevice));
    XP_HIP(hipMemset(attn_part, 0, (size_t(B) * attn_part_seq + 1) * 4));
    XP_HIP(hipMemset(attn_tickets, 0, attn_words * 4));
    XP_HIP(hipDeviceSynchronize());
    logits_valid = false;
    return set_error(XP_E_DEVICE, "xp_batch_forward: a decode attention wait ran past its "
                     "limit (another kernel held CUs of this GPU); the step's results and "
                     "the KV rows it appended are not valid, positions are unchanged");
}

// The sample-first draw from the last step's candidates (decode.cpp:1830-1850),
// on the host: greedy takes each sequence's best candidate; sampling draws
// with Philox(seed, seq_id + i, step) and advances the step.
void Batch::host_draw(uint32_t* tokens_out) {
    const xp_config& c = w.cfg;
    std::vector<float> val(kCand);
    std::vector<uint32_t> idx(kCand);
    for (uint32_t i = 0; i < B; ++i) {
        const float* cv = h_val + size_t(i) * kCand;
        const uint32_t* ci = h_idx + size_t(i) * kCand;
        if (c.sample_mode == 0) {
            tokens_out[i] = ci[0];    // the maximum, lowest index on ties
            continue;
        }
        uint32_t n = 0;
        for (uint32_t j = 0; j < kCand; ++j)
            if (ci[j] != 0xFFFFFFFFu) { val[n] = cv[j]; idx[n] = ci[j]; ++n; }
        const double u = philox_uniform(c.seed, c.seq_id + i, steps[i]++);
        tokens_out[i] = draw(val.data(), idx.data(), n, c.temperature, c.top_k, c.top_p, u);
    }
}

// n sample-first steps (n x xp_batch_decode_step, the same tokens): the
// first draw on the host from the last candidates, the next n - 1 on the
// device at the end of each step's graph, the steps replayed back to back
// with no host round trip between them; the last step is the plain graph,
// so its candidates are in the pinned arrays as after xp_batch_forward.
int Batch::decode_steps(uint32_t n, uint32_t* out) {
    XP_REQUIRE(logits_valid, "xp_batch_decode_steps: no logits yet (run xp_batch_forward first)");
    if (n == 0) return XP_OK;
    if (step_kernel || prefill || n == 1) {
        for (uint32_t k = 0; k < n; ++k) {
            host_draw(out + size_t(k) * B);
            if (const int rc = forward(out + size_t(k) * B); rc != XP_OK) return rc;
        }
        return XP_OK;
    }
    for (uint32_t i = 0; i < B; ++i)
        XP_REQUIRE(pos[i] + n <= S, "xp_batch_decode_steps: sequence %u at position %u + %u steps > max_seq %u",
                   i, pos[i], n, S);
    if (!graph)
        if (const int rc = capture(false, &graph); rc != XP_OK) return rc;
    if (!graph_fd)
        if (const int rc = capture(true, &graph_fd); rc != XP_OK) return rc;
    float total_ms = 0.0f;
    for (uint32_t k0 = 0; k0 < n;) {
        const uint32_t m = std::min(n - k0, kHistCap + 1u);   // steps in this chain
        uint32_t* o = out + size_t(k0) * B;
        host_draw(o);
        for (uint32_t i = 0; i < B; ++i)
            XP_REQUIRE(o[i] < w.cfg.vocab, "xp_batch_decode_steps: token %u of sequence %u >= vocab", o[i], i);
        const std::vector<uint32_t> s0 = steps;   // the device draws' first counters
        XP_HIP(hipMemcpyAsync(d_tok, o, B * 4, hipMemcpyHostToDevice, st));
        XP_HIP(hipMemcpyAsync(d_steps, s0.data(), B * 4, hipMemcpyHostToDevice, st));
        XP_HIP(hipEventRecord(ev[0], st));
        for (uint32_t k = 1; k < m; ++k) XP_HIP(hipGraphLaunch(graph_fd, st));
        // the last step reads its tokens from the pinned array
        XP_HIP(hipMemcpyAsync(h_tok, d_tok, B * 4, hipMemcpyDeviceToHost, st));
        XP_HIP(hipGraphLaunch(graph, st));
        XP_HIP(hipEventRecord(ev[1], st));
        const size_t attn_words = size_t(B) * w.cfg.n_kv_heads * kAttnTicketsPerHead;
        if (any_xchg) XP_HIP(hipMemcpyAsync(h_attn, attn_tickets, attn_words * 4, hipMemcpyDeviceToHost, st));
        std::vector<uint32_t> hist(size_t(kHistCap) * B);
        XP_HIP(hipMemcpyAsync(hist.data(), d_hist, hist.size() * 4, hipMemcpyDeviceToHost, st));
        XP_HIP(hipStreamSynchronize(st));
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, ev[0], ev[1]);
        total_ms += ms;
        if (const int rc = attn_error_check(); rc != XP_OK) return rc;
        for (uint32_t k = 1; k < m; ++k)
            for (uint32_t i = 0; i < B; ++i)
                o[size_t(k) * B + i] = hist[size_t((s0[i] + k - 1u) % kHistCap) * B + i];
        if (w.cfg.sample_mode != 0)
            for (uint32_t i = 0; i < B; ++i) steps[i] += m - 1u;
        for (uint32_t i = 0; i < B; ++i) pos[i] += m;
        k0 += m;
    }
    last_ms = total_ms / float(n);
    logits_valid = true;
    return XP_OK;
}

int Batch::forward(const uint32_t* tokens) {
    for (uint32_t i = 0; i < B; ++i) {
        XP_REQUIRE(pos[i] < S, "xp_batch_forward: sequence %u is at position %u of max_seq %u", i,
                   pos[i], S);
        XP_REQUIRE(tokens[i] < w.cfg.vocab, "xp_batch_forward: token %u of sequence %u >= vocab",
                   tokens[i], i);
    }
    if (!graph)
        if (const int rc = capture(false, &graph); rc != XP_OK) return rc;
    // the tokens go to the device as the graph's embedding gather reads them
    // from this pinned array; the previous step has finished (synchronised
    // below), so nothing reads it while it changes
    std::memcpy(h_tok, tokens, B * 4);
    XP_HIP(hipEventRecord(ev[0], st));
    XP_HIP(hipGraphLaunch(graph, st));
    XP_HIP(hipEventRecord(ev[1], st));
    const size_t attn_words = size_t(B) * w.cfg.n_kv_heads * kAttnTicketsPerHead;
    if (step_kernel) XP_HIP(hipMemcpyAsync(h_status, bs.status, 4, hipMemcpyDeviceToHost, st));
    else if (any_xchg) XP_HIP(hipMemcpyAsync(h_attn, attn_tickets, attn_words * 4, hipMemcpyDeviceToHost, st));
    XP_HIP(hipStreamSynchronize(st));
    (void)hipEventElapsedTime(&last_ms, ev[0], ev[1]);
    if (!step_kernel)
        if (const int rc = attn_error_check(); rc != XP_OK) return rc;
    if (step_kernel && h_status[0] != 0u) {
        // a wait ran past its limit (the grid was not resident at once): the
        // step's results are not valid
        // positions stay where they were (the graph advanced the device's).
        // With waits given up, tiles of different layers ran at once and
        // may have left the arrival tickets they share counted wrong: the
        // combine state (attention records, tickets and epochs, the GEMMs'
        // tickets and partials) starts over as at creation.
        const uint32_t code = h_status[0];
        h_status[0] = 0u;
        XP_HIP(hipMemcpyAsync(bs.status, h_status, 4, hipMemcpyHostToDevice, st));
        XP_HIP(hipStreamSynchronize(st));
        XP_HIP(hipMemcpy(d_pos, pos.data(), B * 4, hipMemcpyHostToDevice));
        XP_HIP(hipMemset(attn_part, 0, (size_t(B) * attn_part_seq + 1) * 4));
        XP_HIP(hipMemset(attn_tickets, 0, size_t(B) * w.cfg.n_kv_heads * kAttnTicketsPerHead * 4));
        XP_HIP(hipMemset(tickets, 0, size_t(tickets_cap) * 4));
        XP_HIP(hipMemset(part, 0, std::max<size_t>(part_cap, 1) * 4));
        XP_HIP(hipDeviceSynchronize());
        logits_valid = false;
        return set_error(XP_E_DEVICE, "xp_batch_forward: the step kernel's wait ran past its limit "
                         "(status %u; another kernel held CUs of this GPU); the step's results and "
                         "the KV rows it appended are not valid, positions are unchanged", code);
    }
    for (uint32_t i = 0; i < B; ++i) ++pos[i];
    logits_valid = true;
    return XP_OK;
}

// Releases a batch's resources (the object itself is freed by its owner).
void release(Batch* b) {
    if (!b) return;
    if (b->st) (void)hipStreamSynchronize(b->st);
    if (b->graph) (void)hipGraphExecDestroy(b->graph);
    if (b->graph_fd) (void)hipGraphExecDestroy(b->graph_fd);
    for (auto& e : b->ev)
        if (e) (void)hipEventDestroy(e);
    if (b->arena) (void)hipFree(b->arena);
    if (b->step_arena) (void)hipFree(b->step_arena);
    if (b->d_trace) (void)hipFree(b->d_trace);
    if (b->h_status) (void)hipHostFree(b->h_status);
    if (b->h_attn) (void)hipHostFree(b->h_attn);
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
               xp_batch** out, int exec = XP_EXEC_AUTO) {
    XP_REQUIRE(weights && out, "null pointer");
    XP_REQUIRE(exec == XP_EXEC_AUTO || exec == XP_EXEC_GRAPH || exec == XP_EXEC_TOKEN,
               "exec_mode=%d: XP_EXEC_AUTO, XP_EXEC_GRAPH or XP_EXEC_TOKEN", exec);
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
        size_t(B) * kHarvest * 4, size_t(B) * kHarvest * 4, size_t(B) * 4,
        size_t(B) * kCand * 4, size_t(B) * kCand * 4, size_t(B) * 4, size_t(B) * 4,
        size_t(kHistCap) * B * 4};
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
    b.d_pos = reinterpret_cast<uint32_t*>(nxt());
    b.d_val = reinterpret_cast<float*>(nxt());
    b.d_idx = reinterpret_cast<uint32_t*>(nxt());
    b.d_tok = reinterpret_cast<uint32_t*>(nxt());
    b.d_steps = reinterpret_cast<uint32_t*>(nxt());
    b.d_hist = reinterpret_cast<uint32_t*>(nxt());
    const unsigned mapped = hipHostMallocMapped | hipHostMallocCoherent;
    if (hipHostMalloc(reinterpret_cast<void**>(&b.h_tok), B * 4, mapped) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&b.h_val), size_t(B) * kCand * 4, mapped) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&b.h_idx), size_t(B) * kCand * 4, mapped) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&b.h_attn),
                      size_t(B) * c.n_kv_heads * kAttnTicketsPerHead * 4) != hipSuccess)
        return fail(XP_E_NOMEM, "pinned host memory");
    if (hipHostGetDevicePointer(reinterpret_cast<void**>(&b.m_tok), b.h_tok, 0) != hipSuccess ||
        hipHostGetDevicePointer(reinterpret_cast<void**>(&b.m_val), b.h_val, 0) != hipSuccess ||
        hipHostGetDevicePointer(reinterpret_cast<void**>(&b.m_idx), b.h_idx, 0) != hipSuccess)
        return fail(XP_E_HIP, "device addresses of the pinned token / candidate arrays");
    // no candidates before the first step
    std::fill(b.h_val, b.h_val + size_t(B) * kCand, -INFINITY);
    std::fill(b.h_idx, b.h_idx + size_t(B) * kCand, 0xFFFFFFFFu);
    if (hipEventCreate(&b.ev[0]) != hipSuccess || hipEventCreate(&b.ev[1]) != hipSuccess)
        return fail(XP_E_HIP, "hipEventCreate failed");
    if (!prefill && exec == XP_EXEC_TOKEN) {
        if (int rc2 = b.setup_step(exec); rc2 != XP_OK) {
            const std::string msg = xp_last_error();
            release(&h->b);
            delete h;
            return set_error(rc2, "%s", msg.c_str());
        }
    }
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

int xp_batch_create2(const xp_session* weights, uint32_t n_seq, uint32_t max_seq, int32_t exec_mode,
                     xp_batch** out) {
    return make_batch(weights, n_seq, max_seq, false, out, exec_mode);
}

int xp_batch_step_trace(xp_batch* h, int enable) {
    XP_REQUIRE(h, "null pointer");
    Batch& b = h->b;
    XP_REQUIRE(b.step_kernel, "xp_batch_step_trace: the batch does not run the step kernel");
    XP_HIP(hipStreamSynchronize(b.st));
    if (b.graph) {
        (void)hipGraphExecDestroy(b.graph);   // recaptured with the new arguments
        b.graph = nullptr;
    }
    if (!enable) {
        b.bs.trace = nullptr;
        return XP_OK;
    }
    const size_t n = (size_t(b.w.cfg.n_layers) * kBsStages * 2 + 1) * size_t(b.w.n_cu);
    if (!b.d_trace) {
        if (hipMalloc(reinterpret_cast<void**>(&b.d_trace), n * 8) != hipSuccess)
            return set_error(XP_E_NOMEM, "xp_batch_step_trace: device memory");
        b.trace_n = n;
    }
    XP_HIP(hipMemset(b.d_trace, 0, n * 8));
    b.bs.trace = b.d_trace;
    return XP_OK;
}

int xp_batch_set_spin_limit(xp_batch* h, uint32_t rounds) {
    XP_REQUIRE(h, "null pointer");
    Batch& b = h->b;
    XP_REQUIRE(rounds <= (1u << 24), "xp_batch_set_spin_limit: rounds=%u > 2^24", rounds);
    XP_HIP(hipStreamSynchronize(b.st));
    if (b.graph) {
        (void)hipGraphExecDestroy(b.graph);   // recaptured with the new limit
        b.graph = nullptr;
    }
    b.bs.spin_limit = rounds;   // the step kernel's waits
    b.attn_spin = rounds;       // the graph's exchange-mode attention
    return XP_OK;
}

int xp_batch_step_trace_read(xp_batch* h, unsigned long long* out, size_t n, size_t* n_out) {
    XP_REQUIRE(h && n_out, "null pointer");
    Batch& b = h->b;
    *n_out = b.trace_n;
    if (!out) return XP_OK;
    XP_REQUIRE(b.d_trace && n >= b.trace_n, "xp_batch_step_trace_read: no trace, or n < %zu", b.trace_n);
    XP_HIP(hipStreamSynchronize(b.st));
    XP_HIP(hipMemcpy(out, b.d_trace, b.trace_n * 8, hipMemcpyDeviceToHost));
    return XP_OK;
}

int xp_batch_exec_mode(const xp_batch* h, int32_t* mode) {
    XP_REQUIRE(h && mode, "null pointer");
    *mode = h->b.step_kernel ? XP_EXEC_TOKEN : XP_EXEC_GRAPH;
    return XP_OK;
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
    b.host_draw(tokens_out);
    return b.forward(tokens_out);
}

int xp_batch_decode_steps(xp_batch* h, uint32_t n, uint32_t* tokens_out) {
    XP_REQUIRE(h && tokens_out, "null pointer");
    return h->b.decode_steps(n, tokens_out);
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
