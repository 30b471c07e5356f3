// One decode token as ONE persistent cooperative kernel on gfx950.
//
// The reference records 838 dispatches per token into one Vulkan submit
// (examples/llm/decode.cpp:1634-1780, agent-docs/llm-inference.md:88-103).
// On MI355X a kernel boundary costs ~1.7 us even inside a HIP graph, and a
// Gemma-3-1B token is only ~0.56 GB of int4 weights (~70 us at 8 TB/s), so the
// whole token step — embedding, 26 layers, final norm, lm_head and argmax — is
// one launch of one 512-thread workgroup per CU. record_token's order
// (decode.cpp:1668-1752) becomes six dataflow stages per layer:
//
//   QKV -> attention -> softmax combine -> O -> gate/up -> down -> next QKV
//
// Synchronisation is dataflow, not barriers. Every value that crosses
// workgroups lives in an 8-byte slot holding (launch tag, fp32 bits), written
// with one device-coherent store; a consumer re-reads the slots it needs
// until every tag is this launch's (the low-latency protocol of collective
// libraries). A stage therefore waits one store-to-load latency for exactly
// the data it uses, and nothing waits for workgroups it does not depend on.
// Each workgroup walks the stages in order and skips those it has no work
// in; every stage's inputs are produced by earlier stages, so the walk is a
// topological order and the grid cannot deadlock. Waits are bounded: past the
// spin limit a workgroup records an error in state[2] and continues, so the
// grid always drains; the host reports the error.
//
// Other design points:
//  * The residual stream is carried between stages through the xa / xb slots
//    (x entering the layer, x after the attention block); the consumers
//    recompute the 1152-wide RMSNorms themselves.
//  * Each stage's weights (the attention stage's KV rows) are loaded into
//    registers before the workgroup waits for the stage's inputs: weights
//    do not depend on activations, so HBM streaming overlaps the waiting.
//  * Matvec tiles are (64-column group, <= 16 quads of k); the 8 waves of the
//    workgroup take quads w and w + 8 (the int4 x fixed-point dot of
//    matvec.hip) and reduce through LDS in a fixed order. The down projection
//    (k = 6912) is split into chunks of 16 quads whose partial sums the next
//    layer adds in chunk order, so every result is deterministic.
//  * Attention: one workgroup per 32 keys of [kv_start, pos]; each computes
//    QK-norm + RoPE of q and k itself, scores, a chunk softmax (max, sum of
//    exp) and the unnormalised weighted values; 4 workgroups per query head
//    then combine the chunks (softmax_rows_finish's rescale,
//    llm_transformer.cl:385-405). The current key/value come from registers
//    (fp16-rounded, as the cache holds them) and are appended to the cache by
//    the chunk that contains them, for later tokens.
//  * RoPE cos/sin for the token's position are computed once per workgroup
//    at kernel start (256 accurate sincosf, one per thread).
#include "xp_device.hpp"
#include "xp_launch.hpp"

namespace xp {

namespace {

constexpr int      kTkThreads   = kTokThreads;
constexpr int      kTkWaves     = kTkThreads / kWave;    // 8
constexpr int      kTkHD        = 256;                   // head_dim
constexpr int      kTkMaxQH     = 8;                     // query heads (one kv head)
constexpr int      kTkC         = 32;                    // keys per attention workgroup
constexpr int      kTkMaxHidden = 2048;
constexpr int      kTkMaxBlk    = 64;                    // staged 32-blocks of x (2048 k)
constexpr int      kTkMaxGrid   = 1024;
constexpr uint32_t kSpinLimit   = 1u << 24;
constexpr int      kTkBig       = 17408;                 // floats of stage scratch
constexpr int      kTkFetch     = 12;                    // slot loads in flight per thread
constexpr int      kTkMaxLayers = 64;

typedef unsigned long long ll_t;

struct TkSmem {
    // The layer table, copied from device memory at kernel start. Read from
    // global memory at each use, its pointers cost a dependent load that
    // also waits for every outstanding weight prefetch (in-order vmcnt).
    TokLayer lt[kTkMaxLayers];
    float    xs[kTkMaxHidden];               // residual stream
    float    xn[kTkMaxHidden];               // input of the current stage
    float    xt[kTkMaxHidden];               // second input (o / down sums)
    QxBlock  qx[kTkMaxBlk];                  // fixed-point staging of xn
    float    sx[kTkMaxBlk];
    float    red[kTkWaves][kWave];           // per-wave tile partials
    float    rs[kTkWaves];                   // block reductions
    float    rt[kTkWaves];
    float    cs[2][kTkHD / 2];               // RoPE cos / sin at this position,
    float    sn[2][kTkHD / 2];               // [0] local theta, [1] global theta
    float    qh[kTkMaxQH][kTkHD];            // normed, rotated q
    float    kn[kTkHD];                      // current key / value (fp16-rounded)
    float    vn[kTkHD];
    float    sc[kTkMaxQH][kTkC];             // scores, then exp
    // Stage scratch: the down chunks of the residual add, the value partials
    // of attention's 4 key groups ([4][n_heads][256]), the combine's inputs.
    float    big[kTkBig];
    float    mh[kTkMaxQH];
    float    lh[kTkMaxQH];
    float    fm[2 * kTkMaxGrid];             // combine: per-chunk factors; argmax slots
    float    amv[kTkWaves];
    uint32_t ami[kTkWaves];
};

// ---- exchange slots -------------------------------------------------------------
__device__ __forceinline__ void ll_put(ll_t* p, float v, uint32_t tag) {
    st_dev64(p, (ll_t(tag) << 32) | ll_t(__float_as_uint(v)));
}
__device__ __forceinline__ float ll_val(ll_t v) { return __uint_as_float(uint32_t(v)); }

// dst[i] = value of slot at(i) for i < n, waiting until every slot carries
// this launch's tag. Up to kTkFetch loads per thread are issued together and
// only the stale ones are re-issued, so data that is ready costs one
// round trip. Bounded: past the spin limit the workgroup records an error in
// state[2] and keeps whatever the slots hold. All threads; ends with a
// workgroup barrier.
template <class At>
__device__ __forceinline__ void ll_fetch_at(float* dst, uint32_t n, uint32_t tag, uint32_t* state, At at) {
    for (uint32_t base = 0; base < n; base += kTkFetch * kTkThreads) {
        ll_t v[kTkFetch];
#pragma unroll
        for (int r = 0; r < kTkFetch; ++r) {
            const uint32_t i = base + r * kTkThreads + threadIdx.x;
            v[r] = i < n ? ld_dev64(at(i)) : (ll_t(tag) << 32);
        }
        uint32_t spins = 0;
        for (;;) {
            bool ok = true;
#pragma unroll
            for (int r = 0; r < kTkFetch; ++r) ok &= uint32_t(v[r] >> 32) == tag;
            if (ok) break;
            ++spins;
            if ((spins & 255u) == 0) {
                if (ld_dev(state + 2) != 0u) break;
                if (spins > kSpinLimit) {
                    st_dev(state + 2, 1u);
                    break;
                }
            }
#pragma unroll
            for (int r = 0; r < kTkFetch; ++r) {
                const uint32_t i = base + r * kTkThreads + threadIdx.x;
                if (uint32_t(v[r] >> 32) != tag) v[r] = ld_dev64(at(i));
            }
        }
#pragma unroll
        for (int r = 0; r < kTkFetch; ++r) {
            const uint32_t i = base + r * kTkThreads + threadIdx.x;
            if (i < n) dst[i] = ll_val(v[r]);
        }
    }
    __syncthreads();
}

// Contiguous slots p[0 .. n).
__device__ __forceinline__ void ll_fetch(float* dst, const ll_t* p, uint32_t n, uint32_t tag,
                                         uint32_t* state) {
    ll_fetch_at(dst, n, tag, state, [=](uint32_t i) { return p + i; });
}
// Two contiguous ranges at once: dst[0 .. n0) from p0, dst[n0 .. n0 + n1) from p1.
__device__ __forceinline__ void ll_fetch2(float* dst, const ll_t* p0, uint32_t n0, const ll_t* p1,
                                          uint32_t n1, uint32_t tag, uint32_t* state) {
    ll_fetch_at(dst, n0 + n1, tag, state,
                [=](uint32_t i) { return i < n0 ? p0 + i : p1 + (i - n0); });
}

__device__ __forceinline__ void tk_trace(const TokArgs& a, uint32_t event) {
    if (a.trace && threadIdx.x == 0)
        a.trace[size_t(event) * gridDim.x + blockIdx.x] = __builtin_amdgcn_s_memrealtime();
}

// ---- small block-wide helpers (512 threads) -------------------------------------
__device__ __forceinline__ float tk_block_sum(float v, float* rs) {
    v = wave_sum(v);
    const uint32_t w = threadIdx.x / kWave;
    if (threadIdx.x % kWave == 0) rs[w] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < kTkWaves; ++i) t += rs[i];
    __syncthreads();
    return t;
}
__device__ __forceinline__ float tk_block_max(float v, float* rs) {
    v = wave_max(v);
    const uint32_t w = threadIdx.x / kWave;
    if (threadIdx.x % kWave == 0) rs[w] = v;
    __syncthreads();
    float t = -INFINITY;
#pragma unroll
    for (int i = 0; i < kTkWaves; ++i) t = fmaxf(t, rs[i]);
    __syncthreads();
    return t;
}

// A norm weight vector held in registers: element tid + r * 512 in v[r].
// Loaded before a stage waits for its inputs, like the matvec weights.
struct TkNormW {
    float v[kTkMaxHidden / kTkThreads];
};
__device__ __forceinline__ void tk_load_norm(TkNormW& w, const float* p, uint32_t n) {
#pragma unroll
    for (int r = 0; r < kTkMaxHidden / kTkThreads; ++r) {
        const uint32_t i = threadIdx.x + r * kTkThreads;
        w.v[r] = i < n ? ldgf(p + i) : 0.0f;
    }
}

// Gemma RMSNorm of S.xs into S.xn: xn = xs * rsqrt(mean(xs^2) + eps) * (1 + w).
__device__ __forceinline__ void tk_norm(const TokArgs& a, TkSmem& S, const TkNormW& w) {
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < a.hidden; i += kTkThreads) ss += S.xs[i] * S.xs[i];
    ss = tk_block_sum(ss, S.rs);
    const float scale = 1.0f / sqrtf(ss / float(a.hidden) + a.eps);
#pragma unroll
    for (int r = 0; r < kTkMaxHidden / kTkThreads; ++r) {
        const uint32_t i = threadIdx.x + r * kTkThreads;
        if (i < a.hidden) S.xn[i] = S.xs[i] * scale * (1.0f + w.v[r]);
    }
    __syncthreads();
}

// S.xs = S.xn + S.xt * rsqrt(mean(xt^2) + eps) * (1 + w_post): the residual
// add of a normed sublayer output (decode.cpp:1739-1751).
__device__ __forceinline__ void tk_residual(const TokArgs& a, TkSmem& S, const TkNormW& w_post) {
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < a.hidden; i += kTkThreads) ss += S.xt[i] * S.xt[i];
    ss = tk_block_sum(ss, S.rs);
    const float scale = 1.0f / sqrtf(ss / float(a.hidden) + a.eps);
#pragma unroll
    for (int r = 0; r < kTkMaxHidden / kTkThreads; ++r) {
        const uint32_t i = threadIdx.x + r * kTkThreads;
        if (i < a.hidden) S.xs[i] = S.xn[i] + S.xt[i] * scale * (1.0f + w_post.v[r]);
    }
    __syncthreads();
}

__device__ __forceinline__ float tk_scale(u32x2 raw, int i, int fmt) {
    const uint32_t w = (i < 2) ? raw.x : raw.y;
    if (fmt == XP_SCALE_F16_QUAD) return f16_bits_to_f32((i & 1) ? (w >> 16) : w);
    return (i & 1) ? bf16hi(w) : bf16lo(w);
}

// ---- matvec tiles ------------------------------------------------------------------
struct TkTile {
    const u32x4* wq;
    const void*  sc;
    uint32_t     nblk;     // k / 32 of the matrix
    uint32_t     cols;
    uint32_t     g;        // column group
    uint32_t     qa, qb;   // quads [qa, qb) of k
    uint32_t     m;        // matrix index (XP_T_Q .. XP_T_DOWN)
};

// Wave w's blocks of a tile: 4 qa + w + 8 r for r < 8 (tiles hold at most
// 16 quads = 64 blocks), each with its scale quad (the block's scale is
// component b % 4). Spreading blocks rather than quads over the 8 waves keeps
// a 9-quad tile at 5 blocks per wave.
struct TkQuads {
    u32x4 w[8];
    u32x2 s[8];
};

__device__ __forceinline__ void tk_prefetch(const TkTile& t, TkQuads& p, uint32_t wave,
                                            uint32_t lane) {
    const uint32_t b1 = 4u * t.qb;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const uint32_t b = 4u * t.qa + wave + 8u * r;
        if (b < b1) {
            p.w[r] = ldg_stream4(t.wq + (size_t(t.g) * t.nblk + b) * kGrp + lane);
            p.s[r] = ldg_stream2(reinterpret_cast<const u32x2*>(t.sc) + size_t(b / 4u) * t.cols +
                                 t.g * kGrp + lane);
        }
    }
}

// Stages S.xn[0 .. nb*32) (k relative to the tile's first block) as
// fixed-point planes S.qx[0 .. nb).
__device__ __forceinline__ void tk_stage(TkSmem& S, uint32_t nb) {
    for (uint32_t i = threadIdx.x; i < nb * 4; i += kTkThreads) {
        const float4* p = reinterpret_cast<const float4*>(S.xn) + 2 * i;
        stage_x8(S.qx, S.sx, i, p[0], p[1]);
    }
    __syncthreads();
}

// The wave's share of tile t (staged planes start at quad qbase), reduced over
// the 8 waves in order; the result is valid in wave 0 (lane = column).
__device__ __forceinline__ float tk_tile(const TkTile& t, const TkQuads& p, TkSmem& S, uint32_t qbase, int fmt,
                         uint32_t wave, uint32_t lane) {
    float acc = 0.0f;
    const uint32_t b1 = 4u * t.qb;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const uint32_t b = 4u * t.qa + wave + 8u * r;
        if (b < b1) {
            const uint32_t lb = b - 4u * qbase;
            const float f = tk_scale(p.s[r], int(b % 4u), fmt) * S.sx[lb];
            acc = fmaf(f, float(block_dot(p.w[r], S.qx[lb])), acc);
        }
    }
    S.red[wave][lane] = acc;
    __syncthreads();
    float r = 0.0f;
    if (wave == 0) {
#pragma unroll
        for (int w = 0; w < kTkWaves; ++w) r += S.red[w][lane];
    }
    __syncthreads();
    return r;
}

// QKV: tile = one 64-column group of q|k|v over all of k.
__device__ __forceinline__ TkTile tk_qkv_tile(const TokArgs& a, const TokLayer& L, uint32_t t) {
    const uint32_t qg = a.n_heads * kTkHD / kGrp, kg = kTkHD / kGrp;
    const uint32_t m = t < qg ? 0u : (t < qg + kg ? 1u : 2u);
    const uint32_t g = m == 0 ? t : (m == 1 ? t - qg : t - qg - kg);
    return TkTile{static_cast<const u32x4*>(L.w[m]), L.s[m], a.hidden / kBlk,
                  m == 0 ? a.n_heads * kTkHD : uint32_t(kTkHD), g, 0u, a.hidden / 128u, m};
}
__device__ __forceinline__ TkTile tk_o_tile(const TokArgs& a, const TokLayer& L, uint32_t t) {
    return TkTile{static_cast<const u32x4*>(L.w[3]), L.s[3], a.n_heads * kTkHD / kBlk,
                  a.hidden, t, 0u, a.n_heads * kTkHD / 128u, 3u};
}
__device__ __forceinline__ TkTile tk_gu_tile(const TokArgs& a, const TokLayer& L, uint32_t t) {
    const uint32_t ng = a.ffn / kGrp;
    const uint32_t m = t < ng ? 4u : 5u;
    return TkTile{static_cast<const u32x4*>(L.w[m]), L.s[m], a.hidden / kBlk, a.ffn,
                  t < ng ? t : t - ng, 0u, a.hidden / 128u, m};
}
// Down: tile = (column group, chunk of 16 quads = 2048 k).
__device__ __forceinline__ uint32_t tk_down_chunks(uint32_t ffn) { return (ffn / 128u + 15u) / 16u; }
__device__ __forceinline__ TkTile tk_down_tile(const TokArgs& a, const TokLayer& L, uint32_t t) {
    const uint32_t nq = a.ffn / 128u, nch = tk_down_chunks(a.ffn);
    const uint32_t g = t / nch, c = t % nch;
    return TkTile{static_cast<const u32x4*>(L.w[6]), L.s[6], a.ffn / kBlk, a.hidden, g, 16u * c,
                  min(16u * c + 16u, nq), 6u};
}

// ---- embedding (decode.cpp:1618-1627, as a gather from the tied int4 table) ----
__device__ __forceinline__ void tk_embed(const TokArgs& a, TkSmem& S, uint32_t tok) {
    const uint32_t nblk = a.hidden / kBlk;
    const u32x4* wq = static_cast<const u32x4*>(a.lm_w);
    for (uint32_t k = threadIdx.x; k < a.hidden; k += kTkThreads) {
        const uint32_t b = k / kBlk, t = k % kBlk;
        const u32x4 w = ldg4(wq + (size_t(tok / kGrp) * nblk + b) * kGrp + (tok % kGrp));
        const uint32_t word = (t < 8) ? w.x : (t < 16) ? w.y : (t < 24) ? w.z : w.w;
        const float q = float(int((word >> ((t & 7u) * 4u)) & 15u) - 8);
        const uint16_t h =
            ldg16(static_cast<const uint16_t*>(a.lm_s) + (size_t(b / 4) * a.vocab + tok) * 4 + (b % 4));
        const float s = a.fmt == XP_SCALE_F16_QUAD ? f16_bits_to_f32(h)
                                                   : __uint_as_float(uint32_t(h) << 16);
        S.xs[k] = (q * s) * a.embed_scale;
    }
    __syncthreads();
}

// S.xs = x entering layer l + 1 from layer l's slots: xb + post_ffw_norm(sum
// of the down chunks, in chunk order). The chunks are contiguous slots
// (dnp follows xb's layer block at a fixed offset); fetched with xb in one
// batch.
__device__ __forceinline__ void tk_after_ffn(const TokArgs& a, TkSmem& S, const TokLL& lay, uint32_t l,
                             const TkNormW& w_post) {
    const ll_t* base = a.ll + size_t(l) * a.ll_layer;
    const uint32_t nch = tk_down_chunks(a.ffn), H = a.hidden;
    // big[0 .. H) = xb, big[H + c H .. ) = chunk c
    ll_fetch2(S.big, base + lay.xb, H, base + lay.dnp, nch * H, a.tag, a.state);
    for (uint32_t i = threadIdx.x; i < H; i += kTkThreads) {
        float t = S.big[H + i];
        for (uint32_t c = 1; c < nch; ++c) t += S.big[H + c * H + i];
        S.xn[i] = S.big[i];
        S.xt[i] = t;
    }
    __syncthreads();
    tk_residual(a, S, w_post);
}

__device__ __forceinline__ float f16_round(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }

}  // namespace

__global__ __launch_bounds__(kTkThreads) void token_kernel(TokArgs a) {
    extern __shared__ __align__(16) unsigned char tk_lds[];
    TkSmem& S = *reinterpret_cast<TkSmem*>(tk_lds);
    const uint32_t tid  = threadIdx.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const uint32_t lane = tid % kWave;
    const uint32_t wg   = blockIdx.x;
    const uint32_t nwg  = gridDim.x;
    const uint32_t tag  = a.tag;
    tk_trace(a, 0);

    const uint32_t pos = a.state[0];
    uint32_t tok = a.state[1];
    if (tok >= a.vocab) tok = 0;                 // the host validates ids
    if (wg == 0 && tid == 0) a.hist[pos] = tok;

    const uint32_t H = a.hidden;
    const uint32_t qd = a.n_heads * kTkHD;
    const uint32_t seq = pos + 1u;
    const TokLL lay = tok_ll_layout(H, a.ffn, a.n_heads, kTkHD, nwg);

    {
        static_assert(sizeof(TokLayer) % 8 == 0, "layer table copies in 8-byte words");
        const unsigned long long* src = reinterpret_cast<const unsigned long long*>(a.layers);
        unsigned long long* dst = reinterpret_cast<unsigned long long*>(S.lt);
        const uint32_t nw = a.n_layers * uint32_t(sizeof(TokLayer) / 8);
        for (uint32_t i = tid; i < nw; i += kTkThreads) dst[i] = src[i];
    }
    // RoPE rotation for this position, both thetas (llm_transformer.cl:158-179).
    if (tid < kTkHD) {
        const uint32_t th = tid / (kTkHD / 2), d = tid % (kTkHD / 2);
        const float ang = float(pos) * (th ? a.freq_global : a.freq_local)[d];
        float sv, cv;
        sincosf(ang, &sv, &cv);
        S.cs[th][d] = cv;
        S.sn[th][d] = sv;
    }
    __syncthreads();

    const uint32_t n_qkv  = (qd + 2u * kTkHD) / kGrp;
    const uint32_t n_comb = a.n_heads * 4u;
    const uint32_t n_o    = H / kGrp;
    const uint32_t n_gu   = 2u * a.ffn / kGrp;
    const uint32_t nch    = tk_down_chunks(a.ffn);
    const uint32_t n_dn   = (H / kGrp) * nch;
    // Workgroup -> tile maps: tile t of a stage runs on workgroup (off + t) %
    // grid, so this workgroup's first tile is (wg - off) mod grid.
    const uint32_t off_comb = n_qkv % nwg, off_gu = (n_qkv + n_comb) % nwg;
    const uint32_t t_qkv = wg, t_comb = (wg + nwg - off_comb) % nwg, t_o = wg;
    const uint32_t t_gu = (wg + nwg - off_gu) % nwg, t_dn = wg;
    TkQuads pre;

    for (uint32_t l = 0; l < a.n_layers; ++l) {
        const TokLayer& L = S.lt[l];
        ll_t* LL = a.ll + size_t(l) * a.ll_layer;
        // ================= QKV =================
        for (uint32_t t = t_qkv; t < n_qkv; t += nwg) {
            const TkTile tt = tk_qkv_tile(a, L, t);
            tk_prefetch(tt, pre, wave, lane);
            TkNormW w_in, w_post;
            tk_load_norm(w_in, L.norm[0], H);
            if (l > 0) tk_load_norm(w_post, S.lt[l - 1u].norm[3], H);
            if (l == 0) tk_embed(a, S, tok);
            else tk_after_ffn(a, S, lay, l - 1u, w_post);
            if (t == 0) {
                for (uint32_t i = tid; i < H; i += kTkThreads) ll_put(LL + lay.xa + i, S.xs[i], tag);
            }
            tk_norm(a, S, w_in);
            tk_stage(S, H / kBlk);
            const float r = tk_tile(tt, pre, S, 0u, a.fmt, wave, lane);
            if (wave == 0) {
                const uint32_t o = tt.m == 0u ? 0u : (tt.m == 1u ? qd : qd + kTkHD);
                ll_put(LL + lay.qkv + o + tt.g * kGrp + lane, r, tag);
            }
        }
        tk_trace(a, 1u + 6u * l);

        // ================= attention =================
        const bool glob = L.global != 0u;
        const uint32_t kv0 = (glob || a.window == 0u || seq <= a.window) ? 0u : seq - a.window;
        const uint32_t span = seq - kv0;
        const uint32_t n_att = (span + kTkC - 1u) / kTkC;
        const uint32_t s_att = nwg - 1u - wg;
        if (s_att < n_att) {
            const uint32_t j0 = s_att * kTkC;
            // score mapping: key jk = tid / 16, 16 dims at part * 16
            const uint32_t jk = tid / 16u, part = tid % 16u;
            // value mapping: dims 2*dp, 2*dp+1 of keys kgv*8 .. kgv*8+7
            const uint32_t dp = tid % 128u, kgv = tid / 128u;
            u32x4 kr[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
            uint32_t vw[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) vw[i] = 0u;
            if (j0 + jk < span) {
                const u32x4* kp = reinterpret_cast<const u32x4*>(
                    L.kc + size_t(kv0 + j0 + jk) * kTkHD + part * 16u);
                kr[0] = ldg4(kp);
                kr[1] = ldg4(kp + 1);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t jj = j0 + kgv * 8u + i;
                if (jj < span)
                    vw[i] = ldg32(L.vc + size_t(kv0 + jj) * kTkHD + 2u * dp);
            }
            // QK-norm weights of this wave's first head, then q_raw | k_raw | v
            float wqk[4];
            {
                const float* w = wave < a.n_heads ? L.norm[4] : L.norm[5];
#pragma unroll
                for (int c = 0; c < 4; ++c) wqk[c] = wave <= a.n_heads ? ldgf(w + lane + 64 * c) : 0.0f;
            }
            ll_fetch(S.xn, LL + lay.qkv, qd + 2u * kTkHD, tag, a.state);
            const uint32_t th = glob ? 1u : 0u;
            // QK-norm + RoPE, one wave per head (q heads, then the kv head)
            for (uint32_t hh = wave; hh <= a.n_heads; hh += kTkWaves) {
                const bool isq = hh < a.n_heads;
                const float* src = isq ? S.xn + hh * kTkHD : S.xn + qd;
                float wc[4];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    wc[c] = hh == wave ? wqk[c] : ldgf((isq ? L.norm[4] : L.norm[5]) + lane + 64 * c);
                float e[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) e[c] = src[lane + 64 * c];
                float ss = e[0] * e[0] + e[1] * e[1] + e[2] * e[2] + e[3] * e[3];
                ss = wave_sum(ss);
                const float scale = 1.0f / sqrtf(ss / float(kTkHD) + a.eps);
#pragma unroll
                for (int c = 0; c < 4; ++c) e[c] = e[c] * scale * (1.0f + wc[c]);
                // rotate-half pairs (d, d + 128): (e0, e2) at d = lane, (e1, e3) at lane + 64
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const float cv = S.cs[th][lane + 64 * c], sv = S.sn[th][lane + 64 * c];
                    const float lo = e[c], hi = e[c + 2];
                    e[c] = lo * cv - hi * sv;
                    e[c + 2] = lo * sv + hi * cv;
                }
                if (isq) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) S.qh[hh][lane + 64 * c] = e[c];
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) S.kn[lane + 64 * c] = f16_round(e[c]);
                }
            }
            if (tid < kTkHD) S.vn[tid] = f16_round(S.xn[qd + kTkHD + tid]);
            __syncthreads();
            if (s_att == n_att - 1u && tid < kTkHD) {
                stg16(L.kc + size_t(pos) * kTkHD + tid, f32_to_f16_bits(S.kn[tid]));
                stg16(L.vc + size_t(pos) * kTkHD + tid, f32_to_f16_bits(S.vn[tid]));
            }
            // scores
            {
                const uint32_t jj = j0 + jk;
                const bool valid = jj < span;
                const bool cur = kv0 + jj == pos;
                float kf[16];
                const uint32_t kw[8] = {kr[0].x, kr[0].y, kr[0].z, kr[0].w,
                                        kr[1].x, kr[1].y, kr[1].z, kr[1].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    kf[2 * e] = cur ? S.kn[part * 16u + 2 * e] : f16_bits_to_f32(kw[e]);
                    kf[2 * e + 1] = cur ? S.kn[part * 16u + 2 * e + 1] : f16_bits_to_f32(kw[e] >> 16);
                }
                for (uint32_t h = 0; h < a.n_heads; ++h) {
                    const float* qp = &S.qh[h][part * 16u];
                    float d = 0.0f;
#pragma unroll
                    for (int e = 0; e < 16; ++e) d = fmaf(qp[e], kf[e], d);
                    d = row16_sum(d);   // the 16 lanes of key jk are one DPP row
                    if (part == 0) S.sc[h][jk] = valid ? d * a.attn_scale : -INFINITY;
                }
            }
            __syncthreads();
            // chunk softmax, one wave per head
            for (uint32_t h = wave; h < a.n_heads; h += kTkWaves) {
                const float v = lane < uint32_t(kTkC) ? S.sc[h][lane] : -INFINITY;
                const float m = wave_max(v);
                const float e = (lane < uint32_t(kTkC) && v != -INFINITY) ? expf(v - m) : 0.0f;
                const float l2 = wave_sum(e);
                if (lane < uint32_t(kTkC)) S.sc[h][lane] = e;
                if (lane == 0) { S.mh[h] = m; S.lh[h] = l2; }
            }
            __syncthreads();
            // weighted values
            {
                float o0[kTkMaxQH], o1[kTkMaxQH];
#pragma unroll
                for (int h = 0; h < kTkMaxQH; ++h) o0[h] = o1[h] = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t jl = kgv * 8u + i, jj = j0 + jl;
                    if (jj < span) {
                        const bool cur = kv0 + jj == pos;
                        const float v0 = cur ? S.vn[2 * dp] : f16_bits_to_f32(vw[i]);
                        const float v1 = cur ? S.vn[2 * dp + 1] : f16_bits_to_f32(vw[i] >> 16);
#pragma unroll
                        for (int h = 0; h < kTkMaxQH; ++h) {
                            if (uint32_t(h) < a.n_heads) {
                                const float p = S.sc[h][jl];
                                o0[h] = fmaf(p, v0, o0[h]);
                                o1[h] = fmaf(p, v1, o1[h]);
                            }
                        }
                    }
                }
#pragma unroll
                for (int h = 0; h < kTkMaxQH; ++h) {
                    if (uint32_t(h) < a.n_heads) {
                        float* vr = S.big + (kgv * a.n_heads + h) * kTkHD;
                        vr[2 * dp] = o0[h];
                        vr[2 * dp + 1] = o1[h];
                    }
                }
            }
            __syncthreads();
            ll_t* pb = LL + lay.attp + size_t(s_att) * a.n_heads * (2u + kTkHD);
            for (uint32_t i = tid; i < a.n_heads * kTkHD; i += kTkThreads) {
                const uint32_t h = i / kTkHD, d = i % kTkHD;
                const uint32_t hs = a.n_heads * kTkHD;
                const float* vr = S.big + h * kTkHD + d;
                const float o = ((vr[0] + vr[hs]) + vr[2 * hs]) + vr[3 * hs];
                ll_put(pb + h * (2u + kTkHD) + 2u + d, o, tag);
            }
            if (tid < a.n_heads) {
                ll_put(pb + tid * (2u + kTkHD), S.mh[tid], tag);
                ll_put(pb + tid * (2u + kTkHD) + 1u, S.lh[tid], tag);
            }
        }
        tk_trace(a, 2u + 6u * l);

        // ================= combine =================
        for (uint32_t c = t_comb; c < n_comb; c += nwg) {
            const uint32_t h = c / 4u, d0 = (c % 4u) * 64u;
            const size_t rstride = size_t(a.n_heads) * (2u + kTkHD);
            const ll_t* base = LL + lay.attp + size_t(h) * (2u + kTkHD);
            // big[s * 66 + 0 / 1] = (max, sum of exp) of chunk s,
            // big[s * 66 + 2 + d] = its unnormalised output at dim d0 + d.
            ll_fetch_at(S.big, n_att * 66u, tag, a.state, [=](uint32_t i) {
                const uint32_t sidx = i / 66u, e = i % 66u;
                return base + sidx * rstride + (e < 2u ? e : d0 + e);
            });
            float m = -INFINITY;
            for (uint32_t s = tid; s < n_att; s += kTkThreads) m = fmaxf(m, S.big[s * 66u]);
            const float M = tk_block_max(m, S.rs);
            float lsum = 0.0f;
            for (uint32_t s = tid; s < n_att; s += kTkThreads) {
                const float f = expf(S.big[s * 66u] - M);
                S.fm[s] = f;
                lsum += f * S.big[s * 66u + 1u];
            }
            const float Ltot = tk_block_sum(lsum, S.rt);   // also orders the fm writes
            const uint32_t d = tid % 64u, sg = tid / 64u;
            float o = 0.0f;
            for (uint32_t s = sg; s < n_att; s += kTkWaves) o = fmaf(S.big[s * 66u + 2u + d], S.fm[s], o);
            S.red[sg][d] = o;
            __syncthreads();
            if (sg == 0) {
                float r = 0.0f;
#pragma unroll
                for (int w = 0; w < kTkWaves; ++w) r += S.red[w][d];
                ll_put(LL + lay.atto + h * kTkHD + d0 + d, r / Ltot, tag);
            }
            __syncthreads();
        }
        tk_trace(a, 3u + 6u * l);

        // ================= O projection =================
        for (uint32_t t = t_o; t < n_o; t += nwg) {
            const TkTile tt = tk_o_tile(a, L, t);
            tk_prefetch(tt, pre, wave, lane);
            ll_fetch(S.xn, LL + lay.atto, qd, tag, a.state);
            tk_stage(S, qd / kBlk);
            const float r = tk_tile(tt, pre, S, 0u, a.fmt, wave, lane);
            if (wave == 0) ll_put(LL + lay.o + tt.g * kGrp + lane, r, tag);
        }
        tk_trace(a, 4u + 6u * l);

        // ================= gate / up =================
        for (uint32_t t = t_gu; t < n_gu; t += nwg) {
            const TkTile tt = tk_gu_tile(a, L, t);
            tk_prefetch(tt, pre, wave, lane);
            TkNormW w_post, w_in;
            tk_load_norm(w_post, L.norm[1], H);
            tk_load_norm(w_in, L.norm[2], H);
            ll_fetch2(S.big, LL + lay.xa, H, LL + lay.o, H, tag, a.state);
            for (uint32_t i = tid; i < H; i += kTkThreads) {
                S.xn[i] = S.big[i];
                S.xt[i] = S.big[H + i];
            }
            __syncthreads();
            tk_residual(a, S, w_post);
            if (t == 0) {
                for (uint32_t i = tid; i < H; i += kTkThreads) ll_put(LL + lay.xb + i, S.xs[i], tag);
            }
            tk_norm(a, S, w_in);
            tk_stage(S, H / kBlk);
            const float r = tk_tile(tt, pre, S, 0u, a.fmt, wave, lane);
            if (wave == 0) {
                const uint32_t o = tt.m == 4u ? 0u : a.ffn;
                ll_put(LL + lay.gu + o + tt.g * kGrp + lane, r, tag);
            }
        }
        tk_trace(a, 5u + 6u * l);

        // ================= down =================
        for (uint32_t t = t_dn; t < n_dn; t += nwg) {
            const TkTile tt = tk_down_tile(a, L, t);
            tk_prefetch(tt, pre, wave, lane);
            const uint32_t k0 = tt.qa * 128u, nk = (tt.qb - tt.qa) * 128u;
            ll_fetch2(S.big, LL + lay.gu + k0, nk, LL + lay.gu + a.ffn + k0, nk, tag, a.state);
            for (uint32_t i = tid; i < nk; i += kTkThreads)
                S.xn[i] = gelu_tanh(S.big[i]) * S.big[nk + i];
            __syncthreads();
            tk_stage(S, nk / kBlk);
            const float r = tk_tile(tt, pre, S, tt.qa, a.fmt, wave, lane);
            if (wave == 0)
                ll_put(LL + lay.dnp + size_t(t % nch) * H + tt.g * kGrp + lane, r, tag);
        }
        tk_trace(a, 6u + 6u * l);
    }

    if (!a.want_logits) {
        if (wg == 0 && tid == 0) a.state[0] = pos + 1u;
        return;
    }

    // ================= final norm, lm_head, argmax =================
    const uint32_t ng = a.vocab / kGrp;
    const uint32_t gw = wg * kTkWaves + wave, nw = nwg * kTkWaves;
    const uint32_t nqh = H / 128u;
    const u32x4* lmw = static_cast<const u32x4*>(a.lm_w);
    // Quad stream of this wave: groups gw, gw + nw, ...; k/128 quads each.
    const uint32_t my_groups = gw < ng ? (ng - gw + nw - 1u) / nw : 0u;
    const uint32_t nu = my_groups * nqh;
    u32x4 w3[3][4];
    u32x2 s3[3];
    auto load_u = [&](int r, uint32_t u) {
        const uint32_t uc = min(u, nu - 1u);
        const uint32_t g = gw + (uc / nqh) * nw, q = uc % nqh;
        const u32x4* wp = lmw + (size_t(g) * (H / kBlk) + 4u * q) * kGrp + lane;
#pragma unroll
        for (int i = 0; i < 4; ++i) w3[r][i] = ldg_stream4(wp + i * kGrp);
        s3[r] = ldg_stream2(reinterpret_cast<const u32x2*>(a.lm_s) + size_t(q) * a.vocab +
                            g * kGrp + lane);
    };
    if (nu > 0) {
        load_u(0, 0);
        load_u(1, 1);
        load_u(2, 2);
    }
    TkNormW wf_post, wf_in;
    tk_load_norm(wf_post, S.lt[a.n_layers - 1u].norm[3], H);
    tk_load_norm(wf_in, a.final_norm, H);
    tk_after_ffn(a, S, lay, a.n_layers - 1u, wf_post);
    tk_norm(a, S, wf_in);
    tk_stage(S, H / kBlk);
    float bv = -INFINITY;
    uint32_t bi = 0u;
    float acc = 0.0f;
    auto mul_u = [&](int r, uint32_t u) {
        const uint32_t q = u % nqh;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lb = 4u * q + i;
            const float f = tk_scale(s3[r], i, a.fmt) * S.sx[lb];
            acc = fmaf(f, float(block_dot(w3[r][i], S.qx[lb])), acc);
        }
        if (q == nqh - 1u) {
            const uint32_t j = (gw + (u / nqh) * nw) * kGrp + lane;
            a.logits[j] = acc;
            am_better(bv, bi, acc, j);
            acc = 0.0f;
        }
    };
    for (uint32_t u = 0; u < nu; u += 3) {
        mul_u(0, u);
        if (u + 3 < nu) load_u(0, u + 3);
        if (u + 1 < nu) {
            mul_u(1, u + 1);
            if (u + 4 < nu) load_u(1, u + 4);
        }
        if (u + 2 < nu) {
            mul_u(2, u + 2);
            if (u + 5 < nu) load_u(2, u + 5);
        }
    }
    am_wave(bv, bi);
    if (lane == 0) { S.amv[wave] = bv; S.ami[wave] = bi; }
    __syncthreads();
    ll_t* am = a.ll + size_t(a.n_layers) * a.ll_layer;
    if (tid == 0) {
        for (int w = 1; w < kTkWaves; ++w) am_better(bv, bi, S.amv[w], S.ami[w]);
        ll_put(am + 2u * wg, bv, tag);
        ll_put(am + 2u * wg + 1u, __uint_as_float(bi), tag);
    }
    tk_trace(a, 1u + 6u * a.n_layers);
    if (wg != 0) return;
    __syncthreads();
    ll_fetch(S.fm, am, 2u * nwg, tag, a.state);
    bv = -INFINITY;
    bi = 0u;
    for (uint32_t i = tid; i < nwg; i += kTkThreads)
        am_better(bv, bi, S.fm[2 * i], __float_as_uint(S.fm[2 * i + 1]));
    am_wave(bv, bi);
    if (lane == 0) { S.amv[wave] = bv; S.ami[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kTkWaves; ++w) am_better(bv, bi, S.amv[w], S.ami[w]);
        if (a.greedy) a.state[1] = bi;
        a.state[0] = pos + 1u;
        a.state[3] = bi;
        reinterpret_cast<float*>(a.state)[4] = bv;
    }
    tk_trace(a, 2u + 6u * a.n_layers);
}

size_t tok_lds_bytes() {
    // Over half of the 160 KiB a gfx950 CU has, so that each CU holds exactly
    // one workgroup of the grid.
    static_assert(sizeof(TkSmem) <= 160 * 1024, "token kernel LDS exceeds a gfx950 CU");
    const size_t need = (sizeof(TkSmem) + 1023) & ~size_t(1023);
    return need > 96 * 1024 ? need : 96 * 1024;
}

int tok_supported(uint32_t n_layers, uint32_t hidden, uint32_t ffn, uint32_t n_heads,
                  uint32_t n_kv_heads, uint32_t head_dim, uint32_t vocab, uint32_t max_seq,
                  int fmt, int n_cu) {
    if (head_dim != uint32_t(kTkHD) || n_kv_heads != 1 || n_heads == 0 ||
        n_heads > uint32_t(kTkMaxQH))
        return set_error(XP_E_ARG, "token kernel: needs head_dim 256, one kv head, <= 8 q heads");
    if (hidden > uint32_t(kTkMaxHidden) || hidden % 128 || ffn % 128 || vocab % kGrp)
        return set_error(XP_E_ARG, "token kernel: hidden <= 2048, multiples of 128");
    if (fmt != XP_SCALE_F16_QUAD && fmt != XP_SCALE_BF16_QUAD)
        return set_error(XP_E_ARG, "token kernel: fp16 or bf16 quad scales only");
    const uint32_t nch = (ffn / 128u + 15u) / 16u;
    if (uint64_t(nch + 1u) * hidden > uint64_t(kTkBig) ||
        uint64_t(max_seq + kTkC - 1u) / kTkC * 66u > uint64_t(kTkBig))
        return set_error(XP_E_ARG, "token kernel: stage scratch too small for this shape");
    if (n_layers == 0 || n_layers > uint32_t(kTkMaxLayers))
        return set_error(XP_E_ARG, "token kernel: at most %d layers", kTkMaxLayers);
    if (n_cu < 64 || n_cu > kTkMaxGrid || uint64_t(n_cu) * kTkC < max_seq)
        return set_error(XP_E_ARG, "token kernel: %d CUs cannot cover max_seq %u", n_cu, max_seq);
    return XP_OK;
}

int launch_token(const TokArgs& a, uint32_t grid, hipStream_t st) {
    static bool attr_set = false;
    const size_t lds = tok_lds_bytes();
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(token_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess)
            return set_error(XP_E_HIP, "token kernel: %zu B of LDS -> %s", lds,
                             hipGetErrorString(e));
        attr_set = true;
    }
    TokArgs copy = a;
    void* args[] = {&copy};
    hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(token_kernel),
                                              dim3(grid), dim3(kTkThreads), args, lds, st);
    if (e != hipSuccess)
        return set_error(XP_E_HIP, "token kernel: cooperative launch of %u workgroups -> %s", grid,
                         hipGetErrorString(e));
    return XP_OK;
}

}  // namespace xp
