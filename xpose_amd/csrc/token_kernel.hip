// One decode token as ONE persistent kernel on gfx950.
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
// workgroups lives in an 8-byte slot holding (launch tag, fp32 bits); slots
// are written two at a time with one 16-byte device-coherent store (sc1), and
// a consumer re-reads the 16-byte pairs it needs (sc1 loads) until every tag
// is this launch's (the low-latency protocol of collective libraries). A
// stage therefore waits one store-to-load latency for exactly the data it
// uses, and nothing waits for workgroups it does not depend on. Each
// workgroup walks the stages in order and skips those it has no work in;
// every stage's inputs are produced by earlier stages, so the walk is a
// topological order and the grid cannot deadlock. Waits are bounded: past the
// spin limit a workgroup records an error in state[2] and continues, so the
// grid always drains; the host reports the error.
//
// The kernel is compiled for one model shape (hidden, ffn, query heads) at a
// time, so every per-thread loop has a compile-time trip count and no
// branches on the shape. Latency, not bandwidth, sets the time of a stage
// (each moves 0.1-8 MB of weights across 256 CUs), so the design keeps every
// stage's dependent chain short:
//  * Vectors crossing a stage boundary are owned by threads: thread i holds
//    elements 4i .. 4i+3 (kOwn) in registers from the slot fetch through the
//    residual add, the RMSNorm and the fixed-point staging (a block of 32 is
//    then eight lanes). Only the staged planes go through LDS.
//  * Block reductions take one barrier (rotating partial buffers).
//  * Each stage's weights (the attention stage's KV rows) are loaded into
//    registers before the workgroup waits for the stage's inputs: weights
//    do not depend on activations, so HBM streaming overlaps the waiting.
//  * Matvec tiles: gate/up tiles are 32 ffn indices of the gate (lanes 0-31)
//    and the up projection (lanes 32-63) over the whole k, ending with the
//    GeGLU of those indices; q|k|v and o tiles are column slices (32 columns
//    of a 64-column group over the whole k, lane l taking column l % 32 and
//    block slot l / 32 of each two-block step); down tiles are 32-column
//    slices of kTokDownQuads-quad k chunks, whose partial sums the next
//    layer adds in chunk order. Wave w takes the steps w, w + 8, ...
//    (clamped to the range, the repeats weighted zero, so the loop has no
//    branches) and the 8 wave partials are summed through LDS in a fixed
//    order, so every result is deterministic.
//  * Attention, local layers (span <= 512, placement verified): 32
//    workgroups of one XCD, each one query head x 64 keys, exchanging their
//    chunk records through that XCD's L2 with 16 combine tiles of 64 dims;
//    global layers: a head pair x 64 keys a workgroup (128 keys past span
//    6656), 32 combine tiles of 32 dims; without a verified placement, all
//    heads x 32 / 16 keys a workgroup. Each attention workgroup computes
//    QK-norm + RoPE of its query head(s) and of the key itself, scores, a
//    chunk softmax (max, sum of exp) and the unnormalised weighted values;
//    the combine tiles rescale and sum the chunks (softmax_rows_finish,
//    llm_transformer.cl:385-405). The current key/value are used from LDS
//    (fp16-rounded, as the cache holds them) and appended to the cache by the
//    chunk that contains them, for later tokens.
//  * RoPE cos/sin for the token's position are computed once per workgroup
//    at kernel start (256 accurate sincosf, one per thread).
#include "xp_device.hpp"
#include "xp_launch.hpp"

namespace xp {

namespace {

constexpr int      kTkThreads   = kTokThreads;
constexpr int      kTkWaves     = kTkThreads / kWave;    // 8
constexpr uint32_t kTkHD        = 256;                   // head_dim
constexpr uint32_t kTkMaxQH     = 8;                     // query heads (one kv head)
// Keys per attention workgroup in global layers (and in local layers that
// do not exchange through one XCD); a build-time knob (32 or 64) for sweeps.
#ifndef XP_TOK_GLOBAL_KEYS
#define XP_TOK_GLOBAL_KEYS 64
#endif
constexpr uint32_t kTkC         = XP_TOK_GLOBAL_KEYS;
static_assert(kTkC == 32 || kTkC == 64, "32 or 64 keys per global attention chunk");
// Global layers' chunks split by head pair when the grid has room (1), or
// all heads per chunk (0).
#ifndef XP_TOK_GLOBAL_PAIRS
#define XP_TOK_GLOBAL_PAIRS 1
#endif
constexpr bool kTkGlobalPairs = XP_TOK_GLOBAL_PAIRS != 0;
// Dims per combine tile in global layers (32 or 64; local layers use 64).
#ifndef XP_TOK_GLOBAL_CD
#define XP_TOK_GLOBAL_CD 32
#endif
constexpr uint32_t kTkGlobalCD  = XP_TOK_GLOBAL_CD;
constexpr uint32_t kTkMaxBlk    = 64;                    // staged 32-blocks (2048 k)
constexpr int      kTkMaxGrid   = 1024;
constexpr int      kTkBig       = 17408;                 // floats of stage scratch
constexpr int      kTkMaxLayers = 64;
constexpr int      kTkLmDepth   = 3;     // lm_head units in flight per wave (4 and 6 measured no faster)
// Slot buffer operations use device scope (sc1, kAuxDev) on raw buffer
// resources (kRsrcWord3).
// Poll back-off of the first phase of the gate/up stage's wait (one thread
// watching for the layer's attention output), in units of 64 cycles.
constexpr int      kGuSleep     = 32;
// Column slices of the q|k|v, o and down tiles: a tile covers 64 / S columns
// of a column group over its whole k range, lane l taking column l / S and
// block slot l % S of each S-block step, so a wave's S-block step is one dot
// per lane and the tile's outputs are complete without more k splits (a
// consumer re-reads fewer partials while it polls). Gate/up keeps whole
// column groups. Build-time knobs (-D) for sweeps.
#ifndef XP_TOK_QKV_SLICES
#define XP_TOK_QKV_SLICES 2
#endif
#ifndef XP_TOK_O_SLICES
#define XP_TOK_O_SLICES 2
#endif
#ifndef XP_TOK_DOWN_SLICES
#define XP_TOK_DOWN_SLICES 2
#endif
constexpr uint32_t kTkSQ = XP_TOK_QKV_SLICES;
constexpr uint32_t kTkSO = XP_TOK_O_SLICES;
constexpr uint32_t kTkSD = XP_TOK_DOWN_SLICES;
static_assert((kTkSQ == 1 || kTkSQ == 2 || kTkSQ == 4) && (kTkSO == 1 || kTkSO == 2 || kTkSO == 4) &&
              (kTkSD == 1 || kTkSD == 2 || kTkSD == 4), "1, 2 or 4 column slices");

typedef unsigned long long ll_t;

// The model shape the kernel is compiled for.
template <uint32_t H_, uint32_t FFN_, uint32_t NH_>
struct TkShape {
    static constexpr uint32_t H = H_, FFN = FFN_, NH = NH_;
    static constexpr uint32_t QD = NH * kTkHD;              // q width
    static constexpr uint32_t QKVD = QD + 2 * kTkHD;        // q | k | v
    static constexpr uint32_t HB = H / kBlk;                // 32-blocks of a hidden vector
    static constexpr uint32_t HO = H / 4;                   // owner threads of a hidden vector
    static constexpr uint32_t QO = QD / 4;                  // owner threads of the attention output
    static constexpr uint32_t DQ = kTokDownQuads;           // quads per down chunk
    static constexpr uint32_t NQF = FFN / 128;              // quads of ffn
    static constexpr uint32_t NCH = (NQF + DQ - 1) / DQ;    // down chunks
    static constexpr uint32_t KQ = kTokQkvSplit;            // k halves of q|k|v
    static constexpr uint32_t KO = kTokOSplit;              // k halves of o
    static constexpr uint32_t QB = HB / KQ;                 // blocks per q|k|v tile
    static constexpr uint32_t OB = QD / kBlk / KO;          // blocks per o tile
    static constexpr uint32_t NOG = H / kGrp;               // o column groups
    static constexpr uint32_t SQ = kTkSQ, SO = kTkSO, SD = kTkSD;   // column slices
    static constexpr uint32_t N_QKV = QKVD / kGrp * KQ * SQ;
    static constexpr uint32_t N_COMB = NH * 4;              // local layers' combine tiles
    static constexpr uint32_t N_O = NOG * KO * SO;
    static constexpr uint32_t N_GU = FFN / (kGrp / 2);          // gate|up tiles of 32 ffn indices
    static constexpr uint32_t N_DN = (H / kGrp) * NCH * SD;
    // S-block steps per wave of a tile (blocks / (8 waves x S slots), rounded up)
    static constexpr int RK = int((QB + 8 * SQ - 1) / (8 * SQ));
    static constexpr int RO = int((OB + 8 * SO - 1) / (8 * SO));
    static constexpr int RD = int((DQ * 4 + 8 * SD - 1) / (8 * SD));
    static constexpr int RQ = int((HB + 7) / 8);
    static constexpr uint32_t NQH = H / 128;                // lm_head quads per column
    static_assert(H % 128 == 0 && FFN % 128 == 0, "hidden and ffn must be multiples of 128");
    static_assert(HO <= uint32_t(kTkThreads) && QO <= uint32_t(kTkThreads) &&
                  DQ * 128 / 4 <= uint32_t(kTkThreads), "vector too wide for four per thread");
    static_assert(HB <= kTkMaxBlk && QD / kBlk <= kTkMaxBlk && DQ * 4 <= kTkMaxBlk, "staging");
    static_assert(NH >= 1 && NH <= kTkMaxQH, "1..8 query heads");
    static_assert(tok_down_chunks(FFN) == NCH, "chunk count must match the slot layout");
    static_assert(HB % KQ == 0 && (QD / kBlk) % KO == 0, "k splits must divide the blocks");
    static_assert(NOG <= N_QKV && NOG <= N_GU, "x is stored by the first H / 64 tiles");
};

struct TkSmem {
    // The layer table, copied from device memory at kernel start. Read from
    // global memory at each use, its pointers cost a dependent load that
    // also waits for every outstanding weight prefetch (in-order vmcnt).
    TokLayer lt[kTkMaxLayers];
    QxBlock  qx[kTkMaxBlk];                  // fixed-point staging of a stage's input
    float    sx[kTkMaxBlk];
    alignas(16) float rs[4][kTkWaves];       // block reductions (rotating)
    float    red[kTkWaves][kWave];           // per-wave tile partials
    float    cs[2][kTkHD / 2];               // RoPE cos / sin at this position,
    float    sn[2][kTkHD / 2];               // [0] local theta, [1] global theta
    alignas(16) float qh[kTkMaxQH][kTkHD];   // normed, rotated q
    float    kn[kTkHD];                      // current key (fp16-rounded)
    float    vn[kTkHD];
    alignas(16) float sc[kTkC][kTkMaxQH];    // scores, then exp ([key][head])
    float    mh[kTkMaxQH];
    float    lh[kTkMaxQH];
    // Stage scratch: the value partials of attention's 4 key groups
    // ([4][n_heads][256]), the combine's chunk data ([chunk][66]).
    alignas(16) float big[kTkBig];
    float    fm[2 * kTkMaxGrid];             // combine: per-chunk factors; argmax slots
    float    amv[kTkWaves];
    uint32_t ami[kTkWaves];
    alignas(16) uint16_t kn16[kTkHD];       // current key as fp16 bits (head-split chunks)
    float    pc[kTkMaxQH];                   // weight of the current key (head-split chunks)
};

// ---- exchange slots -------------------------------------------------------------
// A 16-byte pair of slots: x = value 0, y = tag 0, z = value 1, w = tag 1.
__device__ __forceinline__ u32x4 ll_ld2(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), int(soff), kAuxDev);
}
__device__ __forceinline__ void ll_st2(rsrc_t r, uint32_t voff, uint32_t soff, float a, float b,
                                       uint32_t tag) {
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(a), tag, __float_as_uint(b), tag},
                                           r, int(voff), int(soff), kAuxDev);
}
// The same store kept in the XCD's L2 (written back, not through): visible
// to loads of any scope issued on the same XCD only.
__device__ __forceinline__ void ll_st2_xcd(rsrc_t r, uint32_t voff, uint32_t soff, float a, float b,
                                           uint32_t tag) {
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(a), tag, __float_as_uint(b), tag},
                                           r, int(voff), int(soff), 0);
}
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 0xFu;
}
__device__ __forceinline__ void ll_st1(rsrc_t r, uint32_t voff, uint32_t soff, float a, uint32_t tag) {
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(a), tag}, r, int(voff), int(soff),
                                          kAuxDev);
}
__device__ __forceinline__ bool ll_ok(u32x4 v, uint32_t tag) { return (v.y == tag) & (v.w == tag); }

// Loads the N slot pairs at byte offsets off[i] (+ soff) that are active and
// re-reads them until both tags of every pair are `tag`, sleeping SLEEP x 64
// cycles between rounds (a wait that is long by construction can poll less).
// Bounded: past `limit` re-reads the thread records an error in state[2] and
// keeps what it has; once any wait has recorded one, every other wait gives
// up within 256 rounds (or at its own limit), so the grid drains. A limit of
// 0 fails every wait that is not satisfied by its first read (the forced
// error path of the tests). Per thread; no barrier.
template <int N, int SLEEP = 0>
__device__ __forceinline__ void ll_wait(rsrc_t r, uint32_t soff, const uint32_t (&off)[N],
                                        const bool (&act)[N], u32x4 (&v)[N], uint32_t tag,
                                        uint32_t* state, uint32_t limit) {
    const u32x4 ready = {0u, tag, 0u, tag};
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = act[i] ? ll_ld2(r, off[i], soff) : ready;
    uint32_t spins = 0;
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; ++i) ok &= ll_ok(v[i], tag);
        if (ok) break;
        if (++spins > limit) {
            __hip_atomic_fetch_or((XP_GLOBAL uint32_t*)(state + 2), 1u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        if ((spins & 255u) == 0u && ld_dev(state + 2) != 0u) break;
        // The slots change under us: re-read them all (a stale-only re-read
        // does not unroll, and the ready pairs cannot change).
        if constexpr (SLEEP > 0) __builtin_amdgcn_s_sleep(SLEEP);
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = act[i] ? ll_ld2(r, off[i], soff) : ready;
    }
}

// Owner layout: thread i holds elements kOwn i .. kOwn i + kOwn - 1 of a
// vector crossing a stage boundary, kOwn / 2 slot pairs.
constexpr uint32_t kOwn  = 4;
constexpr uint32_t kOwnP = kOwn / 2;

// Byte offsets of this thread's kOwn consecutive slots starting at slot s0.
__device__ __forceinline__ void own_offsets(uint32_t* off, uint32_t s0) {
#pragma unroll
    for (uint32_t j = 0; j < kOwnP; ++j) off[j] = (s0 + 2u * j) * 8u;
}
__device__ __forceinline__ void own_unpack(float (&x)[kOwn], const u32x4* v) {
#pragma unroll
    for (uint32_t j = 0; j < kOwnP; ++j) {
        x[2 * j] = __uint_as_float(v[j].x);
        x[2 * j + 1] = __uint_as_float(v[j].z);
    }
}
// Owner put: x[0 .. kOwn) into slots s0 .. s0 + kOwn.
__device__ __forceinline__ void own_put(rsrc_t r, uint32_t soff, uint32_t s0, const float (&x)[kOwn],
                                        uint32_t tag) {
#pragma unroll
    for (uint32_t j = 0; j < kOwnP; ++j) ll_st2(r, (s0 + 2u * j) * 8u, soff, x[2 * j], x[2 * j + 1], tag);
}

__device__ __forceinline__ void tk_trace(const TokArgs& a, uint32_t wg, uint32_t event) {
    if (a.trace && threadIdx.x == 0)
        a.trace[size_t(event) * gridDim.x + wg] = __builtin_amdgcn_s_memrealtime();
}
// Stage end of layer l, stage k (event 1 + 6 l + k) and the time this
// workgroup's inputs of that stage had all arrived (event 3 + 6 n_layers +
// 6 l + k; 0 when the workgroup had no work in the stage).
__device__ __forceinline__ void tk_trace_stage(const TokArgs& a, uint32_t wg, uint32_t l, uint32_t k,
                                               unsigned long long t_in) {
    if (a.trace && threadIdx.x == 0) {
        a.trace[size_t(1u + 6u * l + k) * gridDim.x + wg] = __builtin_amdgcn_s_memrealtime();
        a.trace[size_t(3u + 6u * a.n_layers + 6u * l + k) * gridDim.x + wg] = t_in;
    }
}
__device__ __forceinline__ unsigned long long tk_now(const TokArgs& a) {
    return a.trace ? __builtin_amdgcn_s_memrealtime() : 0ull;
}

// rcp_hw / rsq_hw / exp_hw (xp_device.hpp) replace the correctly rounded
// division, square root and expf, some 15-30 dependent instructions each on
// a stage's critical path. The quantiser's r = range * rcp(m) keeps
// |q| <= 2^18 + 1, inside the digit planes' range.

// Wave maximum of floats through order-preserving int32 keys (a float's bits,
// the magnitude bits flipped when negative): v_max_i32 takes its DPP operand
// in place, where fmaxf first quiets both inputs (two more instructions a
// step). -inf orders below every finite value; the identity is INT32_MIN.
__device__ __forceinline__ int32_t f2ord(float v) {
    const int32_t k = __float_as_int(v);
    return k ^ ((k >> 31) & 0x7FFFFFFF);
}
__device__ __forceinline__ float ord2f(int32_t k) { return __int_as_float(k ^ ((k >> 31) & 0x7FFFFFFF)); }
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int32_t dpp_i(int32_t v, int32_t old) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xF, false);
}
__device__ __forceinline__ float wave_max_ord(float v) {
    constexpr int32_t lo = INT32_MIN;
    int32_t k = f2ord(v);
    k = max(k, dpp_i<0xB1, 0xF>(k, lo));    // quad_perm [1,0,3,2]
    k = max(k, dpp_i<0x4E, 0xF>(k, lo));    // quad_perm [2,3,0,1]
    k = max(k, dpp_i<0x141, 0xF>(k, lo));   // row_half_mirror
    k = max(k, dpp_i<0x140, 0xF>(k, lo));   // row_mirror
    k = max(k, dpp_i<0x142, 0xA>(k, lo));   // row_bcast:15 -> rows 1, 3
    k = max(k, dpp_i<0x143, 0xC>(k, lo));   // row_bcast:31 -> rows 2, 3
    return ord2f(__builtin_amdgcn_readlane(k, 63));
}

// ---- block-wide reductions (512 threads, one barrier) ---------------------------
// Every thread returns the same total, summed in a fixed order. rs must not be
// written again before another barrier has passed (the kernel rotates four).
__device__ __forceinline__ float blk_sum(float v, float* rs) {
    v = wave_sum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) rs[threadIdx.x / kWave] = v;
    __syncthreads();
    const float4 p = *reinterpret_cast<const float4*>(rs);
    const float4 q = *reinterpret_cast<const float4*>(rs + 4);
    return ((p.x + p.y) + (p.z + p.w)) + ((q.x + q.y) + (q.z + q.w));
}
__device__ __forceinline__ float blk_max(float v, float* rs) {
    v = wave_max(v);
    if ((threadIdx.x & (kWave - 1)) == 0) rs[threadIdx.x / kWave] = v;
    __syncthreads();
    const float4 p = *reinterpret_cast<const float4*>(rs);
    const float4 q = *reinterpret_cast<const float4*>(rs + 4);
    return fmaxf(fmaxf(fmaxf(p.x, p.y), fmaxf(p.z, p.w)), fmaxf(fmaxf(q.x, q.y), fmaxf(q.z, q.w)));
}

// kOwn consecutive floats of a vector in global memory (owner layout).
__device__ __forceinline__ void ld_own(float (&w)[kOwn], const float* p) {
#pragma unroll
    for (uint32_t j = 0; j < kOwn / 4; ++j) {
        const u32x4 v = ldg4(p + 4 * j);
        w[4 * j + 0] = __uint_as_float(v.x);
        w[4 * j + 1] = __uint_as_float(v.y);
        w[4 * j + 2] = __uint_as_float(v.z);
        w[4 * j + 3] = __uint_as_float(v.w);
    }
}

// Owner-layout Gemma RMSNorm steps (non-owner threads hold zeros and take part
// in the reduction). x = a + t * rsqrt(mean(t^2) + eps) * (1 + w): the residual
// add of a normed sublayer output (decode.cpp:1739-1751).
template <uint32_t H>
__device__ __forceinline__ void own_residual(float (&x)[kOwn], const float (&a)[kOwn],
                                             const float (&t)[kOwn], const float (&w)[kOwn], float eps,
                                             float* rs) {
    float ss = 0.0f;
#pragma unroll
    for (uint32_t e = 0; e < kOwn; ++e) ss = fmaf(t[e], t[e], ss);
    ss = blk_sum(ss, rs);
    const float scale = rsq_hw(ss * (1.0f / float(H)) + eps);
#pragma unroll
    for (uint32_t e = 0; e < kOwn; ++e) x[e] = a[e] + t[e] * scale * (1.0f + w[e]);
}
// RMSNorm feeding a matvec (rmsnorm_apply_gemma, y = x * rsqrt(mean(x^2) +
// eps) * (1 + w)), with its scalar deferred: the matvec of y is that scalar
// times the matvec of x (1 + w), and the block fixed-point staging is
// invariant to a common scale. own_norm_defer returns x (1 + w) and leaves
// each wave's partial sum of x^2 in rs; after the staging barrier,
// norm_scale(rs) is the scalar the caller multiplies its dot products by.
// The sum is then formed while the vector is staged, not before.
__device__ __forceinline__ void own_norm_defer(float (&y)[kOwn], const float (&x)[kOwn],
                                               const float (&w)[kOwn], float* rs) {
    float ss = 0.0f;
#pragma unroll
    for (uint32_t e = 0; e < kOwn; ++e) {
        ss = fmaf(x[e], x[e], ss);
        y[e] = x[e] * (1.0f + w[e]);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & (kWave - 1)) == 0) rs[threadIdx.x / kWave] = ss;
}
template <uint32_t H>
__device__ __forceinline__ float norm_scale(const float* rs, float eps) {
    const float4 p = *reinterpret_cast<const float4*>(rs);
    const float4 q = *reinterpret_cast<const float4*>(rs + 4);
    const float ss = ((p.x + p.y) + (p.z + p.w)) + ((q.x + q.y) + (q.z + q.w));
    return rsq_hw(ss * (1.0f / float(H)) + eps);
}

// Fixed-point staging (the planes of stage_x8, xp_device.hpp) from four
// consecutive activations per thread: task i covers elements 4 (i % 8) .. + 3
// of block i / 8, i.e. half h = i % 2 of word c = (i / 2) % 4 of each digit
// plane; the eight tasks of a block are adjacent lanes of one wave. The
// block maximum, the scale and every digit are those stage_x8 computes.
__device__ __forceinline__ void stage_x4(QxBlock* qx, float* sx, uint32_t i, const float (&v)[4]) {
    // |v| as bits: non-negative floats order as unsigned integers, so the
    // maximum is an integer max whose DPP operand needs no quieting
    uint32_t mb = max(max(__float_as_uint(v[0]) & 0x7FFFFFFFu, __float_as_uint(v[1]) & 0x7FFFFFFFu),
                      max(__float_as_uint(v[2]) & 0x7FFFFFFFu, __float_as_uint(v[3]) & 0x7FFFFFFFu));
    // max over the block's eight tasks: quad_perm xor 1, xor 2, then row_half_mirror
    mb = max(mb, uint32_t(__builtin_amdgcn_update_dpp(0, int(mb), 0xB1, 0xF, 0xF, false)));
    mb = max(mb, uint32_t(__builtin_amdgcn_update_dpp(0, int(mb), 0x4E, 0xF, 0xF, false)));
    mb = max(mb, uint32_t(__builtin_amdgcn_update_dpp(0, int(mb), 0x141, 0xF, 0xF, false)));
    const float m = __uint_as_float(mb);
    const float r = m > 0.0f ? kQxRange * rcp_hw(m) : 0.0f;
    uint32_t t[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) t[e] = uint32_t(__float2int_rn(v[e] * r) + int32_t(kQxBias)) ^ kQxBias;
    const uint32_t lb = i >> 3, hw = i & 7u;   // half-word 2 c + h of each plane
    // Plane p's half-word is digit p of t[0..3] at nibbles 0..3. Byte k of
    // a (b) pairs digit 2 k (2 k + 1) of t[0] and t[1]; c, d the same for
    // t[2], t[3]; a byte permute then joins a pair's byte with the matching
    // t[2] / t[3] byte, two planes per dword.
    const uint32_t a = (t[0] & 0x0F0F0Fu) | ((t[1] & 0x0F0F0Fu) << 4);
    const uint32_t b = ((t[0] >> 4) & 0x0F0F0Fu) | (t[1] & 0xF0F0F0u);
    const uint32_t c = (t[2] & 0x0F0F0Fu) | ((t[3] & 0x0F0F0Fu) << 4);
    const uint32_t d = ((t[2] >> 4) & 0x0F0F0Fu) | (t[3] & 0xF0F0F0u);
    const uint32_t p02 = __builtin_amdgcn_perm(c, a, 0x05010400u);   // planes 0 | 2
    const uint32_t p13 = __builtin_amdgcn_perm(d, b, 0x05010400u);   // planes 1 | 3
    reinterpret_cast<uint16_t*>(&qx[lb].p[0])[hw] = uint16_t(p02);
    reinterpret_cast<uint16_t*>(&qx[lb].p[1])[hw] = uint16_t(p13);
    reinterpret_cast<uint16_t*>(&qx[lb].p[2])[hw] = uint16_t(p02 >> 16);
    reinterpret_cast<uint16_t*>(&qx[lb].p[3])[hw] = uint16_t(p13 >> 16);
    if constexpr (kQxPlanes == 5)
        reinterpret_cast<uint16_t*>(&qx[lb].p[4])[hw] = uint16_t(__builtin_amdgcn_perm(c, a, 0x07030602u));
    if (hw == 0) sx[lb] = m * (1.0f / kQxRange);
}
// Stages an owner vector as fixed-point planes in S.qx / S.sx: task i (i <
// nblocks * 32 / kOwn, eight adjacent lanes per block) holds elements
// kOwn i .. kOwn i + kOwn - 1 of the staged range. The caller then waits at a
// barrier.
__device__ __forceinline__ void own_stage(TkSmem& S, const float (&x)[kOwn], uint32_t i) {
    static_assert(kOwn == 4, "staging from four elements per thread");
    stage_x4(S.qx, S.sx, i, x);
}

// Scale i (0..3) of a block quad's four fp16 / bf16 scales, without branches.
template <int FMT>
__device__ __forceinline__ float tk_scale(u32x2 raw, uint32_t i) {
    const uint32_t w = (i & 2u) ? raw.y : raw.x;
    const uint32_t h = (w >> (16u * (i & 1u))) & 0xFFFFu;
    if constexpr (FMT == XP_SCALE_F16_QUAD) return f16_bits_to_f32(h);
    else return __uint_as_float(h << 16);
}

// ---- matvec tiles ------------------------------------------------------------------
// A tile: columns h CW .. h CW + CW - 1 (CW = 64 / S) of column group g of a
// KM4 matrix (nblk 32-blocks of k, cols columns), k blocks [b0, b0 + nb).
// Lane l takes column h CW + l % CW and block slot q = l / CW (a slot is
// whole 16-lane rows); wave w takes the S-block steps w + 8 r (r < R), i.e.
// block b0 + min(S (w + 8 r) + q, nb - 1); a repeated (clamped) block is
// computed and weighted by zero. S = 1 is one whole column group, lane = column.
template <int R>
struct TkW {
    u32x4 w[R];
    u32x2 s[R];
};

template <int R, uint32_t S = 1>
__device__ __forceinline__ void tile_prefetch(TkW<R>& p, const void* wq, const void* sc, uint32_t nblk,
                                              uint32_t cols, uint32_t g, uint32_t h, uint32_t b0,
                                              uint32_t nb, uint32_t wave, uint32_t lane) {
    constexpr uint32_t CW = kGrp / S;
    const u32x4* w = static_cast<const u32x4*>(wq);
    const u32x2* s = static_cast<const u32x2*>(sc);
    const uint32_t cl = h * CW + lane % CW, q = lane / CW;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t b = b0 + min(S * (wave + 8u * r) + q, nb - 1u);
        p.w[r] = ldg_stream4(w + (size_t(g) * nblk + b) * kGrp + cl);
        p.s[r] = ldg_stream2(s + size_t(b / 4u) * cols + g * kGrp + cl);
    }
}

// Readies a prefetched tile for tile_dot: the weight nibbles as two's
// complement (xor 0x88888888) and in s[r].x the float scale of the lane's
// block of step r (the scale of block b0 + S (w + 8 r) + q is component
// (b0 + S w + q) % 4 of its quad, the same for all r; zero for a clamped
// repeat). Called before the stage's wait: the wait's loads return after the
// prefetch's, so this work is done while the inputs are on their way instead
// of after they arrive.
template <int FMT, int R, uint32_t S = 1>
__device__ __forceinline__ void tile_prep(TkW<R>& p, uint32_t b0, uint32_t nb, uint32_t wave,
                                          uint32_t lane) {
    const uint32_t q = lane / (kGrp / S);
    const uint32_t sc = (b0 + S * wave + q) % 4u;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        p.w[r] ^= 0x88888888u;
        float f = tk_scale<FMT>(p.s[r], sc);
        if (S * (wave + 8u * uint32_t(r)) + q >= nb) f = 0.0f;
        p.s[r].x = __float_as_uint(f);
        // done here, not sunk to the dot past the wait
        asm volatile("" : "+v"(p.w[r]), "+v"(p.s[r].x));
    }
}

// Dot of the wave's blocks with the staged planes (S.qx[0] = block b0) for a
// tile readied by tile_prep, then reduced over the 8 waves and the S slots
// in order. The result is valid in wave 0, lane l < CW holding column l; the
// caller publishes it. Starts after the staging barrier; ends with a barrier.
template <int R, uint32_t S = 1>
__device__ __forceinline__ float tile_dot(const TkW<R>& p, TkSmem& Sm, uint32_t nb, uint32_t wave,
                                          uint32_t lane) {
    constexpr uint32_t CW = kGrp / S;
    constexpr uint32_t NW = 2u * kQxPlanes;   // lanes of a row holding a block's words
    static_assert(NW <= 16u && 2u * NW >= 16u, "a block's words fill one row's lanes");
    const uint32_t q = lane / CW, j = lane % 16u;
    const uint32_t jw = j >= NW ? j - NW : j;   // the other lanes repeat words (unused)
    // Every block's words and scale are read before any is used: the reads
    // return in order while the first blocks are multiplied.
    u32x2 aw[R];
    float sxv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t lb = min(S * (wave + 8u * r) + q, nb - 1u);
        sxv[r] = Sm.sx[lb];
        aw[r] = reinterpret_cast<const u32x2*>(&Sm.qx[lb])[jw];
    }
    __builtin_amdgcn_sched_barrier(0);
    // A DPP operation must follow a write of exec by five wait states, which
    // the compiler does not provide for inline assembly: one s_nop 4 before
    // the first, ordered after the loads by the tied operands.
#pragma unroll
    for (int r = 0; r < R; ++r) asm volatile("s_nop 4" : "+v"(aw[r].x), "+v"(aw[r].y));
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r += 2) {
        if (r + 1 < R) {
            const u32x4 w2[2] = {p.w[r], p.w[r + 1]};
            const u32x2 a2[2] = {aw[r], aw[r + 1]};
            int32_t d[2];
            block_dot_bc<2>(w2, a2, d);
            acc = fmaf(__uint_as_float(p.s[r].x) * sxv[r], float(d[0]), acc);
            acc = fmaf(__uint_as_float(p.s[r + 1].x) * sxv[r + 1], float(d[1]), acc);
        } else {
            const u32x4 w1[1] = {p.w[r]};
            const u32x2 a1[1] = {aw[r]};
            int32_t d[1];
            block_dot_bc<1>(w1, a1, d);
            acc = fmaf(__uint_as_float(p.s[r].x) * sxv[r], float(d[0]), acc);
        }
    }
    Sm.red[wave][lane] = acc;
    __syncthreads();
    float y = 0.0f;
    if (wave == 0) {
        // all partials in flight at once, then summed in wave, slot order
        const uint32_t c = lane % CW;
        float pw[kTkWaves * S];
#pragma unroll
        for (int w = 0; w < kTkWaves; ++w)
#pragma unroll
            for (uint32_t sl = 0; sl < S; ++sl) pw[w * S + sl] = Sm.red[w][c + sl * CW];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (uint32_t i = 0; i < kTkWaves * S; ++i) y += pw[i];
    }
    return y;
}

// Wave 0 publishes its CW = 64 / S column results y (lane l < CW holding
// column l) at slots s0 + column: lane 2 m stores columns 2 m and 2 m + 1,
// the second read from lane 2 m + 1 (quad_perm xor 1).
template <uint32_t S = 1>
__device__ __forceinline__ void tile_put(rsrc_t r, uint32_t soff, uint32_t s0, float y, uint32_t lane,
                                         uint32_t tag) {
    constexpr uint32_t CW = kGrp / S;
    const float yn = dpp_f<0xB1, 0xF>(y, 0.0f);
    if (lane < CW && lane % 2u == 0u) ll_st2(r, (s0 + lane) * 8u, soff, y, yn, tag);
}

__device__ __forceinline__ float f16_round(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }

// An attention wave's vector after QK-norm / RoPE (lane l holds elements
// 2 l, 2 l + 1, 2 l + 128, 2 l + 129): slot v < NH is query head v (fp32 in
// qh[v], or qh[0] when the chunk takes one head), slot NH the key (fp16 bits,
// as the cache will hold it), slot NH + 1 the value (fp16-rounded fp32).
template <class Smem>
__device__ __forceinline__ void own_kv_put(Smem& S, uint32_t v, uint32_t nh, uint32_t lane, float (&e)[4]) {
    constexpr uint32_t HD = 256;
    if (v == nh) {
        const uint32_t lo = uint32_t(f32_to_f16_bits(e[0])) | (uint32_t(f32_to_f16_bits(e[1])) << 16);
        const uint32_t hi = uint32_t(f32_to_f16_bits(e[2])) | (uint32_t(f32_to_f16_bits(e[3])) << 16);
        *reinterpret_cast<uint32_t*>(&S.kn16[2u * lane]) = lo;
        *reinterpret_cast<uint32_t*>(&S.kn16[HD / 2u + 2u * lane]) = hi;
    }
    float* dst = v < nh ? S.qh[v] : (v == nh ? S.kn : S.vn);
    if (v >= nh) {
#pragma unroll
        for (int c = 0; c < 4; ++c) e[c] = f16_round(e[c]);
    }
    *reinterpret_cast<float2*>(dst + 2u * lane) = float2{e[0], e[1]};
    *reinterpret_cast<float2*>(dst + HD / 2u + 2u * lane) = float2{e[2], e[3]};
}

// v, as a value the compiler cannot see through.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

}  // namespace

template <class Sh, int FMT>
__global__ __launch_bounds__(kTkThreads) void token_kernel(TokArgs a) {
    constexpr uint32_t H = Sh::H, FFN = Sh::FFN, NH = Sh::NH, QD = Sh::QD;
    constexpr uint32_t NCH = Sh::NCH;
    extern __shared__ __align__(16) unsigned char tk_lds[];
    TkSmem& S = *reinterpret_cast<TkSmem*>(tk_lds);
    // Thread-derived values are re-derived through an opaque copy at every
    // layer, so that the compiler recomputes per-thread offsets inside each
    // stage instead of keeping them all in registers across the layer loop.
    uint32_t tid = threadIdx.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    uint32_t lane = tid % kWave;
    // The workgroup's role id. With the XCD-local exchange on, role w must
    // run on the XCD the host's probe found residue w % 8 on. The hardware
    // deals a launch's workgroups to the eight XCDs in a fixed cyclic order,
    // but the XCD it starts from moves between launches (measured), so each
    // workgroup takes, within its aligned group of eight, the slot of the
    // XCD it actually runs on: a bijection whenever each aligned group of
    // eight covers the eight XCDs. A workgroup on an XCD the probe never saw
    // reports status bit 2 at once (every wait then gives up), and the host
    // stops using the XCD-local exchange.
    const uint32_t nwg  = gridDim.x;
    uint32_t wg = blockIdx.x;
    bool on_xcd = true;
    if (a.xcd_local) {
        const uint32_t x = xcc_id();
        uint32_t slot = 8u;
#pragma unroll
        for (uint32_t r = 0; r < 8u; ++r)
            if (((a.xcd_ids >> (4u * r)) & 15u) == x) slot = r;
        on_xcd = slot < 8u;
        if (on_xcd) wg = (wg & ~7u) | slot;
        else if (tid == 0)
            __hip_atomic_fetch_or((XP_GLOBAL uint32_t*)(a.state + 2), 2u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
    }
    const uint32_t tag  = a.tag;
    const float    eps  = a.eps;
    tk_trace(a, wg, 0);

    const uint32_t pos = a.state[0];
    uint32_t tok = a.state[1];
    if (tok >= a.vocab) tok = 0;                 // the host validates ids
    if (wg == 0 && tid == 0) a.hist[pos] = tok;

    const uint32_t seq = pos + 1u;
    const TokLL lay = tok_ll_layout(H, FFN, NH, kTkHD, nwg);
    const uint32_t lstride = uint32_t(a.ll_layer) * 8u;   // bytes per layer of slots
    const rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
        a.ll, short(0), int(a.n_layers * lstride + 16u * nwg), kRsrcWord3);
    uint32_t rk = 0;                              // rotating reduction buffer
    auto RS = [&]() { return S.rs[(rk++) & 3u]; };

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

    // Workgroup -> tile maps: tile t of a stage runs on workgroup (off + t) %
    // grid, so this workgroup's first tile is (wg - off) mod grid. QKV,
    // combine, O and down start at workgroup 0 (combine's workgroups have no
    // other work until O, which waits for all of combine anyway); gate/up
    // starts past the O workgroups, whose O tile would otherwise delay their
    // gate/up weight prefetch; attention runs from the last workgroup down.
    const uint32_t off_gu = Sh::N_O % nwg;
    const uint32_t t_comb = wg, t_o = wg;
    // QKV tiles run on workgroups past the down tiles' (from N_DN on, skipping
    // those of residue 7 mod 8, the local attention's XCD), when the grid has
    // room: a workgroup with both a down and a QKV tile would request its QKV
    // weights ahead of one of the two waits, and memory requests complete in
    // order. Otherwise tile t on workgroup t.
    uint32_t t_qkv = wg, qkv_above = 0u;
    const bool qsep = Sh::N_DN + (Sh::N_QKV * 8u + 6u) / 7u + 8u <= nwg;
    if (qsep) {
        // rank of wg among the workgroups >= b whose residue is not 7 (the
        // residue-7 workgroups below x number x / 8)
        const uint32_t b = Sh::N_DN;
        auto rank = [&](uint32_t x) { return (x - b) - (x / 8u - b / 8u); };
        t_qkv = (wg < b || wg % 8u == 7u) ? Sh::N_QKV : rank(wg);
        // QKV workgroups above this one (ranks rank(wg + 1) .. N_QKV - 1)
        qkv_above = wg + 1u <= b ? Sh::N_QKV : Sh::N_QKV - min(Sh::N_QKV, rank(wg + 1u));
    }
    const uint32_t t_gu = (wg + nwg - off_gu) % nwg, t_dn = wg;
    bool hown = tid < Sh::HO;                     // owns kOwn elements of a hidden vector

    // x entering layer l (l > 0) from layer l - 1's slots, in owner registers:
    // xb + post_ffw_norm(sum of the down chunks, in chunk order).
    auto after_ffn = [&](float (&x)[kOwn], uint32_t lp, const float (&w_post)[kOwn]) {
        const uint32_t soff = lp * lstride;
        float xb[kOwn] = {}, t[kOwn] = {};
        if (hown) {
            // xb (written in the gate/up stage, a stage before the down
            // chunks) first, so that the polls of the chunks carry only them
            {
                uint32_t off[kOwnP];
                bool act[kOwnP];
                u32x4 v[kOwnP];
                own_offsets(&off[0], uint32_t(lay.xb) + kOwn * tid);
#pragma unroll
                for (uint32_t i = 0; i < kOwnP; ++i) act[i] = true;
                ll_wait(rr, soff, off, act, v, tag, a.state, a.spin_limit);
                own_unpack(xb, &v[0]);
            }
            constexpr uint32_t NL = kOwnP * NCH;
            uint32_t off[NL];
            bool act[NL];
            u32x4 v[NL];
#pragma unroll
            for (uint32_t c = 0; c < NCH; ++c)
                own_offsets(&off[kOwnP * c], uint32_t(lay.dnp) + c * H + kOwn * tid);
#pragma unroll
            for (uint32_t i = 0; i < NL; ++i) act[i] = true;
            ll_wait(rr, soff, off, act, v, tag, a.state, a.spin_limit);
            own_unpack(t, &v[0]);
#pragma unroll
            for (uint32_t c = 1; c < NCH; ++c) {
                float u[kOwn];
                own_unpack(u, &v[kOwnP * c]);
#pragma unroll
                for (uint32_t e = 0; e < kOwn; ++e) t[e] += u[e];
            }
        }
        own_residual<H>(x, xb, t, w_post, eps, RS());
    };

    // Weight prefetch. A workgroup's first QKV tile of layer l + 1 is loaded
    // before it waits in layer l's down stage, and its down tile before it
    // waits in the gate/up stage: a workgroup busy in the previous stage
    // would otherwise start streaming those weights only when its inputs are
    // already there.
    constexpr int RQ = Sh::RQ;                        // gate/up blocks per wave
    constexpr int RK = Sh::RK;                        // QKV S-block steps per wave
    constexpr int RD = Sh::RD;                        // down S-block steps per wave
    constexpr int RO = Sh::RO;                        // o S-block steps per wave
    // QKV tile t = ((column group of q | k | v) KQ + k part c) SQ + slice h:
    // matrix m (q, k, v), its column group g.
    auto qkv_tile = [&](uint32_t t, uint32_t& m, uint32_t& g, uint32_t& c, uint32_t& h) {
        constexpr uint32_t qg = QD / kGrp, kg = kTkHD / kGrp;
        h = t % Sh::SQ;
        const uint32_t tc = t / Sh::SQ;
        const uint32_t tt = tc / Sh::KQ;
        c = tc % Sh::KQ;
        m = tt < qg ? 0u : (tt < qg + kg ? 1u : 2u);
        g = m == 0 ? tt : (m == 1 ? tt - qg : tt - qg - kg);
    };
    auto prefetch_qkv = [&](TkW<RK>& p, uint32_t l, uint32_t t) {
        uint32_t m, g, c, h;
        qkv_tile(t, m, g, c, h);
        tile_prefetch<RK, Sh::SQ>(p, S.lt[l].w[m], S.lt[l].s[m], Sh::HB, m == 0 ? QD : kTkHD, g, h,
                                  c * Sh::QB, Sh::QB, wave, lane);
    };
    // down tile t = (column group g NCH + k chunk c) SD + slice h
    auto prefetch_dn = [&](TkW<RD>& p, uint32_t l, uint32_t t) {
        const uint32_t h = t % Sh::SD, tc = t / Sh::SD;
        const uint32_t g = tc / NCH, q0 = Sh::DQ * (tc % NCH);
        tile_prefetch<RD, Sh::SD>(p, S.lt[l].w[6], S.lt[l].s[6], FFN / kBlk, H, g, h, 4u * q0,
                                  4u * min(Sh::DQ, Sh::NQF - q0), wave, lane);
    };
    TkW<RK> pq;
    if (t_qkv < Sh::N_QKV) prefetch_qkv(pq, 0u, t_qkv);

    for (uint32_t l = 0; l < a.n_layers; ++l) {
        tid = opaque(threadIdx.x);
        lane = tid % kWave;
        hown = tid < Sh::HO;
        const TokLayer& L = S.lt[l];
        const uint32_t soff = l * lstride;
        // ================= QKV =================
        unsigned long long t_in = 0;
        for (uint32_t t = t_qkv; t < Sh::N_QKV; t += nwg) {
            uint32_t m, g, c, h;
            qkv_tile(t, m, g, c, h);
            if (t != t_qkv) prefetch_qkv(pq, l, t);
            tile_prep<FMT, RK, Sh::SQ>(pq, c * Sh::QB, Sh::QB, wave, lane);
            float w_in[kOwn] = {}, w_post[kOwn] = {}, x[kOwn] = {};
            if (hown) {
                ld_own(w_in, L.norm[0] + kOwn * tid);
                if (l > 0) ld_own(w_post, S.lt[l - 1u].norm[3] + kOwn * tid);
            }
            if (l == 0 && a.embed_f32) {
                // embedding (decode.cpp:1618-1627) from the model's fp32 rows
                if (hown) {
                    const float4 e4 = *reinterpret_cast<const float4*>(
                        a.embed_f32 + size_t(tok) * H + kOwn * tid);
                    x[0] = e4.x * a.embed_scale;
                    x[1] = e4.y * a.embed_scale;
                    x[2] = e4.z * a.embed_scale;
                    x[3] = e4.w * a.embed_scale;
                }
            } else if (l == 0) {
                // embedding (decode.cpp:1618-1627) as a gather from the tied int4 table
                if (hown) {
                    // element k = kOwn tid + e: block k / 32, word (k % 32) / 8, nibble k % 8
                    const uint32_t k0 = kOwn * tid, b = k0 / kBlk, c = (k0 % kBlk) / 8u, n0 = k0 % 8u;
                    const uint32_t* wq = static_cast<const uint32_t*>(a.lm_w);
                    const uint32_t word =
                        ldg32(wq + ((size_t(tok / kGrp) * Sh::HB + b) * kGrp + (tok % kGrp)) * 4u + c);
                    const uint16_t h = ldg16(static_cast<const uint16_t*>(a.lm_s) +
                                             (size_t(b / 4u) * a.vocab + tok) * 4u + (b % 4u));
                    const float s = FMT == XP_SCALE_F16_QUAD ? f16_bits_to_f32(h)
                                                             : __uint_as_float(uint32_t(h) << 16);
#pragma unroll
                    for (uint32_t e = 0; e < kOwn; ++e) {
                        const float q = float(int((word >> (4u * (n0 + e))) & 15u) - 8);
                        x[e] = (q * s) * a.embed_scale;
                    }
                }
            } else {
                after_ffn(x, l - 1u, w_post);
            }
            if (t == t_qkv) t_in = tk_now(a);
            float xn[kOwn];
            float* rsn = RS();
            own_norm_defer(xn, x, w_in, rsn);
            {
                // stage this tile's k half: blocks c QB .. c QB + QB - 1
                constexpr uint32_t tpb = kBlk / kOwn;   // owner threads per block
                const uint32_t i = tid - c * Sh::QB * tpb;
                if (hown && i < Sh::QB * tpb) own_stage(S, xn, i);
            }
            __syncthreads();
            float y = tile_dot<RK, Sh::SQ>(pq, S, Sh::QB, wave, lane);
            if (wave == 0) {
                y *= norm_scale<H>(rsn, eps);
                const uint32_t o = c * Sh::QKVD + (m == 0u ? 0u : (m == 1u ? QD : QD + kTkHD));
                tile_put<Sh::SQ>(rr, soff, uint32_t(lay.qkv) + o + g * kGrp + h * (kGrp / Sh::SQ), y,
                                 lane, tag);
            }
            // x entering the layer, for the gate/up stage: tile t < H / 64
            // stores elements 64 t .. 64 t + 63 (spread so that no workgroup
            // issues many stores). Stored last: a later wait on this wave's
            // memory counter also waits for its stores.
            if (t < Sh::NOG && tid / (kGrp / kOwn) == t) own_put(rr, soff, uint32_t(lay.xa) + kOwn * tid, x, tag);
        }
        tk_trace_stage(a, wg, l, 0u, t_in);
        t_in = 0;

        // The O tile's weights are requested here, before the attention and
        // combine stages: a workgroup with an attention chunk or a combine tile
        // as well as an O tile would otherwise request them only after those.
        TkW<RO> po;
        auto o_tile = [&](uint32_t t, uint32_t& g, uint32_t& c, uint32_t& h) {
            // t = (column group g KO + k part c) SO + slice h
            h = t % Sh::SO;
            const uint32_t tc = t / Sh::SO;
            g = tc / Sh::KO;
            c = tc % Sh::KO;
        };
        if (t_o < Sh::N_O) {
            uint32_t g, c, h;
            o_tile(t_o, g, c, h);
            tile_prefetch<RO, Sh::SO>(po, L.w[3], L.s[3], QD / kBlk, H, g, h, c * Sh::OB, Sh::OB, wave, lane);
        }

        // ================= attention =================
        const bool glob = L.global != 0u;
        const uint32_t kv0 = (glob || a.window == 0u || seq <= a.window) ? 0u : seq - a.window;
        const uint32_t span = seq - kv0;
        // Local layers, when the XCD map was verified: chunk s on workgroup
        // grid - 1 - 8 s and combine tile c on grid - 1 - 8 c, all on one XCD,
        // so the chunk records cross that XCD's L2 only; the chunks hold 16
        // keys when that XCD has a workgroup for each (half the score and
        // value work per workgroup), else kTkC. Otherwise chunk s on
        // the s-th workgroup from the last down that has no QKV tile (a QKV
        // workgroup would issue its chunk's key / value loads only after its
        // tile, ahead of its wait for q | k | v), or on grid - 1 - s when the
        // grid has too few of those; combine tile c on workgroup c.
        const bool xl_ok = a.xcd_local != 0u && !glob && Sh::N_COMB * 8u <= nwg;
        // Local layers on one XCD split by head when that XCD has a
        // workgroup for every (head, 64-key chunk): each workgroup polls one
        // head of q, and a combine tile reads a head's few chunk records.
        constexpr uint32_t kHK = 64u;                    // keys per head-split chunk
        const bool hsplit = xl_ok && (span + kHK - 1u) / kHK * NH * 8u <= nwg;
        // Global layers split by head pair when the grid holds a workgroup
        // for every (pair, chunk) beside the QKV tiles: each workgroup scores
        // and sums its keys for two heads instead of all NH; 64-key chunks
        // while those fit (span <= 6656 on 256 CUs), else 128-key chunks
        // (half the workgroups, half the records a combine tile reads).
        const bool gpair = kTkGlobalPairs && glob && NH % 2u == 0u;
        const bool g64 = gpair && (span + 63u) / 64u * (NH / 2u) + Sh::N_QKV <= nwg;
        const bool g128 = gpair && !g64 && (span + 127u) / 128u * (NH / 2u) + Sh::N_QKV <= nwg;
        const bool gsplit = g64 || g128;
        const uint32_t cw = hsplit ? kHK
                          : g64   ? 64u
                          : g128  ? 128u
                                  : (xl_ok && (span + 15u) / 16u * 8u <= nwg ? 16u : kTkC);
        const uint32_t n_att = (span + cw - 1u) / cw;    // chunk records per head
        const uint32_t n_wga = hsplit ? n_att * NH : gsplit ? n_att * (NH / 2u) : n_att;   // attention workgroups
        const bool xl = xl_ok && n_wga * 8u <= nwg;
        const uint32_t rx = nwg - 1u - wg;
        const bool ask = qsep && n_wga + Sh::N_QKV <= nwg;
        const uint32_t s_att = xl ? (rx % 8u == 0u ? rx / 8u : ~0u)
                                  : !ask ? rx : (t_qkv < Sh::N_QKV ? ~0u : rx - qkv_above);
        const bool xl_st = xl && on_xcd;
        // one chunk of CW keys (CW = 16 or kTkC)
        auto attend = [&](auto cw_c) {
            constexpr uint32_t CW = decltype(cw_c)::value;
            constexpr uint32_t TPK = kTkThreads / CW;        // threads per key (scores)
            constexpr uint32_t NCK = kTkHD / (4u * TPK);      // float4 of a key per thread
            constexpr uint32_t HK = CW / 2u;                  // keys per lane half (values)
            static_assert(TPK == 8u || TPK == 16u || TPK == 32u,
                          "a key's parts span half a DPP row, one row or two");
            static_assert(kTkHD == 32u * kTkWaves, "values: 32 dims per wave");
            static_assert(NH % 4u == 0u, "values: each lane stores one of four heads");
            const uint32_t j0 = s_att * CW;
            // score mapping: key jk = tid / TPK; part p holds dims 4 TPK c + 4 p .. + 3,
            // c < NCK (the parts of a key read consecutive float4 of q: no LDS
            // bank conflicts)
            const uint32_t jk = tid / TPK, part = tid % TPK;
            // value mapping: wave w, lane l: dim dv = 32 w + l % 32 of keys
            // kh HK .. kh HK + HK - 1, kh = l / 32, all query heads; the two
            // key halves meet across lanes l and l ^ 32
            const uint32_t dv = 32u * wave + lane % 32u, kh = lane / 32u;
            // Key / value rows past the span are clamped to its last row and
            // every load is unconditional (a guarded load becomes a branch
            // that waits for it); whatever such a row holds (the last one is
            // the current position, not yet appended) is dropped by selects.
            u32x2 kr[NCK];
            uint32_t vh[HK];
            {
                const uint16_t* kp = L.kc + size_t(kv0 + min(j0 + jk, span - 1u)) * kTkHD + 4u * part;
#pragma unroll
                for (uint32_t c = 0; c < NCK; ++c) kr[c] = *(const XP_GLOBAL u32x2*)(kp + 4u * TPK * c);
            }
#pragma unroll
            for (uint32_t i = 0; i < HK; ++i)
                vh[i] = ldg16(L.vc + size_t(kv0 + min(j0 + kh * HK + i, span - 1u)) * kTkHD + dv);
            // Wave h <= NH + 1 takes vector h of q | k | v (the q heads, the
            // key, the value): lane l holds elements 2 l, 2 l + 1, 2 l + 128,
            // 2 l + 129 (slot pairs l and l + 64), so its rotate-half pairs
            // (d, d + 128) are its own. QK-norm weights at the same elements.
            static_assert(NH + 2u <= uint32_t(kTkWaves), "one wave per q head, the key and the value");
            static_assert(kTkHD == 256u, "two slot pairs per lane per head");
            float wqk[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (wave <= NH) {
                const float* w = (wave < NH ? L.norm[4] : L.norm[5]) + 2u * lane;
                const u32x2 w0 = *(const XP_GLOBAL u32x2*)(w);
                const u32x2 w1 = *(const XP_GLOBAL u32x2*)(w + kTkHD / 2u);
                wqk[0] = __uint_as_float(w0.x); wqk[1] = __uint_as_float(w0.y);
                wqk[2] = __uint_as_float(w1.x); wqk[3] = __uint_as_float(w1.y);
            }
            const uint32_t th = glob ? 1u : 0u;
            if (wave <= NH + 1u) {
                static_assert(Sh::KQ == 1u, "attention reads q | k | v whole (no k parts)");
                uint32_t off[2];
                const bool act[2] = {true, true};
                u32x4 v[2];
                const uint32_t p0 = uint32_t(lay.qkv) + wave * kTkHD + 2u * lane;
                off[0] = p0 * 8u;
                off[1] = (p0 + kTkHD / 2u) * 8u;
                ll_wait(rr, soff, off, act, v, tag, a.state, a.spin_limit);
                float e[4] = {__uint_as_float(v[0].x), __uint_as_float(v[0].z), __uint_as_float(v[1].x),
                              __uint_as_float(v[1].z)};
                if (wave <= NH) {
                    // QK-norm (wave sum) and RoPE of this head, in registers
                    float ss = e[0] * e[0] + e[1] * e[1] + e[2] * e[2] + e[3] * e[3];
                    ss = wave_sum(ss);
                    const float scale = rsq_hw(ss * (1.0f / float(kTkHD)) + eps);
#pragma unroll
                    for (int c = 0; c < 4; ++c) e[c] = e[c] * scale * (1.0f + wqk[c]);
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const float cv = S.cs[th][2u * lane + c], sv = S.sn[th][2u * lane + c];
                        const float lo = e[c], hi = e[c + 2];
                        e[c] = lo * cv - hi * sv;
                        e[c + 2] = lo * sv + hi * cv;
                    }
                }
                own_kv_put(S, wave, NH, lane, e);
            }
            __syncthreads();
            t_in = tk_now(a);
            // scores (the current key comes from S.kn, read unconditionally so
            // that the choice is a select, not a branch)
            {
                const uint32_t jj = j0 + jk;
                const bool valid = jj < span;
                const bool cur = kv0 + jj == pos;
                float kf[4 * NCK];
#pragma unroll
                for (uint32_t c = 0; c < NCK; ++c) {
                    const float4 kc = *reinterpret_cast<const float4*>(&S.kn[4u * TPK * c + 4u * part]);
                    kf[4 * c + 0] = cur ? kc.x : f16_bits_to_f32(kr[c].x);
                    kf[4 * c + 1] = cur ? kc.y : f16_bits_to_f32(kr[c].x >> 16);
                    kf[4 * c + 2] = cur ? kc.z : f16_bits_to_f32(kr[c].y);
                    kf[4 * c + 3] = cur ? kc.w : f16_bits_to_f32(kr[c].y >> 16);
                }
                float d[NH];
#pragma unroll
                for (uint32_t h = 0; h < NH; ++h) {
                    float acc = 0.0f;
#pragma unroll
                    for (uint32_t c = 0; c < NCK; ++c) {
                        const float4 q = *reinterpret_cast<const float4*>(&S.qh[h][4u * TPK * c + 4u * part]);
                        acc = fmaf(q.x, kf[4 * c + 0], acc);
                        acc = fmaf(q.y, kf[4 * c + 1], acc);
                        acc = fmaf(q.z, kf[4 * c + 2], acc);
                        acc = fmaf(q.w, kf[4 * c + 3], acc);
                    }
                    d[h] = acc;
                }
                // key jk's lanes: half a DPP row (TPK 8), one (TPK 16), or two
                // (TPK 32: rows 2 r, 2 r + 1)
#pragma unroll
                for (uint32_t h = 0; h < NH; ++h) {
                    if constexpr (TPK == 8u) {
                        d[h] += dpp_f<0xB1, 0xF>(d[h], 0.0f);    // quad_perm [1,0,3,2]
                        d[h] += dpp_f<0x4E, 0xF>(d[h], 0.0f);    // quad_perm [2,3,0,1]
                        d[h] += dpp_f<0x141, 0xF>(d[h], 0.0f);   // row_half_mirror
                    } else {
                        d[h] = row16_sum(d[h]);
                    }
                    if constexpr (TPK == 32u)
                        d[h] += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(d[h]), 0x401F));
                }
                if (part == 0) {
#pragma unroll
                    for (uint32_t h = 0; h < NH; ++h) S.sc[jk][h] = valid ? d[h] * a.attn_scale : -INFINITY;
                }
            }
            __syncthreads();
            // chunk softmax, one wave per head
            if (wave < NH) {
                const uint32_t h = wave;
                const float v = S.sc[lane % CW][h];
                const bool in = lane < CW && v != -INFINITY;
                const float m = wave_max_ord(in ? v : -INFINITY);
                const float e = in ? exp_hw(v - m) : 0.0f;
                const float l2 = wave_sum(e);
                if (lane < CW) S.sc[lane][h] = e;
                if (lane == 0) { S.mh[h] = m; S.lh[h] = l2; }
            }
            __syncthreads();
            // weighted values (keys past the span have weight 0 and value 0)
            const uint32_t pb = uint32_t(lay.attp) + s_att * NH * (2u + kTkHD);
            {
                const float vc = S.vn[dv];
                float o[NH];
#pragma unroll
                for (uint32_t h = 0; h < NH; ++h) o[h] = 0.0f;
#pragma unroll
                for (uint32_t i = 0; i < HK; ++i) {
                    const uint32_t jl = kh * HK + i;
                    const float vr = kv0 + j0 + jl == pos ? vc : f16_bits_to_f32(vh[i]);
                    const float vv = j0 + jl < span ? vr : 0.0f;
                    float pr[NH];
                    if constexpr (NH % 4 == 0) {
#pragma unroll
                        for (uint32_t h4 = 0; h4 < NH; h4 += 4) {
                            const float4 q = *reinterpret_cast<const float4*>(&S.sc[jl][h4]);
                            pr[h4] = q.x; pr[h4 + 1] = q.y; pr[h4 + 2] = q.z; pr[h4 + 3] = q.w;
                        }
                    } else {
#pragma unroll
                        for (uint32_t h = 0; h < NH; ++h) pr[h] = S.sc[jl][h];
                    }
#pragma unroll
                    for (uint32_t h = 0; h < NH; ++h) o[h] = fmaf(pr[h], vv, o[h]);
                }
                // the other key half (lane ^ 32), then the neighbouring dim (lane ^ 1)
#pragma unroll
                for (uint32_t h = 0; h < NH; ++h) o[h] = add_xor32(o[h]);
                // chunk record: per head (max, sum of exp, unnormalised output[256]);
                // lane l stores dims (dv & ~1, dv | 1) of head 2 kh + (l & 1) (and
                // of the heads NH / 2 further on when NH > 4)
#pragma unroll
                for (uint32_t h0 = 0; h0 < NH; h0 += 4) {
                    // lanes l and l ^ 1 store different heads: each takes the
                    // value of the head it stores from its own registers and
                    // from the neighbour's (quad_perm xor 1, one per head)
                    const uint32_t hs = h0 + 2u * kh + (lane & 1u);
                    float mine = o[h0], nb = 0.0f;
#pragma unroll
                    for (uint32_t k = 0; k < 4; ++k) {
                        const float t = dpp_f<0xB1, 0xF>(o[h0 + k], 0.0f);
                        if (h0 + k == hs) { mine = o[h0 + k]; nb = t; }
                    }
                    {
                        const bool ev = (lane & 1u) == 0u;
                        const float r0 = ev ? mine : nb, r1 = ev ? nb : mine;
                        const uint32_t vo = (pb + hs * (2u + kTkHD) + 2u + (dv & ~1u)) * 8u;
                        if (xl_st) ll_st2_xcd(rr, vo, soff, r0, r1, tag);
                        else ll_st2(rr, vo, soff, r0, r1, tag);
                    }
                }
            }
            if (tid < NH) {
                const uint32_t vo = (pb + tid * (2u + kTkHD)) * 8u;
                if (xl_st) ll_st2_xcd(rr, vo, soff, S.mh[tid], S.lh[tid], tag);
                else ll_st2(rr, vo, soff, S.mh[tid], S.lh[tid], tag);
            }
            // the chunk holding the current position appends its key / value
            // to the caches for later tokens (after the results: stores)
            if (s_att == n_att - 1u && tid < kTkHD) {
                stg16(L.kc + size_t(pos) * kTkHD + tid, S.kn16[tid]);
                stg16(L.vc + size_t(pos) * kTkHD + tid, f32_to_f16_bits(S.vn[tid]));
            }
            __syncthreads();
        };
        // HPW query heads h0 .. h0 + HPW - 1 over keys c CW .. c CW + CW - 1
        // (head-split chunks: one head in local layers, a head pair in global
        // ones). Each head's record has the layout of the all-heads chunks'
        // (chunk c's entry for head h), so the combine is the same. The key
        // and value loads are shared by the HPW heads (one KV head).
        auto attend_heads = [&](auto hpw_c, auto cw_c, uint32_t h0, uint32_t c) {
            constexpr uint32_t HPW = decltype(hpw_c)::value;
            constexpr uint32_t CW = decltype(cw_c)::value;
            constexpr uint32_t TPK = kTkThreads / CW;        // threads per key (scores)
            constexpr uint32_t DPT = kTkHD / TPK;            // dims per thread
            constexpr uint32_t NKQ = kWave / 16u;            // key quarters (values)
            constexpr uint32_t KQ4 = CW / NKQ;               // keys per quarter
            constexpr uint32_t NCH = 4u / HPW;               // FMA chains per head
            static_assert(HPW == 1u || HPW == 2u, "one head or a head pair");
            constexpr uint32_t KPL = (CW + kWave - 1u) / kWave;   // keys per lane (softmax)
            static_assert(TPK == 4u || TPK == 8u || TPK == 16u, "a key's parts span a quad, half a DPP row or one");
            static_assert(HPW * CW <= sizeof(S.sc) / sizeof(float), "scores of the chunk's heads");
            static_assert(KQ4 % 4u == 0u, "a key quarter's weights are read as float4");
            static_assert(kTkHD == 32u * kTkWaves, "values: 16 dim pairs per wave");
            const uint32_t j0 = c * CW;
            const uint32_t jk = tid / TPK, part = tid % TPK;
            // the chunk's scores, then weights: [head][key] (a key quarter's
            // weights are read as float4: no bank conflicts)
            float* ps = &S.sc[0][0];
            // values: wave w, lane l: dims 2 dp, 2 dp + 1 (dp = 16 w + l % 16)
            // of keys kq KQ4 .. kq KQ4 + KQ4 - 1, kq = l / 16
            const uint32_t dp = 16u * wave + lane % 16u, kq = lane / 16u;
            // Rows are read up to the last appended one (span - 2): the key
            // and value loads read only rows this token attends to, the
            // current key (row span - 1, not yet appended) comes from LDS, and
            // every key from span - 1 on is weighted 0 in the value sum, its
            // loaded row being a finite context row. With span 1 the only key
            // is the current one and the loaded values are zeroed.
            // Key part p takes dims 4 TPK i + 4 p .. + 3 (i < DPT / 4): the
            // parts of a key read consecutive float4 of q (no LDS bank conflicts)
            const uint32_t rlast = span >= 2u ? span - 2u : 0u;
            u32x2 kr[DPT / 4u];
            uint32_t vw[KQ4];
            {
                const uint16_t* kp = L.kc + size_t(kv0 + min(j0 + jk, rlast)) * kTkHD + 4u * part;
#pragma unroll
                for (uint32_t i = 0; i < DPT / 4u; ++i) kr[i] = *(const XP_GLOBAL u32x2*)(kp + 4u * TPK * i);
            }
#pragma unroll
            for (uint32_t i = 0; i < KQ4; ++i)
                vw[i] = ldg32(L.vc + size_t(kv0 + min(j0 + kq * KQ4 + i, rlast)) * kTkHD + 2u * dp);
            if (span < 2u) {
#pragma unroll
                for (uint32_t i = 0; i < KQ4; ++i) vw[i] = 0u;
            }
            // waves 0 .. HPW - 1: the query heads, wave HPW: the key, wave
            // HPW + 1: the value (lane l holds elements 2 l, 2 l + 1, 2 l + 128,
            // 2 l + 129)
            float wqk[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (wave <= HPW) {
                const float* w = (wave < HPW ? L.norm[4] : L.norm[5]) + 2u * lane;
                const u32x2 w0 = *(const XP_GLOBAL u32x2*)(w);
                const u32x2 w1 = *(const XP_GLOBAL u32x2*)(w + kTkHD / 2u);
                wqk[0] = __uint_as_float(w0.x); wqk[1] = __uint_as_float(w0.y);
                wqk[2] = __uint_as_float(w1.x); wqk[3] = __uint_as_float(w1.y);
            }
            const uint32_t th = glob ? 1u : 0u;
            if (wave <= HPW + 1u) {
                uint32_t off[2];
                const bool act[2] = {true, true};
                u32x4 v[2];
                const uint32_t vec = wave < HPW ? h0 + wave : NH + wave - HPW;   // q heads, k, v
                const uint32_t p0 = uint32_t(lay.qkv) + vec * kTkHD + 2u * lane;
                off[0] = p0 * 8u;
                off[1] = (p0 + kTkHD / 2u) * 8u;
                ll_wait(rr, soff, off, act, v, tag, a.state, a.spin_limit);
                float e[4] = {__uint_as_float(v[0].x), __uint_as_float(v[0].z), __uint_as_float(v[1].x),
                              __uint_as_float(v[1].z)};
                if (wave <= HPW) {
                    float ss = e[0] * e[0] + e[1] * e[1] + e[2] * e[2] + e[3] * e[3];
                    ss = wave_sum(ss);
                    const float scale = rsq_hw(ss * (1.0f / float(kTkHD)) + eps);
#pragma unroll
                    for (int q = 0; q < 4; ++q) e[q] = e[q] * scale * (1.0f + wqk[q]);
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        const float cv = S.cs[th][2u * lane + q], sv = S.sn[th][2u * lane + q];
                        const float lo = e[q], hi = e[q + 2];
                        e[q] = lo * cv - hi * sv;
                        e[q + 2] = lo * sv + hi * cv;
                    }
                }
                own_kv_put(S, wave < HPW ? wave : NH + wave - HPW, NH, lane, e);
            }
            __syncthreads();
            t_in = tk_now(a);
            // scores: key jk, dims DPT part .. + DPT - 1, summed over the key's
            // TPK lanes (a quad, half a DPP row or one)
            {
                const uint32_t jj = j0 + jk;
                const bool valid = jj < span;
                // the current key's lanes take it from LDS, before the loop
                if (kv0 + jj == pos) {
#pragma unroll
                    for (uint32_t i = 0; i < DPT / 4u; ++i)
                        kr[i] = *reinterpret_cast<const u32x2*>(&S.kn16[4u * TPK * i + 4u * part]);
                }
                float dd[HPW][NCH];   // independent chains
#pragma unroll
                for (uint32_t hh = 0; hh < HPW; ++hh)
#pragma unroll
                    for (uint32_t r = 0; r < NCH; ++r) dd[hh][r] = 0.0f;
#pragma unroll
                for (uint32_t i = 0; i < DPT / 4u; ++i) {
                    const uint32_t d0 = 4u * TPK * i + 4u * part;
                    const u32x2 kb = kr[i];
                    const float k0 = f16_bits_to_f32(kb.x);
                    const float k1 = f16_bits_to_f32(kb.x >> 16);
                    const float k2 = f16_bits_to_f32(kb.y);
                    const float k3 = f16_bits_to_f32(kb.y >> 16);
#pragma unroll
                    for (uint32_t hh = 0; hh < HPW; ++hh) {
                        const float4 q = *reinterpret_cast<const float4*>(&S.qh[hh][d0]);
                        float& acc = dd[hh][i % NCH];
                        acc = fmaf(q.x, k0, acc);
                        acc = fmaf(q.y, k1, acc);
                        acc = fmaf(q.z, k2, acc);
                        acc = fmaf(q.w, k3, acc);
                    }
                }
#pragma unroll
                for (uint32_t hh = 0; hh < HPW; ++hh) {
                    float d = dd[hh][0];
#pragma unroll
                    for (uint32_t r = 1; r < NCH; ++r) d += dd[hh][r];
                    if constexpr (TPK <= 8u) {
                        d += dpp_f<0xB1, 0xF>(d, 0.0f);    // quad_perm [1,0,3,2]
                        d += dpp_f<0x4E, 0xF>(d, 0.0f);    // quad_perm [2,3,0,1]
                        if constexpr (TPK == 8u) d += dpp_f<0x141, 0xF>(d, 0.0f);   // row_half_mirror
                    } else {
                        d = row16_sum(d);
                    }
                    if (part == 0) ps[hh * CW + jk] = valid ? d * a.attn_scale : -INFINITY;
                }
            }
            __syncthreads();
            // the chunk's softmax: wave hh takes head hh, keys lane, lane + 64
            // (KPL per lane); the current key's weight is kept apart (S.pc)
            // and 0 in ps
            if (wave < HPW) {
                float v[KPL], e[KPL];
                float mv = -INFINITY;
#pragma unroll
                for (uint32_t k = 0; k < KPL; ++k) {
                    const uint32_t idx = k * kWave + lane;
                    v[k] = idx < CW ? ps[wave * CW + idx] : -INFINITY;
                    mv = fmaxf(mv, v[k]);
                }
                const float m = wave_max_ord(mv);
                float es = 0.0f;
#pragma unroll
                for (uint32_t k = 0; k < KPL; ++k) {
                    e[k] = v[k] != -INFINITY ? exp_hw(v[k] - m) : 0.0f;
                    es += e[k];
                }
                const float l2 = wave_sum(es);
                const uint32_t jc = pos - kv0 - j0;   // the current key's index, if < CW
                float pcur = 0.0f;
#pragma unroll
                for (uint32_t k = 0; k < KPL; ++k)
                    if (jc < CW && jc / kWave == k) pcur = __shfl(e[k], int(jc % kWave), kWave);
#pragma unroll
                for (uint32_t k = 0; k < KPL; ++k) {
                    const uint32_t idx = k * kWave + lane;
                    if (idx < CW) ps[wave * CW + idx] = idx == jc ? 0.0f : e[k];
                }
                if (lane == 0) { S.mh[wave] = m; S.lh[wave] = l2; S.pc[wave] = pcur; }
            }
            __syncthreads();
            {
                // loaded rows from span - 1 on have weight 0 (see the loads), so
                // the sum needs no selects: one fma with an fp16 operand per dim
                const float2 vc = *reinterpret_cast<const float2*>(&S.vn[2u * dp]);
#pragma unroll
                for (uint32_t hh = 0; hh < HPW; ++hh) {
                    float pw[KQ4];
#pragma unroll
                    for (uint32_t i = 0; i < KQ4; i += 4) {
                        const float4 q = *reinterpret_cast<const float4*>(&ps[hh * CW + kq * KQ4 + i]);
                        pw[i] = q.x; pw[i + 1] = q.y; pw[i + 2] = q.z; pw[i + 3] = q.w;
                    }
                    float oa[2] = {0.0f, 0.0f}, ob[2] = {0.0f, 0.0f};   // even / odd keys
#pragma unroll
                    for (uint32_t i = 0; i < KQ4; ++i) {
                        oa[i % 2u] = fmaf(pw[i], f16_bits_to_f32(vw[i]), oa[i % 2u]);
                        ob[i % 2u] = fmaf(pw[i], f16_bits_to_f32(vw[i] >> 16), ob[i % 2u]);
                    }
                    float o0 = oa[0] + oa[1], o1 = ob[0] + ob[1];
                    // the four key quarters: lanes l ^ 16 (swizzle within 32), l ^ 32
                    o0 += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(o0), 0x401F));
                    o1 += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(o1), 0x401F));
                    o0 = add_xor32(o0);
                    o1 = add_xor32(o1);
                    const float pcur = S.pc[hh];
                    o0 = fmaf(pcur, vc.x, o0);
                    o1 = fmaf(pcur, vc.y, o1);
                    if (kq == 0u) {
                        const uint32_t pb = uint32_t(lay.attp) + (c * NH + h0 + hh) * (2u + kTkHD);
                        const uint32_t vo = (pb + 2u + 2u * dp) * 8u;
                        if (xl_st) ll_st2_xcd(rr, vo, soff, o0, o1, tag);
                        else ll_st2(rr, vo, soff, o0, o1, tag);
                    }
                }
            }
            if (tid < HPW) {
                const uint32_t pb = uint32_t(lay.attp) + (c * NH + h0 + tid) * (2u + kTkHD);
                if (xl_st) ll_st2_xcd(rr, pb * 8u, soff, S.mh[tid], S.lh[tid], tag);
                else ll_st2(rr, pb * 8u, soff, S.mh[tid], S.lh[tid], tag);
            }
            // the first heads of the chunk holding the current position append
            // its key / value to the caches for later tokens
            if (h0 == 0u && c == n_att - 1u && tid < kTkHD) {
                stg16(L.kc + size_t(pos) * kTkHD + tid, S.kn16[tid]);
                stg16(L.vc + size_t(pos) * kTkHD + tid, f32_to_f16_bits(S.vn[tid]));
            }
            __syncthreads();
        };
        if (hsplit) {
            if (s_att < n_wga)
                attend_heads(std::integral_constant<uint32_t, 1u>{}, std::integral_constant<uint32_t, kHK>{},
                             s_att % NH, s_att / NH);
        } else if (gsplit) {
            if (s_att < n_wga) {
                if (g64)
                    attend_heads(std::integral_constant<uint32_t, 2u>{}, std::integral_constant<uint32_t, 64u>{},
                                 2u * (s_att % (NH / 2u)), s_att / (NH / 2u));
                else
                    attend_heads(std::integral_constant<uint32_t, 2u>{}, std::integral_constant<uint32_t, 128u>{},
                                 2u * (s_att % (NH / 2u)), s_att / (NH / 2u));
            }
        } else if (s_att < n_att) {
            if (cw == 16u) attend(std::integral_constant<uint32_t, 16u>{});
            else attend(std::integral_constant<uint32_t, kTkC>{});
        }
        tk_trace_stage(a, wg, l, 1u, t_in);
        t_in = 0;

        // ================= combine =================
        // Tile (h, d0): head h, CD dims from d0: 64 in local layers (16 tiles,
        // on the attention XCD when it exchanges there), 32 in global layers
        // (32 tiles): a global layer's span is up to 256 chunk records, and
        // halving each tile's share of them halves its fetch (measured: the
        // global combine 5.3 -> 4.2 us; local layers keep 64, whose O wait
        // grew with 32).
        auto combine = [&](auto cd_c) {
            constexpr uint32_t CD = decltype(cd_c)::value;
            constexpr uint32_t PP = 1u + CD / 2u;       // slot pairs per chunk: stats, then CD / 2
            constexpr uint32_t CS = 2u * PP;            // floats per chunk in big
            constexpr uint32_t NG = kTkThreads / CD;    // chunk groups of the weighted sum
            constexpr uint32_t NCB = NH * (kTkHD / CD);
            static_assert(NG * CD <= sizeof(S.red) / sizeof(float), "weighted-sum scratch");
            const uint32_t c0 = !xl ? t_comb : (rx % 8u == 0u ? rx / 8u : NCB);
            for (uint32_t c = c0; c < NCB; c += nwg) {
                const uint32_t h = c / (kTkHD / CD), d0 = (c % (kTkHD / CD)) * CD;
                const uint32_t rstride = NH * (2u + kTkHD);
                const uint32_t base = uint32_t(lay.attp) + h * (2u + kTkHD);
                // big[s CS + 0 / 1] = (max, sum of exp) of chunk s,
                // big[s CS + 2 + d] = its unnormalised output at dim d0 + d:
                // PP slot pairs per chunk, fetched 4 per thread at a time.
                const uint32_t np = n_att * PP;
                for (uint32_t b = 0; b < np; b += 4u * kTkThreads) {
                    uint32_t off[4];
                    bool act[4];
                    u32x4 v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint32_t i = b + uint32_t(r) * kTkThreads + tid;
                        act[r] = i < np;
                        const uint32_t ic = act[r] ? i : 0u;
                        const uint32_t s = ic / PP, e = ic % PP;
                        off[r] = (base + s * rstride + (e == 0u ? 0u : 2u + d0 + 2u * (e - 1u))) * 8u;
                    }
                    ll_wait(rr, soff, off, act, v, tag, a.state, a.spin_limit);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint32_t i = b + uint32_t(r) * kTkThreads + tid;
                        if (act[r])
                            *reinterpret_cast<float2*>(&S.big[2u * i]) =
                                float2{__uint_as_float(v[r].x), __uint_as_float(v[r].z)};
                    }
                }
                __syncthreads();
                if (c == c0) t_in = tk_now(a);
                // wave 0 forms the rescale factors exp(m_s - max m) and the
                // softmax denominator (chunk records <= a few hundred: lane
                // reductions, no block-wide ones)
                float* rl = RS();
                if (wave == 0) {
                    float m = -INFINITY;
                    for (uint32_t s = lane; s < n_att; s += kWave) m = fmaxf(m, S.big[s * CS]);
                    const float M = wave_max_ord(m);
                    float lsum = 0.0f;
                    for (uint32_t s = lane; s < n_att; s += kWave) {
                        const float f = exp_hw(S.big[s * CS] - M);
                        S.fm[s] = f;
                        lsum += f * S.big[s * CS + 1u];
                    }
                    lsum = wave_sum(lsum);
                    if (lane == 0) rl[0] = lsum;
                }
                __syncthreads();
                const float Ltot = rl[0];
                const uint32_t d = tid % CD, sg = tid / CD;
                float o = 0.0f;
                for (uint32_t s = sg; s < n_att; s += NG) o = fmaf(S.big[s * CS + 2u + d], S.fm[s], o);
                float* red = &S.red[0][0];
                red[sg * CD + d] = o;
                __syncthreads();
                if (sg == 0) {
                    float r = 0.0f;
#pragma unroll
                    for (uint32_t w = 0; w < NG; ++w) r += red[w * CD + d];
                    tile_put(rr, soff, uint32_t(lay.atto) + h * kTkHD + d0, r * rcp_hw(Ltot), lane, tag);
                }
                __syncthreads();
            }
        };
        if (glob) combine(std::integral_constant<uint32_t, kTkGlobalCD>{});
        else combine(std::integral_constant<uint32_t, 64u>{});
        tk_trace_stage(a, wg, l, 2u, t_in);
        t_in = 0;

        // ================= O projection =================
        for (uint32_t t = t_o; t < Sh::N_O; t += nwg) {
            // attention output [c QD / KO, (c + 1) QD / KO)
            uint32_t g, c, h;
            o_tile(t, g, c, h);
            constexpr uint32_t nb = Sh::OB;
            if (t != t_o) tile_prefetch<RO, Sh::SO>(po, L.w[3], L.s[3], QD / kBlk, H, g, h, c * nb, nb, wave, lane);
            TkW<RO>& p = po;
            tile_prep<FMT, RO, Sh::SO>(p, c * nb, nb, wave, lane);
            if (tid < Sh::QO / Sh::KO) {
                uint32_t off[kOwnP];
                bool act[kOwnP];
                u32x4 v[kOwnP];
#pragma unroll
                for (uint32_t j = 0; j < kOwnP; ++j) act[j] = true;
                own_offsets(off, uint32_t(lay.atto) + c * (QD / Sh::KO) + kOwn * tid);
                ll_wait(rr, soff, off, act, v, tag, a.state, a.spin_limit);
                float x[kOwn];
                own_unpack(x, v);
                own_stage(S, x, tid);
            }
            __syncthreads();
            if (t == t_o) t_in = tk_now(a);
            const float y = tile_dot<RO, Sh::SO>(p, S, nb, wave, lane);
            if (wave == 0)
                tile_put<Sh::SO>(rr, soff, uint32_t(lay.o) + c * H + g * kGrp + h * (kGrp / Sh::SO), y,
                                 lane, tag);
        }
        tk_trace_stage(a, wg, l, 3u, t_in);
        t_in = 0;

        // ================= gate / up =================
        TkW<RD> pdn;
        if (t_dn < Sh::N_DN) prefetch_dn(pdn, l, t_dn);
        for (uint32_t t = t_gu; t < Sh::N_GU; t += nwg) {
            // Tile t: ffn indices 32 t .. 32 t + 31 (column group g = t / 2,
            // half t % 2) of the gate (lanes 0..31) and the up projection
            // (lanes 32..63) over the whole k, so the tile ends with the
            // GeGLU of its 32 indices (gelu(gate) * up, llm_transformer.cl:213-231).
            const uint32_t g = t / 2u, cl = (t % 2u) * 32u + lane % 32u;
            const uint32_t m = lane < 32u ? 4u : 5u;
            TkW<RQ> p;
            {
                const u32x4* w = static_cast<const u32x4*>(L.w[m]);
                const u32x2* sc = static_cast<const u32x2*>(L.s[m]);
#pragma unroll
                for (int r = 0; r < RQ; ++r) {
                    const uint32_t b = min(wave + 8u * uint32_t(r), Sh::HB - 1u);
                    p.w[r] = ldg_stream4(w + (size_t(g) * Sh::HB + b) * kGrp + cl);
                    p.s[r] = ldg_stream2(sc + size_t(b / 4u) * FFN + g * kGrp + cl);
                }
            }
            tile_prep<FMT, RQ>(p, 0u, Sh::HB, wave, lane);
            float w_post[kOwn] = {}, w_in[kOwn] = {}, xa[kOwn] = {}, o[kOwn] = {};
            if (hown) {
                ld_own(w_post, L.norm[1] + kOwn * tid);
                ld_own(w_in, L.norm[2] + kOwn * tid);
            }
            // This wait spans QKV, attention, combine and O. Until the layer's
            // attention output exists (the combine stage's first pair, written
            // about two stages before the O partials) one thread polls it with
            // back-off; only then do the owners poll every input without
            // sleeping. Two hundred workgroups polling all their inputs for the
            // whole span load the fabric that the other stages' exchanges cross.
            if (tid == 0) {
                const uint32_t off1[1] = {uint32_t(lay.atto) * 8u};
                const bool act1[1] = {true};
                u32x4 v1[1];
                ll_wait<1, kGuSleep>(rr, soff, off1, act1, v1, tag, a.state, a.spin_limit);
            }
            __syncthreads();
            if (hown) {
                // xa (written in the QKV stage) first, then the o partials alone
                {
                    uint32_t off[kOwnP];
                    bool act[kOwnP];
                    u32x4 v[kOwnP];
#pragma unroll
                    for (uint32_t j = 0; j < kOwnP; ++j) act[j] = true;
                    own_offsets(&off[0], uint32_t(lay.xa) + kOwn * tid);
                    ll_wait(rr, soff, off, act, v, tag, a.state, a.spin_limit);
                    own_unpack(xa, &v[0]);
                }
                constexpr uint32_t NL = Sh::KO * kOwnP;
                uint32_t off[NL];
                bool act[NL];
                u32x4 v[NL];
#pragma unroll
                for (uint32_t j = 0; j < NL; ++j) act[j] = true;
#pragma unroll
                for (uint32_t c = 0; c < Sh::KO; ++c)
                    own_offsets(&off[kOwnP * c], uint32_t(lay.o) + c * H + kOwn * tid);
                ll_wait(rr, soff, off, act, v, tag, a.state, a.spin_limit);
                own_unpack(o, &v[0]);
#pragma unroll
                for (uint32_t c = 1; c < Sh::KO; ++c) {
                    float u[kOwn];
                    own_unpack(u, &v[kOwnP * c]);
#pragma unroll
                    for (uint32_t e = 0; e < kOwn; ++e) o[e] += u[e];
                }
            }
            float x[kOwn], xn[kOwn];
            own_residual<H>(x, xa, o, w_post, eps, RS());
            if (t == t_gu) t_in = tk_now(a);
            float* rsn = RS();
            own_norm_defer(xn, x, w_in, rsn);
            if (hown) own_stage(S, xn, tid);
            __syncthreads();
            float y = tile_dot<RQ, 1u>(p, S, Sh::HB, wave, lane);
            if (wave == 0) {
                y *= norm_scale<H>(rsn, eps);
                const float up = from_lane_plus32(y);   // lanes 0..31 use it
                const float hv = gelu_hw(y) * up;   // lanes 0..31: index 32 t + lane
                const float hn = dpp_f<0xB1, 0xF>(hv, 0.0f);
                if (lane < 32u && (lane & 1u) == 0u)
                    ll_st2(rr, (uint32_t(lay.gu) + 32u * t + lane) * 8u, soff, hv, hn, tag);
            }
            // x after the attention block, for the next layer: spread and stored last, as xa
            if (t < Sh::NOG && tid / (kGrp / kOwn) == t) own_put(rr, soff, uint32_t(lay.xb) + kOwn * tid, x, tag);
        }
        tk_trace_stage(a, wg, l, 4u, t_in);
        t_in = 0;

        // ================= down =================
        for (uint32_t t = t_dn; t < Sh::N_DN; t += nwg) {
            const uint32_t h = t % Sh::SD, tc = t / Sh::SD;
            const uint32_t g = tc / NCH, c = tc % NCH;
            const uint32_t q0 = Sh::DQ * c, nq = min(Sh::DQ, Sh::NQF - q0);
            const uint32_t nb = 4u * nq, k0 = 128u * q0;
            if (t != t_dn) prefetch_dn(pdn, l, t);
            if (t == t_dn && l + 1u < a.n_layers && t_qkv < Sh::N_QKV) prefetch_qkv(pq, l + 1u, t_qkv);
            tile_prep<FMT, RD, Sh::SD>(pdn, 4u * q0, nb, wave, lane);
            if (tid < nb * (kBlk / kOwn)) {
                // GeGLU output h of this chunk's k range (the gate/up tiles apply it)
                uint32_t off[kOwnP];
                bool act[kOwnP];
                u32x4 v[kOwnP];
#pragma unroll
                for (uint32_t j = 0; j < kOwnP; ++j) act[j] = true;
                own_offsets(&off[0], uint32_t(lay.gu) + k0 + kOwn * tid);
                ll_wait(rr, soff, off, act, v, tag, a.state, a.spin_limit);
                float hx[kOwn];
                own_unpack(hx, &v[0]);
                own_stage(S, hx, tid);
            }
            __syncthreads();
            if (t == t_dn) t_in = tk_now(a);
            const float y = tile_dot<RD, Sh::SD>(pdn, S, nb, wave, lane);
            if (wave == 0)
                tile_put<Sh::SD>(rr, soff, uint32_t(lay.dnp) + c * H + g * kGrp + h * (kGrp / Sh::SD), y,
                                 lane, tag);
        }
        if (t_dn >= Sh::N_DN && l + 1u < a.n_layers && t_qkv < Sh::N_QKV) prefetch_qkv(pq, l + 1u, t_qkv);
        tk_trace_stage(a, wg, l, 5u, t_in);
    }

    if (!a.want_logits) {
        if (wg == 0 && tid == 0) a.state[0] = pos + 1u;
        return;
    }

    // ================= final norm, lm_head, argmax =================
    const uint32_t ng = a.vocab / kGrp;
    const uint32_t gw = wg * kTkWaves + wave, nw = nwg * kTkWaves;
    constexpr uint32_t nqh = Sh::NQH;
    const u32x4* lmw = static_cast<const u32x4*>(a.lm_w);
    // Quad stream of this wave: groups gw, gw + nw, ...; k/128 quads each.
    const uint32_t my_groups = gw < ng ? (ng - gw + nw - 1u) / nw : 0u;
    const uint32_t nu = my_groups * nqh;
    // units in flight per wave (each 4 blocks of 64 columns: 18 VGPRs)
    constexpr int LD = kTkLmDepth;
    u32x4 w3[LD][4];
    u32x2 s3[LD];
    auto load_u = [&](int r, uint32_t u) {
        const uint32_t uc = min(u, nu - 1u);
        const uint32_t g = gw + (uc / nqh) * nw, q = uc % nqh;
        const u32x4* wp = lmw + (size_t(g) * Sh::HB + 4u * q) * kGrp + lane;
#pragma unroll
        for (int i = 0; i < 4; ++i) w3[r][i] = ldg_stream4(wp + i * kGrp);
        s3[r] = ldg_stream2(reinterpret_cast<const u32x2*>(a.lm_s) + size_t(q) * a.vocab +
                            g * kGrp + lane);
    };
    if (nu > 0) {
#pragma unroll
        for (int r = 0; r < LD; ++r) load_u(r, uint32_t(r));
    }
    float* rsn_lm;
    {
        float wf_post[kOwn] = {}, wf_in[kOwn] = {}, x[kOwn], xn[kOwn];
        if (hown) {
            ld_own(wf_post, S.lt[a.n_layers - 1u].norm[3] + kOwn * tid);
            ld_own(wf_in, a.final_norm + kOwn * tid);
        }
        after_ffn(x, a.n_layers - 1u, wf_post);
        rsn_lm = RS();
        own_norm_defer(xn, x, wf_in, rsn_lm);
        if (hown) own_stage(S, xn, tid);
        __syncthreads();
    }
    const float lm_scale = norm_scale<H>(rsn_lm, eps);
    float bv = -INFINITY;
    uint32_t bi = 0u;
    float acc = 0.0f;
    // the staged words of a block through the row's lanes (block_dot_bc)
    constexpr uint32_t NWL = 2u * kQxPlanes;
    const uint32_t jl = lane % 16u, jwl = jl >= NWL ? jl - NWL : jl;
    auto mul_u = [&](int r, uint32_t u) {
        const uint32_t q = u % nqh;
        u32x2 aw[4];
        float sxv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sxv[i] = S.sx[4u * q + i];
            aw[i] = reinterpret_cast<const u32x2*>(&S.qx[4u * q + i])[jwl];
        }
        // exec may have been written just before (see tile_dot)
#pragma unroll
        for (int i = 0; i < 4; ++i) asm volatile("s_nop 4" : "+v"(aw[i].x), "+v"(aw[i].y));
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
            const u32x4 w2[2] = {w3[r][i] ^ 0x88888888u, w3[r][i + 1] ^ 0x88888888u};
            const u32x2 a2[2] = {aw[i], aw[i + 1]};
            int32_t d[2];
            block_dot_bc<2>(w2, a2, d);
            acc = fmaf(tk_scale<FMT>(s3[r], i) * sxv[i], float(d[0]), acc);
            acc = fmaf(tk_scale<FMT>(s3[r], i + 1) * sxv[i + 1], float(d[1]), acc);
        }
        if (q == nqh - 1u) {
            const uint32_t j = (gw + (u / nqh) * nw) * kGrp + lane;
            acc *= lm_scale;
            a.logits[j] = acc;
            am_better(bv, bi, acc, j);
            acc = 0.0f;
        }
    };
    for (uint32_t u = 0; u < nu; u += LD) {
#pragma unroll
        for (int r = 0; r < LD; ++r) {
            if (u + r < nu) {
                mul_u(r, u + r);
                if (u + r + LD < nu) load_u(r, u + r + LD);
            }
        }
    }
    am_wave(bv, bi);
    if (lane == 0) { S.amv[wave] = bv; S.ami[wave] = bi; }
    __syncthreads();
    const uint32_t am_off = a.n_layers * lstride;   // argmax slots: (value, index) per workgroup
    if (tid == 0) {
        for (int w = 1; w < kTkWaves; ++w) am_better(bv, bi, S.amv[w], S.ami[w]);
        ll_st2(rr, 16u * wg, am_off, bv, __uint_as_float(bi), tag);
    }
    tk_trace(a, wg, 1u + 6u * a.n_layers);
    if (wg != 0) return;
    __syncthreads();   // tid 0 has read S.amv
    bv = -INFINITY;
    bi = 0u;
    for (uint32_t i0 = 0; i0 < nwg; i0 += 4u * kTkThreads) {
        uint32_t off[4];
        bool act[4];
        u32x4 v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t i = i0 + uint32_t(r) * kTkThreads + tid;
            act[r] = i < nwg;
            off[r] = 16u * (act[r] ? i : 0u);
        }
        ll_wait(rr, am_off, off, act, v, tag, a.state, a.spin_limit);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (act[r]) am_better(bv, bi, __uint_as_float(v[r].x), v[r].z);
    }
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
    tk_trace(a, wg, 2u + 6u * a.n_layers);
}

namespace {
// The shapes the kernel is built for.
using TkGemma3_1B = TkShape<1152, 6912, 4>;

const void* token_entry(uint32_t hidden, uint32_t ffn, uint32_t n_heads, int fmt) {
    if (hidden == TkGemma3_1B::H && ffn == TkGemma3_1B::FFN && n_heads == TkGemma3_1B::NH) {
        if (fmt == XP_SCALE_F16_QUAD)
            return reinterpret_cast<const void*>(token_kernel<TkGemma3_1B, XP_SCALE_F16_QUAD>);
        if (fmt == XP_SCALE_BF16_QUAD)
            return reinterpret_cast<const void*>(token_kernel<TkGemma3_1B, XP_SCALE_BF16_QUAD>);
    }
    return nullptr;
}
}  // namespace

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
    if (head_dim != kTkHD || n_kv_heads != 1)
        return set_error(XP_E_ARG, "token kernel: needs head_dim 256 and one kv head");
    if (fmt != XP_SCALE_F16_QUAD && fmt != XP_SCALE_BF16_QUAD)
        return set_error(XP_E_ARG, "token kernel: fp16 or bf16 quad scales only");
    if (!token_entry(hidden, ffn, n_heads, fmt))
        return set_error(XP_E_ARG,
                         "token kernel: built for hidden 1152, ffn 6912, 4 query heads (got %u, %u, %u)",
                         hidden, ffn, n_heads);
    if (vocab % kGrp)
        return set_error(XP_E_ARG, "token kernel: vocab must be a multiple of 64");
    if (uint64_t(max_seq + kTkC - 1u) / kTkC * 66u > uint64_t(kTkBig))
        return set_error(XP_E_ARG, "token kernel: stage scratch too small for max_seq %u", max_seq);
    if (n_layers == 0 || n_layers > uint32_t(kTkMaxLayers))
        return set_error(XP_E_ARG, "token kernel: at most %d layers", kTkMaxLayers);
    if (n_cu < 64 || n_cu > kTkMaxGrid || uint64_t(n_cu) * kTkC < max_seq)
        return set_error(XP_E_ARG, "token kernel: %d CUs cannot cover max_seq %u", n_cu, max_seq);
    const TokLL lay = tok_ll_layout(hidden, ffn, n_heads, head_dim, uint32_t(n_cu));
    if ((uint64_t(n_layers) * lay.layer + 2u * uint64_t(n_cu)) * 8u >= (1ull << 31))
        return set_error(XP_E_ARG, "token kernel: exchange slots exceed 2 GiB");
    return XP_OK;
}

// Each workgroup records the XCC (XCD) it runs on and whether the whole grid
// was resident at once: it takes an arrival ticket and waits, bounded, for
// the grid's last arrival (out[w] = XCC id | 0x100 when it saw every
// arrival). Launched exactly as the token kernel is (threads, LDS), so it
// sees the same placement and the same residency.
__global__ __launch_bounds__(kTkThreads) void grid_probe_kernel(uint32_t* out, uint32_t* count,
                                                                uint32_t spin_limit) {
    if (threadIdx.x == 0) {
        const uint32_t n = gridDim.x;
        (void)take_ticket(count);
        uint32_t seen = ld_dev(count), spins = 0;
        while (seen < n && ++spins < spin_limit) {
            __builtin_amdgcn_s_sleep(8);
            seen = ld_dev(count);
        }
        out[blockIdx.x] = xcc_id() | (seen >= n ? 0x100u : 0u);
    }
}

int probe_token_grid(uint32_t grid, hipStream_t st, uint32_t* out) {
    const size_t lds = tok_lds_bytes();
    const void* fn = reinterpret_cast<const void*>(&grid_probe_kernel);
    XP_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    uint32_t* d = nullptr;
    XP_HIP(hipMalloc(&d, size_t(grid + 1) * 4));
    uint32_t* count = d + grid;
    uint32_t limit = 1u << 18;                   // ~0.1 s of 512-cycle sleeps
    void* args[] = {&d, &count, &limit};
    hipError_t e = hipMemsetAsync(count, 0, 4, st);
    if (e == hipSuccess) e = hipLaunchKernel(fn, dim3(grid), dim3(kTkThreads), args, lds, st);
    if (e == hipSuccess) e = hipMemcpyAsync(out, d, size_t(grid) * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    (void)hipFree(d);
    if (e != hipSuccess) return set_error(XP_E_HIP, "token kernel: grid probe -> %s", hipGetErrorString(e));
    return XP_OK;
}

int tok_occupancy(uint32_t hidden, uint32_t ffn, uint32_t n_heads, int fmt, int* blocks_per_cu) {
    const void* fn = token_entry(hidden, ffn, n_heads, fmt);
    if (!fn) return set_error(XP_E_ARG, "token kernel: no build for this shape");
    const size_t lds = tok_lds_bytes();
    XP_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    XP_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, kTkThreads, lds));
    return XP_OK;
}

// A plain launch: the kernel needs its workgroups co-resident (one per CU,
// checked at session set-up by the occupancy query and the grid probe) but
// never waits at a grid barrier, so it needs no cooperative launch. Every
// wait in it is bounded, so a grid that is not resident after all (another
// kernel holding CUs) ends with a status error instead of hanging.
int launch_token(const TokArgs& a, uint32_t grid, hipStream_t st) {
    const void* fn = token_entry(a.hidden, a.ffn, a.n_heads, a.fmt);
    if (!fn) return set_error(XP_E_ARG, "token kernel: no build for this shape");
    // Raised once per kernel instance (the attribute is per function).
    static const void* attr_set[4] = {};
    const size_t lds = tok_lds_bytes();
    bool have = false;
    for (const void* f : attr_set) have |= f == fn;
    if (!have) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess)
            return set_error(XP_E_HIP, "token kernel: %zu B of LDS -> %s", lds,
                             hipGetErrorString(e));
        for (const void*& f : attr_set)
            if (!f) { f = fn; break; }
    }
    TokArgs copy = a;
    void* args[] = {&copy};
    hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(kTkThreads), args, lds, st);
    if (e != hipSuccess)
        return set_error(XP_E_HIP, "token kernel: launch of %u workgroups -> %s", grid,
                         hipGetErrorString(e));
    return XP_OK;
}

}  // namespace xp
