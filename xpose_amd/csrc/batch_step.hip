// EXPERIMENTAL (opt-in XP_EXEC_TOKEN; XP_EXEC_AUTO takes the graph, which
// measures faster: 1.2 vs 1.8 ms a config-5 step).
//
// The batched decode step (up to 16 sequences) as ONE
// persistent kernel on gfx950: every layer's q|k|v GEMM, attention (with
// QK-norm, RoPE and the KV append), o GEMM, residual + RMSNorm staging,
// gate|up GEMM with the GeGLU epilogue, down GEMM and staging, in the order
// of the reference's record_token (examples/llm/decode.cpp:1668-1752) run
// per sequence.
//
// The per-op path (batch.cpp's graph) launches one kernel per stage, 7 a
// layer; each launch pays its workgroups' dispatch, a cold weight request
// and a drain, 5-10 us for work whose weights stream in 0.1-1.1 us. Here one
// 512-thread workgroup per CU (the token kernel's grid, checked resident by
// the same probe) walks the stages in order and runs, in each, the tiles the
// per-op kernel would have run as workgroups (tile t on workgroup t mod
// grid), with the same device code (xp_bmm_device.hpp, xp_attn_device.hpp),
// so results are bit-identical to the per-op path.
//
// Hand-off: a tile writes its outputs with device-scope stores, waits for
// them to complete, and stores this launch's tag into its own flag word; a
// workgroup's first tile of a stage waits (bounded) until every flag of the
// stage before holds the tag, each thread re-reading one flag. (Counters
// that every tile adds to were measured slower: hundreds of device-scope
// atomics on one word serialise.) Every stage's outputs live in buffers
// of their own per layer, written once per launch and read only after their
// counter is complete, so a consumer's L2 cannot hold a stale copy from this
// launch (kernel boundaries write back and invalidate the L2s); its plain
// loads share the XCD's L2 like the per-op kernels' do. Waits only look
// back, every workgroup takes its tiles of a stage before moving on, and the
// grid is resident, so the walk cannot deadlock; a wait past the spin limit
// sets the status word, after which every wait gives up at once, so the grid
// always drains and the host reports XP_E_DEVICE. The tag is one past the
// last launch's, kept in device memory and advanced by the last workgroup
// to exit, so flags never need clearing.
#include "xp_attn_device.hpp"
#include "xp_bmm_device.hpp"

namespace xp {

namespace {

constexpr int kBsThreads = 512;
static_assert(kBsThreads == int(kBmmThreads) && kBsThreads == kAttnThreads,
              "every stage's tile takes the same workgroup shape");

// Tile scratch of the stages, one at a time.
union BsTileSmem {
    BmmSmem<4> g4;
    BmmSmem<1> g1;
    AttnSmem<4, 2> a2;
    AttnSmem<4, 4> a4;
    AttnSmem<4, 8> a8;
    float prep[2][kBsThreads / kWave];
};
struct BsSmem {
    BsTileSmem t;
};

// Waits (bounded) until the first n flags of a stage all hold this launch's
// tag: thread i re-reads flag i (device scope) and the workgroup ANDs the
// results, one barrier a round. Once the status word is set (or past the
// spin limit, which sets it) every wait gives up.
__device__ __forceinline__ void bs_wait(const BstepArgs& a, const uint32_t* flags, uint32_t n,
                                        uint32_t tag) {
    const uint32_t tid = threadIdx.x;
    for (uint32_t spins = 1;; ++spins) {
        const bool ok = tid >= n || ld_dev(flags + tid) == tag;
        if (__syncthreads_and(ok)) return;
        if (spins > a.spin_limit) {
            if (tid == 0)
                __hip_atomic_fetch_or((XP_GLOBAL uint32_t*)a.status, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        if ((spins & 63u) == 0u && __syncthreads_or(ld_dev(a.status) != 0u)) return;
        __builtin_amdgcn_s_sleep(1);
    }
}

// After a tile (device-scope stores of whatever it wrote): every thread's
// stores complete, then the tile's own flag takes the tag. No
// read-modify-write: hundreds of tiles adding to one counter serialise.
__device__ __forceinline__ void bs_signal(uint32_t* flag, uint32_t tag) {
    wait_mem();
    __syncthreads();
    if (threadIdx.x == 0) st_dev(flag, tag);
}

__device__ __forceinline__ void bs_trace(const BstepArgs& a, uint32_t l, uint32_t k, uint32_t e) {
    if (a.trace && threadIdx.x == 0)
        a.trace[(size_t(l * kBsStages + k) * 2u + e) * gridDim.x + blockIdx.x] = __builtin_amdgcn_s_memrealtime();
}

}  // namespace

template <int FMT>
__global__ __launch_bounds__(kBsThreads) void bstep_kernel(BstepArgs a) {
    extern __shared__ __align__(16) unsigned char bs_lds[];
    BsSmem& S = *reinterpret_cast<BsSmem*>(bs_lds);
    const uint32_t wg = blockIdx.x, nwg = gridDim.x;
    // this launch's tag: one past the last launch's, which the last
    // workgroup to exit stores (every workgroup has read it by then; after a
    // wait gave up, workgroup 0 may finish before others have started)
    const uint32_t ep = ld_dev(a.epoch);
    const uint32_t tag = ep + 1u != 0u ? ep + 1u : 1u;
    const uint32_t n_qkv = a.ncb_qkv, n_o = a.ncb_o, n_dn = a.ncb_dn * a.ns_dn;
    if (a.trace && threadIdx.x == 0)
        a.trace[size_t(a.n_layers) * kBsStages * 2u * nwg + wg] = __builtin_amdgcn_s_memrealtime();

    for (uint32_t l = 0; l < a.n_layers; ++l) {
        const BstepLayer* Lp = a.layers + l;
        const BstepLayer& L = *Lp;
        const uint32_t n_att = L.n_att;
        uint32_t* fl = a.flags + size_t(l) * kBsStages * kBsMaxTiles;   // [stage][tile]
        uint32_t* fprev = l > 0 ? fl - kBsMaxTiles : nullptr;           // the previous layer's last stage
        // q|k|v (operand staged by the previous layer's last stage, or, in
        // layer 0, by the launch before this one)
        for (uint32_t t = wg; t < n_qkv; t += nwg) {
            if (t == wg && l > 0) bs_wait(a, fprev, a.batch, tag);
            if (t == wg) bs_trace(a, l, 0, 0);
            __syncthreads();
            (void)bmm_tile<FMT, 1, 0, false, true>(Lp->qkv, t, 0u, n_qkv, S.t.g1);
            bs_signal(fl + 0 * kBsMaxTiles + t, tag);
            if (t + nwg >= n_qkv) bs_trace(a, l, 0, 1);
        }
        // attention over each sequence's own cache
        for (uint32_t t = wg; t < n_att; t += nwg) {
            if (t == wg) bs_wait(a, fl + 0 * kBsMaxTiles, n_qkv, tag);
            if (t == wg) bs_trace(a, l, 1, 0);
            __syncthreads();
            const RopeFreq& f = a.rope[L.att_rope];
            const uint32_t ns = L.att.nsplit, kvh = L.att.kv_heads;
            const uint32_t s = t % ns, g = (t / ns) % kvh, b = t / (ns * kvh);
            if (L.att_u == 2u) (void)attn_tile<4, 2, true, true>(Lp->att, f, s, g, b, S.t.a2);
            else if (L.att_u == 4u) (void)attn_tile<4, 4, true, true>(Lp->att, f, s, g, b, S.t.a4);
            else (void)attn_tile<4, 8, true, true>(Lp->att, f, s, g, b, S.t.a8);
            bs_signal(fl + 1 * kBsMaxTiles + t, tag);
            if (t + nwg >= n_att) bs_trace(a, l, 1, 1);
        }
        // o projection (operand staged from the attention output in the tile);
        // every attention tile done means every combine done
        for (uint32_t t = wg; t < n_o; t += nwg) {
            if (t == wg) bs_wait(a, fl + 1 * kBsMaxTiles, n_att, tag);
            if (t == wg) bs_trace(a, l, 2, 0);
            __syncthreads();
            (void)bmm_tile<FMT, 1, 2, false, true>(Lp->o, t, 0u, n_o, S.t.g1);
            bs_signal(fl + 2 * kBsMaxTiles + t, tag);
            if (t + nwg >= n_o) bs_trace(a, l, 2, 1);
        }
        // x += rmsnorm(o) (1 + w), staged as rmsnorm(x) (1 + w') for gate|up
        for (uint32_t t = wg; t < a.batch; t += nwg) {
            if (t == wg) bs_wait(a, fl + 2 * kBsMaxTiles, n_o, tag);
            if (t == wg) bs_trace(a, l, 3, 0);
            __syncthreads();
            prep_row<kBsThreads, true>(Lp->prep1, t, S.t.prep);
            bs_signal(fl + 3 * kBsMaxTiles + t, tag);
            if (t + nwg >= a.batch) bs_trace(a, l, 3, 1);
        }
        // gate|up with the GeGLU epilogue staging the down operand
        for (uint32_t t = wg; t < a.n_gu; t += nwg) {
            if (t == wg) bs_wait(a, fl + 3 * kBsMaxTiles, a.batch, tag);
            if (t == wg) bs_trace(a, l, 4, 0);
            __syncthreads();
            (void)bmm_tile<FMT, 4, 0, true, true>(Lp->gu, t, 0u, a.n_gu, S.t.g4);
            bs_signal(fl + 4 * kBsMaxTiles + t, tag);
            if (t + nwg >= a.n_gu) bs_trace(a, l, 4, 1);
        }
        // down, k split; the last split of a column block writes it (every
        // split done means every column block written)
        for (uint32_t t = wg; t < n_dn; t += nwg) {
            if (t == wg) bs_wait(a, fl + 4 * kBsMaxTiles, a.n_gu, tag);
            if (t == wg) bs_trace(a, l, 5, 0);
            __syncthreads();
            (void)bmm_tile<FMT, 1, 0, false, true>(Lp->dn, t % a.ncb_dn, t / a.ncb_dn, a.ncb_dn, S.t.g1);
            bs_signal(fl + 5 * kBsMaxTiles + t, tag);
            if (t + nwg >= n_dn) bs_trace(a, l, 5, 1);
        }
        // x += rmsnorm(down) (1 + w), staged for the next layer (or the lm_head)
        for (uint32_t t = wg; t < a.batch; t += nwg) {
            if (t == wg) bs_wait(a, fl + 5 * kBsMaxTiles, n_dn, tag);
            if (t == wg) bs_trace(a, l, 6, 0);
            __syncthreads();
            prep_row<kBsThreads, true>(Lp->prep2, t, S.t.prep);
            bs_signal(fl + 6 * kBsMaxTiles + t, tag);
            if (t + nwg >= a.batch) bs_trace(a, l, 6, 1);
        }
    }
    wait_mem();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t done = __hip_atomic_fetch_add((XP_GLOBAL uint32_t*)a.exit_cnt, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        if (done == nwg - 1u) {
            st_dev(a.exit_cnt, 0u);
            st_dev(a.epoch, tag);
        }
    }
}

int launch_bstep(const BstepArgs& a, int fmt, uint32_t grid, hipStream_t st) {
    if (fmt != XP_SCALE_F16_QUAD && fmt != XP_SCALE_BF16_QUAD)
        return set_error(XP_E_ARG, "batch step: fp16 or bf16 quad scales");
    const size_t lds = tok_lds_bytes();   // the token kernel's: one workgroup per CU, the same probe
    static_assert(sizeof(BsSmem) <= 96 * 1024, "batch step LDS");
    const void* fn = fmt == XP_SCALE_F16_QUAD ? reinterpret_cast<const void*>(&bstep_kernel<XP_SCALE_F16_QUAD>)
                                              : reinterpret_cast<const void*>(&bstep_kernel<XP_SCALE_BF16_QUAD>);
    XP_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    BstepArgs args = a;
    void* kargs[] = {&args};
    const hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(kBsThreads), kargs, lds, st);
    if (e != hipSuccess) return set_error(XP_E_HIP, "batch step: launch -> %s", hipGetErrorString(e));
    return XP_OK;
}

// One workgroup per CU of the step kernel fits: the occupancy query.
int bstep_occupancy(int fmt, int* blocks_per_cu) {
    const size_t lds = tok_lds_bytes();
    const void* fn = fmt == XP_SCALE_F16_QUAD ? reinterpret_cast<const void*>(&bstep_kernel<XP_SCALE_F16_QUAD>)
                                              : reinterpret_cast<const void*>(&bstep_kernel<XP_SCALE_BF16_QUAD>);
    XP_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    XP_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, kBsThreads, lds));
    return XP_OK;
}

}  // namespace xp
