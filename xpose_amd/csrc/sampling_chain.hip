// The full-vocabulary sampling chain (kernels/llm_sampling.cl:130-225,
// 257-281, 349-386, 399-488): temperature, the strided-chain max / exp-sum
// softmax, per-chain top-k with rank selection, the top-k mask, top-p and the
// two multinomial draws. In the reference these are verified building blocks
// that decode does not call; here each is one gfx950 kernel behind an
// xp_<name> entry point with the reference's argument meaning.
//
// Every kernel evaluates what the reference evaluates in the same order:
// chain p is walked k = p, p + nparts, ... by one thread (consecutive threads
// take consecutive chains, so each step of the walk is one coalesced load
// across the wave), and the serial finalisers stay serial. Sums, comparisons,
// the division and the cumulative walks are therefore bit-identical to the
// reference's fp32 arithmetic on the same inputs; only exp (the device libm
// against llvmpipe's) can differ in the last bits.
//
// Where the reference's one-thread-per-chain form would hold a 64-entry array
// per thread (topk_partial), the array lives in LDS, column-major across the
// workgroup's threads so that a step of the insertion touches 64 different
// banks. rank selection stages the candidate list through LDS in tiles.
#include "xp_device.hpp"
#include "xp_launch.hpp"

namespace xp {

namespace {

constexpr uint32_t kScThreads = 256;
constexpr uint32_t kTopkMax = 64;          // XP_TOPK_MAX, llm_sampling.cl:255
constexpr uint32_t kTopkThreads = 64;      // one wave: 64 x 64 x 8 B = 32 KiB of LDS
constexpr uint32_t kRankTile = 2048;       // candidates staged per LDS tile
constexpr uint32_t kNone = 0xFFFFFFFFu;    // unfilled candidate slot

uint32_t blocks(uint32_t n, uint32_t per) { return (n + per - 1) / per; }

}  // namespace

__global__ __launch_bounds__(kScThreads) void temperature_kernel(float* x, float inv_temp, uint32_t n) {
    const uint32_t i = blockIdx.x * kScThreads + threadIdx.x;
    if (i < n) x[i] = x[i] * inv_temp;
}

__global__ __launch_bounds__(kScThreads) void reduce_max_partial_kernel(float* pmax, const float* x,
                                                                        uint32_t n, uint32_t nparts) {
    const uint32_t p = blockIdx.x * kScThreads + threadIdx.x;
    if (p >= nparts) return;
    float m = -INFINITY;
    for (uint32_t k = p; k < n; k += nparts) m = fmaxf(m, x[k]);
    pmax[p] = m;
}

// The maximum is the same in any order (fmax drops NaNs either way), so the
// finaliser is a parallel reduction.
__global__ __launch_bounds__(1024) void reduce_max_final_kernel(float* stats, const float* pmax,
                                                                uint32_t nparts) {
    __shared__ float wm[1024 / kWave];
    float m = -INFINITY;
    for (uint32_t p = threadIdx.x; p < nparts; p += 1024) m = fmaxf(m, pmax[p]);
    m = wave_max(m);
    if (threadIdx.x % kWave == 0) wm[threadIdx.x / kWave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 1024 / kWave; ++w) m = fmaxf(m, wm[w]);
        stats[0] = m;
    }
}

__global__ __launch_bounds__(kScThreads) void softmax_exp_partial_kernel(float* out, float* psum,
                                                                         const float* x,
                                                                         const float* stats,
                                                                         uint32_t n, uint32_t nparts) {
    const uint32_t p = blockIdx.x * kScThreads + threadIdx.x;
    if (p >= nparts) return;
    const float m = stats[0];
    float s = 0.0f;
    for (uint32_t k = p; k < n; k += nparts) {
        const float e = expf(x[k] - m);
        out[k] = e;
        s += e;
    }
    psum[p] = s;
}

__global__ __launch_bounds__(kScThreads) void reduce_sum_partial_kernel(float* out, const float* in,
                                                                        uint32_t n, uint32_t nparts) {
    const uint32_t p = blockIdx.x * kScThreads + threadIdx.x;
    if (p >= nparts) return;
    float s = 0.0f;
    for (uint32_t k = p; k < n; k += nparts) s += in[k];
    out[p] = s;
}

// Serial, as the reference: the fp32 sum depends on its order. The loads are
// issued 16 ahead; the adds stay in order.
__global__ void reduce_sum_final_kernel(float* stats, const float* psum, uint32_t nparts) {
    if (threadIdx.x != 0) return;
    float s = 0.0f;
    uint32_t p = 0;
    for (; p + 16 <= nparts; p += 16) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = psum[p + i];
#pragma unroll
        for (int i = 0; i < 16; ++i) s += v[i];
    }
    for (; p < nparts; ++p) s += psum[p];
    stats[1] = s;
}

__global__ __launch_bounds__(kScThreads) void softmax_normalize_kernel(float* out, const float* stats,
                                                                       uint32_t n) {
    const uint32_t i = blockIdx.x * kScThreads + threadIdx.x;
    if (i < n) out[i] = out[i] / stats[1];
}

// Chain p's best k (descending, strict '>' so the earliest index wins a tie),
// unfilled slots (-inf, none). bv / bi are [slot][thread] in LDS.
__global__ __launch_bounds__(kTopkThreads) void topk_partial_kernel(float* cval, uint32_t* cidx,
                                                                    const float* x, uint32_t n,
                                                                    uint32_t nparts, uint32_t k) {
    __shared__ float bv[kTopkMax][kTopkThreads];
    __shared__ uint32_t bi[kTopkMax][kTopkThreads];
    x += size_t(blockIdx.y) * n;                       // batched rows (grid.y)
    cval += size_t(blockIdx.y) * nparts * k;
    cidx += size_t(blockIdx.y) * nparts * k;
    const uint32_t t = threadIdx.x;
    const uint32_t p = blockIdx.x * kTopkThreads + t;
    for (uint32_t j = 0; j < k; ++j) { bv[j][t] = -INFINITY; bi[j][t] = kNone; }
    if (p >= nparts) return;
    float thr = -INFINITY;                       // bv[k - 1][t]
    for (uint32_t e = p; e < n; e += nparts) {
        const float v = x[e];
        if (!(v > thr)) continue;
        uint32_t j = k - 1u;
        while (j > 0u && v > bv[j - 1u][t]) {
            bv[j][t] = bv[j - 1u][t];
            bi[j][t] = bi[j - 1u][t];
            --j;
        }
        bv[j][t] = v;
        bi[j][t] = e;
        thr = bv[k - 1u][t];
    }
    for (uint32_t j = 0; j < k; ++j) {
        cval[size_t(p) * k + j] = bv[j][t];
        cidx[size_t(p) * k + j] = bi[j][t];
    }
}

// Candidate i's rank = number of filled candidates beating it by (value
// desc, index asc); rank < k writes out[rank]. Candidates pass through LDS in
// tiles that every thread of the workgroup scans.
__global__ __launch_bounds__(kScThreads) void topk_rank_select_kernel(float* oval, uint32_t* oidx,
                                                                      const float* cval,
                                                                      const uint32_t* cidx,
                                                                      uint32_t ncand, uint32_t k) {
    __shared__ float tv[kRankTile];
    __shared__ uint32_t ti[kRankTile];
    cval += size_t(blockIdx.y) * ncand;                 // batched rows (grid.y)
    cidx += size_t(blockIdx.y) * ncand;
    oval += size_t(blockIdx.y) * k;
    oidx += size_t(blockIdx.y) * k;
    const uint32_t i = blockIdx.x * kScThreads + threadIdx.x;
    const bool mine = i < ncand;
    const float v = mine ? cval[i] : -INFINITY;
    const uint32_t d = mine ? cidx[i] : kNone;
    uint32_t rank = 0;
    for (uint32_t base = 0; base < ncand; base += kRankTile) {
        const uint32_t m = min(kRankTile, ncand - base);
        __syncthreads();
        for (uint32_t j = threadIdx.x; j < m; j += kScThreads) {
            tv[j] = cval[base + j];
            ti[j] = cidx[base + j];
        }
        __syncthreads();
        for (uint32_t j = 0; j < m; ++j) {
            const float w = tv[j];
            const uint32_t e = ti[j];
            rank += (e != kNone) & ((w > v) | ((w == v) & (e < d)));
        }
    }
    if (mine && d != kNone && rank < k) {
        oval[rank] = v;
        oidx[rank] = d;
    }
}

__global__ __launch_bounds__(kScThreads) void topk_mask_kernel(float* logits, const float* topk_val,
                                                               uint32_t k, uint32_t n) {
    const uint32_t i = blockIdx.x * kScThreads + threadIdx.x;
    if (i >= n) return;
    const float t = topk_val[k - 1u];
    if (logits[i] < t) logits[i] = -INFINITY;
}

// One thread, serial over k (the reference's top-p is a single work-item).
__global__ void topp_cutoff_kernel(float* w, uint32_t k, float p) {
    if (threadIdx.x != 0) return;
    float total = 0.0f;
    for (uint32_t j = 0; j < k; ++j) total += w[j];
    if (!(total > 0.0f)) return;
    float cum = 0.0f;
    for (uint32_t j = 0; j < k; ++j) {
        if (cum >= p * total) w[j] = 0.0f;
        else cum += w[j];
    }
}

__global__ void multinomial_sample_kernel(float* out, uint32_t* idx_out, const float* w,
                                          const uint32_t* idx, uint32_t k, float u) {
    if (threadIdx.x != 0) return;
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
    out[0] = float(chosen);
    out[1] = cw;
    idx_out[0] = chosen;
}

__global__ void multinomial_strided_kernel(float* out, uint32_t* idx_out, const float* w,
                                           const float* psum, const float* stats, uint32_t n,
                                           uint32_t nparts, float u) {
    if (threadIdx.x != 0) return;
    const float target = u * stats[1];
    float cum = 0.0f;
    uint32_t chain = nparts - 1u;
    for (uint32_t p = 0; p < nparts; ++p) {
        const float s = psum[p];
        if (cum + s > target) { chain = p; break; }
        cum += s;
    }
    uint32_t chosen = chain;
    for (uint32_t e = chain; e < n; e += nparts) {
        chosen = e;
        cum += w[e];
        if (cum > target) break;
    }
    out[0] = float(chosen);
    out[1] = w[chosen];
    idx_out[0] = chosen;
}

// Exact best k of a candidate list, one workgroup per row: a most-significant-
// byte-first radix select finds the k-th largest (value, as an order-preserving
// key); the candidates at or above it (k plus any ties) are gathered in LDS and
// ranked among themselves by (value desc, index asc). Exact while fewer than
// 256 - k candidates tie with the k-th largest value. Logits share their top
// bytes, so most of a wave's keys fall in one bin: the histogram is kept in
// kSelCopies copies, lane l adding to copy l % kSelCopies (a bin's copies in
// consecutive words, different banks), which turns a 64-way same-address
// atomic into a 4-way one, and each thread adds a run of its keys that fall
// in one bin with one atomic; the copies are summed before the scan.
constexpr uint32_t kSelThreads = 1024;
constexpr uint32_t kSelPer = 16;             // candidates per thread (16384 per row)
constexpr uint32_t kSelKeep = 256;           // survivors ranked (k + ties)
static_assert(kTopkMax <= kSelKeep, "the ranked output fits the survivors' slots");
constexpr uint32_t kSelCopies = 16;          // histogram copies
constexpr uint32_t kSelStride = kSelCopies + 1u;   // words per bin (padded: the sum reads bins apart)

__device__ __forceinline__ uint32_t order_key(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(kSelThreads) void select_rows_kernel(float* oval, uint32_t* oidx,
                                                                  const float* cval,
                                                                  const uint32_t* cidx,
                                                                  uint32_t ncand, uint32_t k,
                                                                  uint32_t* pos_inc) {
    __shared__ uint32_t hcopy[256 * kSelStride];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t sel[3];               // prefix, needed, survivors
    __shared__ float sv[kSelKeep];
    __shared__ uint32_t si[kSelKeep];
    // the ranked output, written to oval / oidx once per slot at the end
    // (the outputs may be host memory, where two stores to one slot from
    // different waves need not land in order)
    __shared__ float ov[kSelKeep];
    __shared__ uint32_t oi[kSelKeep];
    const uint32_t r = blockIdx.x, tid = threadIdx.x;
    cval += size_t(r) * ncand;
    cidx += size_t(r) * ncand;
    if (tid < k) {   // slots no candidate reaches stay unfilled
        ov[tid] = -INFINITY;
        oi[tid] = kNone;
    }
    if (pos_inc && tid == 0) pos_inc[r] += 1u;
    // every candidate's value and index loaded at once (unconditionally, an
    // index past the end reads candidate 0), kept in registers for the gather
    uint32_t key[kSelPer], ci[kSelPer];
    float cv[kSelPer];
#pragma unroll
    for (uint32_t j = 0; j < kSelPer; ++j) {
        const uint32_t i = tid + j * kSelThreads;
        const uint32_t ic = i < ncand ? i : 0u;
        cv[j] = cval[ic];
        ci[j] = cidx[ic];
    }
#pragma unroll
    for (uint32_t j = 0; j < kSelPer; ++j) {
        const uint32_t i = tid + j * kSelThreads;
        key[j] = (i < ncand && ci[j] != kNone) ? order_key(cv[j]) : 0u;   // 0: below every value
    }
    uint32_t prefix = 0, mask = 0, need = k;
    const uint32_t copy = tid % kSelCopies;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (uint32_t i = tid; i < 256u * kSelStride; i += kSelThreads) hcopy[i] = 0;
        __syncthreads();
        {   // a thread's run of keys in one bin goes in with one atomic
            uint32_t rb = 0u, rn = 0u;
#pragma unroll
            for (uint32_t j = 0; j < kSelPer; ++j) {
                if (key[j] != 0u && (key[j] & mask) == prefix) {
                    const uint32_t bin = (key[j] >> shift) & 255u;
                    if (bin != rb) {
                        if (rn) atomicAdd(&hcopy[rb * kSelStride + copy], rn);
                        rb = bin;
                        rn = 0u;
                    }
                    ++rn;
                }
            }
            if (rn) atomicAdd(&hcopy[rb * kSelStride + copy], rn);
        }
        __syncthreads();
        if (tid < 256) {
            uint32_t c = 0;
#pragma unroll
            for (uint32_t q = 0; q < kSelCopies; ++q) c += hcopy[tid * kSelStride + q];
            hist[tid] = c;
        }
        __syncthreads();
        if (tid < kWave) {
            // lane l covers bins 255 - 4 l .. 252 - 4 l; inclusive prefix of
            // the lane counts from the top bin down, then the crossing lane
            // walks its own four bins
            const uint32_t l = tid;
            const uint32_t c0 = hist[255 - 4 * l], c1 = hist[254 - 4 * l], c2 = hist[253 - 4 * l],
                           c3 = hist[252 - 4 * l];
            const uint32_t mine = c0 + c1 + c2 + c3;
            uint32_t incl = mine;
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) {
                const uint32_t t = __shfl_up(incl, o, kWave);
                if (l >= uint32_t(o)) incl += t;
            }
            const uint32_t excl = incl - mine;
            if (excl < need && incl >= need) {   // exactly one lane
                uint32_t acc = excl, d = 255 - 4 * l;
                const uint32_t cs[4] = {c0, c1, c2, c3};
                for (int j = 0; j < 4; ++j) {
                    if (acc + cs[j] >= need) { d = 255 - 4 * l - j; break; }
                    acc += cs[j];
                }
                sel[0] = prefix | (d << shift);
                sel[1] = need - acc;
            }
            if (l == kWave - 1 && incl < need) {   // fewer than need keys: keep them all
                sel[0] = prefix;
                sel[1] = need;
            }
        }
        __syncthreads();
        prefix = sel[0];
        need = sel[1];
        mask |= 255u << shift;
        __syncthreads();
    }
    // prefix = the k-th largest key (or 0 when fewer than k candidates exist)
    if (tid == 0) sel[2] = 0;
    __syncthreads();
#pragma unroll
    for (uint32_t j = 0; j < kSelPer; ++j) {
        if (key[j] != 0u && key[j] >= prefix) {
            const uint32_t slot = atomicAdd(&sel[2], 1u);
            if (slot < kSelKeep) { sv[slot] = cv[j]; si[slot] = ci[j]; }
        }
    }
    __syncthreads();
    const uint32_t m = min(sel[2], kSelKeep);
    if (tid < m) {
        const float v = sv[tid];
        const uint32_t d = si[tid];
        uint32_t rank = 0;
        for (uint32_t j = 0; j < m; ++j) rank += (sv[j] > v) | ((sv[j] == v) & (si[j] < d));
        if (rank < k) {
            ov[rank] = v;
            oi[rank] = d;
        }
    }
    __syncthreads();
    if (tid < k) {
        oval[size_t(r) * k + tid] = ov[tid];
        oidx[size_t(r) * k + tid] = oi[tid];
    }
}

// The sample-first draw of a batched step on the device, one wave per
// sequence, in the host draw's arithmetic (session.cpp draw(), after
// decode.cpp:1893-1915), so that steps can follow each other with no host
// round trip: the candidates are select_rows' output, already in the host
// draw's (value desc, index asc) order; e = exp((v - max) / T) in float (the
// exponential in double, rounded once); the sums, the top-p cut and the
// inverse-CDF walk in double, in candidate order, on one lane; u from
// Philox4x32-10 (Salmon et al. 2011) at (seed, seq0 + row, step), 53 bits.
// Greedy (mode 0) takes candidate 0. Writes the token to tok[row] and to
// hist[(steps[row] % hist_cap) * rows + row], and advances steps[row] (in
// greedy mode a history counter only).
__device__ __forceinline__ void philox4x32_10_dev(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                                  uint32_t k0, uint32_t k1, uint32_t (&o)[4]) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
        const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
    }
    o[0] = c0;
    o[1] = c1;
    o[2] = c2;
    o[3] = c3;
}

__global__ __launch_bounds__(kWave) void draw_rows_kernel(const float* val, const uint32_t* idx, uint32_t k,
                                                          int mode, float temperature, uint32_t top_k,
                                                          float top_p, uint32_t seed, uint32_t seq0,
                                                          uint32_t* steps, uint32_t* tok, uint32_t* hist,
                                                          uint32_t hist_cap) {
    __shared__ float sv[kWave], se[kWave];
    __shared__ uint32_t si[kWave];
    const uint32_t row = blockIdx.x, lane = threadIdx.x, rows = gridDim.x;
    if (mode == 0) {
        if (lane == 0) {
            const uint32_t t = idx[size_t(row) * k];
            tok[row] = t;
            hist[(steps[row] % hist_cap) * rows + row] = t;
            steps[row] += 1u;   // the history slot only (greedy draws no uniform)
        }
        return;
    }
    // the valid candidates, compacted in order (the host skips empty slots)
    const float v = lane < k ? val[size_t(row) * k + lane] : -INFINITY;
    const uint32_t d = lane < k ? idx[size_t(row) * k + lane] : 0xFFFFFFFFu;
    const bool ok = d != 0xFFFFFFFFu;
    const unsigned long long m = __ballot(ok);
    const uint32_t at = uint32_t(__popcll(m & ((1ull << lane) - 1ull))), n = uint32_t(__popcll(m));
    if (ok) {
        sv[at] = v;
        si[at] = d;
    }
    __syncthreads();
    const float t = temperature > 0.0f ? temperature : 1.0f;
    const uint32_t kk = top_k ? min(top_k, n) : n;
    float maxl = -INFINITY;
    for (uint32_t i = 0; i < kk; ++i) maxl = maxl < sv[i] ? sv[i] : maxl;
    if (lane < kk) se[lane] = float(exp(double((sv[lane] - maxl) / t)));
    __syncthreads();
    if (lane != 0) return;
    uint32_t token = 0u;
    if (n > 0) {
        uint32_t nn = kk;
        double sum = 0.0;
        for (uint32_t i = 0; i < nn; ++i) sum += double(se[i]);
        if (top_p > 0.0f && top_p < 1.0f && sum > 0.0) {
            double acc = 0.0;
            const double cut = double(top_p) * sum;
            uint32_t keep = 0;
            for (; keep < nn; ++keep) {
                acc += double(se[keep]);
                if (acc >= cut) break;
            }
            nn = min(nn, keep + 1u);
            sum = 0.0;
            for (uint32_t i = 0; i < nn; ++i) sum += double(se[i]);
        }
        uint32_t o[4];
        philox4x32_10_dev(steps[row], 0u, 0u, 0u, seed, seq0 + row, o);
        const uint64_t bits = (uint64_t(o[0]) << 21) | (o[1] >> 11);
        const double u = double(bits) * (1.0 / 9007199254740992.0);
        double r = u * sum;
        token = si[nn - 1u];
        for (uint32_t i = 0; i < nn; ++i) {
            r -= double(se[i]);
            if (r <= 0.0) {
                token = si[i];
                break;
            }
        }
    }
    tok[row] = token;
    hist[(steps[row] % hist_cap) * rows + row] = token;
    steps[row] += 1u;
}

int launch_draw_rows(const float* val, const uint32_t* idx, uint32_t k, uint32_t rows, int mode,
                     float temperature, uint32_t top_k, float top_p, uint32_t seed, uint32_t seq0,
                     uint32_t* steps, uint32_t* tok, uint32_t* hist, uint32_t hist_cap, hipStream_t st) {
    if (k < 1 || k > uint32_t(kWave) || rows == 0 || hist_cap == 0)
        return set_error(XP_E_ARG, "draw rows: k=%u rows=%u hist_cap=%u", k, rows, hist_cap);
    hipLaunchKernelGGL(draw_rows_kernel, dim3(rows), dim3(kWave), 0, st, val, idx, k, mode, temperature,
                       top_k, top_p, seed, seq0, steps, tok, hist, hist_cap);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "draw rows: launch -> %s", hipGetErrorString(e));
    return XP_OK;
}

int launch_select_rows(float* oval, uint32_t* oidx, const float* cval, const uint32_t* cidx,
                       uint32_t ncand, uint32_t k, uint32_t rows, hipStream_t st, uint32_t* pos_inc) {
    if (k < 1 || k > kTopkMax || rows == 0 || ncand == 0 || ncand > kSelThreads * kSelPer)
        return set_error(XP_E_ARG, "select rows: k=%u rows=%u ncand=%u (<= %u)", k, rows, ncand,
                         kSelThreads * kSelPer);
    hipLaunchKernelGGL(select_rows_kernel, dim3(rows), dim3(kSelThreads), 0, st, oval, oidx, cval, cidx,
                       ncand, k, pos_inc);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(XP_E_HIP, "select rows: launch -> %s", hipGetErrorString(e));
    return XP_OK;
}

}  // namespace xp

using namespace xp;

#define XP_SC_LAUNCH(name) \
    do { \
        hipError_t e_ = hipGetLastError(); \
        if (e_ != hipSuccess) return set_error(XP_E_HIP, name ": launch -> %s", hipGetErrorString(e_)); \
        return XP_OK; \
    } while (0)

extern "C" {

int xp_apply_temperature(float* logits, float inv_temp, uint32_t n, xp_stream stream) {
    XP_REQUIRE(logits, "null pointer");
    XP_REQUIRE(n > 0, "n must be positive");
    XP_REQUIRE(std::isfinite(inv_temp), "inv_temp must be finite (route T == 0 to argmax)");
    hipLaunchKernelGGL(temperature_kernel, dim3(blocks(n, kScThreads)), dim3(kScThreads), 0,
                       as_stream(stream), logits, inv_temp, n);
    XP_SC_LAUNCH("xp_apply_temperature");
}

int xp_reduce_max_partial(float* pmax, const float* x, uint32_t n, uint32_t nparts,
                          xp_stream stream) {
    XP_REQUIRE(pmax && x, "null pointer");
    XP_REQUIRE(n > 0 && nparts > 0, "n and nparts must be positive");
    hipLaunchKernelGGL(reduce_max_partial_kernel, dim3(blocks(nparts, kScThreads)), dim3(kScThreads),
                       0, as_stream(stream), pmax, x, n, nparts);
    XP_SC_LAUNCH("xp_reduce_max_partial");
}

int xp_reduce_max_final(float* stats, const float* pmax, uint32_t nparts, xp_stream stream) {
    XP_REQUIRE(stats && pmax, "null pointer");
    XP_REQUIRE(nparts > 0, "nparts must be positive");
    hipLaunchKernelGGL(reduce_max_final_kernel, dim3(1), dim3(1024), 0, as_stream(stream), stats,
                       pmax, nparts);
    XP_SC_LAUNCH("xp_reduce_max_final");
}

int xp_softmax_exp_partial(float* out, float* psum, const float* x, const float* stats, uint32_t n,
                           uint32_t nparts, xp_stream stream) {
    XP_REQUIRE(out && psum && x && stats, "null pointer");
    XP_REQUIRE(n > 0 && nparts > 0, "n and nparts must be positive");
    hipLaunchKernelGGL(softmax_exp_partial_kernel, dim3(blocks(nparts, kScThreads)), dim3(kScThreads),
                       0, as_stream(stream), out, psum, x, stats, n, nparts);
    XP_SC_LAUNCH("xp_softmax_exp_partial");
}

int xp_reduce_sum_partial(float* out, const float* in, uint32_t n, uint32_t nparts,
                          xp_stream stream) {
    XP_REQUIRE(out && in, "null pointer");
    XP_REQUIRE(n > 0 && nparts > 0, "n and nparts must be positive");
    hipLaunchKernelGGL(reduce_sum_partial_kernel, dim3(blocks(nparts, kScThreads)), dim3(kScThreads),
                       0, as_stream(stream), out, in, n, nparts);
    XP_SC_LAUNCH("xp_reduce_sum_partial");
}

int xp_reduce_sum_final(float* stats, const float* psum, uint32_t nparts, xp_stream stream) {
    XP_REQUIRE(stats && psum, "null pointer");
    XP_REQUIRE(nparts > 0, "nparts must be positive");
    hipLaunchKernelGGL(reduce_sum_final_kernel, dim3(1), dim3(64), 0, as_stream(stream), stats, psum,
                       nparts);
    XP_SC_LAUNCH("xp_reduce_sum_final");
}

int xp_softmax_normalize(float* out, const float* stats, uint32_t n, xp_stream stream) {
    XP_REQUIRE(out && stats, "null pointer");
    XP_REQUIRE(n > 0, "n must be positive");
    hipLaunchKernelGGL(softmax_normalize_kernel, dim3(blocks(n, kScThreads)), dim3(kScThreads), 0,
                       as_stream(stream), out, stats, n);
    XP_SC_LAUNCH("xp_softmax_normalize");
}

int xp_topk_partial(float* cval, uint32_t* cidx, const float* x, uint32_t n, uint32_t nparts,
                    uint32_t k, xp_stream stream) {
    XP_REQUIRE(cval && cidx && x, "null pointer");
    XP_REQUIRE(n > 0 && nparts > 0, "n and nparts must be positive");
    XP_REQUIRE(k >= 1 && k <= kTopkMax, "k=%u must be in [1, %u]", k, kTopkMax);
    hipLaunchKernelGGL(topk_partial_kernel, dim3(blocks(nparts, kTopkThreads)), dim3(kTopkThreads), 0,
                       as_stream(stream), cval, cidx, x, n, nparts, k);
    XP_SC_LAUNCH("xp_topk_partial");
}

int xp_topk_rank_select(float* oval, uint32_t* oidx, const float* cval, const uint32_t* cidx,
                        uint32_t ncand, uint32_t k, xp_stream stream) {
    XP_REQUIRE(oval && oidx && cval && cidx, "null pointer");
    XP_REQUIRE(ncand > 0 && k > 0, "ncand and k must be positive");
    hipLaunchKernelGGL(topk_rank_select_kernel, dim3(blocks(ncand, kScThreads)), dim3(kScThreads), 0,
                       as_stream(stream), oval, oidx, cval, cidx, ncand, k);
    XP_SC_LAUNCH("xp_topk_rank_select");
}

int xp_topk_mask(float* logits, const float* topk_val, uint32_t k, uint32_t n, xp_stream stream) {
    XP_REQUIRE(logits && topk_val, "null pointer");
    XP_REQUIRE(n > 0 && k > 0, "n and k must be positive");
    hipLaunchKernelGGL(topk_mask_kernel, dim3(blocks(n, kScThreads)), dim3(kScThreads), 0,
                       as_stream(stream), logits, topk_val, k, n);
    XP_SC_LAUNCH("xp_topk_mask");
}

int xp_topp_cutoff(float* w, uint32_t k, float p, xp_stream stream) {
    XP_REQUIRE(w, "null pointer");
    XP_REQUIRE(k > 0, "k must be positive");
    hipLaunchKernelGGL(topp_cutoff_kernel, dim3(1), dim3(64), 0, as_stream(stream), w, k, p);
    XP_SC_LAUNCH("xp_topp_cutoff");
}

int xp_multinomial_sample(float* out, uint32_t* idx_out, const float* w, const uint32_t* idx,
                          uint32_t k, float u, xp_stream stream) {
    XP_REQUIRE(out && idx_out && w && idx, "null pointer");
    XP_REQUIRE(k > 0, "k must be positive");
    hipLaunchKernelGGL(multinomial_sample_kernel, dim3(1), dim3(64), 0, as_stream(stream), out, idx_out,
                       w, idx, k, u);
    XP_SC_LAUNCH("xp_multinomial_sample");
}

int xp_multinomial_strided(float* out, uint32_t* idx_out, const float* w, const float* psum,
                           const float* stats, uint32_t n, uint32_t nparts, float u,
                           xp_stream stream) {
    XP_REQUIRE(out && idx_out && w && psum && stats, "null pointer");
    XP_REQUIRE(n > 0 && nparts > 0 && nparts <= n, "need 0 < nparts <= n");
    hipLaunchKernelGGL(multinomial_strided_kernel, dim3(1), dim3(64), 0, as_stream(stream), out,
                       idx_out, w, psum, stats, n, nparts, u);
    XP_SC_LAUNCH("xp_multinomial_strided");
}

}  // extern "C"
