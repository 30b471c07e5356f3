// Device code of the split-span decode attention over the fp16 KV cache,
// shared by its kernel (transformer.hip) and the persistent batched step
// kernel (batch_step.hip).
#pragma once

#include "xp_device.hpp"
#include "xp_launch.hpp"

namespace xp {

// ---- decode attention (split-span, fp16 KV) ----------------------------------
// Grid: (nsplit, kv_heads, batch). Workgroup (s, g, b) takes a contiguous chunk
// of sequence b's attended keys for the G query heads that share kv head g,
// reading every key and value once for all G heads (the mq4 idea,
// llm_transformer.cl:418-464, 499-557), in passes of 16 U keys:
//   loads   32 lanes per 512-byte key row (16-byte loads, 8 dims per lane);
//           lane group kp = tid / 32 takes keys kp, kp + 16, ..., and all U
//           K and U V loads of a pass are in flight together
//   scores  each lane dots its 8 dims with the G query heads; the G x U
//           partial dots of a row group are summed by a reduce-scatter over
//           its 32 lanes (each swizzle step halving the values a lane holds),
//           so lane i ends with one (head, key) score
//   softmax one wave per head over the pass, online across passes (running
//           max and sum, the accumulated values rescaled by exp(m_old - m_new))
//   values  the same lanes accumulate p x v for their 8 dims, then the 16 row
//           groups are summed (lane pairs by permlane32 swap, waves through LDS)
// The query is loaded ahead of the first pass's K / V (and, fused, the raw
// q / k / v rows), so the scores wait for q and K while V is in flight.
// U (2, 4 or 8) follows the chunk length, so a 32-key chunk does a quarter
// of a 128-key pass's arithmetic. Up to 128 splits (at least 32 keys each)
// give most CUs a workgroup at one sequence's long spans (256 splits of 32
// keys and 64 of 128 measured slower at span 8192). Each split publishes
// (max, sum of exp, unnormalised o) per head, combined as
// softmax_rows_finish's online combine (llm_transformer.cl:385-405) in one
// of two ways:
//  * tickets (up to 16 splits, or some workgroups not resident at once): the
//    last workgroup of each group of 16 splits to arrive (arrival ticket)
//    rescales and sums the group into one record of the same form, and the
//    last group to arrive combines the group records, so no workgroup reads
//    more than 16 records; records are read with 16-byte device-scope loads
//    spread over all the combining workgroup's threads;
//  * exchange (more splits, every workgroup resident): records as tagged
//    16-byte pairs in a slice-major layout; each split polls its output
//    slice's pairs and its head's statistics in every record and combines
//    them wave-locally (see the exchange block below).
// Either way the sums run in a fixed order (deterministic).
constexpr int kAttnThreads  = 512;
constexpr int kAttnHD       = 256;                        // head_dim
constexpr int kAttnLanes    = kAttnHD / 8;                // lanes per key row
constexpr int kAttnRows     = kAttnThreads / kAttnLanes;  // 16 row groups
constexpr int kAttnMaxPass  = kAttnRows * 8;              // most keys per pass (U = 8)
constexpr int kAttnMinChunk = 32;                         // fewest keys per split
constexpr int kAttnMaxSplit = 256;                        // splits per (sequence, kv head)
constexpr uint32_t kAttnSplitCap = 128;                   // splits the launcher plans at most
constexpr int kAttnFan      = 16;                         // records one combine reads
constexpr int kAttnGroups   = kAttnMaxSplit / kAttnFan;   // level-1 records
constexpr int kAttnMaxG     = 4;                          // query heads per kv head
constexpr int kAttnStat     = 8;                          // floats of (max[4], sum[4]) per record

__host__ __device__ constexpr uint32_t attn_record(uint32_t G) { return kAttnStat + G * kAttnHD; }
// Records per (sequence, kv head): the splits', then the level-1 groups'.
constexpr uint32_t kAttnRecords = kAttnMaxSplit + kAttnGroups;
// Exchange-mode record: G pairs (max, sum of exp) then G * HD / 2 pairs of
// value dims, each pair a 16-byte (v0, tag, v1, tag) slot.
__host__ __device__ constexpr uint32_t attn_xrecord(uint32_t G) { return 4u * (G + G * kAttnHD / 2u); }
// Floats of one (sequence, kv head)'s records in either mode.
__host__ __device__ constexpr uint32_t attn_head_floats(uint32_t G) {
    return kAttnRecords * attn_record(G) > kAttnMaxSplit * attn_xrecord(G) ? kAttnRecords * attn_record(G)
                                                                          : kAttnMaxSplit * attn_xrecord(G);
}
// Exchange mode (at most kAttnSplitCap splits): output dims a split
// combines, the least power of two (at least 2) that covers G * HD over ns
// splits, so a slice never crosses a head. Lane l of a polling wave takes
// records l and l + 64; per record its head's statistics and HPW of the
// slice's value pairs, spread over all eight waves (measured faster than
// fewer waves polling more pairs each: their wave sums then run in series).
__host__ __device__ constexpr uint32_t attn_xdims(uint32_t G, uint32_t ns) {
    uint32_t D = 2u;
    while (D * ns < G * kAttnHD) D *= 2u;
    return D;
}
constexpr uint32_t kAttnXRec = kAttnSplitCap / 64u;   // records a lane
constexpr uint32_t kAttnXPer = 5;                     // pairs a lane polls per record
__host__ __device__ constexpr uint32_t attn_xpairs(uint32_t G, uint32_t ns) {   // HPW
    return (attn_xdims(G, ns) / 2u + 7u) / 8u;
}
static_assert(kAttnXRec == 2u && attn_xpairs(4, kAttnFan + 1) <= kAttnXPer - 1u,
              "exchange polling within one workgroup's waves");
// Floats of one (sequence, kv head)'s exchange records at ns splits: G HD / D
// slices of 1 + D / 2 tagged pairs (16 bytes) per split.
__host__ __device__ constexpr uint32_t attn_xfloats(uint32_t G, uint32_t ns) {
    return 4u * (G * kAttnHD / attn_xdims(G, ns)) * (1u + attn_xdims(G, ns) / 2u) * ns;
}
constexpr bool attn_xfits() {
    for (uint32_t G = 1; G <= uint32_t(kAttnMaxG); G *= 2u)
        for (uint32_t ns = kAttnFan + 1; ns <= kAttnSplitCap; ++ns)
            if (attn_xfloats(G, ns) > attn_head_floats(G)) return false;
    return true;
}
static_assert(attn_xfits(), "exchange records within the partials of a kv head");
constexpr uint32_t kAttnEpoch = kAttnEpochWord;     // ticket word: the last exchange launch's tag
constexpr uint32_t kAttnXErr  = kAttnXErrWord;      // ticket word: set when an exchange wait timed out
static_assert(kAttnTicketsPerHead == 3 + kAttnGroups && kAttnEpoch == 1 + kAttnGroups &&
              kAttnXErr == 2 + kAttnGroups, "tickets: level 2, one per group, epoch, flag");

template <int M>
__device__ __forceinline__ float swz_xor(float x) {   // x of lane ^ M within 32 lanes
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), (M << 10) | 0x1F));
}
// Reduce-scatter of v[0..N) over the 32 lanes of a row group, masks M, M/2 ..
// 1: each step keeps the lower (lane bit clear) or upper half of the values and
// adds the partner's copy of it; once one value is left it is summed plainly.
// Lane l ends with the sum of value (l % 32) / (32 / N) (N <= 32).
template <int N, int M>
__device__ __forceinline__ void reduce_scatter32(float* v, uint32_t lane) {
    if constexpr (M >= 1) {
        if constexpr (N >= 2) {
            constexpr int H = N / 2;
            const bool up = (lane & M) != 0;
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const float keep = up ? v[H + i] : v[i];
                const float send = up ? v[i] : v[H + i];
                v[i] = keep + swz_xor<M>(send);
            }
            reduce_scatter32<H, M / 2>(v, lane);
        } else {
            v[0] += swz_xor<M>(v[0]);
            reduce_scatter32<1, M / 2>(v, lane);
        }
    }
}

__device__ __forceinline__ void attn_range(const AttnArgs& a, uint32_t& span, uint32_t& kv0, uint32_t b) {
    if (a.pos_dev) {
        const uint32_t seq = a.pos_dev[b] + 1u;
        kv0 = (a.window == 0 || seq <= a.window) ? 0u : seq - a.window;
        span = seq - kv0;
    } else {
        span = a.span;
        kv0 = a.kv_start;
    }
}

__device__ __forceinline__ void f16x8(float (&f)[8], u32x4 w) {
    f[0] = f16_bits_to_f32(w.x); f[1] = f16_bits_to_f32(w.x >> 16);
    f[2] = f16_bits_to_f32(w.y); f[3] = f16_bits_to_f32(w.y >> 16);
    f[4] = f16_bits_to_f32(w.z); f[5] = f16_bits_to_f32(w.z >> 16);
    f[6] = f16_bits_to_f32(w.w); f[7] = f16_bits_to_f32(w.w >> 16);
}

// Combine n <= kAttnFan records (stride REC floats, in device memory) of
// kv head g: f_p = exp(m_p - M), L = sum_p l_p f_p, o = sum_p f_p o_p in
// record order. Final: out[h][d] = o / L. Else a record (M, L, o) at rec_out.
// Thread (r, col) loads float4 column col over records r, r + R, ...; wave h
// reads head h's statistics (one record per lane). All threads take part.
template <int G, bool DEV>
__device__ __forceinline__ void attn_combine(const float* recs, uint32_t n, bool final, float* out,
                                             float* rec_out, float (&red)[kAttnThreads / kWave][G * kAttnHD],
                                             float (&fs)[kAttnFan][G], float (&run)[3][G]) {
    constexpr int HD = kAttnHD;
    constexpr uint32_t REC = attn_record(G);
    constexpr int NCOL = G * HD / 4, R = kAttnThreads / NCOL, B = kAttnFan / R;
    static_assert(kAttnFan % R == 0, "records per thread");
    const int tid = int(DEV ? opaque_tid() : threadIdx.x), lane = tid % kWave,
              wave = int(__builtin_amdgcn_readfirstlane(uint32_t(tid) / kWave));
    const int col = tid % NCOL, r = tid / NCOL, h = col * 4 / HD;
    const rsrc_t rs = make_rsrc(recs, n * REC * 4u);
    const uint32_t off = (kAttnStat + col * 4) * 4u;
    u32x4 v[B];
#pragma unroll
    for (int i = 0; i < B; ++i) {
        const uint32_t p = r + i * R;
        v[i] = p < n ? ld_dev16(rs, p * REC * 4u + off) : u32x4{0u, 0u, 0u, 0u};
    }
    if (wave < G) {
        const int hh = wave;
        const bool live = uint32_t(lane) < n;
        const float m = live ? ld_dev(recs + size_t(lane) * REC + hh) : -INFINITY;
        const float l = live ? ld_dev(recs + size_t(lane) * REC + kAttnMaxG + hh) : 0.0f;
        const float mm = l > 0.0f ? m : -INFINITY;
        const float M = wave_max(mm);
        const float f = mm == -INFINITY ? 0.0f : exp_hw(mm - M);
        const float L = wave_sum(l * f);
        if (live) fs[lane][hh] = f;
        if (lane == 0) {
            run[0][hh] = M;
            run[1][hh] = L;
        }
    }
    __syncthreads();
    float4 acc = float4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < B; ++i) {
        const uint32_t p = r + i * R;
        const float f = p < n ? fs[p][h] : 0.0f;
        acc.x = fmaf(__uint_as_float(v[i].x), f, acc.x);
        acc.y = fmaf(__uint_as_float(v[i].y), f, acc.y);
        acc.z = fmaf(__uint_as_float(v[i].z), f, acc.z);
        acc.w = fmaf(__uint_as_float(v[i].w), f, acc.w);
    }
    reinterpret_cast<float4*>(&red[0][0])[r * NCOL + col] = acc;
    __syncthreads();
    if (tid < NCOL) {
        const float4* r4 = reinterpret_cast<const float4*>(&red[0][0]);
        float4 t = r4[tid];
#pragma unroll
        for (int q = 1; q < R; ++q) {
            const float4 u = r4[q * NCOL + tid];
            t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
        }
        const int hh = tid * 4 / HD;
        if (final) {
            const float inv = rcp_hw(run[1][hh]);
            st_u4<DEV>(reinterpret_cast<u32x4*>(out) + tid,
                       u32x4{__float_as_uint(t.x * inv), __float_as_uint(t.y * inv),
                             __float_as_uint(t.z * inv), __float_as_uint(t.w * inv)});
        } else {
            float* o = rec_out + kAttnStat + tid * 4;
            st_dev(o, t.x); st_dev(o + 1, t.y); st_dev(o + 2, t.z); st_dev(o + 3, t.w);
        }
    }
    if (!final && tid < G) {
        st_dev(rec_out + tid, run[0][tid]);
        st_dev(rec_out + kAttnMaxG + tid, run[1][tid]);
    }
}

template <int G, int U>
struct AttnSmem {
    float ps[G][kAttnRows * U];
    float run[3][G];                             // running max, running sum, pass rescale
    alignas(16) float red[kAttnThreads / kWave][G * kAttnHD];
    float fs[kAttnFan][G];
    uint32_t last;
};

// One workgroup of the decode attention: split s of kv head g of batched
// sequence b. Returns true when this workgroup wrote the final output of
// its (sequence, kv head) (the only split, the last combine to arrive, or in
// exchange mode a slice of it). DEV: the final output goes out with
// device-scope stores (read by other workgroups of the same launch).
template <int G, int U, bool FQ, bool DEV>
__device__ __forceinline__ bool attn_tile(AttnArgs a, const RopeFreq& f, uint32_t s, uint32_t g,
                                          uint32_t b, AttnSmem<G, U>& sm) {
    constexpr int HD = kAttnHD, NV = G * U, DUP = 32 / NV, PASS = kAttnRows * U;
    constexpr int PV = (PASS + kWave - 1) / kWave;           // softmax values per lane
    constexpr uint32_t REC = attn_record(G);
    static_assert(NV <= 32 && (32 % NV) == 0, "G x U partial dots over 32 lanes");
    auto& ps = sm.ps;
    auto& run = sm.run;
    auto& red = sm.red;
    auto& fs = sm.fs;
    uint32_t& last = sm.last;
    {   // batched sequence b
        a.q += size_t(b) * a.bq;
        a.out += size_t(b) * a.bq;
        a.kc += b * a.bcache;
        a.vc += b * a.bcache;
        if (a.part) a.part += b * a.bpart;
        if (a.tickets) a.tickets += size_t(b) * a.kv_heads * kAttnTicketsPerHead;
    }
    uint32_t span, kv0;
    attn_range(a, span, kv0, b);
    // exchange mode: the last launch's epoch, read before this workgroup's
    // record is written (see the combine); this launch's tag is one past it.
    // Requested here, used only there: nothing waits for it on the way.
    uint32_t xep = opaque_v(0u);
    if (a.xchg) xep = ld_dev(a.tickets + size_t(g) * kAttnTicketsPerHead + kAttnEpoch);
    uint32_t chunk = (span + a.nsplit - 1) / a.nsplit;
    if (chunk < uint32_t(kAttnMinChunk)) chunk = kAttnMinChunk;
    const uint32_t j0 = min(s * chunk, span);
    const int nk = int(min(j0 + chunk, span) - j0);
    const int tid = int(DEV ? opaque_tid() : threadIdx.x), lane = tid % kWave,
              wave = int(__builtin_amdgcn_readfirstlane(uint32_t(tid) / kWave));
    const int sub = tid % kAttnLanes, kp = tid / kAttnLanes;
    const size_t rowstride = size_t(a.kv_heads) * HD;   // fp16 elements per cache row
    const uint16_t* kbase = a.kc + size_t(kv0) * rowstride + size_t(g) * HD + sub * 8;
    const uint16_t* vbase = a.vc + size_t(kv0) * rowstride + size_t(g) * HD + sub * 8;
    // The last row a key of this split may read. With 128-key passes (U =
    // 8) over chunks that can be far shorter (a batch's short sequences),
    // the split's own last row, so the surplus keys re-read it from the
    // cache (config 5's global layers: 52 -> 34 MB fetched a step, 18.8 ->
    // 18.2 us a launch); with shorter passes the span's last row, the
    // surplus keys then reading the next split's rows (one sequence's
    // splits re-reading one row made its local-layer launch 8.3 -> 9.2 us).
    const uint32_t rlast = U >= 8 && nk > 0 ? j0 + uint32_t(nk) - 1u : (span > 0u ? span - 1u : 0u);

    // K / V of one pass: U keys per lane, all loads in flight together. The
    // loads are unconditional: a key past the split's chunk reads a clamped
    // row and is masked where it is used (score -inf, value words zero). Loads under the key test compiled to branches
    // whose merges waited for the loads (a copy of a loaded register inside
    // the branch), so a pass's later loads issued behind its earlier ones.
    u32x4 kw[U], vw[U];
    auto load_pass = [&](int c0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t r = min(j0 + uint32_t(c0 + kp + kAttnRows * u), rlast);
            kw[u] = ldg4(kbase + size_t(r) * rowstride);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t r = min(j0 + uint32_t(c0 + kp + kAttnRows * u), rlast);
            vw[u] = ldg4(vbase + size_t(r) * rowstride);
        }
    };
    float q[G][8], o[G][8];
    if constexpr (!FQ) {
        // q first: the scores then wait for q and K only, V still in flight
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float4* qp = reinterpret_cast<const float4*>(a.q + (size_t(g) * G + h) * HD + sub * 8);
            const float4 q0 = qp[0], q1 = qp[1];
            q[h][0] = q0.x; q[h][1] = q0.y; q[h][2] = q0.z; q[h][3] = q0.w;
            q[h][4] = q1.x; q[h][5] = q1.y; q[h][6] = q1.z; q[h][7] = q1.w;
        }
    }
    // fused QK-norm: the raw q / k / v rows and the norm weights are
    // requested first as well, so the norms and RoPE below run while the
    // first pass's keys and values are still in flight
    // (opaque zeros where a wave loads nothing, so that no use of the rows
    // is moved up to their loads, ahead of the K / V requests)
    const float z = opaque_v(0.0f);
    float e[4] = {z, z, z, z}, w4[4] = {z, z, z, z};
    if constexpr (FQ) {
        if (wave <= G + 1) {
            const float* src = wave < G   ? a.q_raw + size_t(b) * a.bq + (size_t(g) * G + wave) * HD
                               : wave == G ? a.k_raw + size_t(b) * a.bkv + size_t(g) * HD
                                           : a.v_raw + size_t(b) * a.bkv + size_t(g) * HD;
#pragma unroll
            for (int c = 0; c < 4; ++c) e[c] = src[lane + 64 * c];
            if (wave <= G) {
                const float* w = wave < G ? a.qw : a.kw;
#pragma unroll
                for (int c = 0; c < 4; ++c) w4[c] = w[lane + 64 * c];
            }
        }
    }
    // this thread's RoPE frequency (a kernel argument indexed by thread, so
    // a memory load), requested before the keys as well
    float inv_t = 0.0f;
    if constexpr (FQ) inv_t = f.inv[tid % (HD / 2)];
    load_pass(0);   // the first pass's keys do not depend on q

    // Fused QK-norm + RoPE (qk_norm_rope_append_kernel's arithmetic): waves
    // 0 .. G-1 norm and rotate query head g G + wave, wave G the key, wave
    // G + 1 rounds the value; lane l holds dims l + 64 c, so rotate-half pairs
    // (d, d + 128) are (c, c + 2) of one lane. q lands in red[0], cos / sin
    // in red[1], the fp16 key / value in red[2]; each thread then takes its
    // eight dims into registers (red is free again before the combine). The
    // raw rows (e, w4) were requested above, ahead of the first pass's K / V
    // loads, so waiting for them does not wait for the keys.
    u32x4 kcur = {0u, 0u, 0u, 0u}, vcur = {0u, 0u, 0u, 0u};
    if constexpr (FQ) {
        const uint32_t pos = kv0 + span - 1u;   // pos_dev[b], as attn_range read it
        float* cs = &red[1][0];
        uint16_t* kv16 = reinterpret_cast<uint16_t*>(&red[2][0]);   // key [0, HD), value [HD, 2 HD)
        {
            // every thread (frequency tid % (HD / 2)), the first HD / 2 store:
            // computed only where stored, the frequency's load was moved into
            // that branch, behind the keys, and waited for all of them
            float sv, cv;
            sincosf(float(pos) * inv_t, &sv, &cv);
            asm volatile("" ::"v"(sv), "v"(cv));
            if (tid < HD / 2) {
                cs[tid] = cv;
                cs[HD / 2 + tid] = sv;
            }
        }
        __syncthreads();
        if (wave <= G) {
            const float ss = wave_sum(e[0] * e[0] + e[1] * e[1] + e[2] * e[2] + e[3] * e[3]);
            const float scale = rsq_hw(ss * (1.0f / float(HD)) + a.eps);
#pragma unroll
            for (int c = 0; c < 4; ++c) e[c] = e[c] * scale * (1.0f + w4[c]);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const float cv = cs[lane + 64 * c], sv = cs[HD / 2 + lane + 64 * c];
                const float lo = e[c], hi = e[c + 2];
                e[c] = lo * cv - hi * sv;
                e[c + 2] = lo * sv + hi * cv;
            }
            if (wave < G) {
#pragma unroll
                for (int c = 0; c < 4; ++c) red[0][wave * HD + lane + 64 * c] = e[c];
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) kv16[lane + 64 * c] = f32_to_f16_bits(e[c]);
            }
        } else if (wave == G + 1) {
#pragma unroll
            for (int c = 0; c < 4; ++c) kv16[HD + lane + 64 * c] = f32_to_f16_bits(e[c]);
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float4 q0 = *reinterpret_cast<const float4*>(&red[0][h * HD + sub * 8]);
            const float4 q1 = *reinterpret_cast<const float4*>(&red[0][h * HD + sub * 8 + 4]);
            q[h][0] = q0.x; q[h][1] = q0.y; q[h][2] = q0.z; q[h][3] = q0.w;
            q[h][4] = q1.x; q[h][5] = q1.y; q[h][6] = q1.z; q[h][7] = q1.w;
        }
        kcur = *reinterpret_cast<const u32x4*>(kv16 + sub * 8);
        vcur = *reinterpret_cast<const u32x4*>(kv16 + HD + sub * 8);
        // the split holding the current position appends its key / value
        // for later steps (this launch reads them from kcur / vcur)
        if (span > 0 && (span - 1u) / chunk == s && tid < kAttnLanes) {
            const size_t row = size_t(pos) * rowstride + size_t(g) * HD + sub * 8;
            *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(a.kc) + row) = kcur;
            *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(a.vc) + row) = vcur;
        }
        __syncthreads();   // red is rewritten by the combine
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] = 0.0f;
    if (tid < G) {
        run[0][tid] = -INFINITY;
        run[1][tid] = 0.0f;
    }
    for (int c0 = 0; c0 < nk; c0 += PASS) {
        if (c0 > 0) load_pass(c0);
        if constexpr (FQ) {
            // the current position (the span's last key) from registers
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const bool cur = j0 + uint32_t(c0 + kp + kAttnRows * u) == span - 1u;
                kw[u] = cur ? kcur : kw[u];
                vw[u] = cur ? vcur : vw[u];
            }
        }
        // ---- scores
        float sv[NV];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float kf[8];
            f16x8(kf, kw[u]);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) d = fmaf(q[h][e], kf[e], d);
                sv[h * U + u] = d;
            }
        }
        reduce_scatter32<NV, 16>(sv, uint32_t(lane));
        {
            const int idx = (lane % 32) / DUP, h = idx / U, u = idx % U;
            const int j = kp + kAttnRows * u;
            if (lane % DUP == 0) ps[h][j] = (c0 + j < nk) ? sv[0] * a.scale : -INFINITY;
        }
        __syncthreads();
        // ---- softmax of the pass, online across passes: wave h takes head h
        if (wave < G) {
            const int h = wave;
            float sp[PV];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < PV; ++i) {
                const int idx = lane + kWave * i;
                sp[i] = idx < PASS ? ps[h][idx] : -INFINITY;
                mx = fmaxf(mx, sp[i]);
            }
            const float mold = run[0][h];
            const float mnew = fmaxf(mold, wave_max(mx));   // finite: key c0 is live
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < PV; ++i) {
                const int idx = lane + kWave * i;
                const float p = idx < PASS ? exp_hw(sp[i] - mnew) : 0.0f;
                if (idx < PASS) ps[h][idx] = p;
                sum += p;
            }
            sum = wave_sum(sum);
            if (lane == 0) {
                const float alpha = exp_hw(mold - mnew);   // 0 on the first pass
                run[0][h] = mnew;
                run[1][h] = run[1][h] * alpha + sum;
                run[2][h] = alpha;
            }
        }
        __syncthreads();
        // ---- weighted values
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float al = run[2][h];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[h][e] *= al;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = kp + kAttnRows * u;
            float vf[8];
            f16x8(vf, c0 + j < nk ? vw[u] : u32x4{0u, 0u, 0u, 0u});
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float p = ps[h][j];
#pragma unroll
                for (int e = 0; e < 8; ++e) o[h][e] = fmaf(p, vf[e], o[h][e]);
            }
        }
        __syncthreads();   // ps and run[2] are rewritten by the next pass
    }
    // ---- sum the 16 row groups: lane pairs (l, l + 32), then the 8 waves
    // v_permlane32_swap of values k and k + NO/2 (o flattened, NO = 8 G)
    // hands lane l < 32 the pair (o_k[l], o_k[l + 32]) and lane l + 32 the
    // pair of value k + NO/2, so one swap and one add sum two values and
    // every lane writes: lanes 0..31 the first half of the values, 32..63
    // the second (each sum in the order o[l] + o[l + 32]).
    {
        constexpr int NO = G * 8, NH2 = NO / 2;
        const float* of = &o[0][0];
        float sm2[NH2];
#pragma unroll
        for (int k = 0; k < NH2; ++k) {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(of[k]),
                                                            __float_as_uint(of[k + NH2]), false, false);
            sm2[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
        const int kb = lane < 32 ? 0 : NH2;
#pragma unroll
        for (int k = 0; k < NH2; k += 4) {
            const int kk = kb + k, h = kk / 8, e = kk % 8;
            *reinterpret_cast<float4*>(&red[wave][h * HD + sub * 8 + e]) =
                float4{sm2[k], sm2[k + 1], sm2[k + 2], sm2[k + 3]};
        }
    }
    __syncthreads();
    float* out = a.out + size_t(g) * G * HD;
    if (a.nsplit == 1) {
        for (int i = tid; i < G * HD; i += kAttnThreads) {
            float acc = 0.0f;
#pragma unroll
            for (int w = 0; w < kAttnThreads / kWave; ++w) acc += red[w][i];
            st_f<DEV>(out + i, acc / run[1][i / HD]);
        }
        return true;
    }
    uint32_t* tk = a.tickets + size_t(g) * kAttnTicketsPerHead;   // [0] level 2, [1 + grp] level 1
    if (a.xchg) {
        // ---- exchange mode (every workgroup of the launch resident at once):
        // each split publishes its record as tagged pairs, then polls, in
        // every record, its own slice of the value dims and the statistics
        // of the slice's head, and writes that slice of the output: one
        // exchange instead of the ticket chain. Split 0, once it has seen every record (so every
        // split has read the epoch), stores this launch's tag as the epoch.
        constexpr uint32_t NOUT = G * HD;
        const uint32_t xtag = xep + 1u != 0u ? xep + 1u : 1u;
        const uint32_t ns = a.nsplit;
        const uint32_t D = attn_xdims(G, ns);                      // output dims a slice
        const uint32_t NSC = NOUT / D, IT = 1u + D / 2u;           // slices, items a slice
        // Slice-major layout: item t of slice k of record r is the pair at
        // (k IT + t) ns + r (item 0: the slice head's statistics, 1 + c: value
        // dims 2c, 2c + 1 of the slice), so a poller reads each item of its
        // slice for 64 records as 1 KiB contiguous.
        float* xbase = a.part + size_t(g) * attn_head_floats(G);
        const rsrc_t xr = make_rsrc(xbase, NSC * IT * ns * 16u);
        for (uint32_t i = tid; i < NSC * IT; i += kAttnThreads) {
            const uint32_t k = i / IT, t = i % IT;
            float v0, v1;
            if (t == 0u) {
                const uint32_t h = k * D / HD;
                v0 = run[0][h];      // -inf for an empty split
                v1 = run[1][h];      // 0 for an empty split
            } else {
                const uint32_t d = k * D + 2u * (t - 1u);
                v0 = 0.0f;
                v1 = 0.0f;
#pragma unroll
                for (int w = 0; w < kAttnThreads / kWave; ++w) {
                    v0 += red[w][d];
                    v1 += red[w][d + 1u];
                }
            }
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(v0), xtag, __float_as_uint(v1), xtag},
                                                   xr, int((i * ns + s) * 16u), 0, kAuxDev);
        }
        if (s >= NSC) return false;
        const uint32_t d0 = s * D;
        // The slice's combine, wave by wave with no barrier: wave w takes value
        // pairs [c0, c1) of the slice (HPW a wave) in every record, and the
        // statistics of the slice's head. Lane l polls, for records l and
        // l + 64, slot (t, i) = record slot i's item 0 (statistics) for t = 0,
        // item 1 + c0 + t - 1 (value pair c0 + t - 1) for t >= 1.
        const uint32_t HP = D / 2u, HPW = attn_xpairs(G, ns);
        const uint32_t c0 = uint32_t(wave) * HPW, c1 = min(HP, c0 + HPW);
        if (c0 >= c1) return true;
        const uint32_t NI = 1u + (c1 - c0);
        constexpr int RPL = int(kAttnXRec), TP = int(kAttnXPer);
        uint32_t off[TP][RPL];
        bool act[TP][RPL];
#pragma unroll
        for (int t = 0; t < TP; ++t)
#pragma unroll
            for (int i = 0; i < RPL; ++i) {
                const uint32_t r = uint32_t(lane) + kWave * uint32_t(i);
                act[t][i] = r < ns && uint32_t(t) < NI;
                const uint32_t it = t == 0 ? 0u : 1u + c0 + uint32_t(t - 1);
                off[t][i] = act[t][i] ? ((s * IT + it) * ns + r) * 16u : 0u;
            }
        const u32x4 ready = {0u, xtag, 0u, xtag};
        u32x4 v[TP][RPL];
#pragma unroll
        for (int t = 0; t < TP; ++t)
#pragma unroll
            for (int i = 0; i < RPL; ++i) v[t][i] = act[t][i] ? ld_dev16(xr, off[t][i]) : ready;
        bool timed_out = false;
        for (uint32_t spins = 0;; ++spins) {
            bool ok = true;
#pragma unroll
            for (int t = 0; t < TP; ++t)
#pragma unroll
                for (int i = 0; i < RPL; ++i) ok &= (v[t][i].y == xtag) & (v[t][i].w == xtag);
            if (__builtin_amdgcn_ballot_w64(!ok) == 0ull) break;
            if (spins > a.spin_limit) {
                if (lane == 0) {
                    st_dev(tk + kAttnXErr, 1u);
                    if (a.status)
                        __hip_atomic_fetch_or((XP_GLOBAL uint32_t*)a.status, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
                }
                timed_out = true;
                break;
            }
            asm volatile("" ::: "memory");
#pragma unroll
            for (int t = 0; t < TP; ++t)
#pragma unroll
                for (int i = 0; i < RPL; ++i)
                    if (act[t][i] && ((v[t][i].y != xtag) | (v[t][i].w != xtag)))
                        v[t][i] = ld_dev16(xr, off[t][i]);
        }
        // Only after a complete wait: wave 0 of split 0 has then seen a pair
        // of every split's record, each stored after its split read the
        // epoch, so none can take the next launch's tag. After a timed-out
        // wait the epoch stays, the error word is set, and the tickets' owner
        // zeroes the records and the epoch before the next launch.
        if (s == 0 && wave == 0 && lane == 0 && !timed_out) st_dev(tk + kAttnEpoch, xtag);
        // M = max over records, factors exp(m_r - M) (0 for an empty
        // split), L = sum_r l_r f_r
        float fr[RPL];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            const float l = act[0][i] ? __uint_as_float(v[0][i].z) : 0.0f;
            fr[i] = l > 0.0f ? __uint_as_float(v[0][i].x) : -INFINITY;   // the max, for now
            mx = fmaxf(mx, fr[i]);
        }
        const float M = wave_max(mx);
        float ls = 0.0f;
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            fr[i] = fr[i] == -INFINITY ? 0.0f : exp_hw(fr[i] - M);
            if (act[0][i]) ls = fmaf(__uint_as_float(v[0][i].z), fr[i], ls);
        }
        const float inv = rcp_hw(wave_sum(ls));
        // value dims: per lane over its records in order, then the wave sum
#pragma unroll
        for (int t = 1; t < TP; ++t) {
            if (uint32_t(t) >= NI) break;
            float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
            for (int i = 0; i < RPL; ++i) {
                if (act[t][i]) {
                    acc0 = fmaf(fr[i], __uint_as_float(v[t][i].x), acc0);
                    acc1 = fmaf(fr[i], __uint_as_float(v[t][i].z), acc1);
                }
            }
            const float s0 = wave_sum(acc0), s1 = wave_sum(acc1);
            // a timed-out wait (the launch was not resident at once) leaves
            // NaN, not a plausible value, besides the flag word
            if (lane == 0) {
                const uint32_t d = d0 + 2u * (c0 + uint32_t(t - 1));
                st_f<DEV>(out + d, timed_out ? __builtin_nanf("") : s0 * inv);
                st_f<DEV>(out + d + 1u, timed_out ? __builtin_nanf("") : s1 * inv);
            }
        }
        return true;
    }
    float* part = a.part + size_t(g) * attn_head_floats(G);
    float* rec = part + size_t(s) * REC;
    for (int i = tid; i < G * HD; i += kAttnThreads) {
        float acc = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnThreads / kWave; ++w) acc += red[w][i];
        st_dev(rec + kAttnStat + i, acc);
    }
    if (tid < G) {
        st_dev(rec + tid, run[0][tid]);                 // -inf for an empty split
        st_dev(rec + kAttnMaxG + tid, run[1][tid]);     // 0 for an empty split
    }
    // ---- level 1: the last split of its group of kAttnFan combines the group
    const uint32_t grp = s / kAttnFan, ng = (a.nsplit + kAttnFan - 1) / kAttnFan;
    const uint32_t n1 = min(uint32_t(kAttnFan), a.nsplit - grp * kAttnFan);
    wait_mem();
    __syncthreads();
    if (tid == 0) last = take_ticket(&tk[1 + grp]);
    __syncthreads();
    if (last != n1 - 1) return false;
    if (tid == 0) st_dev(&tk[1 + grp], 0u);
    float* grec = part + size_t(kAttnMaxSplit + grp) * REC;
    attn_combine<G, DEV>(part + size_t(grp) * kAttnFan * REC, n1, ng == 1, out, grec, red, fs, run);
    if (ng == 1) return true;
    // ---- level 2: the last group combines the group records
    wait_mem();
    __syncthreads();
    if (tid == 0) last = take_ticket(&tk[0]);
    __syncthreads();
    if (last != ng - 1) return false;
    if (tid == 0) st_dev(&tk[0], 0u);
    attn_combine<G, DEV>(part + size_t(kAttnMaxSplit) * REC, ng, true, out, nullptr, red, fs, run);
    return true;
}

}  // namespace xp
