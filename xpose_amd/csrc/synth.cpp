// Counter-based synthetic inputs for the decode path (host side).
//
// The reference draws its test data from std::mt19937 streams
// (examples/llm/kernel_tests.cpp:136-142, decode.cpp:2466-2476), which cannot
// regenerate one element without replaying the stream. These generators are
// counter-based instead — Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel
// random numbers: as easy as 1, 2, 3", SC'11) — so any element of any tensor
// is a pure function of (seed, tensor id, element index) and the work splits
// over threads with no shared state.
#include "xp_internal.hpp"

#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace xp {
namespace {

inline void mulhilo(uint32_t a, uint32_t b, uint32_t& hi, uint32_t& lo) {
    const uint64_t p = uint64_t(a) * uint64_t(b);
    hi = uint32_t(p >> 32);
    lo = uint32_t(p);
}

inline void philox(const uint32_t c_in[4], const uint32_t k_in[2], uint32_t out[4]) {
    uint32_t c0 = c_in[0], c1 = c_in[1], c2 = c_in[2], c3 = c_in[3];
    uint32_t k0 = k_in[0], k1 = k_in[1];
    for (int r = 0; r < 10; ++r) {
        if (r) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        uint32_t hi0, lo0, hi1, lo1;
        mulhilo(0xD2511F53u, c0, hi0, lo0);
        mulhilo(0xCD9E8D57u, c2, hi1, lo1);
        const uint32_t n0 = hi1 ^ c1 ^ k0;
        const uint32_t n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

// (x + 0.5) / 2^32: uniform on the open interval (0, 1).
inline double u01(uint32_t x) { return (double(x) + 0.5) * (1.0 / 4294967296.0); }

// Box-Muller, first output only: sqrt(-2 ln u1) * cos(2 pi u2).
inline double normal_at(uint64_t i, uint32_t stream, uint32_t seed, uint32_t tensor) {
    const uint32_t c[4] = {uint32_t(i), uint32_t(i >> 32), stream, 0u};
    const uint32_t k[2] = {seed, tensor};
    uint32_t o[4];
    philox(c, k, o);
    const double u1 = u01(o[0]), u2 = u01(o[1]);
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586476925 * u2);
}

template <class F>
void parallel_for(size_t n, F&& f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 16) nt = 16;
    if (n < (size_t(1) << 16) || nt == 1) {
        f(size_t(0), n);
        return;
    }
    std::vector<std::thread> th;
    const size_t per = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const size_t a = t * per, b = std::min(n, a + per);
        if (a >= b) break;
        th.emplace_back([&f, a, b] { f(a, b); });
    }
    for (auto& x : th) x.join();
}

}  // namespace

uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return uint16_t(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) return uint16_t(sign | 0x7C00u);   // >= 65520 rounds to inf
    if (ax >= 0x38800000u) {                                   // normal fp16
        uint32_t r = ax - ((127u - 15u) << 23);
        r = (r + 0x0FFFu + ((r >> 13) & 1u)) >> 13;
        return uint16_t(sign | r);
    }
    if (ax <= 0x33000000u) return uint16_t(sign);              // <= 2^-25 rounds to 0
    // Subnormal fp16: value / 2^-24 rounded to nearest even.
    const uint32_t e = ax >> 23;
    const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - e;                            // 14..24
    uint32_t m = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (m & 1u))) ++m;
    return uint16_t(sign | m);
}

}  // namespace xp

using namespace xp;

extern "C" {

void xp_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    philox(ctr, key, out);
}

uint16_t xp_f32_to_f16(float f) { return f32_to_f16(f); }

int xp_synth_nibbles(uint32_t* wq, uint32_t rows, uint32_t cols, uint32_t seed,
                     uint32_t tensor_id) {
    XP_REQUIRE(wq != nullptr, "wq is null");
    XP_REQUIRE(rows % 32 == 0 && cols % 64 == 0 && rows && cols,
               "rows=%u must be a multiple of 32 and cols=%u a multiple of 64", rows, cols);
    const size_t n4 = size_t(rows) * cols / 32;   // one uint4 per 32 weights
    parallel_for(n4, [&](size_t a, size_t b) {
        const uint32_t k[2] = {seed, tensor_id};
        for (size_t i = a; i < b; ++i) {
            const uint32_t c[4] = {uint32_t(i), uint32_t(uint64_t(i) >> 32), 0u, 0u};
            philox(c, k, wq + 4 * i);
        }
    });
    return XP_OK;
}

int xp_synth_scales(void* sc, int scale_fmt, uint32_t rows, uint32_t cols, float sigma,
                    uint32_t seed, uint32_t tensor_id) {
    XP_REQUIRE(sc != nullptr, "sc is null");
    XP_REQUIRE(rows % 32 == 0 && rows && cols, "rows=%u must be a positive multiple of 32", rows);
    XP_REQUIRE(scale_fmt == XP_SCALE_F16_QUAD || scale_fmt == XP_SCALE_F32,
               "scale_fmt %d: synthetic scales are fp16 (quad plane or widened f32)", scale_fmt);
    const uint32_t nblk = rows / 32;
    XP_REQUIRE(scale_fmt != XP_SCALE_F16_QUAD || nblk % 4 == 0,
               "quad plane needs rows %% 128 == 0 (rows=%u)", rows);
    const size_t n = size_t(nblk) * cols;
    parallel_for(n, [&](size_t a, size_t b) {
        for (size_t e = a; e < b; ++e) {
            const uint16_t h = f32_to_f16(float(std::fabs(double(sigma) *
                                                          normal_at(e, 1u, seed, tensor_id))));
            const size_t blk = e / cols, j = e % cols;
            if (scale_fmt == XP_SCALE_F16_QUAD) {
                static_cast<uint16_t*>(sc)[((blk / 4) * cols + j) * 4 + (blk % 4)] = h;
            } else {
                // The exact fp32 value of the fp16 scale.
                const uint32_t sgn = uint32_t(h & 0x8000u) << 16;
                const uint32_t ex = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
                float v;
                if (ex == 0) v = std::ldexp(float(man), -24);
                else v = std::ldexp(float(man | 0x400u), int(ex) - 25);
                uint32_t bits;
                std::memcpy(&bits, &v, 4);
                bits |= sgn;
                std::memcpy(static_cast<float*>(sc) + e, &bits, 4);
            }
        }
    });
    return XP_OK;
}

int xp_synth_normal(float* out, size_t n, float mean, float sigma, uint32_t seed,
                    uint32_t tensor_id) {
    XP_REQUIRE(out != nullptr || n == 0, "out is null");
    parallel_for(n, [&](size_t a, size_t b) {
        for (size_t i = a; i < b; ++i)
            out[i] = float(double(mean) + double(sigma) * normal_at(i, 2u, seed, tensor_id));
    });
    return XP_OK;
}

int xp_synth_normal_f16(uint16_t* out, size_t n, float mean, float sigma, uint32_t seed,
                        uint32_t tensor_id) {
    XP_REQUIRE(out != nullptr || n == 0, "out is null");
    parallel_for(n, [&](size_t a, size_t b) {
        for (size_t i = a; i < b; ++i)
            out[i] = f32_to_f16(
                float(double(mean) + double(sigma) * normal_at(i, 2u, seed, tensor_id)));
    });
    return XP_OK;
}

}  // extern "C"
