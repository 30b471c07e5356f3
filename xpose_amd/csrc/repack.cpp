// Native GGUF weights (Q8_0, Q5_0, Q4_K, Q6_K) in the slot-interleaved plane
// layout the xp_mv_rq kernels read, host side. Replaces repack(),
// reconstruct() and native_bytes() (examples/llm/quant_repack.cpp:129-239,
// quant_repack.hpp:13-82); the layout is that code's, spelled out beside
// xp_rq_layout in include/xpose.h.
//
// The repack is a pure rearrangement plus the pre-multiplication of each
// sub-block's scale: the Q4_K / Q6_K slot scale is d * sub-scale and the Q4_K
// bias dmin * sub-min, each one fp32 product of the same operands the
// dequantiser forms first, so reconstruct() reproduces xp_dequantize bit for
// bit. Row groups of 64 are independent and are packed in parallel.
#include <cstring>
#include <stdexcept>
#include <string>

#include "gguf.hpp"
#include "xp_internal.hpp"
#include "xp_parallel.hpp"

#pragma clang fp contract(off)

namespace xp::rq {
namespace {

constexpr uint32_t kSlotRows = 64;

inline uint16_t rd16(const uint8_t* p) { uint16_t v; std::memcpy(&v, p, 2); return v; }
inline uint32_t rd32(const uint8_t* p) { uint32_t v; std::memcpy(&v, p, 4); return v; }
inline float rdh(const uint8_t* p) { return gguf::half_to_float(rd16(p)); }

// One 32-element k-block of one row in a common form: the stored (unbiased)
// quants, one or two scales and the Q4_K bias.
struct KBlock {
    uint8_t q[32];
    float scale[2];
    float bias;
};

// Q4_K sub-block j's six-bit scale and min (the 12 packed bytes at s).
inline void k4_pair(const uint8_t* s, uint32_t j, uint32_t& sc, uint32_t& mn) {
    if (j < 4) {
        sc = s[j] & 63u;
        mn = s[j + 4] & 63u;
    } else {
        sc = (s[j + 4] & 15u) | (uint32_t(s[j - 4] >> 6) << 4);
        mn = uint32_t(s[j + 4] >> 4) | (uint32_t(s[j] >> 6) << 4);
    }
}

// k-block kb of a row whose native blocks start at `row`.
void read_kblock(uint32_t type, const uint8_t* row, uint32_t kb, KBlock& o) {
    switch (type) {
        case gguf::kQ8_0: {   // d | 32 x int8
            const uint8_t* b = row + size_t(kb) * 34;
            o.scale[0] = rdh(b);
            std::memcpy(o.q, b + 2, 32);
            break;
        }
        case gguf::kQ5_0: {   // d | qh | 16 B nibbles; element e: nibble of byte e % 16
            const uint8_t* b = row + size_t(kb) * 22;
            o.scale[0] = rdh(b);
            const uint32_t qh = rd32(b + 2);
            for (uint32_t e = 0; e < 32; ++e) {
                const uint32_t lo = e < 16 ? b[6 + e] & 15u : uint32_t(b[6 + e - 16] >> 4);
                o.q[e] = uint8_t(lo | (((qh >> e) & 1u) << 4));
            }
            break;
        }
        case gguf::kQ4_K: {   // super-block kb / 8, sub-block kb % 8
            const uint8_t* b = row + size_t(kb / 8) * 144;
            const uint32_t s = kb % 8;
            uint32_t sc, mn;
            k4_pair(b + 4, s, sc, mn);
            o.scale[0] = rdh(b) * float(sc);
            o.bias = rdh(b + 2) * float(mn);
            const uint8_t* qs = b + 16 + (s / 2) * 32;   // 64-element run s / 2
            for (uint32_t l = 0; l < 32; ++l) o.q[l] = uint8_t((qs[l] >> (4 * (s & 1))) & 15u);
            break;
        }
        case gguf::kQ6_K: {   // super-block kb / 8; elements 32 (kb % 8) + l
            const uint8_t* b = row + size_t(kb / 8) * 210;
            const uint32_t s = kb % 8, h = s / 4, t = s % 4;
            const float d = rdh(b + 208);
            for (uint32_t l = 0; l < 32; ++l) {
                const uint32_t lo = (b[64 * h + l + 32 * (t & 1u)] >> (4 * (t >> 1))) & 15u;
                const uint32_t up = (b[128 + 32 * h + l] >> (2 * t)) & 3u;
                o.q[l] = uint8_t(lo | (up << 4));
            }
            // sixteen-element groups 2 t + l / 16 of half h
            o.scale[0] = d * float(int8_t(b[192 + 8 * h + 2 * t]));
            o.scale[1] = d * float(int8_t(b[192 + 8 * h + 2 * t + 1]));
            break;
        }
    }
}

size_t row_bytes(uint32_t type, uint32_t cols) {
    const gguf::BlockFormat& bf = gguf::block_format(type);
    return size_t(cols / bf.elems) * bf.bytes;
}

}  // namespace

// Plane sizes; false (with the error set) for what repack() refuses.
bool layout(uint32_t type, uint32_t rows, uint32_t cols, xp_rq_layout& l, const char* who) {
    const bool k_quant = type == gguf::kQ4_K || type == gguf::kQ6_K;
    if (type != gguf::kQ8_0 && type != gguf::kQ5_0 && !k_quant) {
        set_error(XP_E_ARG, "%s: type %u (%s) has no repacked form", who, type,
                  gguf::block_format(type).name);
        return false;
    }
    if (rows == 0 || cols == 0 || cols % 32 || (k_quant && cols % 256)) {
        set_error(XP_E_ARG, "%s: %u x %u: cols must be a positive multiple of %u", who, rows,
                  cols, k_quant ? 256u : 32u);
        return false;
    }
    l = xp_rq_layout{};
    l.type = type;
    l.rows = rows;
    l.padded_rows = (rows + kSlotRows - 1) / kSlotRows * kSlotRows;
    l.cols = cols;
    l.nkb = cols / 32;
    const uint64_t slots = uint64_t(l.padded_rows) * l.nkb;
    l.quant_bytes = slots * (type == gguf::kQ8_0 ? 32 : 16);
    l.high_bytes = type == gguf::kQ5_0 ? slots * 4 : type == gguf::kQ6_K ? slots * 8 : 0;
    l.scale_bytes = slots * (type == gguf::kQ6_K ? 8 : 4);
    l.bias_bytes = type == gguf::kQ4_K ? slots * 4 : 0;
    l.native_bytes = uint64_t(rows) * row_bytes(type, cols);
    return true;
}

void repack(const xp_rq_layout& l, const uint8_t* src, uint32_t threads, uint32_t* quant,
            uint32_t* high, float* scale, float* bias) {
    const uint32_t qw = l.type == gguf::kQ8_0 ? 8 : 4;
    const size_t rb = row_bytes(l.type, l.cols);
    parallel_for(l.padded_rows / kSlotRows, n_threads(threads), [&](uint32_t g) {
        KBlock kb{};
        for (uint32_t t = 0; t < kSlotRows; ++t) {
            const uint32_t r = g * kSlotRows + t;
            for (uint32_t b = 0; b < l.nkb; ++b) {
                const size_t idx = (size_t(g) * l.nkb + b) * kSlotRows + t;
                uint32_t* qd = quant + idx * qw;
                std::memset(qd, 0, qw * 4);
                if (r >= l.rows) {   // padding rows: zero planes
                    if (high) {
                        high[idx * (l.type == gguf::kQ6_K ? 2 : 1)] = 0;
                        if (l.type == gguf::kQ6_K) high[idx * 2 + 1] = 0;
                    }
                    if (l.type == gguf::kQ6_K) scale[idx * 2] = scale[idx * 2 + 1] = 0.0f;
                    else scale[idx] = 0.0f;
                    if (bias) bias[idx] = 0.0f;
                    continue;
                }
                read_kblock(l.type, src + size_t(r) * rb, b, kb);
                if (l.type == gguf::kQ8_0) {
                    for (uint32_t j = 0; j < 32; ++j) qd[j / 4] |= uint32_t(kb.q[j]) << (8 * (j % 4));
                    scale[idx] = kb.scale[0];
                    continue;
                }
                uint32_t h0 = 0, h1 = 0;
                for (uint32_t j = 0; j < 32; ++j) {
                    qd[j / 8] |= uint32_t(kb.q[j] & 15u) << (4 * (j % 8));
                    const uint32_t up = kb.q[j] >> 4;
                    if (l.type == gguf::kQ5_0) h0 |= up << j;
                    else if (j < 16) h0 |= up << (2 * j);
                    else h1 |= up << (2 * (j - 16));
                }
                if (l.type == gguf::kQ5_0) {
                    high[idx] = h0;
                    scale[idx] = kb.scale[0];
                } else if (l.type == gguf::kQ6_K) {
                    high[idx * 2] = h0;
                    high[idx * 2 + 1] = h1;
                    scale[idx * 2] = kb.scale[0];
                    scale[idx * 2 + 1] = kb.scale[1];
                } else {
                    scale[idx] = kb.scale[0];
                    bias[idx] = kb.bias;
                }
            }
        }
    });
}

float reconstruct(const xp_rq_layout& l, const uint32_t* quant, const uint32_t* high,
                  const float* scale, const float* bias, uint32_t r, uint32_t k) {
    const uint32_t j = k % 32;
    const size_t idx = (size_t(r / kSlotRows) * l.nkb + k / 32) * kSlotRows + r % kSlotRows;
    if (l.type == gguf::kQ8_0) {
        const int8_t q = int8_t((quant[idx * 8 + j / 4] >> (8 * (j % 4))) & 0xFFu);
        return scale[idx] * float(q);
    }
    uint32_t q = (quant[idx * 4 + j / 8] >> (4 * (j % 8))) & 15u;
    switch (l.type) {
        case gguf::kQ5_0:
            q |= ((high[idx] >> j) & 1u) << 4;
            return scale[idx] * float(int(q) - 16);
        case gguf::kQ6_K:
            q |= ((high[idx * 2 + j / 16] >> (2 * (j % 16))) & 3u) << 4;
            return scale[idx * 2 + j / 16] * float(int(q) - 32);
        default:   // Q4_K
            return scale[idx] * float(q) - bias[idx];
    }
}

}  // namespace xp::rq

using namespace xp;

extern "C" {

int xp_rq_layout_of(uint32_t type, uint32_t rows, uint32_t cols, xp_rq_layout* out) {
    XP_REQUIRE(out, "null pointer");
    return rq::layout(type, rows, cols, *out, "xp_rq_layout_of") ? XP_OK : XP_E_ARG;
}

int xp_rq_repack(const xp_rq_layout* l, const void* src, uint32_t threads, void* quant,
                 uint32_t* high, float* scale, float* bias) {
    XP_REQUIRE(l && src && quant && scale, "null pointer");
    xp_rq_layout chk;
    if (!rq::layout(l->type, l->rows, l->cols, chk, "xp_rq_repack")) return XP_E_ARG;
    XP_REQUIRE(chk.padded_rows == l->padded_rows && chk.nkb == l->nkb,
               "layout does not match its type and shape (use xp_rq_layout_of)");
    XP_REQUIRE(!chk.high_bytes || high, "type %u needs the high plane", l->type);
    XP_REQUIRE(!chk.bias_bytes || bias, "type %u needs the bias plane", l->type);
    try {
        rq::repack(chk, static_cast<const uint8_t*>(src), threads, static_cast<uint32_t*>(quant),
                   chk.high_bytes ? high : nullptr, scale, chk.bias_bytes ? bias : nullptr);
    } catch (const std::exception& e) {
        return set_error(XP_E_NOMEM, "xp_rq_repack: %s", e.what());
    }
    return XP_OK;
}

int xp_rq_reconstruct(const xp_rq_layout* l, const void* quant, const uint32_t* high,
                      const float* scale, const float* bias, float* out) {
    XP_REQUIRE(l && quant && scale && out, "null pointer");
    xp_rq_layout chk;
    if (!rq::layout(l->type, l->rows, l->cols, chk, "xp_rq_reconstruct")) return XP_E_ARG;
    XP_REQUIRE(!chk.high_bytes || high, "type %u needs the high plane", l->type);
    XP_REQUIRE(!chk.bias_bytes || bias, "type %u needs the bias plane", l->type);
    const uint32_t* q = static_cast<const uint32_t*>(quant);
    for (uint32_t r = 0; r < chk.rows; ++r)
        for (uint32_t k = 0; k < chk.cols; ++k)
            out[size_t(r) * chk.cols + k] = rq::reconstruct(chk, q, high, scale, bias, r, k);
    return XP_OK;
}

}  // extern "C"
