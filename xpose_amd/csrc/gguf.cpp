// GGUF reader, ggml block dequantisers and the xp_gguf_* C entry points.
// The file format and block layouts are ggml's (the reference reads them in
// examples/llm/model/gguf.cpp:234-645); everything here is host code.
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>
#include <stdexcept>

#include "xp_internal.hpp"

// Every a * b + c below rounds twice, as the reference's loaders do.
#pragma clang fp contract(off)

namespace xp::gguf {
namespace {

[[noreturn]] void bad(const std::string& what) { throw std::runtime_error("gguf: " + what); }

// Bounds-checked little-endian cursor over the mapping: every length in the
// file is untrusted, so every read is checked against the end first.
struct Cursor {
    const uint8_t* base;
    uint64_t size, at = 0;
    void need(uint64_t n) const {
        if (n > size - at)
            bad("truncated: " + std::to_string(n) + " bytes wanted at offset " + std::to_string(at) +
                " of " + std::to_string(size));
    }
    template <class T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, base + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    std::string_view str() {
        const uint64_t n = get<uint64_t>();
        need(n);
        std::string_view s(reinterpret_cast<const char*>(base + at), size_t(n));
        at += n;
        return s;
    }
};

uint32_t scalar_bytes(uint32_t kind) {
    switch (kind) {
        case kMU8: case kMI8: case kMBool: return 1;
        case kMU16: case kMI16: return 2;
        case kMU32: case kMI32: case kMF32: return 4;
        case kMU64: case kMI64: case kMF64: return 8;
        default: return 0;
    }
}

// One scalar of `kind`; numeric kinds fill u, i and f alike.
void scalar(Cursor& c, uint32_t kind, Value& v) {
    auto set_int = [&](int64_t x) { v.i = x; v.u = uint64_t(x); v.f = double(x); };
    switch (kind) {
        case kMU8: v.u = c.get<uint8_t>(); v.i = int64_t(v.u); v.f = double(v.u); break;
        case kMI8: set_int(c.get<int8_t>()); break;
        case kMU16: v.u = c.get<uint16_t>(); v.i = int64_t(v.u); v.f = double(v.u); break;
        case kMI16: set_int(c.get<int16_t>()); break;
        case kMU32: v.u = c.get<uint32_t>(); v.i = int64_t(v.u); v.f = double(v.u); break;
        case kMI32: set_int(c.get<int32_t>()); break;
        case kMU64: v.u = c.get<uint64_t>(); v.i = int64_t(v.u); v.f = double(v.u); break;
        case kMI64: set_int(c.get<int64_t>()); break;
        case kMF32: v.f = c.get<float>(); v.i = int64_t(v.f); v.u = uint64_t(v.i); break;
        case kMF64: v.f = c.get<double>(); v.i = int64_t(v.f); v.u = uint64_t(v.i); break;
        case kMBool: v.u = c.get<uint8_t>() ? 1 : 0; v.i = int64_t(v.u); v.f = double(v.u); break;
        case kMStr: v.s = c.str(); break;
        default: bad("metadata value of unknown kind " + std::to_string(kind));
    }
}

}  // namespace

const BlockFormat& block_format(uint32_t type) {
    // Block geometry of every ggml type up to BF16 (bytes per block are part
    // of the file format: a wrong entry shifts every later tensor).
    static const BlockFormat f[31] = {
        {"F32", 1, 4, true},        {"F16", 1, 2, true},        {"Q4_0", 32, 18, true},
        {"Q4_1", 32, 20, true},     {"(removed)", 0, 0, false}, {"(removed)", 0, 0, false},
        {"Q5_0", 32, 22, true},     {"Q5_1", 32, 24, true},     {"Q8_0", 32, 34, true},
        {"Q8_1", 32, 40, false},    {"Q2_K", 256, 84, false},   {"Q3_K", 256, 110, false},
        {"Q4_K", 256, 144, true},   {"Q5_K", 256, 176, false},  {"Q6_K", 256, 210, true},
        {"Q8_K", 256, 292, false},  {"IQ2_XXS", 256, 66, false}, {"IQ2_XS", 256, 74, false},
        {"IQ3_XXS", 256, 98, false}, {"IQ1_S", 256, 50, false}, {"IQ4_NL", 32, 18, false},
        {"IQ3_S", 256, 110, false}, {"IQ2_S", 256, 82, false},  {"IQ4_XS", 256, 136, false},
        {"I8", 1, 1, false},        {"I16", 1, 2, false},       {"I32", 1, 4, false},
        {"I64", 1, 8, false},       {"F64", 1, 8, false},       {"IQ1_M", 256, 56, false},
        {"BF16", 1, 2, true},
    };
    static const BlockFormat unknown{"unknown", 0, 0, false};
    return type < 31 ? f[type] : unknown;
}

float half_to_float(uint16_t h) {
    const uint32_t sign = uint32_t(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t bits;
    if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else {   // subnormal: m * 2^-24, exact in fp32
        float f = std::ldexp(float(m), -24);
        std::memcpy(&bits, &f, 4);
        bits |= sign;
    }
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

namespace {

inline uint16_t rd16(const uint8_t* p) { uint16_t v; std::memcpy(&v, p, 2); return v; }
inline uint32_t rd32(const uint8_t* p) { uint32_t v; std::memcpy(&v, p, 4); return v; }
inline float rdh(const uint8_t* p) { return half_to_float(rd16(p)); }

// 4-bit quants of a 32-element block: element e is the low nibble of byte e
// (e < 16) or the high nibble of byte e - 16.
inline uint32_t nib32(const uint8_t* qs, uint32_t e) {
    return e < 16 ? qs[e] & 15u : uint32_t(qs[e - 16] >> 4);
}

// Q4_K sub-block j (0..7) scale and min from the 12 packed bytes: six bits
// each; j < 4 sits in the low six bits of bytes j / j + 4, j >= 4 takes its
// low four bits from byte j + 4 and its top two from bits 6-7 of byte j - 4
// (scale) or byte j (min).
inline void k4_scale_min(const uint8_t* q, uint32_t j, uint32_t& sc, uint32_t& mn) {
    if (j < 4) {
        sc = q[j] & 63u;
        mn = q[j + 4] & 63u;
    } else {
        sc = (q[j + 4] & 15u) | (uint32_t(q[j - 4] >> 6) << 4);
        mn = uint32_t(q[j + 4] >> 4) | (uint32_t(q[j] >> 6) << 4);
    }
}

}  // namespace

bool dequantize(uint32_t type, const void* src, float* dst, size_t n) {
    const BlockFormat& bf = block_format(type);
    if (!bf.dequant || bf.elems == 0 || n % bf.elems) return false;
    const uint8_t* p = static_cast<const uint8_t*>(src);
    const size_t nb = n / bf.elems;
    switch (type) {
        case kF32:
            std::memcpy(dst, p, n * 4);
            return true;
        case kF16:
            for (size_t i = 0; i < n; ++i) dst[i] = half_to_float(rd16(p + 2 * i));
            return true;
        case kBF16:
            for (size_t i = 0; i < n; ++i) {
                const uint32_t b = uint32_t(rd16(p + 2 * i)) << 16;
                std::memcpy(dst + i, &b, 4);
            }
            return true;
        case kQ4_0:   // d f16 | 16 B nibbles; (q - 8) d
        case kQ4_1:   // d f16 | m f16 | 16 B nibbles; q d + m
            for (size_t b = 0; b < nb; ++b) {
                const uint8_t* blk = p + b * bf.bytes;
                const float d = rdh(blk);
                const bool affine = type == kQ4_1;
                const float m = affine ? rdh(blk + 2) : 0.0f;
                const uint8_t* qs = blk + (affine ? 4 : 2);
                for (uint32_t e = 0; e < 32; ++e) {
                    const uint32_t q = nib32(qs, e);
                    dst[b * 32 + e] = affine ? float(q) * d + m : float(int(q) - 8) * d;
                }
            }
            return true;
        case kQ5_0:   // d f16 | qh u32 | 16 B nibbles; (q - 16) d
        case kQ5_1:   // d f16 | m f16 | qh u32 | 16 B nibbles; q d + m
            for (size_t b = 0; b < nb; ++b) {
                const uint8_t* blk = p + b * bf.bytes;
                const bool affine = type == kQ5_1;
                const float d = rdh(blk);
                const float m = affine ? rdh(blk + 2) : 0.0f;
                const uint32_t qh = rd32(blk + (affine ? 4 : 2));
                const uint8_t* qs = blk + (affine ? 8 : 6);
                for (uint32_t e = 0; e < 32; ++e) {
                    // bit e of qh is the fifth bit of element e
                    const uint32_t q = nib32(qs, e) | (((qh >> e) & 1u) << 4);
                    dst[b * 32 + e] = affine ? float(q) * d + m : float(int(q) - 16) * d;
                }
            }
            return true;
        case kQ8_0:   // d f16 | 32 x i8
            for (size_t b = 0; b < nb; ++b) {
                const uint8_t* blk = p + b * 34;
                const float d = rdh(blk);
                for (uint32_t e = 0; e < 32; ++e)
                    dst[b * 32 + e] = float(int8_t(blk[2 + e])) * d;
            }
            return true;
        case kQ4_K:
            // d f16 | dmin f16 | 12 B six-bit scales and mins | 128 B nibbles.
            // Element e: 64-element run r = e / 64 uses bytes 32 r .. 32 r + 31,
            // low nibbles for its first 32 elements (sub-block 2 r) and high
            // nibbles for the next 32 (sub-block 2 r + 1); value d sc q - dmin mn.
            for (size_t b = 0; b < nb; ++b) {
                const uint8_t* blk = p + b * 144;
                const float d = rdh(blk), dmin = rdh(blk + 2);
                const uint8_t* scl = blk + 4;
                const uint8_t* qs = blk + 16;
                for (uint32_t e = 0; e < 256; ++e) {
                    const uint32_t r = e / 64, hi = (e % 64) / 32, l = e % 32;
                    uint32_t sc, mn;
                    k4_scale_min(scl, 2 * r + hi, sc, mn);
                    const uint32_t q = (qs[32 * r + l] >> (4 * hi)) & 15u;
                    dst[b * 256 + e] = d * float(sc) * float(q) - dmin * float(mn);
                }
            }
            return true;
        case kQ6_K:
            // 128 B low nibbles | 64 B 2-bit highs | 16 x i8 scales | d f16.
            // Element e: half h = e / 128, quarter t = (e % 128) / 32, lane
            // l = e % 32. Low nibble: byte 64 h + l + 32 (t & 1), nibble t / 2;
            // high bits: byte 32 h + l, bits 2 t; scale 8 h + 2 t + l / 16;
            // value d sc (q - 32).
            for (size_t b = 0; b < nb; ++b) {
                const uint8_t* blk = p + b * 210;
                const uint8_t* ql = blk;
                const uint8_t* qh = blk + 128;
                const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192);
                const float d = rdh(blk + 208);
                for (uint32_t e = 0; e < 256; ++e) {
                    const uint32_t h = e / 128, t = (e % 128) / 32, l = e % 32;
                    const uint32_t lo = (ql[64 * h + l + 32 * (t & 1u)] >> (4 * (t >> 1))) & 15u;
                    const uint32_t up = (qh[32 * h + l] >> (2 * t)) & 3u;
                    const int q = int(lo | (up << 4)) - 32;
                    dst[b * 256 + e] = d * float(sc[8 * h + 2 * t + l / 16]) * float(q);
                }
            }
            return true;
        default:
            return false;
    }
}

void dequantize_rows(const Tensor& t, uint64_t row0, uint64_t nrows, float* dst) {
    const BlockFormat& bf = block_format(t.type);
    const uint64_t row = t.dims[0], nrow = t.elements() / (row ? row : 1);
    if (!bf.dequant || bf.elems == 0)
        bad("tensor '" + std::string(t.name) + "' has type " + bf.name + ", which is not dequantised");
    if (row % bf.elems)
        bad("tensor '" + std::string(t.name) + "' rows of " + std::to_string(row) +
            " are not a whole number of " + bf.name + " blocks");
    if (row0 > nrow || nrows > nrow - row0)
        bad("tensor '" + std::string(t.name) + "' rows [" + std::to_string(row0) + ", +" +
            std::to_string(nrows) + ") out of " + std::to_string(nrow));
    const uint64_t row_bytes = row / bf.elems * bf.bytes;
    if (!dequantize(t.type, t.data + row0 * row_bytes, dst, size_t(row * nrows)))
        bad("dequantize failed for '" + std::string(t.name) + "'");
}

// ---- File -----------------------------------------------------------------------
std::unique_ptr<File> File::open(const std::string& path) {
    std::unique_ptr<File> f(new File());
    f->path_ = path;
    f->fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (f->fd_ < 0) bad("cannot open '" + path + "': " + std::strerror(errno));
    struct stat st {};
    if (::fstat(f->fd_, &st) != 0) bad("cannot stat '" + path + "': " + std::strerror(errno));
    if (st.st_size <= 0) bad("'" + path + "' is empty");
    f->size_ = uint64_t(st.st_size);
    void* m = ::mmap(nullptr, size_t(f->size_), PROT_READ, MAP_PRIVATE, f->fd_, 0);
    if (m == MAP_FAILED) bad("cannot map '" + path + "': " + std::strerror(errno));
    f->base_ = static_cast<const uint8_t*>(m);
    ::madvise(m, size_t(f->size_), MADV_SEQUENTIAL);
    f->parse();
    return f;
}

File::~File() {
    if (base_) ::munmap(const_cast<uint8_t*>(base_), size_t(size_));
    if (fd_ >= 0) ::close(fd_);
}

void File::parse() {
    Cursor c{base_, size_};
    if (c.get<uint32_t>() != 0x46554747u) bad("not a GGUF file (bad magic)");
    version_ = c.get<uint32_t>();
    if (version_ != 2 && version_ != 3) bad("version " + std::to_string(version_) + " (2 or 3 supported)");
    const uint64_t n_tensors = c.get<uint64_t>(), n_meta = c.get<uint64_t>();
    if (n_tensors > (1u << 24) || n_meta > (1u << 24)) bad("implausible tensor or metadata count");

    meta_.reserve(size_t(n_meta));
    for (uint64_t k = 0; k < n_meta; ++k) {
        const std::string_view key = c.str();
        Value v;
        v.kind = c.get<uint32_t>();
        if (v.kind == kMArr) {
            v.elem = c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            if (v.elem == kMStr) {
                if (n > size_ / 8) bad("string array longer than the file");
                c.need(n * 8);   // every entry has an 8-byte length
                v.strs.reserve(size_t(n));
                for (uint64_t j = 0; j < n; ++j) v.strs.push_back(c.str());
            } else if (v.elem == kMArr) {
                bad("nested metadata arrays are not supported");
            } else {
                const uint32_t eb = scalar_bytes(v.elem);
                if (eb == 0) bad("metadata array of unknown element kind " + std::to_string(v.elem));
                if (n > size_ / eb) bad("metadata array longer than the file");
                c.need(n * eb);
                v.nums.reserve(size_t(n));
                for (uint64_t j = 0; j < n; ++j) {
                    Value e;
                    scalar(c, v.elem, e);
                    const bool fl = v.elem == kMF32 || v.elem == kMF64;
                    const bool sg = v.elem == kMI8 || v.elem == kMI16 || v.elem == kMI32 || v.elem == kMI64;
                    v.nums.push_back(fl ? e.f : sg ? double(e.i) : double(e.u));
                }
            }
        } else {
            scalar(c, v.kind, v);
        }
        meta_at_.emplace(key, meta_.size());
        meta_.emplace_back(key, std::move(v));
    }
    if (const Value* a = meta("general.alignment")) alignment_ = a->u;
    if (alignment_ == 0 || (alignment_ & (alignment_ - 1))) bad("general.alignment is not a power of two");

    tensors_.reserve(size_t(n_tensors));
    for (uint64_t t = 0; t < n_tensors; ++t) {
        Tensor x;
        x.name = c.str();
        x.n_dims = c.get<uint32_t>();
        if (x.n_dims > 4) bad("tensor '" + std::string(x.name) + "' has " + std::to_string(x.n_dims) + " dims");
        for (uint32_t d = 0; d < x.n_dims; ++d) x.dims[d] = c.get<uint64_t>();
        x.type = c.get<uint32_t>();
        x.offset = c.get<uint64_t>();
        const BlockFormat& bf = block_format(x.type);
        if (bf.elems == 0) bad("tensor '" + std::string(x.name) + "' has unknown type " + std::to_string(x.type));
        uint64_t ne = 1;
        for (uint32_t d = 0; d < x.n_dims; ++d)
            if (x.dims[d] == 0 || __builtin_mul_overflow(ne, x.dims[d], &ne) || ne > (uint64_t(1) << 48))
                bad("tensor '" + std::string(x.name) + "' has a bad shape");
        if (ne % bf.elems) bad("tensor '" + std::string(x.name) + "' is not a whole number of " + bf.name + " blocks");
        x.nbytes = ne / bf.elems * bf.bytes;
        tensor_at_.emplace(x.name, tensors_.size());
        tensors_.push_back(x);
    }
    data_offset_ = (c.at + alignment_ - 1) & ~(alignment_ - 1);
    if (data_offset_ > size_) bad("tensor data starts past the end of the file");
    for (Tensor& x : tensors_) {
        if (x.offset > size_ - data_offset_ || x.nbytes > size_ - data_offset_ - x.offset)
            bad("tensor '" + std::string(x.name) + "' data runs past the end of the file");
        x.data = base_ + data_offset_ + x.offset;
    }
}

const Tensor* File::tensor(std::string_view name) const {
    const auto it = tensor_at_.find(name);
    return it == tensor_at_.end() ? nullptr : &tensors_[it->second];
}

const Value* File::meta(std::string_view key) const {
    const auto it = meta_at_.find(key);
    return it == meta_at_.end() ? nullptr : &meta_[it->second].second;
}

ModelShape File::shape() const {
    ModelShape m;
    const Value* a = meta("general.architecture");
    m.arch = a && a->kind == kMStr ? std::string(a->s) : "unknown";
    const Value* nm = meta("general.name");
    m.name = nm && nm->kind == kMStr ? std::string(nm->s) : "";
    const std::string p = m.arch + ".";
    auto u = [&](const char* key, uint32_t dflt) {
        const Value* v = meta(p + key);
        return v ? uint32_t(v->u) : dflt;
    };
    auto f = [&](const char* key, float dflt) {
        const Value* v = meta(p + key);
        return v ? float(v->f) : dflt;
    };
    m.layers = u("block_count", 0);
    m.heads = u("attention.head_count", 0);
    m.kv_heads = u("attention.head_count_kv", m.heads);
    m.hidden = u("embedding_length", 0);
    m.ffn = u("feed_forward_length", 0);
    m.context = u("context_length", 0);
    m.key_length = u("attention.key_length", 0);
    m.value_length = u("attention.value_length", 0);
    m.sliding_window = u("attention.sliding_window", 0);
    m.rope_base = f("rope.freq_base", 10000.0f);
    m.rms_eps = f("attention.layer_norm_rms_epsilon", 1e-6f);
    // The vocabulary is the token list's length (authoritative); a scalar
    // vocab_size key is the fallback.
    if (const Value* toks = meta("tokenizer.ggml.tokens")) m.vocab = uint32_t(toks->strs.size());
    else m.vocab = u("vocab_size", 0);
    return m;
}

}  // namespace xp::gguf

// ---- C ABI -----------------------------------------------------------------------

namespace {

template <class F>
int guarded(const char* who, F&& fn) {
    try {
        return fn();
    } catch (const std::bad_alloc&) {
        return xp::set_error(XP_E_NOMEM, "%s: out of host memory", who);
    } catch (const std::exception& e) {
        return xp::set_error(XP_E_FORMAT, "%s: %s", who, e.what());
    }
}

void copy_str(std::string_view s, char* out, size_t cap) {
    if (!out || cap == 0) return;
    const size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
    std::memcpy(out, s.data(), n);
    out[n] = '\0';
}

}  // namespace

extern "C" {

int xp_gguf_open(const char* path, xp_gguf** out) {
    XP_REQUIRE(path && out, "null pointer");
    *out = nullptr;
    return guarded("xp_gguf_open", [&] {
        auto g = std::make_unique<xp_gguf>();
        g->f = xp::gguf::File::open(path);
        *out = g.release();
        return XP_OK;
    });
}

int xp_gguf_close(xp_gguf* g) {
    delete g;
    return XP_OK;
}

int xp_gguf_get_info(xp_gguf* g, xp_gguf_info* info) {
    XP_REQUIRE(g && info, "null pointer");
    info->version = g->f->version();
    info->n_tensors = g->f->tensors().size();
    info->n_meta = g->f->n_meta();
    info->alignment = g->f->alignment();
    info->data_offset = g->f->data_offset();
    info->file_size = g->f->size();
    return XP_OK;
}

int xp_gguf_get_model(xp_gguf* g, xp_gguf_model* m) {
    XP_REQUIRE(g && m, "null pointer");
    const xp::gguf::ModelShape s = g->f->shape();
    *m = xp_gguf_model{};
    copy_str(s.arch, m->arch, sizeof m->arch);
    m->n_layers = s.layers;
    m->n_heads = s.heads;
    m->n_kv_heads = s.kv_heads;
    m->hidden = s.hidden;
    m->ffn = s.ffn;
    m->context_length = s.context;
    m->key_length = s.key_length;
    m->value_length = s.value_length;
    m->vocab = s.vocab;
    m->sliding_window = s.sliding_window;
    m->head_dim = s.head_dim();
    m->rope_freq_base = s.rope_base;
    m->rms_eps = s.rms_eps;
    return XP_OK;
}

int xp_gguf_tensor_count(xp_gguf* g, uint64_t* n) {
    XP_REQUIRE(g && n, "null pointer");
    *n = g->f->tensors().size();
    return XP_OK;
}

int xp_gguf_tensor_at(xp_gguf* g, uint64_t i, char* name, size_t cap) {
    XP_REQUIRE(g && name && cap, "null pointer");
    XP_REQUIRE(i < g->f->tensors().size(), "tensor index %llu out of range",
               static_cast<unsigned long long>(i));
    copy_str(g->f->tensors()[size_t(i)].name, name, cap);
    return XP_OK;
}

int xp_gguf_tensor_info(xp_gguf* g, const char* name, uint32_t* type, uint32_t* n_dims,
                        uint64_t* dims, uint64_t* nbytes) {
    XP_REQUIRE(g && name, "null pointer");
    const xp::gguf::Tensor* t = g->f->tensor(name);
    if (!t) return xp::set_error(XP_E_ARG, "xp_gguf_tensor_info: no tensor '%s'", name);
    if (type) *type = t->type;
    if (n_dims) *n_dims = t->n_dims;
    if (dims)
        for (int d = 0; d < 4; ++d) dims[d] = t->dims[d];
    if (nbytes) *nbytes = t->nbytes;
    return XP_OK;
}

int xp_gguf_meta_number(xp_gguf* g, const char* key, double* value) {
    XP_REQUIRE(g && key && value, "null pointer");
    const xp::gguf::Value* v = g->f->meta(key);
    if (!v) return xp::set_error(XP_E_ARG, "xp_gguf_meta_number: no key '%s'", key);
    if (v->kind == xp::gguf::kMStr || v->kind == xp::gguf::kMArr)
        return xp::set_error(XP_E_ARG, "xp_gguf_meta_number: '%s' is not a number", key);
    const bool sg = v->kind == xp::gguf::kMI8 || v->kind == xp::gguf::kMI16 ||
                    v->kind == xp::gguf::kMI32 || v->kind == xp::gguf::kMI64;
    const bool fl = v->kind == xp::gguf::kMF32 || v->kind == xp::gguf::kMF64;
    *value = fl ? v->f : sg ? double(v->i) : double(v->u);
    return XP_OK;
}

int xp_gguf_meta_string(xp_gguf* g, const char* key, char* out, size_t cap, size_t* len) {
    XP_REQUIRE(g && key, "null pointer");
    const xp::gguf::Value* v = g->f->meta(key);
    if (!v || v->kind != xp::gguf::kMStr)
        return xp::set_error(XP_E_ARG, "xp_gguf_meta_string: no string key '%s'", key);
    if (len) *len = v->s.size();
    copy_str(v->s, out, cap);
    return XP_OK;
}

int xp_gguf_meta_array_length(xp_gguf* g, const char* key, uint64_t* n) {
    XP_REQUIRE(g && key && n, "null pointer");
    const xp::gguf::Value* v = g->f->meta(key);
    if (!v || v->kind != xp::gguf::kMArr)
        return xp::set_error(XP_E_ARG, "xp_gguf_meta_array_length: no array key '%s'", key);
    *n = v->length();
    return XP_OK;
}

int xp_dequantize(uint32_t type, const void* src, float* out, uint64_t n) {
    XP_REQUIRE(src && out, "null pointer");
    const xp::gguf::BlockFormat& bf = xp::gguf::block_format(type);
    if (!bf.dequant)
        return xp::set_error(XP_E_ARG, "xp_dequantize: type %u (%s) is not supported", type, bf.name);
    if (n % bf.elems)
        return xp::set_error(XP_E_ARG, "xp_dequantize: %llu elements are not whole %s blocks",
                             static_cast<unsigned long long>(n), bf.name);
    xp::gguf::dequantize(type, src, out, size_t(n));
    return XP_OK;
}

int xp_gguf_dequantize_rows(xp_gguf* g, const char* name, uint64_t row0, uint64_t nrows,
                            float* out) {
    XP_REQUIRE(g && name && out, "null pointer");
    const xp::gguf::Tensor* t = g->f->tensor(name);
    if (!t) return xp::set_error(XP_E_ARG, "xp_gguf_dequantize_rows: no tensor '%s'", name);
    return guarded("xp_gguf_dequantize_rows", [&] {
        xp::gguf::dequantize_rows(*t, row0, nrows, out);
        return XP_OK;
    });
}

}  // extern "C"
