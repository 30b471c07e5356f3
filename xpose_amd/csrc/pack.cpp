// Requantising packer, packed-weight cache and the GGUF load path.
//
// Every matrix of a GGUF model is read at its native type (Q8_0 / Q5_0 /
// Q4_K / Q6_K / F16 / ...), dequantised row by row and requantised to the one
// int4 format the kernels read (the reference's load path,
// examples/llm/decode.cpp:60-229 and 710-1328):
//   * symmetric int4 per 32-block: q = round-half-away(v / s) + 8 clamped to
//     [0, 15] (the kernels read q - 8);
//   * s = amax / 7, then (bf16 scales) whichever of the two bf16 values
//     bracketing it gives the smaller squared block error, so the nibbles are
//     derived from exactly the scale the GPU multiplies back;
//   * KM4 nibble plane uint4[(g nblk + b) 64 + t], word (k >> 3) & 3, nibble
//     (k & 7) 4; bf16 quad scale plane [((b / 4) cols + j) 4 + b % 4] or fp32
//     [b][cols].
// GGUF stores a linear weight [out][in] with rows of `in` elements, so GGUF
// row j is output column j: packing 64 consecutive rows is one column group.
// Column groups are independent, so a matrix packs in parallel over groups.
//
// The cache ("<model>.xpack" or any path) holds the packed bytes of every
// matrix so later loads skip the requantisation: see CacheHeader.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstring>
#include <functional>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "gguf.hpp"
#include "xp_internal.hpp"
#include "xp_parallel.hpp"
#include "xp_launch.hpp"

// The quantiser's arithmetic is part of the packed bytes: every a * b + c
// rounds twice, as in the reference's packer.
#pragma clang fp contract(off)

namespace xp::pack {
namespace {

constexpr uint32_t kQB = 32;        // quantisation block along k
constexpr uint32_t kCG = 64;        // KM4 column group
// Bump when anything that changes the packed bytes changes.
constexpr uint32_t kPackerRev = 1;

double now_ms() {
    using namespace std::chrono;
    return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

// ---- quantiser -----------------------------------------------------------------
inline uint32_t nibble(float v, float inv) {
    const int q = int(std::lround(v * inv)) + 8;
    return uint32_t(q < 0 ? 0 : q > 15 ? 15 : q);
}

inline uint32_t f32_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float bits_f32(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

// Squared reconstruction error of a 32-block at scale s (infinite for s <= 0).
double block_error(const float* v, float s) {
    if (!(s > 0.0f)) return std::numeric_limits<double>::infinity();
    const float inv = 1.0f / s;
    double e = 0.0;
    for (uint32_t t = 0; t < kQB; ++t) {
        const double d = double(int(nibble(v[t], inv)) - 8) * double(s) - double(v[t]);
        e += d * d;
    }
    return e;
}

// The bf16 scale of a block: s0 = amax / 7 truncated to bf16, or the next bf16
// value up, whichever reconstructs the block better (ties to the lower).
float bf16_scale(const float* v, float s0) {
    if (!(s0 > 0.0f)) return 0.0f;
    const uint32_t lo = f32_bits(s0) & 0xFFFF0000u;
    const float a = bits_f32(lo), b = bits_f32(lo + 0x10000u);
    return block_error(v, a) <= block_error(v, b) ? a : b;
}

// Column group g of a matrix: cols64[c][rows] holds output columns 64 g + c.
// Writes its KM4 words and its fp32 scales sf[b][cols] (the value the
// nibbles were derived with).
void pack_group(const float* cols64, uint32_t rows, uint32_t cols, uint32_t g, bool bf16,
                uint32_t* wq, float* sf) {
    const uint32_t nblk = rows / kQB;
    for (uint32_t b = 0; b < nblk; ++b)
        for (uint32_t c = 0; c < kCG; ++c) {
            const float* v = cols64 + size_t(c) * rows + size_t(b) * kQB;
            float amax = 0.0f;
            for (uint32_t t = 0; t < kQB; ++t) amax = std::max(amax, std::fabs(v[t]));
            const float s = bf16 ? bf16_scale(v, amax / 7.0f) : amax / 7.0f;
            sf[size_t(b) * cols + size_t(g) * kCG + c] = s;
            const float inv = s > 0.0f ? 1.0f / s : 0.0f;
            uint32_t w[4] = {0, 0, 0, 0};
            for (uint32_t t = 0; t < kQB; ++t) w[t >> 3] |= nibble(v[t], inv) << ((t & 7u) * 4u);
            uint32_t* dst = wq + ((size_t(g) * nblk + b) * kCG + c) * 4;
            std::memcpy(dst, w, 16);
        }
}

// Scale plane of columns [j0, j1) from the fp32 scales sf[b][cols].
void write_scales(const float* sf, uint32_t nblk, uint32_t cols, uint32_t j0, uint32_t j1,
                  bool bf16, void* sc) {
    if (bf16) {
        uint16_t* o = static_cast<uint16_t*>(sc);
        for (uint32_t b = 0; b < nblk; ++b)
            for (uint32_t j = j0; j < j1; ++j)
                o[(size_t(b / 4) * cols + j) * 4 + b % 4] =
                    uint16_t(f32_bits(sf[size_t(b) * cols + j]) >> 16);
    } else {
        float* o = static_cast<float*>(sc);
        for (uint32_t b = 0; b < nblk; ++b)
            for (uint32_t j = j0; j < j1; ++j) o[size_t(b) * cols + j] = sf[size_t(b) * cols + j];
    }
}

size_t wq_bytes(uint32_t rows, uint32_t cols) { return size_t(rows) * cols / 2; }
size_t sc_bytes(uint32_t rows, uint32_t cols, bool bf16) {
    return size_t(rows / kQB) * cols * (bf16 ? 2 : 4);
}

// One matrix to pack: GGUF tensor `name` as (rows = in, cols = out).
struct Task {
    std::string name;
    const gguf::Tensor* t = nullptr;
    uint32_t rows = 0, cols = 0;
    int layer = -1, id = XP_T_LM_HEAD;
};

struct Packed {
    std::vector<uint32_t> wq;
    std::vector<uint8_t> sc;
};

// Packs a task's GGUF rows (threaded over column groups).
void pack_task(const Task& k, bool bf16, uint32_t threads, Packed& out) {
    const uint32_t nblk = k.rows / kQB, ngroups = k.cols / kCG;
    out.wq.assign(wq_bytes(k.rows, k.cols) / 4, 0u);
    out.sc.assign(sc_bytes(k.rows, k.cols, bf16), 0u);
    std::vector<float> sf(size_t(nblk) * k.cols);
    parallel_for(ngroups, threads, [&](uint32_t g) {
        std::vector<float> cols64(size_t(kCG) * k.rows);
        gguf::dequantize_rows(*k.t, uint64_t(g) * kCG, kCG, cols64.data());
        pack_group(cols64.data(), k.rows, k.cols, g, bf16, out.wq.data(), sf.data());
        write_scales(sf.data(), nblk, k.cols, g * kCG, (g + 1) * kCG, bf16, out.sc.data());
    });
}

// ---- digests -------------------------------------------------------------------
inline uint64_t fmix(uint64_t x) {
    x ^= x >> 33;
    x *= 0xff51afd7ed558ccdull;
    x ^= x >> 33;
    x *= 0xc4ceb9fe1a85ec53ull;
    x ^= x >> 33;
    return x;
}

// 64-bit digest of a byte range: 8-byte lanes, each mixed with its offset and
// folded multiply-rotate; the length seeds the state. Not cryptographic: it
// tells a cache written by this packer from a damaged or foreign one.
uint64_t digest_bytes(const uint8_t* p, size_t n) {
    uint64_t h = fmix(uint64_t(n) ^ 0x9e3779b97f4a7c15ull);
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        uint64_t w;
        std::memcpy(&w, p + i, 8);
        h = (h ^ fmix(w ^ uint64_t(i))) * 0x9e3779b97f4a7c15ull;
        h = (h << 29) | (h >> 35);
    }
    for (; i < n; ++i) h = (h ^ p[i]) * 0x100000001b3ull;
    return fmix(h);
}

// Digest in 1 MiB chunks (hashed in parallel) folded in chunk order, so the
// value does not depend on the thread count.
constexpr size_t kChunk = size_t(1) << 20;
uint64_t digest(const void* data, size_t n, uint32_t threads) {
    const uint8_t* p = static_cast<const uint8_t*>(data);
    const uint32_t nc = uint32_t((n + kChunk - 1) / kChunk);
    std::vector<uint64_t> part(nc);
    parallel_for(nc, threads, [&](uint32_t c) {
        const size_t off = size_t(c) * kChunk;
        part[c] = digest_bytes(p + off, std::min(kChunk, n - off));
    });
    uint64_t h = fmix(uint64_t(n));
    for (uint64_t v : part) h = fmix(h ^ v) + 0x632be59bd9b4e019ull;
    return h;
}

// ---- the cache file ------------------------------------------------------------
// [CacheHeader][payload: wq then sc of each entry, in task order][entry table]
constexpr char kMagic[8] = {'X', 'P', 'O', 'S', 'E', 'P', 'K', '1'};
constexpr uint32_t kCacheVersion = 1;
constexpr uint32_t kNameCap = 88;

struct CacheHeader {
    char magic[8];
    uint32_t version, header_bytes;
    uint64_t src_bytes, src_mtime_ns, src_stamp;   // the model file the cache was packed from
    int32_t scale_fmt;
    uint32_t packer_rev, n_entries, entry_bytes;
    uint64_t table_at, file_bytes;
    uint8_t pad[56];
};
static_assert(sizeof(CacheHeader) == 128, "cache header is 128 bytes");

struct CacheEntry {
    char name[kNameCap];
    uint32_t rows, cols;
    uint64_t at, wq_bytes, sc_bytes, digest;
};
static_assert(sizeof(CacheEntry) == 128, "cache entry is 128 bytes");

// Size, modification time and a digest of the first and last 64 KiB of the
// model file: a replaced or edited model does not match its old cache.
bool stamp(const std::string& path, uint64_t& bytes, uint64_t& mtime_ns, uint64_t& st) {
    struct stat sb {};
    if (::stat(path.c_str(), &sb) != 0) return false;
    bytes = uint64_t(sb.st_size);
    mtime_ns = uint64_t(sb.st_mtim.tv_sec) * 1000000000ull + uint64_t(sb.st_mtim.tv_nsec);
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return false;
    const size_t w = size_t(std::min<uint64_t>(bytes, 64u << 10));
    std::vector<uint8_t> buf(w);
    uint64_t h = bytes;
    for (int end = 0; end < 2; ++end) {
        const off_t off = end ? off_t(bytes - w) : 0;
        if (::pread(fd, buf.data(), w, off) != ssize_t(w)) {
            ::close(fd);
            return false;
        }
        h = fmix(h ^ digest_bytes(buf.data(), w));
    }
    ::close(fd);
    st = h;
    return true;
}

bool read_all(int fd, void* dst, size_t n) {
    uint8_t* p = static_cast<uint8_t*>(dst);
    while (n) {
        const ssize_t r = ::read(fd, p, n);
        if (r <= 0) return false;
        p += r;
        n -= size_t(r);
    }
    return true;
}
bool write_all(int fd, const void* src, size_t n) {
    const uint8_t* p = static_cast<const uint8_t*>(src);
    while (n) {
        const ssize_t r = ::write(fd, p, n);
        if (r <= 0) return false;
        p += r;
        n -= size_t(r);
    }
    return true;
}

CacheHeader expected_header(const std::string& model, int fmt, uint32_t n, bool& ok) {
    CacheHeader h{};
    std::memcpy(h.magic, kMagic, 8);
    h.version = kCacheVersion;
    h.header_bytes = sizeof(CacheHeader);
    h.scale_fmt = fmt;
    h.packer_rev = kPackerRev;
    h.n_entries = n;
    h.entry_bytes = sizeof(CacheEntry);
    ok = stamp(model, h.src_bytes, h.src_mtime_ns, h.src_stamp);
    return h;
}

// Opens `path` and checks everything short of the payload digests against
// what packing `tasks` from the model would produce. Returns the fd
// positioned at the first payload byte and the entry table, or -1 with the
// reason in *why.
int open_cache(const std::string& path, const CacheHeader& want, const std::vector<Task>& tasks,
               bool bf16, std::vector<CacheEntry>& table, std::string* why) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        *why = "no cache file";
        return -1;
    }
    auto reject = [&](const char* r) {
        *why = r;
        ::close(fd);
        return -1;
    };
    struct stat sb {};
    if (::fstat(fd, &sb) != 0) return reject("cannot stat the cache");
    CacheHeader h{};
    if (!read_all(fd, &h, sizeof h)) return reject("truncated header");
    if (std::memcmp(h.magic, kMagic, 8) != 0) return reject("not a cache file");
    if (h.version != want.version || h.header_bytes != want.header_bytes ||
        h.entry_bytes != want.entry_bytes)
        return reject("cache format differs");
    if (h.src_bytes != want.src_bytes || h.src_mtime_ns != want.src_mtime_ns ||
        h.src_stamp != want.src_stamp)
        return reject("the model file changed");
    if (h.scale_fmt != want.scale_fmt) return reject("scale format differs");
    if (h.packer_rev != want.packer_rev) return reject("packer revision differs");
    if (h.n_entries != want.n_entries) return reject("matrix count differs");
    if (h.file_bytes != uint64_t(sb.st_size)) return reject("cache size differs from its header");
    if (h.table_at < sizeof(CacheHeader) ||
        h.table_at + uint64_t(h.n_entries) * sizeof(CacheEntry) != h.file_bytes)
        return reject("entry table does not end the file");
    table.resize(h.n_entries);
    if (::pread(fd, table.data(), table.size() * sizeof(CacheEntry), off_t(h.table_at)) !=
        ssize_t(table.size() * sizeof(CacheEntry)))
        return reject("truncated entry table");
    uint64_t at = sizeof(CacheHeader);
    for (size_t i = 0; i < tasks.size(); ++i) {
        const CacheEntry& e = table[i];
        if (strnlen(e.name, kNameCap) == kNameCap || tasks[i].name != e.name)
            return reject("matrix names or order differ");
        if (e.rows != tasks[i].rows || e.cols != tasks[i].cols) return reject("matrix shape differs");
        if (e.wq_bytes != wq_bytes(e.rows, e.cols) || e.sc_bytes != sc_bytes(e.rows, e.cols, bf16))
            return reject("entry sizes disagree with the shape");
        if (e.at != at) return reject("payload is not contiguous");
        at += e.wq_bytes + e.sc_bytes;
    }
    if (at != h.table_at) return reject("payload does not reach the table");
    if (::lseek(fd, off_t(sizeof(CacheHeader)), SEEK_SET) < 0) return reject("seek failed");
    return fd;
}

// Writes "<path>.tmp" entry by entry, then the table and header, and renames
// it over `path`: a partly written cache is never visible under its name.
class CacheWriter {
public:
    CacheWriter(const std::string& path, const CacheHeader& h) : path_(path), h_(h) {
        tmp_ = path + ".tmp";
        fd_ = ::open(tmp_.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
        const CacheHeader blank{};
        if (fd_ >= 0 && !write_all(fd_, &blank, sizeof blank)) drop();
    }
    ~CacheWriter() { drop(); }
    bool ok() const { return fd_ >= 0; }
    void add(const Task& k, const Packed& p, uint32_t threads) {
        if (fd_ < 0) return;
        CacheEntry e{};
        std::snprintf(e.name, kNameCap, "%s", k.name.c_str());
        e.rows = k.rows;
        e.cols = k.cols;
        e.at = at_;
        e.wq_bytes = p.wq.size() * 4;
        e.sc_bytes = p.sc.size();
        e.digest = fmix(digest(p.wq.data(), e.wq_bytes, threads) ^ (digest(p.sc.data(), e.sc_bytes, threads) * 3));
        if (!write_all(fd_, p.wq.data(), e.wq_bytes) || !write_all(fd_, p.sc.data(), e.sc_bytes)) {
            drop();
            return;
        }
        at_ += e.wq_bytes + e.sc_bytes;
        table_.push_back(e);
    }
    bool finish() {
        if (fd_ < 0 || table_.size() != h_.n_entries) {
            drop();
            return false;
        }
        h_.table_at = at_;
        h_.file_bytes = at_ + table_.size() * sizeof(CacheEntry);
        bool good = write_all(fd_, table_.data(), table_.size() * sizeof(CacheEntry)) &&
                    ::lseek(fd_, 0, SEEK_SET) == 0 && write_all(fd_, &h_, sizeof h_) &&
                    ::fsync(fd_) == 0;
        good = ::close(fd_) == 0 && good;
        fd_ = -1;
        if (good && ::rename(tmp_.c_str(), path_.c_str()) == 0) return true;
        ::unlink(tmp_.c_str());
        return false;
    }

private:
    void drop() {
        if (fd_ >= 0) {
            ::close(fd_);
            ::unlink(tmp_.c_str());
        }
        fd_ = -1;
    }
    std::string path_, tmp_;
    CacheHeader h_;
    int fd_ = -1;
    uint64_t at_ = sizeof(CacheHeader);
    std::vector<CacheEntry> table_;
};

// ---- the model's matrices --------------------------------------------------------
// Validated before anything is packed: present, 2-D with the expected
// (rows, cols), dequantisable row by row, block-divisible.
std::vector<Task> model_tasks(const gguf::File& f, const xp_config& c, bool bf16) {
    const uint32_t H = c.hidden, qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    std::vector<Task> tasks;
    auto add = [&](const std::string& name, uint32_t rows, uint32_t cols, int layer, int id) {
        const gguf::Tensor* t = f.tensor(name);
        if (!t) throw std::runtime_error("the model has no tensor '" + name + "'");
        if (t->n_dims != 2 || t->dims[0] != rows || t->dims[1] != cols)
            throw std::runtime_error("tensor '" + name + "' is not {" + std::to_string(rows) + ", " +
                                     std::to_string(cols) + "}");
        const gguf::BlockFormat& bf = gguf::block_format(t->type);
        if (!bf.dequant)
            throw std::runtime_error("tensor '" + name + "' has type " + bf.name +
                                     ", which this loader does not dequantise");
        if (rows % bf.elems)
            throw std::runtime_error("tensor '" + name + "' rows of " + std::to_string(rows) +
                                     " are not whole " + bf.name + " blocks");
        if (rows % kQB || (bf16 && (rows / kQB) % 4) || cols % kCG)
            throw std::runtime_error("tensor '" + name + "' shape does not fit the packing (rows a " +
                                     "multiple of " + std::to_string(bf16 ? 128 : 32) +
                                     ", columns of 64)");
        if (name.size() >= kNameCap) throw std::runtime_error("tensor name '" + name + "' too long");
        Task k;
        k.name = name;
        k.t = t;
        k.rows = rows;
        k.cols = cols;
        k.layer = layer;
        k.id = id;
        tasks.push_back(k);
    };
    static const char* kName[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate",
                                   "ffn_up", "ffn_down"};
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        const uint32_t rows[7] = {H, H, H, qd, H, H, c.ffn};
        const uint32_t cols[7] = {qd, kvd, kvd, H, c.ffn, c.ffn, H};
        for (int m = 0; m < 7; ++m) add(p + kName[m] + ".weight", rows[m], cols[m], int(l), m);
    }
    // Gemma ties the output head to the embedding; an untied model has output.weight.
    add(f.tensor("output.weight") ? "output.weight" : "token_embd.weight", H, c.vocab, -1,
        XP_T_LM_HEAD);
    return tasks;
}

void check_shape(const gguf::File& f, const xp_config& c) {
    const gguf::ModelShape m = f.shape();
    auto need = [&](const char* what, uint32_t file, uint32_t cfg) {
        if (file && file != cfg)
            throw std::runtime_error(std::string("config ") + what + " = " + std::to_string(cfg) +
                                     " but the model has " + std::to_string(file));
    };
    need("n_layers", m.layers, c.n_layers);
    need("hidden", m.hidden, c.hidden);
    need("ffn", m.ffn, c.ffn);
    need("n_heads", m.heads, c.n_heads);
    need("n_kv_heads", m.kv_heads, c.n_kv_heads);
    need("head_dim", m.head_dim(), c.head_dim);
    need("vocab", m.vocab, c.vocab);
}

bool bf16_fmt(int fmt) {
    if (fmt == XP_SCALE_BF16_QUAD) return true;
    if (fmt == XP_SCALE_F32) return false;
    throw std::runtime_error("a GGUF model packs to bf16 quad or fp32 scales (scale_fmt " +
                             std::to_string(fmt) + ")");
}

// Packs (or reads from a valid cache) every matrix, handing each to `sink`.
void load_matrices(const gguf::File& f, const xp_config& c, const char* cache, bool repack,
                   uint32_t threads, xp_load_stats& st,
                   const std::function<void(const Task&, const Packed&)>& sink) {
    const bool bf16 = bf16_fmt(c.scale_fmt);
    const std::vector<Task> tasks = model_tasks(f, c, bf16);
    st.n_tensors = uint32_t(tasks.size());
    st.threads = threads;
    bool stamped = false;
    const CacheHeader want = expected_header(f.path(), c.scale_fmt, uint32_t(tasks.size()), stamped);
    const bool use_cache = cache && *cache && stamped;
    if (use_cache && !repack) {
        std::vector<CacheEntry> table;
        std::string why;
        const int fd = open_cache(cache, want, tasks, bf16, table, &why);
        if (fd >= 0) {
            const double t0 = now_ms();
            bool good = true;
            Packed p;
            for (size_t i = 0; i < tasks.size() && good; ++i) {
                p.wq.resize(table[i].wq_bytes / 4);
                p.sc.resize(table[i].sc_bytes);
                good = read_all(fd, p.wq.data(), table[i].wq_bytes) &&
                       read_all(fd, p.sc.data(), table[i].sc_bytes) &&
                       fmix(digest(p.wq.data(), table[i].wq_bytes, threads) ^
                            (digest(p.sc.data(), table[i].sc_bytes, threads) * 3)) == table[i].digest;
                if (good) {
                    st.cache_ms += now_ms() - t0;
                    sink(tasks[i], p);
                    st.packed_bytes += table[i].wq_bytes + table[i].sc_bytes;
                }
            }
            ::close(fd);
            if (good) {
                st.from_cache = 1;
                return;
            }
            st.packed_bytes = 0;   // a damaged entry: repack everything below
        }
    }
    std::unique_ptr<CacheWriter> w;
    if (use_cache) {
        w.reset(new CacheWriter(cache, want));
        if (!w->ok()) w.reset();
    }
    Packed p;
    for (const Task& k : tasks) {
        const double t0 = now_ms();
        pack_task(k, bf16, threads, p);
        st.pack_ms += now_ms() - t0;
        if (w) {
            const double t1 = now_ms();
            w->add(k, p, threads);
            st.cache_ms += now_ms() - t1;
        }
        sink(k, p);
        st.packed_bytes += p.wq.size() * 4 + p.sc.size();
    }
    if (w) {
        const double t1 = now_ms();
        st.cache_written = w->finish() ? 1 : 0;
        st.cache_ms += now_ms() - t1;
    }
}

template <class F>
int guarded(const char* who, F&& fn) {
    try {
        return fn();
    } catch (const std::bad_alloc&) {
        return set_error(XP_E_NOMEM, "%s: out of host memory", who);
    } catch (const std::exception& e) {
        return set_error(XP_E_FORMAT, "%s: %s", who, e.what());
    }
}

}  // namespace
}  // namespace xp::pack

using namespace xp;
using namespace xp::pack;

extern "C" {

int xp_config_from_gguf(xp_gguf* g, xp_config* c) {
    XP_REQUIRE(g && c, "null pointer");
    const gguf::ModelShape m = g->f->shape();
    if (m.layers) c->n_layers = m.layers;
    if (m.heads) c->n_heads = m.heads;
    if (m.kv_heads) c->n_kv_heads = m.kv_heads;
    if (m.hidden) c->hidden = m.hidden;
    if (m.ffn) c->ffn = m.ffn;
    if (m.head_dim()) c->head_dim = m.head_dim();
    if (m.vocab) c->vocab = m.vocab;
    c->rms_eps = m.rms_eps;
    c->rope_theta_global = m.rope_base;
    // A window the caller moved off the default is a command-line choice and
    // survives the merge (decode.cpp:1427-1434); otherwise the file's extent.
    xp_config d;
    xp_config_gemma3_1b(&d);
    if (m.sliding_window && c->sliding_window == d.sliding_window)
        c->sliding_window = m.sliding_window;
    return XP_OK;
}

int xp_pack_int4(const float* w, uint32_t rows, uint32_t cols, int scale_fmt, uint32_t threads,
                 void* wq, void* sc) {
    XP_REQUIRE(w && wq && sc, "null pointer");
    XP_REQUIRE(scale_fmt == XP_SCALE_BF16_QUAD || scale_fmt == XP_SCALE_F32,
               "scale_fmt %d: bf16 quad or fp32", scale_fmt);
    const bool bf16 = scale_fmt == XP_SCALE_BF16_QUAD;
    XP_REQUIRE(rows > 0 && rows % (bf16 ? 128 : 32) == 0, "rows=%u must be a positive multiple of %d",
               rows, bf16 ? 128 : 32);
    XP_REQUIRE(cols > 0 && cols % 64 == 0, "cols=%u must be a positive multiple of 64", cols);
    return guarded("xp_pack_int4", [&] {
        const uint32_t nblk = rows / 32;
        std::vector<float> sf(size_t(nblk) * cols);
        parallel_for(cols / 64, n_threads(threads), [&](uint32_t g) {
            pack_group(w + size_t(g) * 64 * rows, rows, cols, g, bf16, static_cast<uint32_t*>(wq),
                       sf.data());
            write_scales(sf.data(), nblk, cols, g * 64, (g + 1) * 64, bf16, sc);
        });
        return XP_OK;
    });
}

int xp_gguf_pack_model(xp_gguf* g, const xp_config* c, const char* cache_path, uint32_t threads,
                       xp_load_stats* st) {
    XP_REQUIRE(g && c && cache_path, "null pointer");
    xp_load_stats local{};
    xp_load_stats& s = st ? *st : local;
    s = xp_load_stats{};
    const double t0 = now_ms();
    const int rc = guarded("xp_gguf_pack_model", [&] {
        check_shape(*g->f, *c);
        load_matrices(*g->f, *c, cache_path, true, n_threads(threads), s,
                      [](const Task&, const Packed&) {});
        if (!s.cache_written) throw std::runtime_error(std::string("could not write ") + cache_path);
        return XP_OK;
    });
    s.total_ms = now_ms() - t0;
    return rc;
}

int xp_gguf_verify_cache(xp_gguf* g, const xp_config* c, const char* cache_path,
                         uint32_t threads, uint32_t* mismatches) {
    XP_REQUIRE(g && c && cache_path && mismatches, "null pointer");
    *mismatches = 0;
    return guarded("xp_gguf_verify_cache", [&] {
        check_shape(*g->f, *c);
        const bool bf16 = bf16_fmt(c->scale_fmt);
        const std::vector<Task> tasks = model_tasks(*g->f, *c, bf16);
        bool stamped = false;
        const CacheHeader want = expected_header(g->f->path(), c->scale_fmt, uint32_t(tasks.size()), stamped);
        if (!stamped) throw std::runtime_error("cannot stamp the model file");
        std::vector<CacheEntry> table;
        std::string why;
        const int fd = open_cache(cache_path, want, tasks, bf16, table, &why);
        if (fd < 0) throw std::runtime_error("no valid cache at " + std::string(cache_path) + " (" + why + ")");
        Packed fresh;
        std::vector<uint8_t> disk;
        uint32_t bad = 0;
        bool short_read = false;
        for (size_t i = 0; i < tasks.size(); ++i) {
            pack_task(tasks[i], bf16, n_threads(threads), fresh);
            const size_t wb = fresh.wq.size() * 4, sb = fresh.sc.size();
            disk.resize(wb + sb);
            if (!read_all(fd, disk.data(), disk.size())) {
                short_read = true;
                bad += uint32_t(tasks.size() - i);
                break;
            }
            if (std::memcmp(disk.data(), fresh.wq.data(), wb) != 0 ||
                std::memcmp(disk.data() + wb, fresh.sc.data(), sb) != 0)
                ++bad;
        }
        ::close(fd);
        *mismatches = bad;
        if (short_read) throw std::runtime_error("cache payload is short");
        return XP_OK;
    });
}

int xp_session_load_gguf(xp_session* s, xp_gguf* g, const char* cache_path, uint32_t flags,
                         uint32_t threads, xp_load_stats* st) {
    XP_REQUIRE(s && g, "null pointer");
    SessionWeights sw;
    int rc = session_weights(s, &sw);
    if (rc != XP_OK) return rc;
    const xp_config c = sw.cfg;
    xp_load_stats local{};
    xp_load_stats& ls = st ? *st : local;
    ls = xp_load_stats{};
    const double t0 = now_ms();
    const uint32_t nt = n_threads(threads);
    rc = guarded("xp_session_load_gguf", [&] {
        const gguf::File& f = *g->f;
        check_shape(f, c);
        int urc = XP_OK;
        auto upload = [&](int layer, int id, const void* host, size_t bytes, size_t off = 0) {
            if (urc != XP_OK) return;
            const double u0 = now_ms();
            urc = xp_session_upload_part(s, layer, id, off, host, bytes);
            ls.upload_ms += now_ms() - u0;
        };
        load_matrices(f, c, cache_path, (flags & XP_LOAD_REPACK) != 0, nt, ls,
                      [&](const Task& k, const Packed& p) {
                          upload(k.layer, k.id, p.wq.data(), p.wq.size() * 4);
                          upload(k.layer, k.id | XP_T_SCALES, p.sc.data(), p.sc.size());
                      });
        if (urc != XP_OK) return urc;
        // Norms: the file holds 1 + w for Gemma's (1 + w) norms; the kernels
        // apply 1 + w to what they are given (decode.cpp:1490-1515).
        auto norm = [&](const std::string& name, int layer, int id, uint32_t n) {
            const gguf::Tensor* t = f.tensor(name);
            if (!t) throw std::runtime_error("the model has no tensor '" + name + "'");
            if (t->elements() != n)
                throw std::runtime_error("norm '" + name + "' has " + std::to_string(t->elements()) +
                                         " elements, want " + std::to_string(n));
            std::vector<float> v(n);
            if (!gguf::dequantize(t->type, t->data, v.data(), n))
                throw std::runtime_error("norm '" + name + "' cannot be dequantised");
            if (!(flags & XP_LOAD_NORM_RAW))
                for (float& x : v) x -= 1.0f;
            upload(layer, id, v.data(), size_t(n) * 4);
        };
        static const char* kNorm[6] = {"attn_norm", "post_attention_norm", "ffn_norm",
                                       "post_ffw_norm", "attn_q_norm", "attn_k_norm"};
        for (uint32_t l = 0; l < c.n_layers; ++l)
            for (int i = 0; i < 6; ++i)
                norm("blk." + std::to_string(l) + "." + kNorm[i] + ".weight", int(l),
                     XP_T_ATTN_NORM + i, i >= 4 ? c.head_dim : c.hidden);
        norm("output_norm.weight", -1, XP_T_FINAL_NORM, c.hidden);
        if (urc != XP_OK) return urc;
        // The embedding rows at the file's own precision, streamed to the
        // device 4096 rows at a time.
        if (!(flags & XP_LOAD_NO_EMBED)) {
            const gguf::Tensor* t = f.tensor("token_embd.weight");
            if (!t) throw std::runtime_error("the model has no tensor 'token_embd.weight'");
            if (t->n_dims != 2 || t->dims[0] != c.hidden || t->dims[1] != c.vocab)
                throw std::runtime_error("token_embd.weight is not {hidden, vocab}");
            constexpr uint32_t kRows = 4096;
            std::vector<float> rows(size_t(kRows) * c.hidden);
            for (uint32_t r0 = 0; r0 < c.vocab && urc == XP_OK; r0 += kRows) {
                const uint32_t n = std::min(kRows, c.vocab - r0);
                const uint32_t per = (n + nt - 1) / nt;
                parallel_for((n + per - 1) / per, nt, [&](uint32_t i) {
                    const uint32_t a = i * per, b = std::min(n, a + per);
                    gguf::dequantize_rows(*t, r0 + a, b - a, rows.data() + size_t(a) * c.hidden);
                });
                upload(-1, XP_T_EMBED, rows.data(), size_t(n) * c.hidden * 4,
                       size_t(r0) * c.hidden * 4);
            }
        }
        return urc;
    });
    ls.total_ms = now_ms() - t0;
    return rc;
}

}  // extern "C"
