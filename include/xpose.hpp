// xpose.hpp — C++ host interface of the MI355X Gemma-3 decode path.
//
// Mirrors vulkore::llm::DecodeSession (examples/llm/decode.hpp:605-676) over
// the C ABI of xpose.h, so the reference's callers (the decode CLI,
// examples/llm/decode.cpp:2720-3006, and the Android JNI layer,
// android/app/src/main/cpp/llm_jni.cpp:110-164) switch by changing the class
// they construct:
//
//   reference                                 here
//   DecodeSession(Paths, DecodeConfig)        DecodeSession(Model, Config, cache) (GGUF,
//                                             requantised or from the pack cache), or
//                                             DecodeSession(Config) + upload / synthesize
//   GGUFFile::open, --verify-cache            Model(path), Model::verify_cache
//   prefill(std::span<const uint32_t>)        prefill(const uint32_t*, size_t) /
//                                             prefill(const std::vector<uint32_t>&)
//   uint32_t decode_step()                    uint32_t decode_step()
//   reset(), position(), config()             same
//   last_metrics(), last_logits()             same (Metrics mirrors the reference's)
//   last_candidates()                         same ((value, index) pairs)
//   weight_bytes(), kv_bytes(), device_name() same
//
// Errors are exceptions, as in the reference (check.hpp:16-35, decode.cpp:
// 46-56): every failing entry point throws std::runtime_error carrying the
// entry point's name and the library's message. Header-only; link libxpose.so.
#ifndef XPOSE_HPP
#define XPOSE_HPP

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "xpose.h"

namespace xpose {

inline void check(int rc, const char* what) {
    if (rc != XP_OK)
        throw std::runtime_error(std::string(what) + " failed (" + std::to_string(rc) +
                                 "): " + xp_last_error());
}

namespace llm {

// The reference's Sampling + DecodeConfig, one struct (decode.hpp:153-436).
struct Config : xp_config {
    Config() { xp_config_gemma3_1b(this); }
    static Config gemma3_1b() { return Config(); }
};

// decode.hpp:573-582, with the execution mode in place of submits.
struct Metrics {
    double   ms             = 0;
    double   gpu_ms         = 0;
    double   sample_ms      = 0;
    double   tokens_per_sec = 0;
    uint32_t dispatches     = 0;   // kernel launches per token step
    uint32_t position       = 0;
    int32_t  exec_mode      = 0;   // XP_EXEC_TOKEN, _GRAPH or _LAUNCH
};

// A GGUF model file (GGUFFile, examples/llm/model/gguf.hpp:173-215).
class Model {
public:
    explicit Model(const std::string& path) : path_(path) {
        check(xp_gguf_open(path.c_str(), &g_), "xp_gguf_open");
    }
    ~Model() {
        if (g_) xp_gguf_close(g_);
    }
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    // The file's shapes over `base` (DecodeConfig::from_model, decode.cpp:258-275);
    // a GGUF model packs to bf16 scales unless fp32 is asked for.
    Config config(Config base = Config()) const {
        check(xp_config_from_gguf(g_, &base), "xp_config_from_gguf");
        if (base.scale_fmt != XP_SCALE_F32) base.scale_fmt = XP_SCALE_BF16_QUAD;
        return base;
    }
    // --verify-cache (decode.cpp:2580-2661): repack and compare the cache
    // byte for byte; returns the number of matrices that differ.
    uint32_t verify_cache(const Config& c, const std::string& cache, uint32_t threads = 0) const {
        uint32_t bad = 0;
        check(xp_gguf_verify_cache(g_, &c, cache.c_str(), threads, &bad), "xp_gguf_verify_cache");
        return bad;
    }
    const std::string& path() const { return path_; }
    xp_gguf* handle() const { return g_; }

private:
    std::string path_;
    xp_gguf* g_ = nullptr;
};

// The model's SentencePiece tokenizer (Tokenizer, model/tokenizer.hpp:46-94).
// Borrows the Model's strings: destroy it before the Model.
class Tokenizer {
public:
    explicit Tokenizer(const Model& m) {
        check(xp_tokenizer_create(m.handle(), &t_), "xp_tokenizer_create");
        check(xp_tokenizer_info(t_, &ids_), "xp_tokenizer_info");
    }
    ~Tokenizer() {
        if (t_) xp_tokenizer_destroy(t_);
    }
    Tokenizer(const Tokenizer&) = delete;
    Tokenizer& operator=(const Tokenizer&) = delete;

    std::vector<uint32_t> encode(const std::string& text, bool add_bos, bool add_eos = false) const {
        size_t n = 0;
        check(xp_tokenize(t_, text.data(), text.size(), add_bos, add_eos, nullptr, 0, &n), "xp_tokenize");
        std::vector<int32_t> ids(n);
        check(xp_tokenize(t_, text.data(), text.size(), add_bos, add_eos, ids.data(), n, &n),
              "xp_tokenize");
        return std::vector<uint32_t>(ids.begin(), ids.end());
    }
    std::string decode(const std::vector<int32_t>& ids, bool skip_special = true) const {
        size_t n = 0;
        check(xp_detokenize(t_, ids.data(), ids.size(), skip_special, nullptr, 0, &n), "xp_detokenize");
        std::string s(n + 1, '\0');
        check(xp_detokenize(t_, ids.data(), ids.size(), skip_special, &s[0], s.size(), &n),
              "xp_detokenize");
        s.resize(n);
        return s;
    }
    std::string decode_one(int32_t id) const {
        size_t n = 0;
        check(xp_token_piece(t_, id, nullptr, 0, &n), "xp_token_piece");
        std::string s(n + 1, '\0');
        check(xp_token_piece(t_, id, &s[0], s.size(), &n), "xp_token_piece");
        s.resize(n);
        return s;
    }
    int32_t id_for(const std::string& spelling) const {
        int32_t id = -1;
        check(xp_token_find(t_, spelling.data(), spelling.size(), &id), "xp_token_find");
        return id;
    }
    int32_t bos_id() const { return ids_.bos; }
    int32_t eos_id() const { return ids_.eos; }
    int32_t unk_id() const { return ids_.unk; }
    size_t vocab_size() const { return ids_.vocab; }

private:
    xp_tokenizer* t_ = nullptr;
    xp_tokenizer_ids ids_{};
};

class DecodeSession {
public:
    explicit DecodeSession(const Config& cfg) : cfg_(cfg) {
        check(xp_init(0), "xp_init");
        check(xp_session_create(&cfg_, &s_), "xp_session_create");
    }
    // The reference's DecodeSession(Paths, DecodeConfig): shapes from the
    // file, policy fields from `cfg`, weights requantised on load or read
    // from the pack cache at `cache` ("" = no cache), packed on `threads`
    // host threads (0 = all, Paths::pack_threads).
    DecodeSession(const Model& m, const Config& cfg, const std::string& cache = std::string(),
                  uint32_t flags = 0, uint32_t threads = 0)
        : DecodeSession(m.config(cfg)) {
        check(xp_session_load_gguf(s_, m.handle(), cache.empty() ? nullptr : cache.c_str(), flags,
                                   threads, &load_),
              "xp_session_load_gguf");
    }
    // Where the load time went (LoadStats, decode.hpp:584-603).
    const xp_load_stats& load_stats() const { return load_; }
    ~DecodeSession() {
        if (s_) xp_session_destroy(s_);
    }
    DecodeSession(const DecodeSession&) = delete;
    DecodeSession& operator=(const DecodeSession&) = delete;

    // Packed weights (KM4 nibble planes, quad scale planes, norm weights
    // stored as multiplier - 1): the reference's upload_packed
    // (decode.cpp:652) with the layout of xpose.h.
    void upload(int layer, int tensor, const void* host, size_t bytes) {
        check(xp_session_upload(s_, layer, tensor, host, bytes), "xp_session_upload");
    }
    // The seeded synthetic model of the benchmark configurations.
    void synthesize(uint32_t seed) { check(xp_session_synthesize(s_, seed), "xp_session_synthesize"); }
    void set_position(uint32_t pos) { check(xp_session_set_position(s_, pos), "xp_session_set_position"); }
    void set_spin_limit(uint32_t rounds) {
        check(xp_session_set_spin_limit(s_, rounds), "xp_session_set_spin_limit");
    }
    void kv_upload(int layer, int which, uint32_t pos0, uint32_t n, const uint16_t* rows) {
        check(xp_session_kv_upload(s_, layer, which, pos0, n, rows), "xp_session_kv_upload");
    }

    void prefill(const uint32_t* ids, size_t n) {
        check(xp_session_prefill(s_, ids, uint32_t(n)), "xp_session_prefill");
    }
    void prefill(const std::vector<uint32_t>& ids) { prefill(ids.data(), ids.size()); }

    uint32_t decode_step() {
        uint32_t t = 0;
        check(xp_session_decode_step(s_, &t), "xp_session_decode_step");
        return t;
    }
    // n greedy steps queued behind one wait (greedy mode only).
    std::vector<uint32_t> decode_steps(uint32_t n) {
        std::vector<uint32_t> out(n);
        check(xp_session_decode_steps(s_, n, out.data()), "xp_session_decode_steps");
        return out;
    }
    void reset() { check(xp_session_reset(s_), "xp_session_reset"); }

    uint32_t position() const {
        uint32_t p = 0;
        check(xp_session_position(s_, &p), "xp_session_position");
        return p;
    }
    const Config& config() const { return cfg_; }
    Metrics last_metrics() const {
        xp_metrics m{};
        check(xp_session_last_metrics(s_, &m), "xp_session_last_metrics");
        Metrics r;
        r.ms = m.ms;
        r.gpu_ms = m.gpu_ms;
        r.sample_ms = m.sample_ms;
        r.tokens_per_sec = m.tokens_per_sec;
        r.dispatches = m.launches;
        r.position = m.position;
        r.exec_mode = m.exec_mode;
        return r;
    }
    std::vector<float> last_logits() const {
        std::vector<float> v(cfg_.vocab);
        check(xp_session_last_logits(s_, v.data(), cfg_.vocab), "xp_session_last_logits");
        return v;
    }
    std::vector<std::pair<float, uint32_t>> last_candidates() const {
        const uint32_t n = 4 * cfg_.topk_parts;
        std::vector<float> v(n);
        std::vector<uint32_t> i(n);
        check(xp_session_last_candidates(s_, v.data(), i.data(), n), "xp_session_last_candidates");
        std::vector<std::pair<float, uint32_t>> r;
        r.reserve(n);
        for (uint32_t k = 0; k < n; ++k)
            if (i[k] != 0xFFFFFFFFu) r.emplace_back(v[k], i[k]);
        return r;
    }
    uint64_t weight_bytes() const {
        size_t b = 0;
        check(xp_session_weight_bytes(s_, &b), "xp_session_weight_bytes");
        return b;
    }
    uint64_t kv_bytes() const {
        size_t b = 0;
        check(xp_session_kv_bytes(s_, &b), "xp_session_kv_bytes");
        return b;
    }
    std::string device_name() const {
        char name[256] = {0}, arch[64] = {0};
        int n_cu = 0;
        size_t hbm = 0;
        check(xp_device_info(name, sizeof name, &n_cu, &hbm, arch, sizeof arch), "xp_device_info");
        return std::string(name) + " (" + arch + ")";
    }

private:
    Config cfg_;
    xp_session* s_ = nullptr;
    xp_load_stats load_{};
};

}  // namespace llm
}  // namespace xpose

#endif  // XPOSE_HPP
