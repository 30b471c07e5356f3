// SentencePiece tokenizer from GGUF metadata, host side. Replaces
// vulkore::llm::Tokenizer (examples/llm/model/tokenizer.hpp:46-94,
// tokenizer.cpp:70-374).
//
// The GGUF file carries the vocabulary: tokenizer.ggml.tokens (spellings,
// U+2581 standing for a space), .scores (merge priority), .token_type (1
// normal, 2 unknown, 3 control, 4 user-defined, 5 unused, 6 byte), the
// bos / eos / unknown / padding ids and the add_bos / add_eos /
// add_space_prefix flags.
//
// encode: control and unknown tokens are cut out of the text first (longest
// spelling wins, probing one lookup per distinct spelling length); each
// remaining fragment is normalised (spaces to U+2581, one leading U+2581 when
// add_space_prefix), split into UTF-8 characters, and adjacent symbols are
// merged while their concatenation is a vocabulary spelling, best score first
// and the leftmost pair on a tie; a symbol left without a spelling falls
// back to its bytes' "<0xAB>" tokens (or the unknown id).
// decode: byte tokens become their byte, U+2581 a space; the first text
// piece loses the space the prefix added; control / unknown tokens are
// skipped on request.
#include <algorithm>
#include <cstring>
#include <memory>
#include <queue>
#include <stdexcept>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "gguf.hpp"
#include "xp_internal.hpp"

namespace xp::tok {
namespace {

constexpr std::string_view kSpace = "\xe2\x96\x81";   // U+2581
enum : int32_t { kNormal = 1, kUnknown = 2, kControl = 3, kByte = 6 };

[[noreturn]] void bad(const std::string& m) { throw std::runtime_error("tokenizer: " + m); }

size_t char_bytes(unsigned char c) {
    return c < 0x80 ? 1 : (c & 0xE0) == 0xC0 ? 2 : (c & 0xF0) == 0xE0 ? 3 : (c & 0xF8) == 0xF0 ? 4 : 1;
}

int hexval(char c) {
    return c >= '0' && c <= '9' ? c - '0' : c >= 'A' && c <= 'F' ? c - 'A' + 10
         : c >= 'a' && c <= 'f' ? c - 'a' + 10 : -1;
}

// A six-character "<0x..>" spelling: its value from one or two hex digits
// after "<0x" (the reference reads it with "%02X"), else -1.
int byte_spelling(std::string_view s) {
    if (s.size() != 6 || s.compare(0, 3, "<0x") != 0 || s[5] != '>') return -1;
    const int hi = hexval(s[3]), lo = hexval(s[4]);
    if (hi < 0) return -1;
    return lo < 0 ? hi : hi * 16 + lo;
}

}  // namespace

class Tokenizer {
public:
    explicit Tokenizer(const gguf::File& f) {
        const gguf::Value* t = f.meta("tokenizer.ggml.tokens");
        if (!t || t->kind != gguf::kMArr || t->elem != gguf::kMStr)
            bad("tokenizer.ggml.tokens is missing or not a string array");
        text_ = t->strs;
        const size_t n = text_.size();
        score_.assign(n, 0.0f);
        if (const gguf::Value* s = f.meta("tokenizer.ggml.scores")) {
            if (s->nums.size() != n) bad("scores and tokens differ in length");
            for (size_t i = 0; i < n; ++i) score_[i] = float(s->nums[i]);
        }
        kind_.assign(n, kNormal);
        if (const gguf::Value* k = f.meta("tokenizer.ggml.token_type")) {
            if (k->nums.size() != n) bad("token_type and tokens differ in length");
            for (size_t i = 0; i < n; ++i) kind_[i] = int32_t(k->nums[i]);
        }
        auto id = [&](const char* key) {
            const gguf::Value* v = f.meta(key);
            return v ? int32_t(v->u) : -1;
        };
        auto flag = [&](const char* key, bool dflt) {
            const gguf::Value* v = f.meta(key);
            return v ? v->u != 0 : dflt;
        };
        bos = id("tokenizer.ggml.bos_token_id");
        eos = id("tokenizer.ggml.eos_token_id");
        unk = id("tokenizer.ggml.unknown_token_id");
        pad = id("tokenizer.ggml.padding_token_id");
        add_bos = flag("tokenizer.ggml.add_bos_token", true);
        add_eos = flag("tokenizer.ggml.add_eos_token", false);
        prefix = flag("tokenizer.ggml.add_space_prefix", true);
        index_.reserve(n * 2);
        std::vector<size_t> lens;
        for (size_t i = 0; i < n; ++i) {
            index_.emplace(text_[i], int32_t(i));   // the lowest id keeps a shared spelling
            if (kind_[i] == kControl || kind_[i] == kUnknown) lens.push_back(text_[i].size());
            if (kind_[i] == kByte) {
                const int b = byte_spelling(text_[i]);
                if (b >= 0) byte_id_[b] = int32_t(i);
            }
        }
        std::sort(lens.begin(), lens.end(), std::greater<size_t>());
        lens.erase(std::unique(lens.begin(), lens.end()), lens.end());
        if (!lens.empty() && lens.back() == 0) lens.pop_back();
        special_lens_ = lens;
    }

    size_t size() const { return text_.size(); }
    int32_t kind(int32_t id) const { return id >= 0 && size_t(id) < kind_.size() ? kind_[id] : 0; }
    float score(int32_t id) const { return id >= 0 && size_t(id) < score_.size() ? score_[id] : 0.0f; }
    std::string_view text(int32_t id) const {
        return id >= 0 && size_t(id) < text_.size() ? text_[id] : std::string_view();
    }
    int32_t find(std::string_view s) const {
        const auto it = index_.find(s);
        return it == index_.end() ? -1 : it->second;
    }

    std::vector<int32_t> encode(std::string_view s, bool with_bos, bool with_eos) const {
        std::vector<int32_t> out;
        if (with_bos && bos >= 0) out.push_back(bos);
        size_t i = 0, start = 0;
        while (i < s.size()) {
            int32_t hit = -1;
            for (size_t len : special_lens_) {
                if (len > s.size() - i) continue;
                const int32_t id = find(s.substr(i, len));
                if (id >= 0 && (kind_[id] == kControl || kind_[id] == kUnknown)) {
                    hit = id;
                    break;
                }
            }
            if (hit < 0) {
                ++i;
                continue;
            }
            fragment(s.substr(start, i - start), out);
            out.push_back(hit);
            i += text_[hit].size();
            start = i;
        }
        fragment(s.substr(start), out);
        if (with_eos && eos >= 0) out.push_back(eos);
        return out;
    }

    std::string piece(int32_t id) const {
        const std::string_view s = text(id);
        if (kind(id) == kByte) {
            const int b = byte_spelling(s);
            return b >= 0 ? std::string(1, char(b)) : std::string(s);
        }
        std::string out;
        out.reserve(s.size());
        for (size_t i = 0; i < s.size();) {
            if (s.compare(i, kSpace.size(), kSpace) == 0) {
                out += ' ';
                i += kSpace.size();
            } else {
                out += s[i++];
            }
        }
        return out;
    }

    std::string decode(const int32_t* ids, size_t n, bool skip_special) const {
        std::string out;
        bool first = true;
        for (size_t i = 0; i < n; ++i) {
            const int32_t k = kind(ids[i]);
            const bool special = k == kControl || k == kUnknown;
            if (skip_special && special) continue;
            std::string p = piece(ids[i]);
            if (first && prefix && !p.empty() && p[0] == ' ') p.erase(0, 1);
            if (!special) first = false;
            out += p;
        }
        return out;
    }

    int32_t bos = -1, eos = -1, unk = -1, pad = -1;
    bool add_bos = true, add_eos = false, prefix = true;

private:
    // The merge loop over one fragment (no special tokens in it).
    void fragment(std::string_view raw, std::vector<int32_t>& out) const {
        if (raw.empty()) return;
        std::string s;
        s.reserve(raw.size() + 8);
        if (prefix) s += kSpace;
        for (char c : raw) {
            if (c == ' ') s += kSpace;
            else s += c;
        }
        // symbols: [at, at + len) of s, doubly linked in order
        struct Sym { size_t at, len; int prev, next; };
        std::vector<Sym> sym;
        for (size_t i = 0; i < s.size();) {
            const size_t len = std::min(char_bytes(static_cast<unsigned char>(s[i])), s.size() - i);
            const int k = int(sym.size());
            sym.push_back({i, len, k - 1, i + len < s.size() ? k + 1 : -1});
            i += len;
        }
        // candidate merges: higher score first, then the leftmost
        struct Cand { float score; int left, right; size_t len; };
        auto later = [](const Cand& a, const Cand& b) {
            return a.score < b.score || (a.score == b.score && a.left > b.left);
        };
        std::priority_queue<Cand, std::vector<Cand>, decltype(later)> q(later);
        auto offer = [&](int l, int r) {
            if (l < 0 || r < 0) return;
            const std::string_view cat(s.data() + sym[l].at, sym[l].len + sym[r].len);
            const int32_t id = find(cat);
            if (id >= 0) q.push({score_[id], l, r, cat.size()});
        };
        for (int k = 1; k < int(sym.size()); ++k) offer(k - 1, k);
        while (!q.empty()) {
            const Cand c = q.top();
            q.pop();
            Sym& l = sym[c.left];
            Sym& r = sym[c.right];
            // skip a candidate one of whose sides has merged since
            if (l.len == 0 || r.len == 0 || l.len + r.len != c.len) continue;
            l.len += r.len;
            r.len = 0;
            l.next = r.next;
            if (r.next >= 0) sym[r.next].prev = c.left;
            offer(l.prev, c.left);
            offer(c.left, l.next);
        }
        for (int k = 0; k >= 0; k = sym[k].next) {
            if (sym[k].len == 0) continue;
            const std::string_view t(s.data() + sym[k].at, sym[k].len);
            const int32_t id = find(t);
            if (id >= 0) {
                out.push_back(id);
                continue;
            }
            // a merged symbol always has a spelling: only single characters
            // reach the byte fallback
            for (unsigned char b : t) {
                if (byte_id_[b] >= 0) out.push_back(byte_id_[b]);
                else if (unk >= 0) out.push_back(unk);
            }
        }
    }

    std::vector<std::string_view> text_;
    std::vector<float> score_;
    std::vector<int32_t> kind_;
    std::unordered_map<std::string_view, int32_t> index_;
    std::vector<size_t> special_lens_;
    int32_t byte_id_[256] = {
#define XP_M1_8 -1, -1, -1, -1, -1, -1, -1, -1
#define XP_M1_64 XP_M1_8, XP_M1_8, XP_M1_8, XP_M1_8, XP_M1_8, XP_M1_8, XP_M1_8, XP_M1_8
        XP_M1_64, XP_M1_64, XP_M1_64, XP_M1_64
#undef XP_M1_64
#undef XP_M1_8
    };
};

}  // namespace xp::tok

struct xp_tokenizer {
    std::unique_ptr<xp::tok::Tokenizer> t;
};

namespace {
template <class F>
int tguard(const char* who, F&& fn) {
    try {
        return fn();
    } catch (const std::bad_alloc&) {
        return xp::set_error(XP_E_NOMEM, "%s: out of host memory", who);
    } catch (const std::exception& e) {
        return xp::set_error(XP_E_FORMAT, "%s: %s", who, e.what());
    }
}

int put_string(const std::string& s, char* out, size_t cap, size_t* len) {
    if (len) *len = s.size();
    if (out && cap) {
        const size_t n = std::min(s.size(), cap - 1);
        std::memcpy(out, s.data(), n);
        out[n] = '\0';
    }
    return XP_OK;
}
}  // namespace

extern "C" {

int xp_tokenizer_create(xp_gguf* g, xp_tokenizer** out) {
    XP_REQUIRE(g && out, "null pointer");
    *out = nullptr;
    return tguard("xp_tokenizer_create", [&] {
        auto t = std::make_unique<xp_tokenizer>();
        t->t = std::make_unique<xp::tok::Tokenizer>(*g->f);
        *out = t.release();
        return XP_OK;
    });
}

int xp_tokenizer_destroy(xp_tokenizer* t) {
    delete t;
    return XP_OK;
}

int xp_tokenizer_info(xp_tokenizer* t, xp_tokenizer_ids* info) {
    XP_REQUIRE(t && info, "null pointer");
    info->vocab = uint32_t(t->t->size());
    info->bos = t->t->bos;
    info->eos = t->t->eos;
    info->unk = t->t->unk;
    info->pad = t->t->pad;
    info->add_bos = t->t->add_bos;
    info->add_eos = t->t->add_eos;
    info->add_space_prefix = t->t->prefix;
    return XP_OK;
}

int xp_tokenize(xp_tokenizer* t, const char* text, size_t len, int add_bos, int add_eos,
                int32_t* ids, size_t cap, size_t* n) {
    XP_REQUIRE(t && (text || len == 0) && n, "null pointer");
    return tguard("xp_tokenize", [&] {
        const std::vector<int32_t> v =
            t->t->encode(std::string_view(text ? text : "", len), add_bos != 0, add_eos != 0);
        *n = v.size();
        if (ids) std::memcpy(ids, v.data(), std::min(cap, v.size()) * 4);
        return v.size() > cap && ids
                   ? xp::set_error(XP_E_ARG, "xp_tokenize: %zu ids do not fit in %zu", v.size(), cap)
                   : XP_OK;
    });
}

int xp_detokenize(xp_tokenizer* t, const int32_t* ids, size_t n, int skip_special, char* out,
                  size_t cap, size_t* len) {
    XP_REQUIRE(t && (ids || n == 0), "null pointer");
    return tguard("xp_detokenize",
                  [&] { return put_string(t->t->decode(ids, n, skip_special != 0), out, cap, len); });
}

int xp_token_piece(xp_tokenizer* t, int32_t id, char* out, size_t cap, size_t* len) {
    XP_REQUIRE(t, "null pointer");
    return tguard("xp_token_piece", [&] { return put_string(t->t->piece(id), out, cap, len); });
}

int xp_token_text(xp_tokenizer* t, int32_t id, char* out, size_t cap, size_t* len) {
    XP_REQUIRE(t, "null pointer");
    return put_string(std::string(t->t->text(id)), out, cap, len);
}

int xp_token_find(xp_tokenizer* t, const char* spelling, size_t len, int32_t* id) {
    XP_REQUIRE(t && spelling && id, "null pointer");
    *id = t->t->find(std::string_view(spelling, len));
    return XP_OK;
}

int xp_token_kind(xp_tokenizer* t, int32_t id, int32_t* kind, float* score) {
    XP_REQUIRE(t, "null pointer");
    if (kind) *kind = t->t->kind(id);
    if (score) *score = t->t->score(id);
    return XP_OK;
}

}  // extern "C"
