// xpose_decode — command-line decode driver over include/xpose.hpp, the
// counterpart of the reference's decode CLI (examples/llm/decode.cpp:
// 2720-3006), with the reference's flag spellings where the two overlap:
//
//   xpose_decode --model FILE [--prompt TEXT | --prompt-file F] [--chat] [-n N]
//                [--pack-cache F | --no-pack-cache] [--repack] [--pack-threads N]
//                [--verify-cache]
//   xpose_decode [--layers N] [--prompt-len N | --ctx P] [-n N] [--weights-seed S]
//   common:      [--max-seq N] [--window N] [--global-every N] [--temp T]
//                [--top-k K] [--top-p P] [--seed S] [--exec token|graph|launch]
//                [--curve] [--ids]
//
// With --model the GGUF file is requantised to int4 with bf16 scales through
// the pack cache (default FILE.xpack); --verify-cache repacks every matrix,
// compares the cache byte for byte and exits (no GPU). The prompt text is
// encoded with the model's tokenizer (BOS first), --chat wraps it in Gemma's
// turn template (decode.cpp:2888-2890), the generated text is streamed and
// generation stops at <eos> or <end_of_turn> unless --curve
// (decode.cpp:2919-2946). Without a prompt, or without --model, the prompt is
// --prompt-len uniform-random ids (benchmark config 3; the seeded synthetic
// model when there is no --model). --ctx P instead pre-fills every layer's KV
// cache with fp16 N(0,1) rows 0..P-1 and decodes from position P (config 4).
// --temp / --top-k / --top-p switch to temperature sampling, --seed sets its
// Philox key (decode.cpp:2800-2806). --curve reports tok/s per 512-position
// bucket and the deepest/shallowest ratio, the reference's flatness metric
// (decode.cpp:2977-2999). Prints per-step gpu ms min / median / mean like the
// reference (decode.cpp:2961-2972).
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "xpose.hpp"

namespace {

double now_ms() {
    using namespace std::chrono;
    return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

int usage() {
    std::fprintf(stderr,
                 "usage: xpose_decode --model FILE [--prompt TEXT | --prompt-file F] [--chat] "
                 "[-n N]\n"
                 "                    [--pack-cache F | --no-pack-cache] [--repack] "
                 "[--pack-threads N] [--verify-cache]\n"
                 "       xpose_decode [--layers N] [--prompt-len N | --ctx P] [-n N] "
                 "[--weights-seed S]\n"
                 "       common: [--max-seq N] [--window N] [--global-every N] [--temp T] "
                 "[--top-k K] [--top-p P]\n"
                 "               [--seed S] [--exec token|graph|launch] [--curve] [--ids]\n");
    return 2;
}

bool read_file(const char* path, std::string& out) {
    std::FILE* fp = std::fopen(path, "rb");
    if (!fp) return false;
    char buf[4096];
    size_t got;
    while ((got = std::fread(buf, 1, sizeof buf, fp)) > 0) out.append(buf, got);
    std::fclose(fp);
    return true;
}

}  // namespace

int main(int argc, char** argv) {
    uint32_t layers = 26, prompt_len = 32, tokens = 128, ctx = 0, seed = 0x5EED0003u;
    uint32_t pack_threads = 0;
    int exec = XP_EXEC_AUTO;
    bool curve = false, print_ids = false, no_cache = false, repack = false, verify = false;
    bool chat = false, have_text = false;
    std::string model, cache, text;
    // Policy fields applied over the model's shapes, as the reference's
    // DecodeConfig fields are: {name, value} pairs kept in flag order.
    std::vector<std::pair<std::string, double>> policy;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&]() -> const char* { return i + 1 < argc ? argv[++i] : nullptr; };
        auto num = [&](uint32_t& dst) {
            const char* v = next();
            if (!v) return false;
            dst = uint32_t(std::strtoul(v, nullptr, 0));
            return true;
        };
        const char* v = nullptr;
        if (a == "--layers") { if (!num(layers)) return usage(); }
        else if (a == "--prompt-len") { if (!num(prompt_len)) return usage(); }
        else if (a == "-n" || a == "--tokens") { if (!num(tokens)) return usage(); }
        else if (a == "--ctx") { if (!num(ctx)) return usage(); }
        else if (a == "--weights-seed") { if (!num(seed)) return usage(); }
        else if (a == "--pack-threads") { if (!num(pack_threads)) return usage(); }
        else if (a == "--exec" && (v = next())) {
            const std::string m = v;
            exec = m == "token" ? XP_EXEC_TOKEN : m == "graph" ? XP_EXEC_GRAPH
                 : m == "launch" ? XP_EXEC_LAUNCH : -1;
            if (exec < 0) return usage();
        } else if (a == "--curve") curve = true;
        else if (a == "--ids") print_ids = true;
        else if (a == "--model" && (v = next())) model = v;
        else if (a == "--pack-cache" && (v = next())) cache = v;
        else if (a == "--no-pack-cache") no_cache = true;
        else if (a == "--repack") repack = true;
        else if (a == "--verify-cache") verify = true;
        else if (a == "--prompt" && (v = next())) { text = v; have_text = true; }
        else if (a == "--prompt-file" && (v = next())) {
            text.clear();
            if (!read_file(v, text)) {
                std::fprintf(stderr, "cannot open %s\n", v);
                return 2;
            }
            have_text = true;
        }
        else if (a == "--chat") chat = true;
        else if ((a == "--max-seq" || a == "--window" || a == "--global-every" || a == "--temp" ||
                  a == "--top-k" || a == "--top-p" || a == "--seed") && (v = next()))
            policy.emplace_back(a, std::strtod(v, nullptr));
        else return usage();
    }
    if ((verify || repack || no_cache || !cache.empty() || have_text || chat) && model.empty())
        return usage();
    if (chat && !have_text) return usage();
    if (!model.empty() && cache.empty() && !no_cache) cache = model + ".xpack";
    auto apply_policy = [&](xpose::llm::Config& c) {
        for (const auto& [name, x] : policy) {
            if (name == "--max-seq") c.max_seq = uint32_t(x);
            else if (name == "--window") c.sliding_window = uint32_t(x);
            else if (name == "--global-every") c.global_every = uint32_t(x);
            else if (name == "--seed") c.seed = uint32_t(x);
            else {
                c.sample_mode = 1;
                if (name == "--temp") c.temperature = float(x);
                else if (name == "--top-k") c.top_k = uint32_t(x);
                else c.top_p = float(x);
            }
        }
    };
    try {
        xpose::llm::Config cfg;
        cfg.n_layers = layers;
        cfg.exec_mode = exec;
        std::unique_ptr<xpose::llm::Model> gguf;
        if (!model.empty()) {
            gguf.reset(new xpose::llm::Model(model));
            cfg = gguf->config(cfg);
            apply_policy(cfg);
            if (verify) {
                const uint32_t bad = gguf->verify_cache(cfg, cache, pack_threads);
                std::printf("%s: %s\n", cache.c_str(),
                            bad ? "FAIL: the cache does not match a fresh pack"
                                : "PASS: cached bytes are identical to a fresh pack");
                return bad ? 1 : 0;
            }
        }
        const double t0 = now_ms();
        std::unique_ptr<xpose::llm::DecodeSession> sp;
        if (gguf)
            sp.reset(new xpose::llm::DecodeSession(*gguf, cfg, no_cache ? std::string() : cache,
                                                   repack ? XP_LOAD_REPACK : 0u, pack_threads));
        else {
            apply_policy(cfg);
            sp.reset(new xpose::llm::DecodeSession(cfg));
        }
        xpose::llm::DecodeSession& sess = *sp;
        if (!gguf) sess.synthesize(seed);
        const double load_ms = now_ms() - t0;
        std::printf("device      %s\n", sess.device_name().c_str());
        if (gguf) {
            const xp_load_stats& ls = sess.load_stats();
            std::printf("weights     %.1f MiB packed int4 + bf16 scales from %s in %.0f ms "
                        "(%s; pack %.0f ms, cache %.0f ms, upload %.0f ms, %u threads)\n",
                        double(sess.weight_bytes()) / (1024.0 * 1024.0), model.c_str(), load_ms,
                        ls.from_cache ? "from the pack cache"
                                      : (ls.cache_written ? "packed, cache written" : "packed"),
                        ls.pack_ms, ls.cache_ms, ls.upload_ms, ls.threads);
        } else {
            std::printf("weights     %.1f MiB packed int4 + fp16 scales (synthesised in %.0f ms)\n",
                        double(sess.weight_bytes()) / (1024.0 * 1024.0), load_ms);
        }
        std::printf("kv cache    %.1f MiB (%u positions)\n",
                    double(sess.kv_bytes()) / (1024.0 * 1024.0), cfg.max_seq);

        std::unique_ptr<xpose::llm::Tokenizer> tok;
        int32_t stop1 = -1, stop2 = -1;
        if (have_text) {
            tok.reset(new xpose::llm::Tokenizer(*gguf));
            if (chat) text = "<start_of_turn>user\n" + text + "<end_of_turn>\n<start_of_turn>model\n";
            stop1 = tok->eos_id();
            stop2 = tok->id_for("<end_of_turn>");
        }
        std::vector<uint32_t> ids;
        if (tok) {
            ids = tok->encode(text, true);
        } else if (ctx > 0) {
            const uint32_t row = cfg.n_kv_heads * cfg.head_dim;
            std::vector<uint16_t> rows(size_t(ctx) * row);
            for (uint32_t l = 0; l < cfg.n_layers; ++l)
                for (int which = 0; which < 2; ++which) {
                    xpose::check(xp_synth_normal_f16(rows.data(), rows.size(), 0.0f, 1.0f, ctx,
                                                     2u * l + uint32_t(which)),
                                 "xp_synth_normal_f16");
                    sess.kv_upload(int(l), which, 0, ctx, rows.data());
                }
            sess.set_position(ctx);
            ids.push_back(4242);
        } else {
            // Prompt ids uniform on [0, vocab): Philox stream 0x7000.
            for (uint32_t i = 0; i < prompt_len; ++i) {
                const uint32_t c[4] = {i, 0u, 0u, 0u}, k[2] = {seed, 0x7000u};
                uint32_t o[4];
                xp_philox4x32_10(c, k, o);
                ids.push_back(o[0] % cfg.vocab);
            }
        }
        if (ids.size() + ctx + tokens > cfg.max_seq) {
            std::fprintf(stderr, "xpose_decode: %zu + %u + %u positions exceed max_seq %u\n",
                         ids.size(), ctx, tokens, cfg.max_seq);
            return 2;
        }
        sess.prefill(ids);
        const auto pm = sess.last_metrics();
        const char* mode = pm.exec_mode == XP_EXEC_TOKEN ? "persistent token kernel"
                         : pm.exec_mode == XP_EXEC_GRAPH ? "captured graph" : "per-op launches";
        std::printf("execution   %s, %u launch(es) per token\n", mode, pm.dispatches);
        std::printf("prefill     %zu tokens in %.2f ms\n\n", ids.size(), pm.ms);

        std::vector<double> step_ms;
        std::vector<uint32_t> pos_of, out;
        double total = 0;
        if (tok) {
            std::printf("%s", text.c_str());
            std::fflush(stdout);
        }
        for (uint32_t i = 0; i < tokens; ++i) {
            out.push_back(sess.decode_step());
            if (tok) {
                // Gemma ends a turn with <end_of_turn>, not <eos> (decode.cpp:2927-2929)
                const int32_t t = int32_t(out.back());
                if (!curve && (t == stop1 || t == stop2)) {
                    out.pop_back();
                    break;
                }
                std::printf("%s", tok->decode_one(t).c_str());
                std::fflush(stdout);
            }
            const auto m = sess.last_metrics();
            step_ms.push_back(m.gpu_ms);
            pos_of.push_back(m.position);
            total += m.ms;
        }
        if (tok) std::printf("\n\n");
        const size_t done = step_ms.size();
        if (done == 0) {
            std::printf("decode      0 tokens\n");
            return 0;
        }
        std::printf("decode      %zu tokens, %.4f ms/token, %.1f tok/s (host wall per step)\n",
                    done, total / double(done), double(done) * 1000.0 / total);
        std::vector<double> s = step_ms;
        std::sort(s.begin(), s.end());
        double sum = 0;
        for (double x : s) sum += x;
        std::printf("gpu ms      min %.4f | median %.4f | mean %.4f   (n=%zu)\n", s.front(),
                    s[s.size() / 2], sum / double(s.size()), s.size());
        if (curve) {
            std::map<uint32_t, std::vector<double>> b;
            for (size_t i = 0; i < step_ms.size(); ++i) b[(pos_of[i] - 1) / 512].push_back(step_ms[i]);
            double lo = 1e30, hi = 0;
            std::printf("\nposition bucket      tok/s     median ms\n");
            for (auto& kv : b) {
                std::sort(kv.second.begin(), kv.second.end());
                const double med = kv.second[kv.second.size() / 2];
                lo = std::min(lo, med);
                hi = std::max(hi, med);
                std::printf("%5u-%-5u      %9.1f    %.4f\n", kv.first * 512, kv.first * 512 + 511,
                            1000.0 / med, med);
            }
            std::printf("deepest / shallowest median ms: %.3f\n", hi / lo);
        }
        if (print_ids) {
            std::printf("ids");
            for (uint32_t t : out) std::printf(" %u", t);
            std::printf("\n");
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "xpose_decode: %s\n", e.what());
        return 1;
    }
    return 0;
}
