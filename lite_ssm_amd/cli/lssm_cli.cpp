// lssm_cli — command-line generation over a .ssm file on one MI355X, the Linux
// counterpart of the reference's apps/lite_ssm_cli.cpp.
//
// Same flags, argument meaning, messages and output contract as the reference
// CLI (lite_ssm_cli.cpp:106-147 flags, :259-329 prefill/decode timing and the
// "[lite-ssm]" lines, :331-337 --dump-logits, :339-346 ids on stdout), with
// three platform differences:
//   * resident set size comes from /proc/self/statm (the reference asks the
//     Mach kernel, lite_ssm_cli.cpp:161-167, which exists only on macOS);
//   * --probe-only touches the mapping once per host page (sysconf), where
//     the reference steps 16 KB, the Apple Silicon page;
//   * the model runs on the GPU through include/lssm.h: the file is uploaded
//     to HBM once, the engine keeps the recurrent state on the device, embeds
//     the ids and takes greedy ids there (the reference embeds and samples on
//     the host, lite_ssm_cli.cpp:237-244, 296-303).  --top-p copies the logits
//     to the host and samples there as the reference does.
// Text prompts need SentencePiece, which this build does not link (the
// reference fetches it at configure time); `python -m lite_ssm_amd.cli`
// tokenizes with the sentencepiece Python module and runs this binary with
// --input-ids.  Given a text prompt, this binary says so and exits 2.
#include "lssm.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <numeric>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace {

struct Args {
    std::string model = "model.ssm";
    std::string tokenizer = "tokenizer.model";
    std::string prompt_text;
    std::vector<uint32_t> input_ids;
    std::string dump_logits;
    uint32_t max_tokens = 200;
    bool greedy = true;
    float top_p = 0.9f;
    float temperature = 1.0f;
    uint64_t seed = 0xCAFEBABEull;
    uint32_t eos_id = 0;
    bool eos_set = false;
    bool quiet = false;
    bool probe_only = false;
};

// usage and input errors exit 2, library errors 1 (as the reference CLI)
[[noreturn]] void die(const std::string& msg) {
    std::fprintf(stderr, "lite-ssm: %s\n", msg.c_str());
    std::exit(2);
}

void usage() {
    std::fprintf(stderr,
                 "usage: lssm_cli [--model PATH] [--tokens N] [--greedy | --top-p P]\n"
                 "                [--temperature T] [--seed S] [--eos ID] [--quiet]\n"
                 "                [--dump-logits PATH] (--input-ids 1,2,3 | --probe-only)\n"
                 "  --model PATH        .ssm weights (default model.ssm)\n"
                 "  --tokens N          tokens to generate, including the first (default 200)\n"
                 "  --greedy            argmax sampling (default)\n"
                 "  --top-p P           nucleus sampling with mass P\n"
                 "  --temperature T     softmax temperature for --top-p (default 1.0)\n"
                 "  --seed S            xorshift64 seed for --top-p (default 0xCAFEBABE; 0 -> 1)\n"
                 "  --input-ids IDS     prompt token ids, comma or space separated\n"
                 "  --eos ID            stop after generating ID\n"
                 "  --dump-logits PATH  write the last step's logits as fp32\n"
                 "  --probe-only        map the file, touch every page, report RSS\n"
                 "  --tokenizer PATH    accepted; text prompts go through python -m lite_ssm_amd.cli\n");
}

std::vector<uint32_t> parse_ids(std::string_view s) {
    std::vector<uint32_t> ids;
    size_t i = 0;
    while (i < s.size()) {
        while (i < s.size() && (s[i] == ',' || s[i] == ' ')) ++i;
        size_t j = i;
        while (j < s.size() && s[j] != ',' && s[j] != ' ') ++j;
        if (j > i) ids.push_back(static_cast<uint32_t>(std::stoul(std::string(s.substr(i, j - i)))));
        i = j;
    }
    return ids;
}

Args parse_args(int argc, char** argv) {
    Args a;
    std::vector<std::string> words;
    for (int i = 1; i < argc; ++i) {
        const std::string_view k = argv[i];
        auto value = [&](const char* flag) -> std::string {
            if (i + 1 >= argc) die(std::string(flag) + " expects an argument");
            return argv[++i];
        };
        if (k == "--model") a.model = value("--model");
        else if (k == "--tokenizer") a.tokenizer = value("--tokenizer");
        else if (k == "--tokens") a.max_tokens = static_cast<uint32_t>(std::stoul(value("--tokens")));
        else if (k == "--greedy") a.greedy = true;
        else if (k == "--top-p") { a.greedy = false; a.top_p = std::stof(value("--top-p")); }
        else if (k == "--temperature") a.temperature = std::stof(value("--temperature"));
        else if (k == "--seed") a.seed = std::stoull(value("--seed"));
        else if (k == "--input-ids") a.input_ids = parse_ids(value("--input-ids"));
        else if (k == "--dump-logits") a.dump_logits = value("--dump-logits");
        else if (k == "--eos") { a.eos_id = static_cast<uint32_t>(std::stoul(value("--eos"))); a.eos_set = true; }
        else if (k == "--quiet") a.quiet = true;
        else if (k == "--probe-only") a.probe_only = true;
        else if (k == "-h" || k == "--help") { usage(); std::exit(0); }
        else if (!k.empty() && k[0] == '-') die("unknown flag: " + std::string(k));
        else words.emplace_back(k);
    }
    if (a.input_ids.empty() && words.empty() && !a.probe_only) {
        usage();
        die("provide a prompt text positionally, --input-ids, or --probe-only");
    }
    if (!a.input_ids.empty() && !words.empty()) die("can't combine --input-ids with a positional prompt");
    for (size_t i = 0; i < words.size(); ++i) a.prompt_text += (i ? " " : "") + words[i];
    return a;
}

void say(bool quiet, const char* fmt, ...) {
    if (quiet) return;
    va_list ap;
    va_start(ap, fmt);
    std::vfprintf(stderr, fmt, ap);
    va_end(ap);
    std::fputc('\n', stderr);
}

// Resident set size: the second field of /proc/self/statm, in pages.
size_t rss_bytes() {
    FILE* f = std::fopen("/proc/self/statm", "r");
    if (!f) return 0;
    unsigned long size = 0, resident = 0;
    const int got = std::fscanf(f, "%lu %lu", &size, &resident);
    std::fclose(f);
    return got == 2 ? static_cast<size_t>(resident) * static_cast<size_t>(sysconf(_SC_PAGESIZE)) : 0;
}

void check(int rc, const char* what) {
    if (rc != LSSM_OK) throw std::runtime_error(std::string(what) + ": " + lssm_last_error());
}

// Logits of the activation dtype as fp32 (the reference's read_logits_fp32).
float half_to_f32(uint16_t h) {
    const uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    float v;
    if (e == 0) v = std::ldexp(static_cast<float>(m), -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = std::ldexp(static_cast<float>(m | 0x400u), static_cast<int>(e) - 25);
    return s ? -v : v;
}
float bf16_to_f32(uint16_t b) {
    const uint32_t u = static_cast<uint32_t>(b) << 16;
    float v;
    std::memcpy(&v, &u, 4);
    return v;
}

// Nucleus sampling as sampler.cpp:39-79 defines it: descending argsort,
// stable softmax at temperature t (t <= 1e-6 -> 1), cut at cumulative mass
// >= top_p, draw r = u * (nucleus mass) with u from xorshift64 (13, 7, 17;
// top 24 bits), first index whose running mass reaches r.
uint32_t sample_top_p(const std::vector<float>& logits, float top_p, float temperature, uint64_t& s) {
    if (logits.empty()) die("sample_top_p: empty logits");
    const float t = temperature > 1e-6f ? temperature : 1.0f;
    std::vector<uint32_t> order(logits.size());
    std::iota(order.begin(), order.end(), 0u);
    std::sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) { return logits[x] > logits[y]; });
    const float top = logits[order[0]] / t;
    std::vector<float> p(order.size());
    float total = 0.0f;
    for (size_t i = 0; i < order.size(); ++i) {
        p[i] = std::exp(logits[order[i]] / t - top);
        total += p[i];
    }
    for (float& v : p) v /= total;
    size_t keep = p.size();
    float run = 0.0f;
    for (size_t i = 0; i < p.size(); ++i) {
        run += p[i];
        if (run >= top_p) { keep = i + 1; break; }
    }
    float mass = 0.0f;
    for (size_t i = 0; i < keep; ++i) mass += p[i];
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    const float r = static_cast<float>(s >> 40) / static_cast<float>(1u << 24) * mass;
    float acc = 0.0f;
    for (size_t i = 0; i < keep; ++i) {
        acc += p[i];
        if (r <= acc) return order[i];
    }
    return order[keep - 1];
}

int probe_only(const Args& args) {
    using clk = std::chrono::steady_clock;
    const auto t0 = clk::now();
    const size_t rss0 = rss_bytes();
    lssm_ssm* f = nullptr;
    check(lssm_ssm_open(&f, args.model.c_str()), "open");   // validates the header and index
    lssm_ssm_header h{};
    check(lssm_ssm_get_header(f, &h), "header");
    const double ms_open = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
    const size_t rss1 = rss_bytes();
    // a read-only mapping of the file of its own: page-touch it
    const int fd = ::open(args.model.c_str(), O_RDONLY);
    if (fd < 0) die("cannot open " + args.model);
    struct stat st {};
    if (::fstat(fd, &st) != 0) { ::close(fd); die("cannot stat " + args.model); }
    const size_t sz = static_cast<size_t>(st.st_size);
    void* base = ::mmap(nullptr, sz, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (base == MAP_FAILED) die("cannot map " + args.model);
    const size_t step = static_cast<size_t>(sysconf(_SC_PAGESIZE));
    const auto t1 = clk::now();
    volatile size_t sink = 0;
    for (size_t i = 0; i < sz; i += step) sink += static_cast<const uint8_t*>(base)[i];
    (void)sink;
    const double ms_scan = std::chrono::duration<double, std::milli>(clk::now() - t1).count();
    const size_t rss2 = rss_bytes();
    ::munmap(base, sz);
    std::printf("== probe-only mmap stress ==\n");
    std::printf("  model file        : %s (%.2f GB)\n", args.model.c_str(), sz / 1e9);
    std::printf("  tensors indexed   : %u\n", h.n_tensors);
    std::printf("  rss pre-mmap      : %.1f MB\n", rss0 / 1048576.0);
    std::printf("  rss after mmap    : %.1f MB   (+%.1f MB, %.1f ms wall)\n", rss1 / 1048576.0,
                (static_cast<double>(rss1) - static_cast<double>(rss0)) / 1048576.0, ms_open);
    std::printf("  rss after scan    : %.1f MB   (page-touched every %zu B, %.1f ms wall)\n", rss2 / 1048576.0,
                step, ms_scan);
    std::printf("  resident fraction : %.1f%% of file (the rest is paged out / cold)\n",
                100.0 * static_cast<double>(rss2) / static_cast<double>(sz));
    lssm_ssm_close(f);
    return 0;
}

int generate(const Args& args) {
    using clk = std::chrono::steady_clock;
    if (!args.prompt_text.empty())
        die("text prompts need SentencePiece, which this build does not link: run "
            "`python -m lite_ssm_amd.cli` (same flags) or pass --input-ids");
    const auto t_boot = clk::now();
    lssm_ssm* f = nullptr;
    check(lssm_ssm_open(&f, args.model.c_str()), "open");
    lssm_ctx* ctx = nullptr;
    check(lssm_ctx_create(&ctx, nullptr), "context");
    void* dbase = nullptr;
    check(lssm_ssm_upload(f, ctx, &dbase), "upload");
    lssm_model_config cfg{};
    const void *embed = nullptr, *norm_f = nullptr, *lm_head = nullptr;
    lssm_ssm_header h{};
    check(lssm_ssm_get_header(f, &h), "header");
    std::vector<lssm_layer_weights> layers(h.n_layer);
    check(lssm_ssm_model(f, dbase, &cfg, &embed, &norm_f, &lm_head, layers.data(), h.n_layer), "model");

    const std::vector<uint32_t>& ids = args.input_ids;
    if (ids.empty()) die("empty prompt after tokenization");
    const uint32_t L = static_cast<uint32_t>(ids.size());
    for (uint32_t id : ids)
        if (id >= cfg.vocab_size) die("input id " + std::to_string(id) + " out of vocab range");
    lssm_engine* eng = nullptr;
    check(lssm_engine_create(&eng, ctx, &cfg, embed, norm_f, lm_head, layers.data(), 1,
                             std::max<uint32_t>(L, cfg.chunk_size)),
          "engine");
    int32_t* d_ids = nullptr;
    check(lssm_malloc(reinterpret_cast<void**>(&d_ids), sizeof(int32_t) * (L + 1)), "malloc");
    std::vector<int32_t> h_ids(ids.begin(), ids.end());
    check(lssm_memcpy_h2d(ctx, d_ids, h_ids.data(), sizeof(int32_t) * L), "copy ids");
    void* d_logits = nullptr;
    check(lssm_engine_logits(eng, &d_logits), "logits");
    const size_t esz = cfg.act == LSSM_F32 ? 4 : 2;
    std::vector<uint8_t> raw(static_cast<size_t>(cfg.vocab_size) * esz);
    std::vector<float> logits(cfg.vocab_size);
    auto read_logits = [&]() {
        check(lssm_memcpy_d2h(ctx, raw.data(), d_logits, raw.size()), "copy logits");
        for (uint32_t i = 0; i < cfg.vocab_size; ++i) {
            if (cfg.act == LSSM_F32) std::memcpy(&logits[i], raw.data() + 4 * i, 4);
            else {
                uint16_t b;
                std::memcpy(&b, raw.data() + 2 * i, 2);
                logits[i] = cfg.act == LSSM_BF16 ? bf16_to_f32(b) : half_to_f32(b);
            }
        }
    };
    int32_t* d_next = d_ids + L;
    uint64_t rng = args.seed ? args.seed : 1u;
    // greedy: the engine's device argmax (first index of the maximum, the
    // reference's sample_greedy tie rule); top-p: sampled on the host
    auto pick = [&]() -> uint32_t {
        if (!args.greedy) {
            read_logits();
            return sample_top_p(logits, args.top_p, args.temperature, rng);
        }
        int32_t v = 0;
        check(lssm_memcpy_d2h(ctx, &v, d_next, sizeof v), "copy id");
        return static_cast<uint32_t>(v);
    };
    const double boot_ms = std::chrono::duration<double, std::milli>(clk::now() - t_boot).count();
    say(args.quiet, "[lite-ssm] boot %.1f ms | prompt=%u raw ids | max_tokens=%u | mode=%s", boot_ms, L,
        args.max_tokens, args.greedy ? "greedy" : "top-p");
    const uint32_t eos = args.eos_set ? args.eos_id : 0xFFFFFFFFu;

    check(lssm_engine_reset(eng), "reset");
    const auto t_prefill = clk::now();
    check(lssm_engine_prefill(eng, d_ids, 1, L, d_next), "prefill");
    uint32_t next = pick();
    const double prefill_ms = std::chrono::duration<double, std::milli>(clk::now() - t_prefill).count();
    std::vector<uint32_t> generated{next};
    const auto t_decode = clk::now();
    for (uint32_t step = 1; step < args.max_tokens; ++step) {
        if (next == eos) break;
        const int32_t v = static_cast<int32_t>(next);
        check(lssm_memcpy_h2d(ctx, d_next, &v, sizeof v), "copy id");
        check(lssm_engine_decode(eng, d_next, 1, d_next), "decode");
        next = pick();
        generated.push_back(next);
    }
    const double decode_ms = std::chrono::duration<double, std::milli>(clk::now() - t_decode).count();
    const double tps = generated.size() <= 1 ? 0.0 : (generated.size() - 1) * 1000.0 / decode_ms;
    say(args.quiet, "[lite-ssm] prefill %.1f ms | decode %.1f ms | %.1f tok/s | generated=%zu", prefill_ms,
        decode_ms, tps, generated.size());
    say(args.quiet, "[lite-ssm] rss %.1f MB", rss_bytes() / 1048576.0);

    if (!args.dump_logits.empty()) {
        if (args.greedy) read_logits();   // top-p already holds them
        std::ofstream out(args.dump_logits, std::ios::binary);
        if (!out) die("cannot open --dump-logits target: " + args.dump_logits);
        out.write(reinterpret_cast<const char*>(logits.data()), static_cast<std::streamsize>(logits.size() * 4));
        if (!out.good()) die("write failed: " + args.dump_logits);
    }
    for (size_t i = 0; i < generated.size(); ++i) std::printf(i ? ",%u" : "%u", generated[i]);
    std::printf("\n");
    std::fflush(stdout);
    lssm_free(d_ids);
    lssm_engine_destroy(eng);
    lssm_ctx_destroy(ctx);
    lssm_ssm_close(f);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const Args args = parse_args(argc, argv);
        return args.probe_only ? probe_only(args) : generate(args);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "lite-ssm: %s\n", e.what());
        return 1;
    }
}
