// tests/cpp/ref_model_run.cpp — the reference's own host code (SSMFile,
// Mamba2Model, Mamba2State, Mamba2Workspace, generate(); compiled unchanged from
// /root/reference/src into oracle/_ref/libref_host.so) driving this repository's
// HIP backend through include/lite_ssm/{ops,allocator}.hpp.
//
// Usage: ref_model_run <model.ssm> <n_new> <logits.bin> <id,id,...>
// Greedy-generates n_new tokens after the prompt exactly as the reference's
// runtime does (src/runtime/inference.cpp:14-70), prints one JSON line
// {"ids": [...], "first_ms": ..., "decode_ms": ...} and writes the fp32 logits
// each id was picked from ([n_new, vocab] float32,
// Mamba2Model::read_logits_fp32) to logits.bin.  first_ms is the time from
// the start of generate() to the first pick (prefill and logits), decode_ms
// the time from the first pick to the last (n_new - 1 decode steps), both
// without the logits file writes.
// Exit 77 (skip) when no GPU is available.

#include "lite_ssm/inference.hpp"
#include "lite_ssm/model.hpp"
#include "lite_ssm/ops.hpp"
#include "lite_ssm/state.hpp"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <sstream>
#include <string>
#include <vector>

int main(int argc, char** argv) {
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s <model.ssm> <n_new> <logits.bin> <id,id,...>\n", argv[0]);
        return 2;
    }
    try {
        lite_ssm::MetalOps probe;
        if (!probe.metallib_loaded()) {
            std::fprintf(stderr, "no GPU / code object: skip\n");
            return 77;
        }
        std::vector<uint32_t> prompt;
        std::stringstream ss(argv[4]);
        for (std::string tok; std::getline(ss, tok, ',');) prompt.push_back((uint32_t)std::stoul(tok));
        const uint32_t n_new = (uint32_t)std::stoul(argv[2]);

        lite_ssm::SSMFile weights(argv[1]);
        lite_ssm::Mamba2Model model(weights);
        lite_ssm::MetalOps ops;
        lite_ssm::Mamba2Workspace ws(model.config(), (uint32_t)prompt.size());
        lite_ssm::Mamba2State state(model.config());

        std::FILE* out = std::fopen(argv[3], "wb");
        if (!out) {
            std::fprintf(stderr, "cannot open %s\n", argv[3]);
            return 2;
        }
        lite_ssm::GenerationConfig gc;
        gc.max_new_tokens = n_new;
        gc.greedy = true;
        // one untimed generation first (each kernel's code is loaded on its
        // first launch), as the reference's benchmark drops its first
        // iteration (examples/benchmark_litessm.cpp); generate() resets the
        // state, so the timed run starts from the same place
        {
            lite_ssm::GenerationConfig warm = gc;
            warm.max_new_tokens = 2;
            lite_ssm::generate(model, ops, ws, state, prompt, warm, [](uint32_t) {});
        }
        // the callback runs right after each pick, while the workspace's fp32
        // scratch still holds the logits the id was taken from
        using clk = std::chrono::steady_clock;
        double first_ms = 0.0, decode_ms = 0.0, io_ms = 0.0;
        const auto t0 = clk::now();
        auto ids = lite_ssm::generate(model, ops, ws, state, prompt, gc, [&](uint32_t) {
            const auto t = clk::now();
            const double at = std::chrono::duration<double, std::milli>(t - t0).count() - io_ms;
            if (first_ms == 0.0) first_ms = at;
            else decode_ms = at - first_ms;
            const std::vector<float>& lg = model.read_logits_fp32(ws);
            std::fwrite(lg.data(), sizeof(float), lg.size(), out);
            io_ms += std::chrono::duration<double, std::milli>(clk::now() - t).count();
        });
        std::fclose(out);
        std::printf("{\"ids\": [");
        for (size_t i = 0; i < ids.size(); ++i) std::printf("%s%u", i ? ", " : "", ids[i]);
        std::printf("], \"first_ms\": %.3f, \"decode_ms\": %.3f}\n", first_ms, decode_ms);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
    return 0;
}
