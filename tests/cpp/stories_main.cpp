// Greedy-stream driver for BASELINE config 4 (TEST INFRASTRUCTURE).
//
// Built by oracle/Makefile twice against the reference's own model code
// (/root/reference/src/model.cpp, ops.cpp, quant.cpp, thread_pool.cpp):
//   oracle/_ref/stories_cpu  with the reference's matmul.cpp (the CPU path)
//   oracle/_ref/stories_gpu  with tests/cpp/gpu_matmul_shim.cpp in place of
//                            matmul.cpp, so Transformer::project
//                            (model.cpp:256-258) -- all 25 products per
//                            token -- runs on this build's GPU kernels
// Everything else (embedding, rmsnorm, RoPE, attention, SwiGLU) is the same
// reference code in both, so the streams can differ only through the matmuls.
//
// usage: stories_{cpu,gpu} <checkpoint> <prompt-file> <f32|q8> <n_decode>
// Prefills the prompt as one batch, then decodes greedily (first maximum,
// as sampler.cpp:28-29), without stopping at BOS. Prints one JSON object:
// tokens (1 + n_decode), the top-1 minus top-2 logit margin of each pick,
// and timings.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "model.h"

namespace {

std::size_t pick(const std::vector<float>& logits, float* margin) {
    const auto best = std::max_element(logits.begin(), logits.end());
    float second = -INFINITY;
    for (auto it = logits.begin(); it != logits.end(); ++it)
        if (it != best) second = std::max(second, *it);
    *margin = *best - second;
    return static_cast<std::size_t>(best - logits.begin());
}

}  // namespace

int main(int argc, char** argv) try {
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s <checkpoint> <prompt-file> <f32|q8> <n_decode>\n", argv[0]);
        return 2;
    }
    const std::string type = argv[3];
    const int n_decode = std::stoi(argv[4]);
    std::vector<int> prompt;
    {
        std::ifstream in(argv[2]);
        for (int t; in >> t;) prompt.push_back(t);
    }
    using Clock = std::chrono::steady_clock;
    const auto t_load = Clock::now();
    Transformer model(load_checkpoint(argv[1]), type == "q8" ? WeightType::q8 : WeightType::f32);
    const auto t0 = Clock::now();
    std::vector<int> tokens;
    std::vector<float> margins;
    float margin = 0.0f;
    tokens.push_back(static_cast<int>(pick(model.prefill(prompt, 0), &margin)));
    margins.push_back(margin);
    const auto t1 = Clock::now();
    for (int s = 0; s < n_decode; ++s) {
        const auto& logits = model.forward(tokens.back(), prompt.size() + static_cast<std::size_t>(s));
        tokens.push_back(static_cast<int>(pick(logits, &margin)));
        margins.push_back(margin);
    }
    const auto t2 = Clock::now();
    auto ms = [](auto a, auto b) { return std::chrono::duration<double, std::milli>(b - a).count(); };
    std::printf("{\"type\": \"%s\", \"prompt\": %zu, \"load_ms\": %.3f, \"prefill_ms\": %.3f, "
                "\"decode_ms_per_token\": %.4f, \"tokens\": [",
                type.c_str(), prompt.size(), ms(t_load, t0), ms(t0, t1),
                n_decode ? ms(t1, t2) / n_decode : 0.0);
    for (std::size_t i = 0; i < tokens.size(); ++i) std::printf("%s%d", i ? ", " : "", tokens[i]);
    std::printf("], \"margins\": [");
    for (std::size_t i = 0; i < margins.size(); ++i) std::printf("%s%.6g", i ? ", " : "", margins[i]);
    std::printf("]}\n");
    return 0;
} catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
}
