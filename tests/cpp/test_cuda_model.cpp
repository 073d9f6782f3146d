// The reference's GPU model test (/root/reference/tests/test_cuda_model.cpp)
// against this build's drop-in header (include/cuda_model.h), with the
// reference's own CPU Transformer as the checker: both are built from the
// reference's model.cpp and friends by oracle/Makefile (target e2e).
//
// Same coverage: multi-head with a tied classifier, grouped-query with a
// separate one, multi-query; fp32 and int8 weights; decode over the whole
// context, prefill in chunks of 1, 1 and 5, a decode step on that cache, a
// whole-context prefill that rewinds; logits within 1e-4; the same
// rejections as the CPU model, after which the cache still works. Exits 77
// (skip) without a GPU. The random checkpoints are written here (llama2.c v0
// layout, model.cpp:115-163) with the value ranges of the reference's model
// fixture: uniform, embedding and classifier +-1, wq/wk/wv +-0.4, wo/w1/w2/w3
// +-0.3, rms_att 1 +- 0.2, rms_ffn +-0.2, rms_final +-1.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <filesystem>
#include <fstream>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "cuda_model.h"
#include "model.h"

namespace {

int failures = 0;

#define CHECK(cond)                                                                    \
    do {                                                                               \
        if (!(cond)) {                                                                 \
            std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                                                \
        }                                                                              \
    } while (0)

constexpr float kTol = 1e-4f;
constexpr int kDim = 16, kHidden = 40, kLayers = 2, kVocab = 29, kSeq = 8;

// Writes a small random checkpoint and returns its path.
std::string write_model(int heads, int kv_heads, bool shared, unsigned seed) {
    std::mt19937 rng(seed);
    const int hs = kDim / heads, kv = kv_heads * hs;
    std::vector<float> floats;
    auto fill = [&](std::size_t n, float scale, float offset) {
        std::uniform_real_distribution<float> dist(-scale, scale);
        for (std::size_t i = 0; i < n; ++i) floats.push_back(offset + dist(rng));
    };
    fill(std::size_t(kVocab) * kDim, 1.0f, 0.0f);                  // embedding
    fill(std::size_t(kLayers) * kDim, 0.2f, 1.0f);                 // rms_att
    fill(std::size_t(kLayers) * kDim * kDim, 0.4f, 0.0f);          // wq
    fill(std::size_t(kLayers) * kv * kDim, 0.4f, 0.0f);            // wk
    fill(std::size_t(kLayers) * kv * kDim, 0.4f, 0.0f);            // wv
    fill(std::size_t(kLayers) * kDim * kDim, 0.3f, 0.0f);          // wo
    fill(std::size_t(kLayers) * kDim, 0.2f, 0.0f);                 // rms_ffn
    fill(std::size_t(kLayers) * kHidden * kDim, 0.3f, 0.0f);       // w1
    fill(std::size_t(kLayers) * kDim * kHidden, 0.3f, 0.0f);       // w2
    fill(std::size_t(kLayers) * kHidden * kDim, 0.3f, 0.0f);       // w3
    fill(kDim, 1.0f, 0.0f);                                        // rms_final
    floats.insert(floats.end(), std::size_t(kSeq) * hs, 123.0f);   // legacy RoPE, ignored
    if (!shared) fill(std::size_t(kVocab) * kDim, 1.0f, 0.0f);     // wcls
    const std::int32_t header[7] = {kDim, kHidden, kLayers, heads, kv_heads,
                                    shared ? kVocab : -kVocab, kSeq};
    const std::string path =
        (std::filesystem::temp_directory_path() / ("em_test_cuda_model_" + std::to_string(seed) + ".bin"))
            .string();
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(header), sizeof header);
    f.write(reinterpret_cast<const char*>(floats.data()), std::streamsize(floats.size() * sizeof(float)));
    return path;
}

Checkpoint load_random(int heads, int kv_heads, bool shared) {
    const std::string path = write_model(heads, kv_heads, shared, unsigned(heads * 10 + kv_heads));
    Checkpoint ckpt = load_checkpoint(path);
    std::filesystem::remove(path);
    return ckpt;
}

bool close(const std::vector<float>& gpu, const std::vector<float>& cpu, const char* what,
           std::size_t pos) {
    float d = 0.0f;
    for (std::size_t i = 0; i < gpu.size(); ++i) d = std::max(d, std::fabs(gpu[i] - cpu[i]));
    if (d <= kTol) return true;
    std::fprintf(stderr, "  %s at pos %zu: max diff %g\n", what, pos, double(d));
    return false;
}

void test_matches_cpu(int heads, int kv_heads, bool shared, WeightType type) {
    const Checkpoint ckpt = load_random(heads, kv_heads, shared);
    Transformer cpu(ckpt, type);
    CudaTransformer gpu(ckpt, type);
    const std::size_t T = ckpt.config.seq_len;
    const int V = int(ckpt.config.vocab_size);
    std::vector<int> tokens;
    for (std::size_t pos = 0; pos < T; ++pos) {
        tokens.push_back(int(pos * 7 + 3) % V);
        CHECK(close(gpu.forward(tokens[pos], pos), cpu.forward(tokens[pos], pos), "forward", pos));
    }
    std::size_t pos = 0;
    for (std::size_t chunk : {1, 1, 5}) {
        const std::vector<int> part(tokens.begin() + long(pos), tokens.begin() + long(pos + chunk));
        CHECK(close(gpu.prefill(part, pos), cpu.prefill(part, pos), "prefill", pos));
        pos += chunk;
    }
    CHECK(close(gpu.forward(tokens[pos], pos), cpu.forward(tokens[pos], pos), "forward after prefill", pos));
    CHECK(close(gpu.prefill(tokens, 0), cpu.prefill(tokens, 0), "full prefill", 0));
}

template <class E, class F>
bool throws(F&& f) {
    try {
        f();
    } catch (const E&) {
        return true;
    }
    return false;
}

void test_bad_inputs() {
    const Checkpoint ckpt = load_random(4, 2, true);
    CudaTransformer gpu(ckpt);
    Transformer cpu(ckpt);
    const int V = int(ckpt.config.vocab_size);
    const std::size_t T = ckpt.config.seq_len;
    CHECK(throws<std::out_of_range>([&] { gpu.forward(V, 0); }));
    CHECK(throws<std::out_of_range>([&] { gpu.forward(-1, 0); }));
    CHECK(throws<std::out_of_range>([&] { gpu.forward(0, 1); }));
    CHECK(throws<std::invalid_argument>([&] { gpu.prefill({}, 0); }));
    CHECK(throws<std::out_of_range>([&] { gpu.prefill(std::vector<int>(T + 1, 0), 0); }));
    CHECK(close(gpu.prefill({1, 2, 3}, 0), cpu.prefill({1, 2, 3}, 0), "after errors", 0));
}

}  // namespace

int main() try {
    if (!em_available()) {
        std::puts("no GPU, skipping");
        return 77;
    }
    for (WeightType type : {WeightType::f32, WeightType::q8}) {
        test_matches_cpu(4, 4, true, type);
        test_matches_cpu(4, 2, false, type);
        test_matches_cpu(4, 1, true, type);
    }
    test_bad_inputs();
    if (failures) {
        std::fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    std::puts("all tests passed");
} catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
}
