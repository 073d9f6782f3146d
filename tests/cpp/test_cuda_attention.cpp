// The reference's GPU attention test (/root/reference/tests/
// test_cuda_attention.cpp) against this build's drop-in header
// (include/cuda_attention.h): the same shapes, kernels, rows and positions,
// a double-precision reference, its tolerance 5e-5 and the bit-identical
// second call; exits 77 (skip) without a GPU, as the reference does
// (:198-202).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <initializer_list>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "cuda_attention.h"
#include "cuda_matmul.h"

namespace {

int failures = 0;

#define CHECK(cond)                                                                    \
    do {                                                                               \
        if (!(cond)) {                                                                 \
            std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                                                \
        }                                                                              \
    } while (0)

constexpr double kTol = 5e-5;

Tensor uniform(std::size_t rows, std::size_t cols, std::mt19937& rng) {
    std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
    Tensor t(rows, cols);
    for (float& x : t.data) x = dist(rng);
    return t;
}

// Causal softmax attention in double, as attention_cuda() is specified.
std::vector<double> expected(const AttentionShape& s, std::size_t rows, int pos, const Tensor& q,
                             const Tensor& kc, const Tensor& vc) {
    const std::size_t hs = s.head_size, group = s.n_heads / s.n_kv_heads;
    const std::size_t dim = std::size_t(s.n_heads) * hs;
    std::vector<double> out(rows * dim, 0.0);
    std::vector<double> w;
    for (std::size_t i = 0; i < rows; ++i) {
        const std::size_t ctx = std::size_t(pos) + i + 1;
        w.assign(ctx, 0.0);
        for (std::size_t h = 0; h < std::size_t(s.n_heads); ++h) {
            const std::size_t kv = (h / group) * hs;
            double top = -INFINITY;
            for (std::size_t t = 0; t < ctx; ++t) {
                double d = 0.0;
                for (std::size_t j = 0; j < hs; ++j)
                    d += double(q.data[i * s.q_stride + h * hs + j]) *
                         double(kc.data[t * s.kv_stride + kv + j]);
                w[t] = d / std::sqrt(double(hs));
                top = std::max(top, w[t]);
            }
            double total = 0.0;
            for (double& x : w) total += x = std::exp(x - top);
            for (std::size_t j = 0; j < hs; ++j) {
                double acc = 0.0;
                for (std::size_t t = 0; t < ctx; ++t) acc += w[t] * double(vc.data[t * s.kv_stride + kv + j]);
                out[i * dim + h * hs + j] = acc / total;
            }
        }
    }
    return out;
}

const char* name(AttentionKernel k) {
    return k == AttentionKernel::single_block ? "single_block"
           : k == AttentionKernel::split      ? "split"
                                              : "automatic";
}

struct Case {
    int heads, kv_heads, head_size, seq_len;
};

void run_case(const Case& c, AttentionKernel kernel, std::initializer_list<int> positions,
              std::size_t rows, std::mt19937& rng) {
    const std::size_t hs = c.head_size, kv = std::size_t(c.kv_heads) * hs;
    const std::size_t dim = std::size_t(c.heads) * hs;
    const AttentionShape s{c.heads, c.kv_heads, c.head_size, c.seq_len, dim + 2 * kv, kv, dim};
    try {
        attention_check(s, kernel);
    } catch (const std::invalid_argument& e) {
        std::fprintf(stderr, "  %s rejected %d/%d x %d: %s\n", name(kernel), c.heads, c.kv_heads,
                     c.head_size, e.what());
        ++failures;
        return;
    }
    const Tensor q = uniform(rows, s.q_stride, rng);
    const Tensor kc = uniform(std::size_t(c.seq_len), kv, rng);
    const Tensor vc = uniform(std::size_t(c.seq_len), kv, rng);
    const DeviceTensor dq(q), dk(kc), dv(vc);
    DeviceTensor out(rows, dim);
    const std::size_t n = attention_scratch_floats(s, rows, kernel);
    DeviceTensor scratch(1, std::max<std::size_t>(1, n));
    void* pos_dev = nullptr;
    if (em_malloc(&pos_dev, sizeof(int)) != EM_OK) throw std::runtime_error(em_last_error());
    for (int pos : positions) {
        if (pos < 0 || std::size_t(pos) + rows > std::size_t(c.seq_len)) continue;
        em_memcpy_h2d(pos_dev, &pos, sizeof pos);
        attention_cuda(s, rows, static_cast<const int*>(pos_dev), dq.data(), dk.data(), dv.data(),
                       out.data(), scratch.data(), kernel);
        const Tensor got = out.download();
        attention_cuda(s, rows, static_cast<const int*>(pos_dev), dq.data(), dk.data(), dv.data(),
                       out.data(), scratch.data(), kernel);
        const Tensor again = out.download();
        const std::vector<double> want = expected(s, rows, pos, q, kc, vc);
        double diff = 0.0;
        for (std::size_t j = 0; j < want.size(); ++j)
            diff = std::max(diff, std::fabs(double(got.data[j]) - want[j]));
        if (diff > kTol) {
            std::fprintf(stderr, "  %s %d/%d x %d, seq_len %d, pos %d, %zu rows: max diff %g\n",
                         name(kernel), c.heads, c.kv_heads, c.head_size, c.seq_len, pos, rows, diff);
            ++failures;
        }
        CHECK(got.data == again.data);
    }
    em_free(pos_dev);
}

void test_kernels() {
    std::mt19937 rng(7);
    const Case cases[] = {{6, 6, 48, 256}, {8, 2, 64, 1000}, {8, 1, 32, 600},
                          {4, 2, 16, 300}, {6, 2, 32, 300}};
    for (const Case& c : cases)
        for (AttentionKernel k : {AttentionKernel::single_block, AttentionKernel::split,
                                  AttentionKernel::automatic})
            for (std::size_t rows : {1, 3, 8, 12})
                run_case(c, k, {0, 31, 32, 33, 200, c.seq_len - int(rows)}, rows, rng);
}

void test_long_context() {
    std::mt19937 rng(11);
    const Case c{4, 1, 128, 20000};
    const AttentionShape s{4, 1, 128, 20000, 4 * 128 + 2 * 128, 128, 4 * 128};
    bool threw = false;
    try {
        attention_check(s, AttentionKernel::single_block);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    CHECK(threw);
    run_case(c, AttentionKernel::split, {0, 5000, 19999}, 1, rng);
    run_case(c, AttentionKernel::automatic, {12345, 19990}, 10, rng);
}

void test_bad_shapes() {
    auto rejects = [](const AttentionShape& s, AttentionKernel k) {
        try {
            attention_check(s, k);
        } catch (const std::invalid_argument&) {
            return true;
        }
        return false;
    };
    CHECK(rejects({2, 2, 6, 64, 36, 12, 12}, AttentionKernel::split));
    CHECK(!rejects({2, 2, 6, 64, 36, 12, 12}, AttentionKernel::single_block));
    CHECK(rejects({6, 4, 8, 64, 96, 32, 48}, AttentionKernel::automatic));
    CHECK(rejects({4, 4, 8, 0, 64, 32, 32}, AttentionKernel::automatic));
}

}  // namespace

int main() try {
    test_bad_shapes();  // host-only checks
    if (!cuda_available()) {
        std::puts("no GPU, skipping");
        return failures ? 1 : 77;
    }
    test_kernels();
    test_long_context();
    cuda_synchronize();
    if (failures) {
        std::fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    std::puts("all tests passed");
} catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
}
