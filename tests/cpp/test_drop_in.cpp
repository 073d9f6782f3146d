// The reference's GPU test (/root/reference/tests/test_cuda.cpp), run
// against this build's drop-in headers (include/cuda_matmul.h, matmul.h,
// quant.h) instead of the CUDA library, with the CPU oracle (oracle/oracle.c,
// linked as liboracle.so) as the reference product. Same shapes, seeds,
// kernels, fusions and tolerance (1e-5 * k); exits 77 (skip) without a GPU,
// as test_cuda.cpp:291-295 does.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <iterator>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "cuda_matmul.h"
#include "matmul.h"
#include "quant.h"

extern "C" {
void orc_quantize_q8(size_t rows, size_t cols, const float* B, int8_t* q, float* scale);
void orc_dequantize(size_t rows, size_t cols, const int8_t* q, const float* scale, float* out);
void orc_matmul_naive(size_t m, size_t n, size_t k, const float* A, const float* B, float* C);
void orc_rmsnorm(size_t rows, size_t cols, const float* x, const float* w, float eps, float* y);
}

namespace {

int failures = 0;

#define CHECK(cond)                                                                    \
    do {                                                                               \
        if (!(cond)) {                                                                 \
            std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                                                \
        }                                                                              \
    } while (0)

Tensor random_tensor(std::size_t rows, std::size_t cols, std::mt19937& rng) {
    std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
    Tensor t(rows, cols);
    for (auto& x : t.data) x = dist(rng);
    return t;
}

// The oracle's products and ops, on Tensors.
Tensor ref_matmul(const Tensor& A, const Tensor& B) {
    Tensor C(A.rows, B.cols);
    orc_matmul_naive(A.rows, B.cols, A.cols, A.data.data(), B.data.data(), C.data.data());
    return C;
}
Tensor ref_rmsnorm(const Tensor& x, const std::vector<float>& w) {
    Tensor y(x.rows, x.cols);
    orc_rmsnorm(x.rows, x.cols, x.data.data(), w.data(), 1e-5f, y.data.data());
    return y;
}
QTensor ref_quantize(const Tensor& B) {
    QTensor q;
    q.rows = B.rows;
    q.cols = B.cols;
    q.data.resize(B.data.size());
    q.scale.resize(B.cols);
    orc_quantize_q8(B.rows, B.cols, B.data.data(), q.data.data(), q.scale.data());
    return q;
}
Tensor ref_dequantize(const QTensor& q) {
    Tensor t(q.rows, q.cols);
    orc_dequantize(q.rows, q.cols, q.data.data(), q.scale.data(), t.data.data());
    return t;
}

bool close_to(const Tensor& got, const Tensor& want, std::size_t k) {
    if (got.rows != want.rows || got.cols != want.cols) return false;
    const float tol = 1e-5f * static_cast<float>(std::max<std::size_t>(k, 1));
    for (std::size_t i = 0; i < got.data.size(); ++i)
        if (!(std::fabs(got.data[i] - want.data[i]) <= tol)) return false;
    return true;
}

struct Kernel {
    const char* name;
    GpuKernel kernel;
    std::size_t max_m;
};
const Kernel kKernels[] = {
    {"naive", GpuKernel::naive, ~std::size_t{0}},
    {"tiled", GpuKernel::tiled, ~std::size_t{0}},
    {"tiled_split", GpuKernel::tiled_split, ~std::size_t{0}},
    {"skinny", GpuKernel::skinny, 8},
    {"automatic", GpuKernel::automatic, ~std::size_t{0}},
};

struct Shape { std::size_t m, k, n; };
constexpr Shape kShapes[] = {
    {1, 1, 1},     {1, 17, 1},     {3, 5, 7},      {8, 8, 128},    {9, 9, 129},
    {127, 300, 129}, {128, 256, 128}, {200, 513, 33}, {130, 70, 1030},
    {1, 4096, 288}, {1, 288, 4096}, {2, 1000, 70},  {4, 4097, 33},  {7, 64, 4111},
    {8, 513, 2049}, {16, 4096, 300}, {33, 1029, 257}, {64, 2000, 4096},
    {1, 0, 5},      {12, 0, 3},
};

void test_against_reference() {
    std::mt19937 rng(42);
    for (const Shape& s : kShapes) {
        const Tensor A = random_tensor(s.m, s.k, rng);
        const Tensor B = random_tensor(s.k, s.n, rng);
        const Tensor want = ref_matmul(A, B);
        for (const Kernel& k : kKernels) {
            if (s.m > k.max_m) continue;
            if (!close_to(matmul_cuda(A, B, k.kernel), want, s.k)) {
                std::fprintf(stderr, "  [%s] mismatch at m=%zu k=%zu n=%zu\n", k.name, s.m, s.k, s.n);
                CHECK(false);
            }
        }
    }
}

void test_reuse() {
    std::mt19937 rng(5);
    DeviceTensor C(3, 3);
    for (const Shape& s : {Shape{1, 2000, 300}, Shape{4, 100, 5000}, Shape{64, 3000, 64},
                           Shape{200, 64, 64}}) {
        const Tensor A = random_tensor(s.m, s.k, rng);
        const Tensor B = random_tensor(s.k, s.n, rng);
        const DeviceTensor dA(A), dB(B);
        matmul_cuda(dA, dB, C);
        CHECK(C.rows() == s.m && C.cols() == s.n);
        CHECK(close_to(C.download(), ref_matmul(A, B), s.k));
    }
}

Tensor add(const Tensor& a, const Tensor& b) {
    Tensor c = a;
    for (std::size_t i = 0; i < c.data.size(); ++i) c.data[i] += b.data[i];
    return c;
}

template <class F>
std::string invalid_argument_of(F&& f) {
    try {
        f();
    } catch (const std::invalid_argument& e) {
        return e.what();
    }
    return "";
}

void test_fusion() {
    std::mt19937 rng(9);
    for (const Shape& s : {Shape{1, 288, 300}, Shape{3, 100, 70}, Shape{8, 513, 129},
                           Shape{9, 64, 33}, Shape{70, 40, 130}}) {
        const Tensor A = random_tensor(s.m, s.k, rng);
        const Tensor B = random_tensor(s.k, s.n, rng);
        const Tensor C0 = random_tensor(s.m, s.n, rng);
        Tensor w_host = random_tensor(1, s.k, rng);
        const std::vector<float> w = w_host.data;
        const DeviceTensor dA(A), dB(B), dW(w_host);
        MatmulFusion acc, norm, norm_acc;
        acc.accumulate = norm_acc.accumulate = true;
        norm.rms_weight = norm_acc.rms_weight = dW.data();
        const Tensor plain = ref_matmul(A, B);
        const Tensor normed = ref_matmul(ref_rmsnorm(A, w), B);
        struct Case {
            const char* name;
            MatmulFusion fusion;
            Tensor want;
        };
        const Case cases[] = {
            {"accumulate", acc, add(C0, plain)},
            {"rms", norm, normed},
            {"rms + accumulate", norm_acc, add(C0, normed)},
        };
        for (const Kernel& k : kKernels) {
            if (s.m > k.max_m) continue;
            for (const Case& c : cases) {
                DeviceTensor dC(C0);
                matmul_cuda(s.m, s.n, s.k, dA.data(), dB.data(), dC.data(), k.kernel, c.fusion);
                if (!close_to(dC.download(), c.want, 2 * s.k)) {
                    std::fprintf(stderr, "  [%s] %s mismatch at m=%zu k=%zu n=%zu\n", k.name, c.name,
                                 s.m, s.k, s.n);
                    CHECK(false);
                }
            }
        }
    }
}

void test_q8() {
    std::mt19937 rng(11);
    std::vector<Shape> shapes(std::begin(kShapes), std::end(kShapes));
    shapes.insert(shapes.end(), {{3, 100, 1028}, {8, 1000, 4100}, {6, 20, 36}, {1, 4096, 4}});
    for (const Shape& s : shapes) {
        const Tensor A = random_tensor(s.m, s.k, rng);
        const Tensor Bf = random_tensor(s.k, s.n, rng);
        const QTensor Bq = quantize_q8(Bf);  // on the GPU
        const QTensor Bq_ref = ref_quantize(Bf);
        CHECK(Bq.data == Bq_ref.data && Bq.scale == Bq_ref.scale);  // bit-exact
        const Tensor want = ref_matmul(A, ref_dequantize(Bq_ref));
        for (const Kernel& k : kKernels) {
            if (s.m > k.max_m) continue;
            if (!close_to(matmul_cuda(A, Bq, k.kernel), want, s.k)) {
                std::fprintf(stderr, "  [%s] q8 mismatch at m=%zu k=%zu n=%zu\n", k.name, s.m, s.k,
                             s.n);
                CHECK(false);
            }
        }
    }
    for (const Shape& s : {Shape{1, 288, 300}, Shape{5, 768, 288}, Shape{2, 20, 64},
                           Shape{3, 288, 30}, Shape{70, 40, 130}}) {
        const Tensor A = random_tensor(s.m, s.k, rng);
        const QTensor Bq = ref_quantize(random_tensor(s.k, s.n, rng));
        const Tensor C0 = random_tensor(s.m, s.n, rng);
        const Tensor w_host = random_tensor(1, s.k, rng);
        const DeviceTensor dA(A), dW(w_host);
        const DeviceQTensor dB(Bq);
        MatmulFusion f;
        f.accumulate = true;
        f.rms_weight = dW.data();
        const Tensor want = add(C0, ref_matmul(ref_rmsnorm(A, w_host.data), ref_dequantize(Bq)));
        for (const Kernel& k : kKernels) {
            if (s.m > k.max_m) continue;
            DeviceTensor dC(C0);
            matmul_cuda(s.m, s.n, s.k, dA.data(), dB.data(), dB.scale(), dC.data(), k.kernel, f);
            if (!close_to(dC.download(), want, 2 * s.k)) {
                std::fprintf(stderr, "  [%s] q8 fused mismatch at m=%zu k=%zu n=%zu\n", k.name, s.m,
                             s.k, s.n);
                CHECK(false);
            }
        }
    }
}

void test_split_k_queue() {
    std::mt19937 rng(13);
    struct Case {
        Shape s;
        bool q8, accumulate;
    };
    const Case cases[] = {
        {{1, 4096, 4096}, false, false}, {{8, 4096, 4100}, true, true},
        {{1, 288, 32000}, true, false},  {{3, 768, 288}, false, true},
        {{1, 288, 864}, true, true},     {{5, 1000, 70}, true, false},
    };
    constexpr int kRepeats = 3;
    for (int round = 0; round < 2; ++round) {
        std::vector<DeviceTensor> outs;
        std::vector<Tensor> wants;
        std::vector<DeviceTensor> keep_a, keep_b;
        std::vector<DeviceQTensor> keep_q;
        for (const Case& c : cases) {
            const Tensor A = random_tensor(c.s.m, c.s.k, rng);
            const Tensor B = random_tensor(c.s.k, c.s.n, rng);
            const Tensor C0 = random_tensor(c.s.m, c.s.n, rng);
            const QTensor Bq = ref_quantize(B);
            const Tensor prod = ref_matmul(A, c.q8 ? ref_dequantize(Bq) : B);
            keep_a.emplace_back(A);
            if (c.q8) {
                keep_q.emplace_back(Bq);
            } else {
                keep_b.emplace_back(B);
            }
            MatmulFusion f;
            f.accumulate = c.accumulate;
            for (int r = 0; r < kRepeats; ++r) {
                outs.emplace_back(C0);
                if (c.q8) {
                    matmul_cuda(c.s.m, c.s.n, c.s.k, keep_a.back().data(), keep_q.back().data(),
                                keep_q.back().scale(), outs.back().data(), GpuKernel::skinny, f);
                } else {
                    matmul_cuda(c.s.m, c.s.n, c.s.k, keep_a.back().data(), keep_b.back().data(),
                                outs.back().data(), GpuKernel::skinny, f);
                }
                wants.push_back(c.accumulate ? add(C0, prod) : prod);
            }
        }
        for (std::size_t i = 0; i < outs.size(); ++i) {
            const Tensor got = outs[i].download();
            const Case& c = cases[i / kRepeats];
            if (!close_to(got, wants[i], 2 * c.s.k)) {
                std::fprintf(stderr, "  split-K queue mismatch at m=%zu k=%zu n=%zu%s\n", c.s.m,
                             c.s.k, c.s.n, c.q8 ? " (q8)" : "");
                CHECK(false);
            }
            if (i % kRepeats) CHECK(got.data == outs[i - 1].download().data);
        }
    }
}

void test_bad_shapes() {
    const std::string msg = invalid_argument_of([] { matmul_cuda(Tensor(2, 3), Tensor(4, 2)); });
    CHECK(msg.find("2x3") != std::string::npos && msg.find("4x2") != std::string::npos);
    CHECK(!invalid_argument_of([] { matmul_cuda(Tensor(2, 3), quantize_q8(Tensor(4, 2))); }).empty());
    CHECK(!invalid_argument_of([] { matmul_cuda(Tensor(9, 2), Tensor(2, 2), GpuKernel::skinny); })
               .empty());
    // matmul.h and quant.h (test_matmul.cpp:40-66, test_quant.cpp:81-90).
    const std::string m2 = invalid_argument_of([] { matmul_parallel(Tensor(2, 3), Tensor(4, 2)); });
    CHECK(m2.find("2x3") != std::string::npos && m2.find("4x2") != std::string::npos);
    const std::string m3 =
        invalid_argument_of([] { matmul_parallel(Tensor(2, 3), quantize_q8(Tensor(4, 2))); });
    CHECK(m3.find("2x3") != std::string::npos && m3.find("4x2") != std::string::npos);
}

// test_matmul.cpp:40-52 on the matmul.h drop-in.
void test_known_values() {
    Tensor A(2, 3), B(3, 2);
    float v = 1.0f;
    for (auto& x : A.data) x = v++;
    for (auto& x : B.data) x = v++;
    for (Tensor C : {matmul_naive(A, B), matmul_blocked(A, B), matmul_parallel(A, B)}) {
        CHECK(C.rows == 2 && C.cols == 2);
        CHECK(C.at(0, 0) == 58.0f && C.at(0, 1) == 64.0f);
        CHECK(C.at(1, 0) == 139.0f && C.at(1, 1) == 154.0f);
    }
}

// test_quant.cpp:33-51 on the GPU quantiser.
void test_round_trip() {
    std::mt19937 rng(3);
    std::uniform_real_distribution<float> dist(-2.0f, 2.0f);
    Tensor B(37, 21);
    for (auto& x : B.data) x = dist(rng);
    for (std::size_t c = 0; c < B.cols; ++c) B.at(5, c) *= float(c + 1);
    for (std::size_t r = 0; r < B.rows; ++r) B.at(r, 4) = 0.0f;
    const QTensor q = quantize_q8(B);
    const Tensor d = dequantize(q);
    const QTensor q_ref = ref_quantize(B);
    CHECK(q.data == q_ref.data && q.scale == q_ref.scale);
    CHECK(q.scale[4] == 0.0f);
    for (std::size_t c = 0; c < B.cols; ++c) {
        int max_q = 0;
        for (std::size_t r = 0; r < B.rows; ++r) {
            max_q = std::max(max_q, std::abs(int(q.data[r * B.cols + c])));
            CHECK(std::fabs(d.at(r, c) - B.at(r, c)) <= q.scale[c] * 0.5f * (1 + 1e-5f));
        }
        CHECK(max_q == (c == 4 ? 0 : 127));
    }
}

}  // namespace

int main() try {
    if (!cuda_available()) {
        std::puts("no GPU device, skipping");
        return 77;
    }
    test_known_values();
    test_round_trip();
    test_against_reference();
    test_reuse();
    test_fusion();
    test_q8();
    test_split_k_queue();
    test_bad_shapes();
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
