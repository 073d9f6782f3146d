// C entry points over the reference's own CPU code, compiled from the source
// files under /root/reference/src by oracle/Makefile into oracle/_ref/.
// TEST INFRASTRUCTURE ONLY: it pins the C oracle (tests/test_oracle.py,
// tests/golden/make_golden.py) and is the CPU baseline that bench.py times
// (cpu_baseline.kind = "reference"). Nothing in the product links it.
//
// Bindings (reference file:line):
//   ref_quantize_q8 / ref_dequantize    quant.h:7-9, quant.cpp:6-36
//   ref_matmul_{naive,blocked,parallel} matmul.h:9-19, matmul.cpp:205-225,310-313
//   ref_matmul_parallel_q8              matmul.h:20-22, matmul.cpp:315-318
//   ref_rmsnorm                         ops.h:12, ops.cpp:8-26
//   ref_pool_size                       thread_pool.h:27-35
//   ref_time_parallel_{f32,q8}          the timing method of bench/bench_matmul.cpp:49-63
//                                       (one warm-up, then the median of reps)
#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "matmul.h"
#include "ops.h"
#include "quant.h"
#include "thread_pool.h"

namespace {

thread_local std::string g_error;

Tensor make_tensor(std::size_t rows, std::size_t cols, const float* data) {
    Tensor t(rows, cols);
    if (rows * cols) std::memcpy(t.data.data(), data, rows * cols * sizeof(float));
    return t;
}

QTensor make_qtensor(std::size_t rows, std::size_t cols, const std::int8_t* q, const float* scale) {
    QTensor t;
    t.rows = rows;
    t.cols = cols;
    t.data.assign(q, q + rows * cols);
    t.scale.assign(scale, scale + cols);
    return t;
}

void copy_out(const Tensor& t, float* out) {
    if (!t.data.empty()) std::memcpy(out, t.data.data(), t.data.size() * sizeof(float));
}

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 1;
    }
}

volatile float g_sink;

template <class F>
double median_seconds(F&& f, int reps) {
    using Clock = std::chrono::steady_clock;
    {
        Tensor warm = f();
        if (!warm.data.empty()) g_sink = warm.data[0];
    }
    std::vector<double> times;
    times.reserve(static_cast<std::size_t>(reps));
    for (int r = 0; r < reps; ++r) {
        const auto t0 = Clock::now();
        Tensor C = f();
        const auto t1 = Clock::now();
        if (!C.data.empty()) g_sink = C.data[0];
        times.push_back(std::chrono::duration<double>(t1 - t0).count());
    }
    std::nth_element(times.begin(), times.begin() + reps / 2, times.end());
    return times[static_cast<std::size_t>(reps / 2)];
}

} // namespace

extern "C" {

const char* ref_last_error() { return g_error.c_str(); }

unsigned ref_pool_size() { return ThreadPool::global().size(); }

int ref_quantize_q8(std::size_t rows, std::size_t cols, const float* B, std::int8_t* q,
                    float* scale) {
    return guarded([&] {
        const QTensor t = quantize_q8(make_tensor(rows, cols, B));
        if (!t.data.empty()) std::memcpy(q, t.data.data(), t.data.size());
        if (!t.scale.empty()) std::memcpy(scale, t.scale.data(), t.scale.size() * sizeof(float));
    });
}

int ref_dequantize(std::size_t rows, std::size_t cols, const std::int8_t* q, const float* scale,
                   float* out) {
    return guarded([&] { copy_out(dequantize(make_qtensor(rows, cols, q, scale)), out); });
}

// which: 0 naive, 1 blocked, 2 parallel.
int ref_matmul_f32(int which, std::size_t m, std::size_t n, std::size_t k, const float* A,
                   const float* B, float* C, unsigned threads) {
    return guarded([&] {
        const Tensor a = make_tensor(m, k, A), b = make_tensor(k, n, B);
        Tensor c = which == 0   ? matmul_naive(a, b)
                   : which == 1 ? matmul_blocked(a, b)
                                : matmul_parallel(a, b, threads);
        copy_out(c, C);
    });
}

int ref_matmul_parallel_q8(std::size_t m, std::size_t n, std::size_t k, const float* A,
                           const std::int8_t* q, const float* scale, float* C, unsigned threads) {
    return guarded([&] {
        copy_out(matmul_parallel(make_tensor(m, k, A), make_qtensor(k, n, q, scale), threads), C);
    });
}

// Shape-error text of matmul_parallel(Tensor(ar, ac), Tensor(br, bc)), for
// the message checks of tests/test_matmul.cpp:56-66.
int ref_shape_error(std::size_t ar, std::size_t ac, std::size_t br, std::size_t bc) {
    return guarded([&] { matmul_parallel(Tensor(ar, ac), Tensor(br, bc)); });
}

int ref_rmsnorm(std::size_t rows, std::size_t cols, const float* x, const float* w, float eps,
                float* y) {
    return guarded([&] {
        copy_out(rmsnorm(make_tensor(rows, cols, x), std::vector<float>(w, w + cols), eps), y);
    });
}

// Median seconds of matmul_parallel(A, B) after one warm-up; A and B are
// copied into the reference's Tensor types once, outside the timed calls.
double ref_time_parallel_f32(std::size_t m, std::size_t n, std::size_t k, const float* A,
                             const float* B, int reps, unsigned threads) {
    const Tensor a = make_tensor(m, k, A), b = make_tensor(k, n, B);
    return median_seconds([&] { return matmul_parallel(a, b, threads); }, reps);
}

double ref_time_parallel_q8(std::size_t m, std::size_t n, std::size_t k, const float* A,
                            const std::int8_t* q, const float* scale, int reps, unsigned threads) {
    const Tensor a = make_tensor(m, k, A);
    const QTensor b = make_qtensor(k, n, q, scale);
    return median_seconds([&] { return matmul_parallel(a, b, threads); }, reps);
}

} // extern "C"
