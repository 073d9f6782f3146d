// The reference's CPU matmul entry points (declared in
// /root/reference/src/matmul.h:9-22), defined over this build's C ABI so
// the reference's own model code runs every product on the MI355X
// (TEST INFRASTRUCTURE: linked into oracle/_ref/stories_gpu in place of
// matmul.cpp).
//
// Weights (the B operand) are uploaded once and kept on the device, keyed
// by their host buffer: the model allocates them at load and never changes
// them. Activations are uploaded per call, and C is downloaded per call,
// which is what a host-resident caller of the drop-in pays. int8 B with
// its scales goes to em_matmul_q8; the scales stay on the device too.
#include <cstdint>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "llm_engine_amd.h"
#include "matmul.h"

namespace {

void check(int rc) {
    if (rc == EM_OK) return;
    if (rc == EM_EINVAL) throw std::invalid_argument(em_last_error());
    throw std::runtime_error(em_last_error());
}

std::string shape(std::size_t r, std::size_t c) { return std::to_string(r) + "x" + std::to_string(c); }

template <class BT>
void check_shapes(const Tensor& A, const BT& B) {
    if (A.cols == B.rows) return;
    throw std::invalid_argument("matmul: inner dimensions differ (A is " + shape(A.rows, A.cols) +
                                ", B is " + shape(B.rows, B.cols) + ")");
}

void* upload(const void* src, std::size_t bytes) {
    void* p = nullptr;
    check(em_malloc(&p, bytes));
    if (bytes) check(em_memcpy_h2d(p, src, bytes));
    return p;
}

// Device copy of a weight buffer, made on first use.
using Key = std::tuple<const void*, std::size_t>;
std::map<Key, void*> g_resident;

const void* resident(const void* host, std::size_t bytes) {
    const Key key{host, bytes};
    auto it = g_resident.find(key);
    if (it == g_resident.end()) it = g_resident.emplace(key, upload(host, bytes)).first;
    return it->second;
}

// Grow-only device buffers for A and C.
struct Buffer {
    void* p = nullptr;
    std::size_t cap = 0;
    void* get(std::size_t bytes) {
        if (bytes > cap) {
            check(em_free(p));
            p = nullptr;
            check(em_malloc(&p, bytes));
            cap = bytes;
        }
        return p;
    }
};
Buffer g_a, g_c;

Tensor product(const Tensor& A, std::size_t n, const void* B, const float* scale, int kernel) {
    const std::size_t m = A.rows, k = A.cols;
    Tensor C(m, n);
    if (m == 0 || n == 0) return C;
    float* dA = static_cast<float*>(g_a.get(m * k * sizeof(float)));
    float* dC = static_cast<float*>(g_c.get(m * n * sizeof(float)));
    if (m * k) check(em_memcpy_h2d(dA, A.data.data(), m * k * sizeof(float)));
    if (scale) {
        check(em_matmul_q8(m, n, k, dA, static_cast<const std::int8_t*>(B), scale, dC, kernel, 0,
                           nullptr, EM_STREAM_PER_THREAD));
    } else {
        check(em_matmul_f32(m, n, k, dA, static_cast<const float*>(B), dC, kernel, 0, nullptr,
                            EM_STREAM_PER_THREAD));
    }
    check(em_memcpy_d2h(C.data.data(), dC, m * n * sizeof(float)));
    return C;
}

Tensor run_f32(const Tensor& A, const Tensor& B, int kernel) {
    check_shapes(A, B);
    return product(A, B.cols, resident(B.data.data(), B.data.size() * sizeof(float)), nullptr,
                   kernel);
}

}  // namespace

Tensor matmul_naive(const Tensor& A, const Tensor& B) { return run_f32(A, B, EM_KERNEL_NAIVE); }

Tensor matmul_blocked(const Tensor& A, const Tensor& B) { return run_f32(A, B, EM_KERNEL_TILED); }

Tensor matmul_parallel(const Tensor& A, const Tensor& B, unsigned) {
    return run_f32(A, B, EM_KERNEL_AUTOMATIC);
}

Tensor matmul_parallel(const Tensor& A, const QTensor& B, unsigned) {
    check_shapes(A, B);
    const void* q = resident(B.data.data(), B.data.size());
    const float* s = static_cast<const float*>(resident(B.scale.data(), B.scale.size() * sizeof(float)));
    return product(A, B.cols, q, s, EM_KERNEL_AUTOMATIC);
}
