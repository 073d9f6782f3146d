// C++ interface of the MI355X matmul path, keeping the names, signatures,
// defaults and exception types of the reference's GPU matmul header
// (/root/reference/src/cuda_matmul.h:1-122) so its callers -- the forward
// pass (cuda_model.cu:164-173), bench_cuda and test_cuda -- build against it
// unchanged. Header-only: everything below forwards to the C ABI in
// llm_engine_amd.h (link libllm_engine_amd.so). The file name is the
// reference's; nothing here is CUDA.
//
// Calls run on the calling thread's default stream (hipStreamPerThread) and
// return before the GPU finishes, except download() and the Tensor
// overloads, which wait. Split-K scratch is library-owned and shared, so,
// as in the reference, calls from several host threads at once race.
//
// Errors: std::invalid_argument for bad shapes (the message names both as
// "RxC"), skinny with m > 8, or > 2^31 elements; std::runtime_error
// ("hip: <op>: <error>") for runtime failures and when no GPU is present.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>

#include "llm_engine_amd.h"
#include "tensor.h"

namespace em_detail {

inline void check(int rc) {
    if (rc == EM_OK) return;
    if (rc == EM_EINVAL) throw std::invalid_argument(em_last_error());
    throw std::runtime_error(em_last_error());
}

inline std::string dims(std::size_t r, std::size_t c) {
    return std::to_string(r) + "x" + std::to_string(c);
}

inline void inner_mismatch(std::size_t ar, std::size_t ac, std::size_t br, std::size_t bc) {
    throw std::invalid_argument("matmul_cuda: inner dimensions differ (A is " + dims(ar, ac) +
                                ", B is " + dims(br, bc) + ")");
}

}  // namespace em_detail

// Row-major fp32 matrix in GPU memory. Move-only; frees on destruction
// (cuda_matmul.h:16-40).
class DeviceTensor {
public:
    DeviceTensor() = default;
    DeviceTensor(std::size_t rows, std::size_t cols) : rows_(rows), cols_(cols) {
        void* p = nullptr;
        em_detail::check(em_malloc(&p, rows * cols * sizeof(float)));
        data_ = static_cast<float*>(p);
    }
    explicit DeviceTensor(const Tensor& t) : DeviceTensor(t.rows, t.cols) { upload(t); }
    ~DeviceTensor() { em_free(data_); }

    DeviceTensor(DeviceTensor&& o) noexcept
        : rows_(std::exchange(o.rows_, 0)), cols_(std::exchange(o.cols_, 0)),
          data_(std::exchange(o.data_, nullptr)) {}
    DeviceTensor& operator=(DeviceTensor&& o) noexcept {
        std::swap(rows_, o.rows_);
        std::swap(cols_, o.cols_);
        std::swap(data_, o.data_);
        return *this;
    }
    DeviceTensor(const DeviceTensor&) = delete;
    DeviceTensor& operator=(const DeviceTensor&) = delete;

    // Copies t in, reallocating if the shape differs.
    void upload(const Tensor& t) {
        if (t.rows != rows_ || t.cols != cols_) *this = DeviceTensor(t.rows, t.cols);
        if (!t.data.empty())
            em_detail::check(em_memcpy_h2d(data_, t.data.data(), t.data.size() * sizeof(float)));
    }
    Tensor download() const {
        Tensor t(rows_, cols_);
        if (!t.data.empty())
            em_detail::check(em_memcpy_d2h(t.data.data(), data_, t.data.size() * sizeof(float)));
        return t;
    }

    std::size_t rows() const { return rows_; }
    std::size_t cols() const { return cols_; }
    float* data() { return data_; }
    const float* data() const { return data_; }

private:
    std::size_t rows_ = 0, cols_ = 0;
    float* data_ = nullptr;
};

// int8 matrix plus one fp32 scale per column in GPU memory, as QTensor.
// Move-only (cuda_matmul.h:42-64). Also registers a strip-layout copy of its
// bytes with the library (em_q8_register; EM_STRIP_COPY=0 turns it off).
class DeviceQTensor {
public:
    DeviceQTensor() = default;
    explicit DeviceQTensor(const QTensor& t) : rows_(t.rows), cols_(t.cols) {
        if (t.data.size() != rows_ * cols_ || t.scale.size() != cols_)
            throw std::invalid_argument("DeviceQTensor: data or scale size doesn't match the shape");
        try {
            void* p = nullptr;
            em_detail::check(em_malloc(&p, t.data.size()));
            data_ = static_cast<std::int8_t*>(p);
            em_detail::check(em_malloc(&p, t.scale.size() * sizeof(float)));
            scale_ = static_cast<float*>(p);
            if (!t.data.empty()) em_detail::check(em_memcpy_h2d(data_, t.data.data(), t.data.size()));
            if (!t.scale.empty())
                em_detail::check(
                    em_memcpy_h2d(scale_, t.scale.data(), t.scale.size() * sizeof(float)));
            // The library's strip copy of the bytes (em_q8_register): products
            // of up to 8 rows over this matrix then run in one launch. The
            // bytes are never written again, so the copy stays valid.
            em_detail::check(em_q8_register(data_, rows_, cols_, EM_STREAM_PER_THREAD));
        } catch (...) {
            em_q8_unregister(data_);
            em_free(data_);
            em_free(scale_);
            throw;
        }
    }
    ~DeviceQTensor() {
        em_q8_unregister(data_);
        em_free(data_);
        em_free(scale_);
    }

    DeviceQTensor(DeviceQTensor&& o) noexcept
        : rows_(std::exchange(o.rows_, 0)), cols_(std::exchange(o.cols_, 0)),
          data_(std::exchange(o.data_, nullptr)), scale_(std::exchange(o.scale_, nullptr)) {}
    DeviceQTensor& operator=(DeviceQTensor&& o) noexcept {
        std::swap(rows_, o.rows_);
        std::swap(cols_, o.cols_);
        std::swap(data_, o.data_);
        std::swap(scale_, o.scale_);
        return *this;
    }
    DeviceQTensor(const DeviceQTensor&) = delete;
    DeviceQTensor& operator=(const DeviceQTensor&) = delete;

    std::size_t rows() const { return rows_; }
    std::size_t cols() const { return cols_; }
    const std::int8_t* data() const { return data_; }
    const float* scale() const { return scale_; }

private:
    std::size_t rows_ = 0, cols_ = 0;
    std::int8_t* data_ = nullptr;
    float* scale_ = nullptr;
};

// cuda_matmul.h:66-72. The values are the C ABI's EM_KERNEL_* codes.
enum class GpuKernel {
    automatic = EM_KERNEL_AUTOMATIC,      // fp32: skinny for m <= 8 (m <= 3 for 2^25 weights or
                                          // more), else tiled_split (tiled if B is unaligned); int8:
                                          // skinny for 1 row and for 2-4 rows of small weights,
                                          // else exact-split bf16 MFMA
    naive = EM_KERNEL_NAIVE,              // one thread per element of C; the reference kernel
    tiled = EM_KERNEL_TILED,              // LDS-tiled fp32 MFMA, 128 x 128 tiles
    tiled_split = EM_KERNEL_TILED_SPLIT,  // MFMA on 16/32-row tiles, B streamed once, k split
    skinny = EM_KERNEL_SKINNY,            // m <= 8: wave64 GEMV, k split across waves and blocks
};

// cuda_matmul.h:85-92.
struct MatmulFusion {
    bool accumulate = false;               // C += A x B
    const float* rms_weight = nullptr;     // multiply rmsnorm(A) * rms_weight (k device floats)
};

inline void matmul_cuda(std::size_t m, std::size_t n, std::size_t k, const float* A,
                        const float* B, float* C, GpuKernel kernel = GpuKernel::automatic,
                        const MatmulFusion& fusion = {}) {
    em_detail::check(em_matmul_f32(m, n, k, A, B, C, static_cast<int>(kernel),
                                   fusion.accumulate ? 1 : 0, fusion.rms_weight,
                                   EM_STREAM_PER_THREAD));
}

inline void matmul_cuda(std::size_t m, std::size_t n, std::size_t k, const float* A,
                        const std::int8_t* B, const float* scale, float* C,
                        GpuKernel kernel = GpuKernel::automatic, const MatmulFusion& fusion = {}) {
    em_detail::check(em_matmul_q8(m, n, k, A, B, scale, C, static_cast<int>(kernel),
                                  fusion.accumulate ? 1 : 0, fusion.rms_weight,
                                  EM_STREAM_PER_THREAD));
}

// C = A x B; C is reallocated if it isn't m x n (cuda_matmul.h:74-78).
inline void matmul_cuda(const DeviceTensor& A, const DeviceTensor& B, DeviceTensor& C,
                        GpuKernel kernel = GpuKernel::automatic) {
    if (A.cols() != B.rows()) em_detail::inner_mismatch(A.rows(), A.cols(), B.rows(), B.cols());
    if (C.rows() != A.rows() || C.cols() != B.cols()) C = DeviceTensor(A.rows(), B.cols());
    matmul_cuda(A.rows(), B.cols(), A.cols(), A.data(), B.data(), C.data(), kernel);
}

inline std::size_t cuda_scratch_generation() { return em_scratch_generation(); }

inline void cuda_synchronize() { em_detail::check(em_synchronize()); }

inline bool cuda_available() { return em_available() != 0; }

// Copies A and B to the GPU, multiplies, copies C back (cuda_matmul.h:114-116).
inline Tensor matmul_cuda(const Tensor& A, const Tensor& B,
                          GpuKernel kernel = GpuKernel::automatic) {
    if (A.cols != B.rows) em_detail::inner_mismatch(A.rows, A.cols, B.rows, B.cols);
    const DeviceTensor dA(A), dB(B);
    DeviceTensor dC;
    matmul_cuda(dA, dB, dC, kernel);
    return dC.download();
}

inline Tensor matmul_cuda(const Tensor& A, const QTensor& B,
                          GpuKernel kernel = GpuKernel::automatic) {
    if (A.cols != B.rows) em_detail::inner_mismatch(A.rows, A.cols, B.rows, B.cols);
    const DeviceTensor dA(A);
    const DeviceQTensor dB(B);
    DeviceTensor dC(A.rows, B.cols);
    matmul_cuda(A.rows, B.cols, A.cols, dA.data(), dB.data(), dB.scale(), dC.data(), kernel);
    return dC.download();
}
