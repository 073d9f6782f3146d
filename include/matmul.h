// The reference's CPU matmul entry points (/root/reference/src/matmul.h:1-22)
// with the same signatures, computed on the MI355X, so a caller written for
// them -- bench_matmul, test_matmul, Transformer::project (model.cpp:256-258)
// -- runs on the GPU unchanged. Each call uploads A and B, multiplies and
// downloads C (synchronously).
//
//   matmul_naive     -> GpuKernel::naive (one thread per element)
//   matmul_blocked   -> GpuKernel::tiled (LDS-tiled fp32 MFMA)
//   matmul_parallel  -> GpuKernel::automatic; `threads` is accepted and
//                       ignored (the GPU's parallelism is not a thread count)
//
// Shape mismatches throw std::invalid_argument naming both shapes, as the
// reference's check_shapes (matmul.cpp:54-64) does.
#pragma once

#include "cuda_matmul.h"

inline Tensor matmul_naive(const Tensor& A, const Tensor& B) {
    return matmul_cuda(A, B, GpuKernel::naive);
}

inline Tensor matmul_blocked(const Tensor& A, const Tensor& B) {
    return matmul_cuda(A, B, GpuKernel::tiled);
}

inline Tensor matmul_parallel(const Tensor& A, const Tensor& B, unsigned threads = 0) {
    (void)threads;
    return matmul_cuda(A, B, GpuKernel::automatic);
}

inline Tensor matmul_parallel(const Tensor& A, const QTensor& B, unsigned threads = 0) {
    (void)threads;
    return matmul_cuda(A, B, GpuKernel::automatic);
}
