/*
 * llm_engine_amd.h -- C ABI of the MI355X (gfx950) matmul hot path.
 *
 * Plain pointers and sizes only. Every entry point validates its arguments on
 * the host before it touches the GPU, returns EM_OK or an error code, and
 * leaves a message for em_last_error(). Device pointers are plain HIP device
 * allocations (em_malloc, hipMalloc or a torch tensor's data_ptr()).
 *
 * Streams: `stream` is a hipStream_t passed through as is. NULL is HIP's
 * legacy null stream; EM_STREAM_PER_THREAD is the calling thread's default
 * stream, which is what the reference's library uses (it is compiled with
 * --default-stream per-thread, /root/reference/CMakeLists.txt:100-105), and
 * what the C++ layer in cuda_matmul.h passes. Calls are queued and return
 * before the GPU finishes. Calls that use split-K share one library-owned
 * scratch buffer: concurrent calls on different streams race, as in the
 * reference (cuda_matmul.h:7-12).
 *
 * Layout (cuda_matmul.h:94-107): A is m x k, B is k x n, C is m x n, all
 * dense row-major fp32 with no leading dimensions; int8 B carries n fp32
 * column scales. rms_weight, when not NULL, holds k floats.
 */
#ifndef LLM_ENGINE_AMD_H
#define LLM_ENGINE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define EM_OK 0
#define EM_EINVAL 1  /* bad arguments: shapes, kernel choice, sizes (std::invalid_argument) */
#define EM_EDEVICE 2 /* a HIP runtime error (std::runtime_error "cuda: <op>: <err>") */
#define EM_ENODEV 3  /* no usable GPU */

/* Kernel choice; replaces enum class GpuKernel, cuda_matmul.h:61-67. */
#define EM_KERNEL_AUTOMATIC 0   /* skinny for m <= 8, else tiled_split (tiled if B is unaligned) */
#define EM_KERNEL_NAIVE 1       /* one thread per element of C; the reference kernel */
#define EM_KERNEL_TILED 2       /* LDS-tiled fp32 MFMA GEMM, 128 x 128 tiles */
#define EM_KERNEL_TILED_SPLIT 3 /* MFMA over 16/32-row tiles, B streamed from HBM/L2, k split */
#define EM_KERNEL_SKINNY 4      /* m <= 8 only: wave64 GEMV, k split across waves and blocks */

#define EM_STREAM_PER_THREAD ((void*)2) /* hipStreamPerThread */

/* Message of the last failed call on this thread ("" if none). */
const char* em_last_error(void);

/* 1 if a usable GPU is present; replaces cuda_available(), cuda_matmul.h:121-122. */
int em_available(void);

/* Waits for all queued GPU work; replaces cuda_synchronize(), cuda_matmul.h:118-119. */
int em_synchronize(void);

/* Bumped whenever the library reallocates its split-K / norm scratch; a HIP
 * graph captured before the bump must be captured again. Replaces
 * cuda_scratch_generation(), cuda_matmul.h:109-112, cuda_matmul.cu:268-297,567. */
size_t em_scratch_generation(void);

/* Device memory, for DeviceTensor / DeviceQTensor (cuda_matmul.cu:452-525):
 * allocation, free, and the synchronous copies of upload() / download(). */
int em_malloc(void** ptr, size_t bytes);
int em_free(void* ptr);
int em_memcpy_h2d(void* dst, const void* src, size_t bytes);
int em_memcpy_d2h(void* dst, const void* src, size_t bytes);

/* C = A x B (C += A x B if accumulate), A optionally replaced by
 * rmsnorm(A) * rms_weight (eps 1e-5). Replaces
 *   void matmul_cuda(size_t m, size_t n, size_t k, const float* A, const float* B,
 *                    float* C, GpuKernel, const MatmulFusion&)   cuda_matmul.h:94-99
 * Errors (before any launch): skinny with m > 8; m*k, k*n or m*n >= 2^31;
 * a NULL pointer where the shape needs one; an unknown kernel. m == 0 or
 * n == 0 does nothing; k == 0 zeroes C unless accumulating
 * (cuda_matmul.cu:406-422). Results are bit-identical across repeats. */
int em_matmul_f32(size_t m, size_t n, size_t k, const float* A, const float* B, float* C,
                  int kernel, int accumulate, const float* rms_weight, void* stream);

/* Same with int8 B and n column scales: C = A x dequantize(B). Replaces
 *   void matmul_cuda(size_t m, size_t n, size_t k, const float* A, const int8_t* B,
 *                    const float* scale, float* C, GpuKernel, const MatmulFusion&)
 *                                                                 cuda_matmul.h:101-107 */
int em_matmul_q8(size_t m, size_t n, size_t k, const float* A, const int8_t* B,
                 const float* scale, float* C, int kernel, int accumulate,
                 const float* rms_weight, void* stream);

/* Symmetric per-column int8 quantisation on the GPU, bit-exact with
 *   QTensor quantize_q8(const Tensor& B)   quant.h:7, quant.cpp:6-28
 * B is rows x cols fp32 on the device; q receives rows x cols int8 and scale
 * cols floats: scale = max|B[:,c]| / 127, inv = 1 / scale (0 for a zero
 * column), q = clamp(lround(B * inv), -127, 127), rounding half away from zero. */
int em_quantize_q8(size_t rows, size_t cols, const float* B, int8_t* q, float* scale,
                   void* stream);

/* out = q * scale[c] on the GPU; replaces Tensor dequantize(const QTensor&),
 * quant.h:9, quant.cpp:30-36. */
int em_dequantize_q8(size_t rows, size_t cols, const int8_t* q, const float* scale, float* out,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LLM_ENGINE_AMD_H */
