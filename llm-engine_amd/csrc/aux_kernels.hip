// Small kernels around the products:
//   naive_kernel    GpuKernel::naive, one thread per element of C
//                   (reference sgemm_naive, cuda_matmul.cu:34-47)
//   reduce_slices   fixed-order split-K sum, scale and residual add
//                   (reference sum_slices, cuda_matmul.cu:245-254)
//   rmsnorm_rows    the separate norm pass for kernels that don't fuse it
//                   (reference rmsnorm_rows, cuda_matmul.cu:256-266)
//   fill_zero       k == 0 output (cuda_matmul.cu:419-422), as a kernel so a
//                   captured graph holds no memset node
//   quantize_q8     quant.cpp:6-28 on the GPU, bit-exact: column absmax in
//                   slices + an order-free max, then scale = absmax / 127 and
//                   inv = 1 / scale with IEEE division, then
//                   q = clamp(round-half-away(B * inv), -127, 127)
//   dequantize_q8   quant.cpp:30-36
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

template <class BT>
__device__ __forceinline__ float load_b(const BT* B, int idx, const float* scale, int col) {
    if constexpr (std::is_same<BT, float>::value) {
        return B[idx];
    } else {
        return static_cast<float>(B[idx]) * scale[col];
    }
}

template <class BT>
__global__ __launch_bounds__(kThreads) void naive_kernel(int m, int n, int k, const float* A,
                                                         const BT* B, const float* scale,
                                                         float* C, int accumulate) {
    const int col = blockIdx.x * 64 + threadIdx.x % 64;
    const int row = blockIdx.y * 4 + threadIdx.x / 64;
    if (row >= m || col >= n) return;
    float acc = 0.0f;
    for (int p = 0; p < k; ++p) acc = fmaf(A[row * k + p], load_b(B, p * n + col, scale, col), acc);
    float* c = C + static_cast<size_t>(row) * n + col;
    *c = accumulate ? *c + acc : acc;
}

__global__ __launch_bounds__(kThreads) void reduce_slices_kernel(int mn, int n, int slices,
                                                                 const float* partial,
                                                                 const float* scale, float* C,
                                                                 int accumulate) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= mn) return;
    float total = ordered_sum(partial + i, static_cast<size_t>(mn), slices);
    if (scale) total *= scale[i % n];
    C[i] = accumulate ? C[i] + total : total;
}

__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(int k, const float* A,
                                                                const float* w, float* out) {
    __shared__ float part[4];
    const float* in = A + static_cast<size_t>(blockIdx.x) * k;
    float* o = out + static_cast<size_t>(blockIdx.x) * k;
    float ss = 0.0f;
    for (int j = threadIdx.x; j < k; j += kThreads) ss = fmaf(in[j], in[j], ss);
    const float s = 1.0f / sqrtf(block_sum(ss, part) / static_cast<float>(k) + kRmsEps);
    for (int j = threadIdx.x; j < k; j += kThreads) o[j] = in[j] * s * w[j];
}

__global__ __launch_bounds__(kThreads) void fill_zero_kernel(float* p, size_t count) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < count;
         i += static_cast<size_t>(gridDim.x) * kThreads)
        p[i] = 0.0f;
}

// --- quantize_q8 -----------------------------------------------------------

// Column maxima of |B| over one slice of rows: partial[slice][c].
__global__ __launch_bounds__(kThreads) void colmax_kernel(int rows, int cols, int span,
                                                          const float* B, float* partial) {
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= cols) return;
    const int r0 = blockIdx.y * span, r1 = min(rows, r0 + span);
    float mx = 0.0f;
    // fmaxf keeps the running value when |B| is NaN, as std::max(scale, v)
    // does in quant.cpp:14; on ordered values max is exact in any order.
    for (int r = r0; r < r1; ++r) mx = fmaxf(mx, fabsf(B[static_cast<size_t>(r) * cols + c]));
    partial[static_cast<size_t>(blockIdx.y) * cols + c] = mx;
}

// scale[c] = absmax / 127 and inv[c] = 1 / scale (0 for a zero column), both
// correctly rounded (the library is built with IEEE fp32 division).
__global__ __launch_bounds__(kThreads) void scale_kernel(int cols, int slices,
                                                         const float* partial, float* scale,
                                                         float* inv) {
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= cols) return;
    float mx = 0.0f;
    for (int s = 0; s < slices; ++s) mx = fmaxf(mx, partial[static_cast<size_t>(s) * cols + c]);
    const float sc = mx / 127.0f;
    scale[c] = sc;
    inv[c] = sc > 0.0f ? 1.0f / sc : 0.0f;
}

// lround for the range that matters: half away from zero, as a float. The
// product is rounded to fp32 before anything else reads it (no contraction
// into the subtraction), as quant.cpp:23 computes B * inv first.
__device__ __forceinline__ float round_half_away(float x) {
#pragma clang fp contract(off)
    const float t = truncf(x);
    return fabsf(x - t) >= 0.5f ? t + copysignf(1.0f, x) : t;
}

// total < 2^31 (checked by the entry point), so int indices suffice.
__global__ __launch_bounds__(kThreads) void quantize_kernel(int total, int cols, const float* B,
                                                            const float* inv, int8_t* q) {
#pragma clang fp contract(off)
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < total; i += gridDim.x * kThreads) {
        const int c = i % cols;
        const float x = B[i] * inv[c];
        const float r = fminf(fmaxf(round_half_away(x), -127.0f), 127.0f);
        q[i] = static_cast<int8_t>(static_cast<int>(r));
    }
}

__global__ __launch_bounds__(kThreads) void dequantize_kernel(int total, int cols,
                                                              const int8_t* q, const float* scale,
                                                              float* out) {
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < total; i += gridDim.x * kThreads)
        out[i] = static_cast<float>(q[i]) * scale[i % cols];
}

int grid_for(size_t count) {
    const size_t blocks = (count + kThreads - 1) / kThreads;
    const size_t cap = static_cast<size_t>(cu_count()) * 16;
    return static_cast<int>(blocks < cap ? (blocks ? blocks : 1) : cap);
}

}  // namespace

template <class BT>
void run_naive(const MatmulArgs& a) {
    const dim3 grid(ceil_div(a.n, 64), ceil_div(a.m, 4));
    hipLaunchKernelGGL((naive_kernel<BT>), grid, dim3(kThreads), 0, a.stream, a.m, a.n, a.k, a.A,
                       static_cast<const BT*>(a.B), a.scale, a.C, a.accumulate ? 1 : 0);
}

template void run_naive<float>(const MatmulArgs&);
template void run_naive<int8_t>(const MatmulArgs&);

void run_reduce_slices(int m, int n, int slices, const float* partial, const float* scale,
                       float* C, bool accumulate, hipStream_t stream) {
    const int mn = m * n;
    hipLaunchKernelGGL(reduce_slices_kernel, dim3(ceil_div(mn, kThreads)), dim3(kThreads), 0,
                       stream, mn, n, slices, partial, scale, C, accumulate ? 1 : 0);
}

void run_rmsnorm_rows(int m, int k, const float* A, const float* w, float* out,
                      hipStream_t stream) {
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(m), dim3(kThreads), 0, stream, k, A, w, out);
}

void run_fill_zero(float* p, size_t count, hipStream_t stream) {
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(count)), dim3(kThreads), 0, stream, p,
                       count);
}

void run_quantize_q8(int rows, int cols, const float* B, int8_t* q, float* scale,
                     hipStream_t stream) {
    // Enough row slices for ~4 workgroups per CU over the column tiles.
    const int tiles = ceil_div(cols, kThreads);
    const int want = ceil_div(4LL * cu_count(), tiles);
    const int slices = rows ? std::max(1, std::min(want, ceil_div(rows, 16))) : 1;
    const int span = rows ? ceil_div(rows, slices) : 0;
    const int used = rows ? ceil_div(rows, span) : 1;
    float* work = scratch(kQuant, static_cast<size_t>(used) * cols + cols);
    float* inv = work + static_cast<size_t>(used) * cols;
    if (rows) {
        hipLaunchKernelGGL(colmax_kernel, dim3(tiles, used), dim3(kThreads), 0, stream, rows, cols,
                           span, B, work);
    } else {
        run_fill_zero(work, cols, stream);
    }
    hipLaunchKernelGGL(scale_kernel, dim3(tiles), dim3(kThreads), 0, stream, cols, used, work,
                       scale, inv);
    const size_t total = static_cast<size_t>(rows) * cols;
    if (total)
        hipLaunchKernelGGL(quantize_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream,
                           static_cast<int>(total), cols, B, inv, q);
}

void run_dequantize_q8(int rows, int cols, const int8_t* q, const float* scale, float* out,
                       hipStream_t stream) {
    const size_t total = static_cast<size_t>(rows) * cols;
    if (total)
        hipLaunchKernelGGL(dequantize_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream,
                           static_cast<int>(total), cols, q, scale, out);
}

}  // namespace em
