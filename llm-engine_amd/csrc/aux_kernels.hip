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
//   stream_read     a read-only pass over a buffer (probes.hip's read kernel
//                   in its fastest shape): the HBM ceiling that the GEMV is
//                   compared with (no counterpart in the reference, whose
//                   bench times a device-to-device copy instead,
//                   bench_cuda.cpp:79-88)
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

// One output per thread. C and the scale are loaded with the first
// partials, so no round trip waits on them alone. With ssq,
// each wave (outputs 64w .. 64w + 63, one row of C when n is a multiple of
// 64) also writes the sum of their squares, by a fixed butterfly.
// 256-thread workgroups: 64-thread ones measured 0.5 us slower per call.
static_assert(kSsqChunk == kWave, "one sum of squares per wave");

__global__ __launch_bounds__(kThreads) void reduce_slices_kernel(
    int mn, int n, int slices, const float* __restrict__ partial, const float* __restrict__ scale,
    float* __restrict__ C, int accumulate, float* __restrict__ ssq) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    const bool in = i < mn;
    const int ii = in ? i : mn - 1;
    const float prior = accumulate ? C[ii] : 0.0f;
    const float sc = scale ? scale[ii % n] : 1.0f;
    float total = ordered_sum(partial, static_cast<uint32_t>(ii), static_cast<uint32_t>(mn), slices);
    if (scale) total *= sc;
    const float out = accumulate ? prior + total : total;
    if (in) C[i] = out;
    if (ssq) {
        const float sq = wave_sum(in ? out * out : 0.0f);
        if (in && threadIdx.x % kWave == 0) ssq[i / kSsqChunk] = sq;
    }
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

// Column maxima of |B| over one slice of rows: partial[slice][c]. With V4
// (cols % 4 == 0, B 16-byte aligned) a thread owns four adjacent columns
// and reads them as one float4; eight rows are loaded before any is used.
template <bool V4>
__global__ __launch_bounds__(kThreads) void colmax_kernel(int rows, int cols, int span,
                                                          const float* B, float* partial) {
    constexpr int W = V4 ? 4 : 1;
    const int c = (blockIdx.x * kThreads + threadIdx.x) * W;
    if (c >= cols) return;
    const int r0 = blockIdx.y * span, r1 = min(rows, r0 + span);
    // fmaxf keeps the running value when |B| is NaN, as std::max(scale, v)
    // does in quant.cpp:14; on ordered values max is exact in any order.
    float mx[W];
#pragma unroll
    for (int e = 0; e < W; ++e) mx[e] = 0.0f;
    auto take = [&](int r) {
        const float* row = B + static_cast<size_t>(r) * cols + c;
        if constexpr (V4) {
            const float4 v = *reinterpret_cast<const float4*>(row);
            mx[0] = fmaxf(mx[0], fabsf(v.x));
            mx[1] = fmaxf(mx[1], fabsf(v.y));
            mx[2] = fmaxf(mx[2], fabsf(v.z));
            mx[3] = fmaxf(mx[3], fabsf(v.w));
        } else {
            mx[0] = fmaxf(mx[0], fabsf(*row));
        }
    };
    int r = r0;
    for (; r + 8 <= r1; r += 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) take(r + u);
    }
    for (; r < r1; ++r) take(r);
#pragma unroll
    for (int e = 0; e < W; ++e) partial[static_cast<size_t>(blockIdx.y) * cols + c + e] = mx[e];
}

// scale[c] = absmax / 127 and inv[c] = 1 / scale (0 for a zero column), both
// correctly rounded (the library is built with IEEE fp32 division). The
// slice maxima are loaded 16 at a time (max is exact in any order).
__global__ __launch_bounds__(kThreads) void scale_kernel(int cols, int slices,
                                                         const float* partial, float* scale,
                                                         float* inv) {
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= cols) return;
    float mx = 0.0f;
    int s = 0;
    for (; s + 16 <= slices; s += 16) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = partial[static_cast<size_t>(s + i) * cols + c];
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, v[i]);
    }
    for (; s < slices; ++s) mx = fmaxf(mx, partial[static_cast<size_t>(s) * cols + c]);
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

__device__ __forceinline__ int8_t quantize_one(float b, float inv) {
#pragma clang fp contract(off)
    const float x = b * inv;
    const float r = fminf(fmaxf(round_half_away(x), -127.0f), 127.0f);
    return static_cast<int8_t>(static_cast<int>(r));
}

// total < 2^31 (checked by the entry point), so int indices suffice. With
// V4 (cols % 4 == 0, B 16-byte and q 4-byte aligned) a thread takes four
// consecutive elements of one row: one float4 load and one 32-bit store.
template <bool V4>
__global__ __launch_bounds__(kThreads) void quantize_kernel(int total, int cols, const float* B,
                                                            const float* inv, int8_t* q) {
    if constexpr (V4) {
        const int quads = total / 4;
        for (int i = blockIdx.x * kThreads + threadIdx.x; i < quads; i += gridDim.x * kThreads) {
            const int c = (4 * i) % cols;
            const float4 b = reinterpret_cast<const float4*>(B)[i];
            const float4 s = *reinterpret_cast<const float4*>(inv + c);
            const uint32_t w = static_cast<uint8_t>(quantize_one(b.x, s.x)) |
                               static_cast<uint32_t>(static_cast<uint8_t>(quantize_one(b.y, s.y))) << 8 |
                               static_cast<uint32_t>(static_cast<uint8_t>(quantize_one(b.z, s.z))) << 16 |
                               static_cast<uint32_t>(static_cast<uint8_t>(quantize_one(b.w, s.w))) << 24;
            reinterpret_cast<uint32_t*>(q)[i] = w;
        }
    } else {
        for (int i = blockIdx.x * kThreads + threadIdx.x; i < total; i += gridDim.x * kThreads)
            q[i] = quantize_one(B[i], inv[i % cols]);
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
                       float* C, bool accumulate, hipStream_t stream, float* ssq) {
    const int mn = m * n;
    hipLaunchKernelGGL(reduce_slices_kernel, dim3(ceil_div(mn, kThreads)), dim3(kThreads), 0,
                       stream, mn, n, slices, partial, scale, C, accumulate ? 1 : 0,
                       n % kSsqChunk == 0 ? ssq : nullptr);
}

// The read ceiling: 1024 workgroups, 16 loads in flight per thread, each
// workgroup on one contiguous chunk -- the fastest shape of the floor
// study's sweep over a 600 MiB buffer (6.95-6.98 TB/s against 5.1-5.4 for
// a 2048-workgroup grid stride with 8 loads in flight).
void run_stream_read(const void* buf, std::size_t bytes, uint32_t* sink, hipStream_t stream) {
    const std::size_t per = static_cast<std::size_t>(kThreads) * 16 * 16;
    const int blocks = static_cast<int>(std::max<std::size_t>(
        1, std::min<std::size_t>(1024, (bytes + per - 1) / per)));
    run_probe_read(buf, bytes, blocks, 16, true, sink, stream);
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
    const bool v4 = cols % 4 == 0 && reinterpret_cast<uintptr_t>(B) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(q) % 4 == 0;
    // Enough row slices for ~4 workgroups per CU over the column tiles.
    const int tiles = ceil_div(cols, kThreads * (v4 ? 4 : 1));
    const int want = ceil_div(4LL * cu_count(), tiles);
    const int slices = rows ? std::max(1, std::min(want, ceil_div(rows, 16))) : 1;
    const int span = rows ? ceil_div(rows, slices) : 0;
    const int used = rows ? ceil_div(rows, span) : 1;
    float* work = scratch(kQuant, static_cast<size_t>(used) * cols + cols);
    float* inv = work + static_cast<size_t>(used) * cols;
    if (rows) {
        if (v4) {
            hipLaunchKernelGGL(colmax_kernel<true>, dim3(tiles, used), dim3(kThreads), 0, stream,
                               rows, cols, span, B, work);
        } else {
            hipLaunchKernelGGL(colmax_kernel<false>, dim3(tiles, used), dim3(kThreads), 0, stream,
                               rows, cols, span, B, work);
        }
    } else {
        run_fill_zero(work, cols, stream);
    }
    hipLaunchKernelGGL(scale_kernel, dim3(ceil_div(cols, kThreads)), dim3(kThreads), 0, stream,
                       cols, used, work, scale, inv);
    const size_t total = static_cast<size_t>(rows) * cols;
    if (total == 0) return;
    if (v4) {
        hipLaunchKernelGGL(quantize_kernel<true>, dim3(grid_for(total / 4)), dim3(kThreads), 0,
                           stream, static_cast<int>(total), cols, B, inv, q);
    } else {
        hipLaunchKernelGGL(quantize_kernel<false>, dim3(grid_for(total)), dim3(kThreads), 0,
                           stream, static_cast<int>(total), cols, B, inv, q);
    }
}

void run_dequantize_q8(int rows, int cols, const int8_t* q, const float* scale, float* out,
                       hipStream_t stream) {
    const size_t total = static_cast<size_t>(rows) * cols;
    if (total)
        hipLaunchKernelGGL(dequantize_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream,
                           static_cast<int>(total), cols, q, scale, out);
}

}  // namespace em
