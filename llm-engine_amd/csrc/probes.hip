// Measurement kernels for the floor study in bench.py (--floor): what one
// dependent launch costs with no work, and how fast one launch can read a
// buffer, by grid size, loads in flight and access pattern (contiguous
// chunks, a grid stride, or the column segments of a row-major matrix). No counterpart in
// the reference; the reference's bench times a device-to-device copy as its
// ceiling (bench_cuda.cpp:79-88).
#include <algorithm>

#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

__global__ __launch_bounds__(kThreads) void empty_kernel() {}

// DEPTH nontemporal 16-byte loads in flight per thread per step, folded into
// an xor so none is dead; the one store is taken only if the xor hits a
// fixed value (about never). CONTIG: workgroup b reads one contiguous chunk
// (its threads side by side, DEPTH x 4 KiB per step); otherwise the grid
// strides over the whole buffer. Indices past the end are clamped to the
// last vector (read again, never out of bounds).
template <int DEPTH, bool CONTIG>
__global__ __launch_bounds__(kThreads) void read_probe_kernel(const uint4* p, size_t n16,
                                                              size_t chunk, uint32_t* sink) {
    uint32_t acc = 0;
    size_t begin, end, step, lane_stride;
    if constexpr (CONTIG) {
        begin = static_cast<size_t>(blockIdx.x) * chunk + threadIdx.x;
        end = std::min(static_cast<size_t>(blockIdx.x + 1) * chunk, n16);
        lane_stride = kThreads;
    } else {
        begin = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
        end = n16;
        lane_stride = static_cast<size_t>(gridDim.x) * kThreads;
    }
    step = lane_stride * DEPTH;
    for (size_t i = begin; i < end; i += step) {
        uint4 v[DEPTH];
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) v[u] = stream_load(p + std::min(i + u * lane_stride, n16 - 1));
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9e3779b9u) *sink = acc;
}

template <int DEPTH>
void launch_read(const void* buf, std::size_t n16, int blocks, bool contig, uint32_t* sink,
                 hipStream_t s) {
    const std::size_t per = static_cast<std::size_t>(kThreads) * DEPTH;
    std::size_t chunk = (n16 + blocks - 1) / blocks;
    chunk = (chunk + per - 1) / per * per;
    const uint4* p = static_cast<const uint4*>(buf);
    if (contig) {
        hipLaunchKernelGGL((read_probe_kernel<DEPTH, true>), dim3(blocks), dim3(kThreads), 0, s, p,
                           n16, chunk, sink);
    } else {
        hipLaunchKernelGGL((read_probe_kernel<DEPTH, false>), dim3(blocks), dim3(kThreads), 0, s, p,
                           n16, chunk, sink);
    }
}

// A rows x row_bytes matrix read by column segments: workgroup b owns the
// SEG-byte run [group * SEG, (group + 1) * SEG) of every row of its k slice
// (rows [slice * span, (slice + 1) * span)), 256 threads as SEG / 16 lanes
// across the run and 256 / (SEG / 16) rows per load round, DEPTH rounds in
// flight per thread; with xcd, the workgroups of one XCD own consecutive
// (group, slice) pairs, a band of columns. The layouts a GEMV over row-major
// weights can give its workgroups, read with nothing else done. Rows past
// the slice are clamped to its last (read again, never out of bounds).
template <int SEG, int DEPTH>
__global__ __launch_bounds__(kThreads) void read_columns_kernel(const char* p, int rows,
                                                                int row_bytes, int span,
                                                                int slices, int xcd,
                                                                uint32_t* sink) {
    constexpr int kLanes = SEG / 16;
    constexpr int kRound = kThreads / kLanes;
    const int total = gridDim.x;
    const int id = xcd ? (blockIdx.x & 7) * (total / 8) + (blockIdx.x >> 3) : blockIdx.x;
    const int group = id / slices, slice = id - group * slices;
    const int rb = slice * span, re = min(rb + span, rows);
    const size_t col = static_cast<size_t>(group) * SEG + 16 * (threadIdx.x % kLanes);
    uint32_t acc = 0;
    for (int r = rb + threadIdx.x / kLanes; r < re; r += kRound * DEPTH) {
        uint4 v[DEPTH];
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) {
            const int rr = min(r + u * kRound, re - 1);
            v[u] = stream_load(reinterpret_cast<const uint4*>(p + static_cast<size_t>(rr) * row_bytes + col));
        }
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9e3779b9u) *sink = acc;
}

template <int SEG>
void launch_columns(const void* buf, int rows, int row_bytes, int span, int slices, int blocks,
                    int xcd, int depth, uint32_t* sink, hipStream_t s) {
    const char* p = static_cast<const char*>(buf);
    if (depth == 8) {
        hipLaunchKernelGGL((read_columns_kernel<SEG, 8>), dim3(blocks), dim3(kThreads), 0, s, p,
                           rows, row_bytes, span, slices, xcd, sink);
    } else {
        hipLaunchKernelGGL((read_columns_kernel<SEG, 16>), dim3(blocks), dim3(kThreads), 0, s, p,
                           rows, row_bytes, span, slices, xcd, sink);
    }
}

}  // namespace

bool run_probe_read_columns(const void* buf, int rows, int row_bytes, int seg_bytes, int slices,
                            int depth, bool xcd, uint32_t* sink, hipStream_t stream) {
    if (depth != 8 && depth != 16) return false;
    const int groups = row_bytes / seg_bytes;
    const int blocks = groups * slices;
    const int span = (rows + slices - 1) / slices;
    const int x = xcd && blocks % 8 == 0 ? 1 : 0;
    switch (seg_bytes) {
        case 64: launch_columns<64>(buf, rows, row_bytes, span, slices, blocks, x, depth, sink, stream); return true;
        case 128: launch_columns<128>(buf, rows, row_bytes, span, slices, blocks, x, depth, sink, stream); return true;
        case 256: launch_columns<256>(buf, rows, row_bytes, span, slices, blocks, x, depth, sink, stream); return true;
        case 512: launch_columns<512>(buf, rows, row_bytes, span, slices, blocks, x, depth, sink, stream); return true;
        case 1024: launch_columns<1024>(buf, rows, row_bytes, span, slices, blocks, x, depth, sink, stream); return true;
        default: return false;
    }
}

void run_probe_empty(int blocks, hipStream_t stream) {
    hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(kThreads), 0, stream);
}

bool run_probe_read(const void* buf, std::size_t bytes, int blocks, int depth, bool contig,
                    uint32_t* sink, hipStream_t stream) {
    const std::size_t n16 = bytes / 16;
    switch (depth) {
        case 4: launch_read<4>(buf, n16, blocks, contig, sink, stream); return true;
        case 8: launch_read<8>(buf, n16, blocks, contig, sink, stream); return true;
        case 16: launch_read<16>(buf, n16, blocks, contig, sink, stream); return true;
        default: return false;
    }
}

}  // namespace em
