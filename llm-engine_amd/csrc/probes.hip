// Measurement kernels for the floor study in bench.py (--floor): what one
// dependent launch costs with no work, and how fast one launch can read a
// buffer, by grid size, loads in flight and access pattern. No counterpart in
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

}  // namespace

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
