// Device helpers shared by the gfx950 kernels: wave64 reductions, vector
// types and the int8 -> fp32 widening.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace em {

// RMSNorm's eps (ops.h:12 of the reference: rmsnorm(..., eps = 1e-5f)).
constexpr float kRmsEps = 1e-5f;

// Every kernel here runs 256-thread workgroups: four wave64s, one per SIMD.
constexpr int kThreads = 256;
constexpr int kWave = 64;

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Streaming loads of weights that one call reads exactly once: the
// nontemporal hint marks the lines evict-first, so a pass over a large
// matrix does not displace what the caches hold for the rest of the call
// (measured 0.45 us faster per 16 MiB GEMV on gfx950).
__device__ __forceinline__ uint4 stream_load(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 stream_load(const float4* p) {
    const floatx4 v = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
template <class T>
__device__ __forceinline__ T stream_load(const T* p) {
    return __builtin_nontemporal_load(p);
}

// Butterfly sum over the 64 lanes of a wave. The pattern is fixed, so the
// result does not depend on timing.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Maximum over the 64 lanes of a wave.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Maximum over a 256-thread workgroup; every thread gets the result. `part`
// is 4 floats of LDS; the leading barrier lets a previous call finish.
__device__ __forceinline__ float block_max(float v, float* part) {
    v = wave_max(v);
    const int wave = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x % kWave) == 0) part[wave] = v;
    __syncthreads();
    return fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
}

// Sum over a 256-thread workgroup; every thread gets the result. The four
// wave sums are added in wave order. `part` is 4 floats of LDS; the leading
// barrier lets a previous call finish reading it.
__device__ __forceinline__ float block_sum(float v, float* part) {
    v = wave_sum(v);
    const int wave = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x % kWave) == 0) part[wave] = v;
    __syncthreads();
    return (part[0] + part[1]) + (part[2] + part[3]);
}

// Halving steps of a cross-lane reduce-scatter (gfx950 lane swaps, no LDS).
// fold32(x, y): lanes 0-31 get x + x of lane + 32, lanes 32-63 get y of lane
// - 32 + y; fold16(x, y): the same between rows of 16 (even rows x, odd rows
// y). Each sum is formed in exactly one lane, so the result is fixed.
__device__ __forceinline__ float fold32(float x, float y) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float fold16(float x, float y) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// DPP move inside rows of 16 lanes: row_shl:8 (0x108) reads lane + 8,
// row_shr:8 (0x118) lane - 8, row_shl:4 (0x104) lane + 4, row_shr:4 (0x114)
// lane - 4. The control must be a constant of the instruction.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// One step of lane_reduce16 over lane bit BIT (5, 4, 3 or 2). With N > 1
// values the list is halved: a lane whose bit is clear keeps items
// [0, N/2), a lane whose bit is set items [N/2, N), each summed with its
// partner's copy of the same item. With one value left the partner's value
// is added (both lanes form the same bits: a + b == b + a).
template <int BIT, int N>
__device__ __forceinline__ void lane_step(const float (&in)[N], float (&out)[N > 1 ? N / 2 : 1]) {
    const bool hi = (threadIdx.x >> BIT) & 1;
    constexpr int H = N > 1 ? N / 2 : 1;
#pragma unroll
    for (int t = 0; t < H; ++t) {
        const float x = in[t], y = in[N > 1 ? t + H : t];
        if constexpr (BIT == 5) {
            out[t] = fold32(x, y);
        } else if constexpr (BIT == 4) {
            out[t] = fold16(x, y);
        } else if constexpr (BIT == 3) {
            const float lo_sum = x + dpp_row<0x108>(x), hi_sum = y + dpp_row<0x118>(y);
            out[t] = hi ? hi_sum : lo_sum;
        } else {
            const float lo_sum = x + dpp_row<0x104>(x), hi_sum = y + dpp_row<0x114>(y);
            out[t] = hi ? hi_sum : lo_sum;
        }
    }
}

// Sum of N values (a power of two) over the 16 lanes of a wave that share
// lane & 3 (lane bits 5 .. 2), in a fixed pattern: reduce-scatter steps
// while more than one value is left, then butterflies. Each lane ends with
// max(N / 16, 1) sums; slot s holds list item lane_item<N>(lane, s).
template <int N>
__device__ __forceinline__ void lane_reduce16(const float (&v)[N], float (&out)[N >= 16 ? N / 16 : 1]) {
    constexpr int N1 = N > 1 ? N / 2 : 1, N2 = N1 > 1 ? N1 / 2 : 1, N3 = N2 > 1 ? N2 / 2 : 1;
    float a[N1], b[N2], c[N3];
    lane_step<5, N>(v, a);
    lane_step<4, N1>(a, b);
    lane_step<3, N2>(b, c);
    lane_step<2, N3>(c, out);
}
template <int N>
__host__ __device__ constexpr int lane_item(int lane, int s) {
    int t = s, count = N;
    for (int bit = 5; bit >= 2; --bit) {
        if (count > 1) {
            count /= 2;
            if ((lane >> bit) & 1) t += count;
        }
    }
    return t;
}
// Whether this lane holds the one copy that is written out: lanes that
// differ only in bits summed by butterflies hold the same sums.
template <int N>
__host__ __device__ constexpr bool lane_writes(int lane) {
    int count = N;
    for (int bit = 5; bit >= 2; --bit) {
        if (count > 1) count /= 2;
        else if ((lane >> bit) & 1) return false;
    }
    return true;
}

// Four int8 in one 32-bit word, widened to fp32. hipcc turns each into one
// v_cvt_f32_i32 with an SDWA sign-extended byte select.
__device__ __forceinline__ void widen4(uint32_t w, float* out) {
    out[0] = static_cast<float>(static_cast<int8_t>(w));
    out[1] = static_cast<float>(static_cast<int8_t>(w >> 8));
    out[2] = static_cast<float>(static_cast<int8_t>(w >> 16));
    out[3] = static_cast<float>(static_cast<int8_t>(w >> 24));
}

// base[idx] + base[idx + stride] + ... (slices terms), added in slice order
// from +0 (so every caller gets the same bits), with the loads issued 16 at
// a time so the sum waits on one memory latency per 16 slices. The last
// partial batch is one more batch of 16 with its loads guarded by the slice
// count (uniform across the wave) and +0 in the registers past it: adding
// +0 leaves a sum that started at +0 unchanged (such a sum is never -0). A
// tail of single load-then-add steps took 11 round trips for a GEMV over
// k = 11008 (43 slices). The code stays small on purpose: the kernels that
// call it wait on little else, and one batch of up to 64 measured slower at
// 32 and 64 slices than two or four of 16.
__device__ __forceinline__ float ordered_sum(const float* __restrict__ base, uint32_t idx,
                                             uint32_t stride, int slices) {
    const float* p = base + idx;
    float total = 0.0f;
    int s = 0;
    for (; s + 16 <= slices; s += 16) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = p[static_cast<size_t>(s + i) * stride];
#pragma unroll
        for (int i = 0; i < 16; ++i) total += v[i];
    }
    if (s < slices) {
        const int left = slices - s;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (i < left) v[i] = p[static_cast<size_t>(s + i) * stride];
#pragma unroll
        for (int i = 0; i < 16; ++i) total += v[i];
    }
    return total;
}

// A product's output as a consumer reads it: C itself (one k slice, or a
// kernel that writes C), or the skinny GEMV's partials [slice][m][n] summed
// in slice order and scaled by the column scale: reduce_slices' arithmetic.
struct Summed {
    const float* c;
    const float* partial;
    const float* scale;  // int8 column scales, null for fp32
    int slices, n;
    size_t mn;
};

__device__ __forceinline__ float summed(const Summed& s, int row, int col) {
    const size_t idx = static_cast<size_t>(row) * s.n + col;
    if (s.slices == 1) return s.c[idx];
    float t = ordered_sum(s.partial, static_cast<uint32_t>(idx), static_cast<uint32_t>(s.mn),
                          s.slices);
    if (s.scale) t *= s.scale[col];
    return t;
}

// One RoPE rotation of the pair (x0, x1) by the angle with cosine c and
// sine s (model.cpp:93-103), with its two roundings spelled out, so that every
// kernel that rotates a key (prefill, decode) caches the same bits.
__device__ __forceinline__ float2 rope_pair(float x0, float x1, float c, float s) {
    return make_float2(fmaf(x0, c, -(x1 * s)), fmaf(x0, s, x1 * c));
}

// summed() of four consecutive columns (col % 4 == 0, n % 4 == 0, 16-byte
// aligned buffers): float4 loads, each component added in slice order as
// ordered_sum adds it, then scaled: the same bits as four summed() calls.
__device__ __forceinline__ floatx4 summed4(const Summed& s, int row, int col) {
    const size_t idx = static_cast<size_t>(row) * s.n + col;
    if (s.slices == 1) return *reinterpret_cast<const floatx4*>(s.c + idx);
    const floatx4* p = reinterpret_cast<const floatx4*>(s.partial + idx);
    const size_t stride4 = s.mn / 4;
    floatx4 t{0.f, 0.f, 0.f, 0.f};
    int sl = 0;
    for (; sl + 16 <= s.slices; sl += 16) {
        floatx4 v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = p[static_cast<size_t>(sl + i) * stride4];
#pragma unroll
        for (int i = 0; i < 16; ++i) t += v[i];
    }
    if (sl < s.slices) {
        const int left = s.slices - sl;
        floatx4 v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (i < left) v[i] = p[static_cast<size_t>(sl + i) * stride4];
#pragma unroll
        for (int i = 0; i < 16; ++i) t += v[i];
    }
    if (s.scale) t *= *reinterpret_cast<const floatx4*>(s.scale + col);
    return t;
}

// SwiGLU of one (gate, up) pair, silu(g) * u (model.cpp:306-310): the one
// expression every kernel that forms it uses, so they agree bit for bit.
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// Split attention (one workgroup per chunk of the context): at least
// kSplitMinChunk positions per chunk, and a row of n_ctx positions over at
// most `splits` chunks has ceil(n_ctx / split_chunk(n_ctx, splits)) of them
// (cuda_attention.cu:25-31).
//
// The least chunk is 64 positions when each split workgroup serves one
// query head, 32 when it serves a group of heads sharing a kv head (their
// keys and values are a quarter or less of the bytes per position, so a
// longer chunk mostly adds latency: 8 kv heads at contexts 128 / 512 / 1024
// took 10.6 / 11.9 / 12.7 us with 64, 8.9 / 10.1 / 11.1 with 32; one head
// per workgroup measured even or slower with 32 outside 256-512).
constexpr int kSplitMinChunk = 64;
constexpr int kSplitMinChunkGrouped = 32;
__host__ __device__ __forceinline__ int split_chunk(int n_ctx, int splits, int min_chunk) {
    const int c = (n_ctx + splits - 1) / splits;
    return c > min_chunk ? c : min_chunk;
}

// One decode row's split attention output before its merge. Chunk c of
// head h leaves its max score and its sum of e^(score - max) in
// ml[h * splits + c] and its unnormalised output in
// o[(h * splits + c) * head_size, + head_size); a row whose positions fit
// one chunk is written, normalised, to out[h * head_size + d] instead.
// The row sits at position *pos, so n_ctx = *pos + 1.
struct SplitRow {
    const float* o;
    const float2* ml;
    const float* out;
    const int* pos;
    int splits, n_heads, head_size, min_chunk;
};

// The split merge (cuda_attention.cu:234-255: m = max m_c,
// l = sum e^(m_c - m) l_c, out = sum e^(m_c - m) o_c / l), one batch of eight chunks into a running max m, sum l and output acc: chunk
// u counts when c0 + u * stride < n. Every kernel that merges chunks runs
// this and merge_combine, so they give the same bits.
template <class T>
__device__ __forceinline__ void merge_batch8(float& m, float& l, T& acc, const float2* ml,
                                             const T* o, int c0, int stride, int n) {
    float mb = m;
#pragma unroll
    for (int u = 0; u < 8; ++u)
        if (c0 + u * stride < n) mb = fmaxf(mb, ml[u].x);
    // mb is finite: chunk c0 < n holds at least one position.
    const float alpha = expf(m - mb);  // 0 while m = -inf
    l *= alpha;
    acc *= alpha;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        if (c0 + u * stride < n) {
            const float w = expf(ml[u].x - mb);
            l += w * ml[u].y;
            acc += w * o[u];
        }
    }
    m = mb;
}

// Slots 0 .. used - 1 of (max, sum) ml(r) and output acc(r), combined in
// slot order: sum_r e^(m_r - M) acc_r / sum_r e^(m_r - M) l_r, M = max m_r.
template <class T, class ML, class ACC>
__device__ __forceinline__ T merge_combine(int used, T zero, ML ml, ACC acc) {
    float M = ml(0).x;
    for (int r = 1; r < used; ++r) M = fmaxf(M, ml(r).x);
    T total = zero;
    float l = 0.0f;
    for (int r = 0; r < used; ++r) {
        const float2 v = ml(r);
        const float f = expf(v.x - M);
        total += f * acc(r);
        l += f * v.y;
    }
    return total * (1.0f / l);
}

// Tile of workgroup `id` of a 1-D grid. Workgroups are dispatched to the
// eight XCDs in turn (id % 8), each XCD with its own L2. With xcd_order the
// ids are renumbered so that each XCD receives a contiguous run of tiles,
// row tile fastest: the row tiles that stream the same 256 columns of B run
// side by side on one XCD and share its L2, instead of landing on eight
// different L2s. The renumbering is a bijection for any grid size.
struct TileId {
    int row, col, slice;
};
__device__ __forceinline__ TileId tile_of(int id, int total, int row_tiles, int col_tiles,
                                          bool xcd_order) {
    constexpr int kXcds = 8;
    int idx = id;
    if (xcd_order) {
        const int per = total / kXcds, rem = total % kXcds;
        const int x = id % kXcds, seq = id / kXcds;
        idx = (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + seq;
        TileId t;
        t.row = idx % row_tiles;
        t.col = (idx / row_tiles) % col_tiles;
        t.slice = idx / (row_tiles * col_tiles);
        return t;
    }
    TileId t;
    t.col = idx % col_tiles;
    t.slice = (idx / col_tiles) % (total / (row_tiles * col_tiles));
    t.row = idx / (total / row_tiles);
    return t;
}

__device__ __forceinline__ floatx4 mfma16x16x4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

}  // namespace em
