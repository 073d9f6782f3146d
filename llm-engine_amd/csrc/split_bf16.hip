// int8-weight products on bf16 matrix cores with fp32 results: what
// GpuKernel::automatic runs for int8 B above 8 rows, and for fewer rows
// where split_bf16_preferred says it beats the GEMV
// (reference: tiled_split / tiled, /root/reference/src/cuda_matmul.cu:49-125,
// 350-363; CPU pack_b dequantisation, matmul.cpp:73-90).
//
// Exact splitting. Every int8 weight q (|q| <= 127) is exactly a bf16. Every
// fp32 activation a is exactly hi + mid + lo, three bf16 values: hi keeps a's
// top 8 significant bits (truncated), mid the next 8 bits of the exact
// remainder a - hi, lo the last 8 (a 24-bit significand needs no more). So
// each product hi*q, mid*q, lo*q is exact in fp32 (8 x 8 significant bits),
// and v_mfma_f32_16x16x32_bf16 sums them into fp32 accumulators. Nothing is
// dropped: the result differs from an fp32 FMA chain only in summation order,
// as any reordered fp32 sum does, and the column scale is applied to the
// finished sum as in the GEMV path.
//
// Range. gfx950's bf16 MFMA keeps subnormal operands, products and sums
// (checked on the device), so the split stays exact while every term is a
// bf16 value: down to |a| = 2^-110 (the lo term's last bit at 2^-133,
// bf16's smallest subnormal). Smaller values (fp32 subnormals, or rows near
// 1e-37) would lose low bits. The pre-pass, which holds each row, scales it
// by 2^s, s = max(0, 64 - e) for its largest finite magnitude 2^e, and the
// kernel scales each sum of the row back by 2^-s (after the column scale
// when it writes C): both exact in fp32 short of a subnormal result, which
// rounds once, so a row that needs no scaling gets the same bits either way.
// The kernel that splits A itself runs unscaled, ORs its lo remainders
// (their low half is non-zero iff bits were dropped) and checks its sums;
// a 16-row block with dropped bits or a non-finite sum is computed again by
// fp32 multiply-adds (fma_block), whose products of such values keep their
// relative precision. An infinite activation passes through the pre-pass as
// hi = a, mid = lo = 0 (and through fma_block as itself), so C gets +-inf,
// NaN where its weight is 0, as fp32 arithmetic gives; a NaN gives NaN. The
// products sum a * q before the column scale, as the GEMV does, so
// |a| * 127 * k past fp32's range overflows where a * (q * scale) might not.
//
// Speed. At 16 cycles per 8192 multiply-adds
// the three terms cost 3/16 of fp32 MFMA time (16x16x4 f32: 32 cycles per
// 1024); measured against the fp32-MFMA tiled_split kernel at 4096^2 it is
// 1.1x faster at m = 9-16, 1.9x at m = 64 and 2.6x at m = 512. VALU work
// does not overlap the MFMA pipe on gfx950 (each VALU op beside a bf16 MFMA
// adds ~1.4 ns to it), so the kernel's speed is set by VALU ops per MFMA:
// widening the weights (1.5 per byte, once per row tile) and splitting A
// (5.5 per value, once per column tile).
//
//  * split_a_row_kernel (split_a_kernel past 8192 values a row), when
//    RMSNorm is fused or A's rows are not whole 16-byte groups: writes the
//    three bf16 planes
//    A3[term][m_pad][k_pad], zero-padded to whole tiles. Otherwise the main
//    kernel loads fp32 A and splits each 8-value group in registers.
//  * split_bf16_kernel<RB>: as tiled_split, B streams from HBM straight into
//    MFMA operands. A lane (g, j) loads 16 consecutive bytes of 8 rows of a
//    32-row chunk; MFMA t takes byte t of each, i.e. column 16j + t, as the
//    8 k-values lane group g supplies (the k order inside the chunk is the
//    same for A and B). Each byte is widened once and feeds 3 x RB MFMAs
//    (one per term of A and 16-row block). Chunks ring through two register
//    sets per wave; the epilogue stages the four waves' sums in LDS and
//    writes coalesced float4 runs; k slices go through reduce_slices.
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kTile = 256;               // columns per workgroup
constexpr int kChunk = 32;               // k rows per MFMA step of a wave
constexpr int kStep = 4 * kChunk;        // the four waves' chunks
constexpr int kDepth = 2;                // chunks in flight per wave
// The epilogue tile in LDS: rows of kTile floats as 64 granules of four;
// granule q of a row is stored at q ^ ((q >> 3) & 7). A lane's 16 columns
// are granules 4j .. 4j + 3, so without the swizzle the 16-byte writes of
// lanes j and j + 2 (and the reads of threads 16 columns apart) fall on the
// same banks; with it, every eight consecutive lanes cover all 32 banks.
__device__ __forceinline__ int granule(int q) { return q ^ ((q >> 3) & 7); }

// --- A -> three bf16 planes -------------------------------------------------

__device__ __forceinline__ uint32_t bits(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ float from_bits(uint32_t u) { return __builtin_bit_cast(float, u); }

// a = hi + mid + lo exactly for |a| >= 2^-110; each part's bits are the top
// half of an fp32. +-inf: hi = a, mid = lo = 0 (a - hi would be NaN).
__device__ __forceinline__ void split3(float a, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
#pragma clang fp contract(off)
    hi = bits(a) >> 16;
    const float h = from_bits(hi << 16);
    const float r1 = a == h ? 0.0f : a - h;
    mid = bits(r1) >> 16;
    const float r2 = r1 - from_bits(mid << 16);
    lo = bits(r2) >> 16;
}

// The row scale's exponent: the largest finite magnitude is brought to
// [2^64, 2^65) when it lies below (values down to 2^-174 of it then split
// exactly, and a sum of k < 2^31 scaled products stays below 2^103).
constexpr int kShiftTarget = 64;

__device__ __forceinline__ float finite_mag(float x) {
    const float m = fabsf(x);
    return m < __builtin_inff() ? m : 0.0f;  // NaN and inf count as 0
}

__device__ __forceinline__ int row_shift(float max_mag) {
    const uint32_t u = bits(max_mag);
    if (u == 0) return 0;
    const int e = u >= 0x00800000u ? static_cast<int>(u >> 23) - 127 : 31 - __clz(u) - 149;
    return max(0, kShiftTarget - e);
}

// block_sum(ss) and block_max(mx) over one pair of barriers (the sum in
// block_sum's order). `part` is 8 floats of LDS.
__device__ __forceinline__ void block_sum_max(float& ss, float& mx, float* part) {
    ss = wave_sum(ss);
    mx = wave_max(mx);
    const int wave = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x % kWave) == 0) {
        part[wave] = ss;
        part[4 + wave] = mx;
    }
    __syncthreads();
    ss = (part[0] + part[1]) + (part[2] + part[3]);
    mx = fmaxf(fmaxf(part[4], part[5]), fmaxf(part[6], part[7]));
}

// Row r of A3 (three planes, m_pad x k_pad each): rmsnorm(A[r]) * w when w is
// given (the arithmetic of rmsnorm_rows: x * s * w[j]), times 2^shifts[r];
// zeros past m and k. The shift comes from the row's largest finite |x|, or
// with the norm from s * max |x * w[j]| (within rounding of the normed
// row's largest, found in the sum of squares' pass).
__global__ __launch_bounds__(kThreads) void split_a_kernel(int m, int k, int m_pad, int k_pad,
                                                           const float* A, const float* w,
                                                           uint16_t* A3, int* shifts) {
    __shared__ float part[8];
    const int r = blockIdx.x;
    const float* in = A + static_cast<std::size_t>(r) * k;
    float s = 1.0f, top = 0.0f;
    if (r < m) {
        float ss = 0.0f, mx = 0.0f;
        if (w) {
            for (int j = threadIdx.x; j < k; j += kThreads) {
                ss = fmaf(in[j], in[j], ss);
                mx = fmaxf(mx, finite_mag(in[j] * w[j]));
            }
            block_sum_max(ss, mx, part);
            s = 1.0f / sqrtf(ss / static_cast<float>(k) + kRmsEps);
            top = s * mx;
        } else {
            for (int j = threadIdx.x; j < k; j += kThreads) mx = fmaxf(mx, finite_mag(in[j]));
            top = block_max(mx, part);
        }
    }
    const int shift = row_shift(top);
    if (threadIdx.x == 0) shifts[r] = shift;
    const std::size_t plane = static_cast<std::size_t>(m_pad) * k_pad;
    uint16_t* o = A3 + static_cast<std::size_t>(r) * k_pad;
    // Eight k per thread per step: one 16-byte store per plane.
    for (int j0 = threadIdx.x * 8; j0 < k_pad; j0 += kThreads * 8) {
        uint32_t h[8], md[8], l[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int j = j0 + e;
            float a = 0.0f;
            if (r < m && j < k) a = w ? in[j] * s * w[j] : in[j];
            split3(__builtin_ldexpf(a, shift), h[e], md[e], l[e]);
        }
        auto pack = [](const uint32_t* v) {
            return make_uint4(v[0] | v[1] << 16, v[2] | v[3] << 16, v[4] | v[5] << 16,
                              v[6] | v[7] << 16);
        };
        *reinterpret_cast<uint4*>(o + j0) = pack(h);
        *reinterpret_cast<uint4*>(o + plane + j0) = pack(md);
        *reinterpret_cast<uint4*>(o + 2 * plane + j0) = pack(l);
    }
}

// The same planes in one pass, for rows of at most S x 2048 values: the row
// is held in registers (eight values per thread per step, float4 loads when
// rows are 16-byte groups), so A is read once and the norm costs one block
// reduction (the loop above reads A twice with scalar loads: 15.5 us at
// m = 512, k = 4096). The sum of squares adds each thread's values in step
// and element order, then block_sum.
template <int S>
__global__ __launch_bounds__(kThreads) void split_a_row_kernel(int m, int k, int m_pad, int k_pad,
                                                               int vec4,
                                                               const float* __restrict__ A,
                                                               const float* __restrict__ w,
                                                               uint16_t* __restrict__ A3,
                                                               int* __restrict__ shifts) {
    __shared__ float part[8];
    const int r = blockIdx.x;
    const bool live = r < m;  // rows past m are zeros
    const float* in = A + static_cast<std::size_t>(live ? r : 0) * k;
    // The row and, with a norm, its weights (1 past k), all loaded before
    // the reduction's barriers.
    float v[S][8], wv[S][8];
#pragma unroll
    for (int st = 0; st < S; ++st) {
        const int j0 = (st * kThreads + threadIdx.x) * 8;
        if (live && vec4 && j0 + 8 <= k) {
            const floatx4 x0 = *reinterpret_cast<const floatx4*>(in + j0);
            const floatx4 x1 = *reinterpret_cast<const floatx4*>(in + j0 + 4);
            v[st][0] = x0.x; v[st][1] = x0.y; v[st][2] = x0.z; v[st][3] = x0.w;
            v[st][4] = x1.x; v[st][5] = x1.y; v[st][6] = x1.z; v[st][7] = x1.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[st][e] = live && j0 + e < k ? in[j0 + e] : 0.0f;
        }
        if (w && vec4 && j0 + 8 <= k) {
            const floatx4 g0 = *reinterpret_cast<const floatx4*>(w + j0);
            const floatx4 g1 = *reinterpret_cast<const floatx4*>(w + j0 + 4);
            wv[st][0] = g0.x; wv[st][1] = g0.y; wv[st][2] = g0.z; wv[st][3] = g0.w;
            wv[st][4] = g1.x; wv[st][5] = g1.y; wv[st][6] = g1.z; wv[st][7] = g1.w;
        } else if (w) {
#pragma unroll
            for (int e = 0; e < 8; ++e) wv[st][e] = j0 + e < k ? w[j0 + e] : 1.0f;
        }
    }
    // The norm and the shift, as split_a_kernel finds them, with one
    // reduction (values past k are 0, weights there 1).
    float s = 1.0f, top = 0.0f;
    if (live) {
        float ss = 0.0f, mx = 0.0f;
#pragma unroll
        for (int st = 0; st < S; ++st)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (w) {
                    ss = fmaf(v[st][e], v[st][e], ss);
                    mx = fmaxf(mx, finite_mag(v[st][e] * wv[st][e]));
                } else {
                    mx = fmaxf(mx, finite_mag(v[st][e]));
                }
            }
        if (w) {
            block_sum_max(ss, mx, part);
            s = 1.0f / sqrtf(ss / static_cast<float>(k) + kRmsEps);
            top = s * mx;
        } else {
            top = block_max(mx, part);
        }
    }
    const int shift = row_shift(top);
    if (threadIdx.x == 0) shifts[r] = shift;
    const std::size_t plane = static_cast<std::size_t>(m_pad) * k_pad;
    uint16_t* o = A3 + static_cast<std::size_t>(r) * k_pad;
#pragma unroll
    for (int st = 0; st < S; ++st) {
        const int j0 = (st * kThreads + threadIdx.x) * 8;
        if (j0 >= k_pad) continue;
        uint32_t h[8], md[8], l[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int j = j0 + e;
            const float a = w && j < k ? v[st][e] * s * wv[st][e] : v[st][e];
            split3(__builtin_ldexpf(a, shift), h[e], md[e], l[e]);
        }
        auto pack = [](const uint32_t* x) {
            return make_uint4(x[0] | x[1] << 16, x[2] | x[3] << 16, x[4] | x[5] << 16,
                              x[6] | x[7] << 16);
        };
        *reinterpret_cast<uint4*>(o + j0) = pack(h);
        *reinterpret_cast<uint4*>(o + plane + j0) = pack(md);
        *reinterpret_cast<uint4*>(o + 2 * plane + j0) = pack(l);
    }
}

// --- the product ---------------------------------------------------------------

struct SbParams {
    int m, n, k, k_span, m_pad, k_pad;
    const uint16_t* A3;  // the three planes (pre-pass) and their rows' shifts, or
    const int* shifts;
    const float* A;      // fp32 A, split in registers (RAW kernels)
    const int8_t* B;
    const float* scale;
    float* out;  // C (direct) or partials [slice][m][n]
    int accumulate, direct;
    int row_tiles, col_tiles, xcd_order;
    int col_base;  // first column tile of this launch
    // PAIR kernels (the forward pass's w13 with its SwiGLU): B's first
    // `pair` columns are gates and the next `pair` ups; a column tile holds
    // 128 gates and their 128 ups, and out (m x pair) gets silu(g) * u.
    int pair;
    RopeFuse rope;  // direct only: rope.pos non-null fuses RoPE and the cache write
};

// rope_cache_kernel's work on columns c .. c + 3 of row `row` (c % 4 == 0,
// head_size % 4 == 0): two q or k pairs rotated by rope_pair with the
// tables' row of this position, q back into C, k into the key cache; v
// into the value cache.
// The angles of columns c .. c + 3 at position pos (q or k columns): the
// cosines and sines of pairs (cc / 2) % half and the next, which is
// (cc / 2) % half + 1 (cc % 4 == 0 and half even), loaded as float2s.
// {cos0, cos1, sin0, sin1}; zeros for value columns.
__device__ __forceinline__ floatx4 rope_angles(const RopeFuse& r, int pos, int c) {
    if (c >= r.dim + r.kv_dim) return floatx4{0.f, 0.f, 0.f, 0.f};
    const int cc = c >= r.dim ? c - r.dim : c, half = r.head_size / 2;
    const int a0 = pos * half + (cc / 2) % half;
    const float2 cs = *reinterpret_cast<const float2*>(r.cos_t + a0);
    const float2 sn = *reinterpret_cast<const float2*>(r.sin_t + a0);
    return floatx4{cs.x, cs.y, sn.x, sn.y};
}

// The same without a branch: value columns load the angles of their offset
// in the value part (any valid pair; rope_put does not read them), so the
// loads are unconditional and no merge of loaded and constant values makes
// a later instruction wait for them.
__device__ __forceinline__ floatx4 rope_angles_any(const RopeFuse& r, int pos, int c) {
    const int kv_end = r.dim + r.kv_dim;
    const int cc = c >= kv_end ? c - kv_end : c >= r.dim ? c - r.dim : c;
    const int half = r.head_size / 2;
    const int a0 = pos * half + (cc / 2) % half;
    const float2 cs = *reinterpret_cast<const float2*>(r.cos_t + a0);
    const float2 sn = *reinterpret_cast<const float2*>(r.sin_t + a0);
    return floatx4{cs.x, cs.y, sn.x, sn.y};
}

__device__ __forceinline__ void rope_put(const SbParams& p, int row, int pos, int c, floatx4 v,
                                         const floatx4& ang) {
    const RopeFuse& r = p.rope;
    if (c < r.dim + r.kv_dim) {
        const bool is_k = c >= r.dim;
        const int cc = is_k ? c - r.dim : c;
        const float2 y0 = rope_pair(v[0], v[1], ang[0], ang[2]);
        const float2 y1 = rope_pair(v[2], v[3], ang[1], ang[3]);
        float* dst = is_k ? r.kc + static_cast<std::size_t>(pos) * r.kv_dim + cc
                          : p.out + static_cast<std::size_t>(row) * p.n + c;
        *reinterpret_cast<floatx4*>(dst) = floatx4{y0.x, y0.y, y1.x, y1.y};
    } else {
        *reinterpret_cast<floatx4*>(r.vc + static_cast<std::size_t>(pos) * r.kv_dim +
                                    (c - r.dim - r.kv_dim)) = v;
    }
}

__device__ __forceinline__ void rope_store(const SbParams& p, int row, int c, floatx4 v) {
    const int pos = *p.rope.pos + row;
    rope_put(p, row, pos, c, v, rope_angles(p.rope, pos, c));
}

// One 16-row block of split_bf16_kernel's tile (columns c0 .. c0 + 255,
// rows m0 .. m0 + 15, k in [kb, ke)) by fp32 multiply-adds of a * q, for a
// block whose A the three-term split cannot hold (values below 2^-110, or
// non-finite): fp32 products of such values keep their relative precision,
// and inf * q gives +-inf (NaN at q = 0) as fp32 arithmetic does. Each lane
// takes four adjacent columns (one 32-bit word of B per k) and every fourth
// row (rows w, w + 4, ...; the A values of a row are the same in every lane
// of the wave). Output as the kernel's epilogue writes it: scaled into C
// (with the accumulation or the RoPE epilogue) or unscaled into the
// partials. Slow (16 multiply-adds per lane per k), small in registers.
__device__ __forceinline__ void fma_block(const SbParams& p, int c0, int m0, int kb, int ke,
                                          int slice) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int c = c0 + 4 * (threadIdx.x % kWave);
    const bool live = c < p.n;  // n % 16 == 0: all four columns or none
    const int8_t* b = p.B + (live ? c : 0);
    const float* a_row[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        a_row[i] = p.A + static_cast<std::size_t>(min(m0 + 4 * i + w, p.m - 1)) * p.k;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][e] = 0.0f;
    for (int kk = kb; kk < ke; ++kk) {
        float q[4];
        widen4(*reinterpret_cast<const uint32_t*>(b + static_cast<std::size_t>(kk) * p.n), q);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = a_row[i][kk];
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][e] = fmaf(a, q[e], acc[i][e]);
        }
    }
    if (!live) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = m0 + 4 * i + w;
        if (row >= p.m) break;
        floatx4 v{acc[i][0], acc[i][1], acc[i][2], acc[i][3]};
        if (p.direct) {
            v *= *reinterpret_cast<const floatx4*>(p.scale + c);
            if (p.rope.pos) {
                rope_store(p, row, c, v);
                continue;
            }
            floatx4* o = reinterpret_cast<floatx4*>(p.out + static_cast<std::size_t>(row) * p.n + c);
            *o = p.accumulate ? *o + v : v;
        } else {
            *reinterpret_cast<floatx4*>(
                p.out + (static_cast<std::size_t>(slice) * p.m + row) * p.n + c) = v;
        }
    }
}

template <int RB, bool RAW>
struct Chunk {
    uint4 b[8];         // rows 8g + e of the chunk, 16 columns each
    uint4 a[RB][3];     // 8 bf16 of each term, row 16 rb + j
};

// RAW: the 8 fp32 values of row 16 rb + j as loaded; split in multiply().
template <int RB>
struct Chunk<RB, true> {
    uint4 b[8];
    floatx4 a[RB][2];
    bool aok;           // false past k: the A values count as zero
};

// Eight fp32 values -> the three bf16 terms, packed as MFMA A operands: the
// split3 arithmetic, with each term's top halves paired by one byte permute
// (4.5 VALU ops per value; the MFMA pipe does not hide VALU work, so this
// count sets the kernel's speed as much as the MFMAs do). The lo remainders
// are ORed into `lost`, whose low half is then non-zero iff some lo term
// dropped bits (half an op per value); an infinite value gives a NaN sum.
__device__ __forceinline__ void split8(const floatx4& x0, const floatx4& x1, uint4 (&t)[3],
                                       uint32_t& lost) {
#pragma clang fp contract(off)
    const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    uint32_t a[8], r1[8], r2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = bits(v[e]);
        const float f1 = v[e] - from_bits(a[e] & 0xffff0000u);
        r1[e] = bits(f1);
        r2[e] = bits(f1 - from_bits(r1[e] & 0xffff0000u));
    }
#pragma unroll
    for (int e = 0; e < 8; e += 2) lost = lost | r2[e] | r2[e + 1];
    auto pair = [](const uint32_t* x, int e) {
        return __builtin_amdgcn_perm(x[e + 1], x[e], 0x07060302u);  // top halves, x[e] low
    };
    t[0] = make_uint4(pair(a, 0), pair(a, 2), pair(a, 4), pair(a, 6));
    t[1] = make_uint4(pair(r1, 0), pair(r1, 2), pair(r1, 4), pair(r1, 6));
    t[2] = make_uint4(pair(r2, 0), pair(r2, 2), pair(r2, 4), pair(r2, 6));
}

// The 8 k-values of column byte t, widened and packed as MFMA's B operand.
__device__ __forceinline__ bf16x8 column(const uint4 (&b)[8], int t) {
    const int word = t >> 2, shift = 8 * (t & 3);
    uint32_t f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t w = word == 0 ? b[e].x : word == 1 ? b[e].y : word == 2 ? b[e].z : b[e].w;
        f[e] = bits(static_cast<float>(static_cast<int8_t>(w >> shift)));
    }
    uint4 packed;
    packed.x = __builtin_amdgcn_perm(f[1], f[0], 0x07060302u);
    packed.y = __builtin_amdgcn_perm(f[3], f[2], 0x07060302u);
    packed.z = __builtin_amdgcn_perm(f[5], f[4], 0x07060302u);
    packed.w = __builtin_amdgcn_perm(f[7], f[6], 0x07060302u);
    return __builtin_bit_cast(bf16x8, packed);
}

// RAW: A arrives as fp32 and is split in registers (else as the three planes
// of split_a_kernel). WHOLE: k is a multiple of the chunk, so every chunk
// lies inside k and no row or value needs a clamp or a mask.
// PAIR (pre-split planes only, one slice): lanes j < 8 load gate columns
// c0 + 16j .., lanes j >= 8 the up columns of the same gates, so tile
// column t < 128 is gate c0 + t and column 128 + t its up; the epilogue
// writes silu(g) * u of the finished, scaled values: the bits of the
// product written to C followed by the forward pass's SwiGLU kernel.
// EPI, the direct product's epilogue: kStore (C = the sums, or partials
// when k is split), kAccumulate (C += the sums), kRope (the qkv epilogue).
constexpr int kStore = 0, kAccumulate = 1, kRope = 2;

template <int RB, bool RAW, bool WHOLE, bool PAIR = false, int EPI = kStore>
__global__ __launch_bounds__(kThreads) void split_bf16_kernel(SbParams p) {
    static_assert(!(PAIR && RAW), "the SwiGLU pair reads pre-split planes");
    static_assert(!(PAIR && EPI != kStore), "the SwiGLU pair writes its own output");
    __shared__ __attribute__((aligned(16))) floatx4 tile[4 * 16 * kTile / 4];

    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int g = lane >> 4, j = lane & 15;
    const TileId place = tile_of(blockIdx.x, gridDim.x, p.row_tiles, p.col_tiles,
                                 p.xcd_order != 0);
    const int c0 = (place.col + p.col_base) * (PAIR ? kTile / 2 : kTile);
    const int m0 = place.row * 16 * RB;
    const int kb = place.slice * p.k_span;
    const int ke = min(p.k, kb + p.k_span);

    // The epilogue's column scales (the same columns in every row block)
    // and row shifts, loaded before the first chunk: issued after the
    // chunks, their wait would also wait for the ring's re-reads past the
    // last chunk, and their registers could only be written once those
    // re-reads had landed. Thread (orow, ocol) ends up with row orow,
    // columns ocol .. ocol + 15 of each block; PAIR: gates pp .. pp + 7 of
    // the tile (and their ups).
    const int orow = tid / 16, ocol = (tid % 16) * 16;
    const int pp = (tid % 16) * 8;
    floatx4 esc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        esc[q] = floatx4{1.f, 1.f, 1.f, 1.f};
        if constexpr (PAIR) {
            // q = 0, 1: the gates' scales; 2, 3: the ups'.
            const int c = min(c0 + pp + 4 * (q & 1), p.pair - 4);
            esc[q] = *reinterpret_cast<const floatx4*>(p.scale + (q < 2 ? c : p.pair + c));
        } else {
            // Unused when k is split (reduce_slices scales the sums).
            const int c = min(c0 + ocol + 4 * q, p.n - 4);
            esc[q] = *reinterpret_cast<const floatx4*>(p.scale + c);
        }
    }
    int esh[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
        esh[rb] = RAW ? 0 : -p.shifts[m0 + 16 * rb + (PAIR ? tid / 16 : orow)];  // < m_pad
    const int rpos0 = EPI == kRope ? *p.rope.pos : 0;

    floatx4 acc[RB][16];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int t = 0; t < 16; ++t) acc[rb][t] = floatx4{0.f, 0.f, 0.f, 0.f};

    // A lane whose columns lie past n reads column 0 (its sums are never
    // stored); rows past k read row k - 1, whose A3 entries are zero. No
    // load is predicated, so each multiply waits only for its own chunk.
    int col = c0 + 16 * j < p.n ? c0 + 16 * j : 0;
    if constexpr (PAIR) {
        const int gate = c0 + 16 * (j & 7);
        col = gate < p.pair ? (j < 8 ? gate : p.pair + gate) : 0;
    }
    const std::size_t plane = static_cast<std::size_t>(p.m_pad) * p.k_pad;
    // This lane's rows of A (rows past m read row m - 1; their sums are
    // never stored), from which each chunk is one offset away.
    const float* a_row[RB];
    const uint16_t* a3_row[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        if constexpr (RAW) {
            a_row[rb] = p.A + static_cast<std::size_t>(min(m0 + 16 * rb + j, p.m - 1)) * p.k + 8 * g;
        } else {
            a3_row[rb] = p.A3 + static_cast<std::size_t>(m0 + 16 * rb + j) * p.k_pad + 8 * g;
        }
    }
    const int8_t* b_lane = p.B + static_cast<uint32_t>(8 * g * p.n + col);
    auto fetch = [&](Chunk<RB, RAW>& c, int k0) {
        if constexpr (RAW) {
            // k % 8 == 0, so a lane's 8 values are all inside k or all past
            // it; past k it reads valid memory and is masked.
            int kl = k0;
            if constexpr (!WHOLE) {
                c.aok = k0 + 8 * g < p.k;
                kl = c.aok ? k0 : p.k - 8 - 8 * g;
            }
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const floatx4* src = reinterpret_cast<const floatx4*>(a_row[rb] + kl);
                c.a[rb][0] = src[0];
                c.a[rb][1] = src[1];
            }
        } else {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int term = 0; term < 3; ++term)
                    c.a[rb][term] = *reinterpret_cast<const uint4*>(a3_row[rb] + k0 + term * plane);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if constexpr (WHOLE) {
                c.b[e] = stream_load(reinterpret_cast<const uint4*>(
                    b_lane + static_cast<uint32_t>((k0 + e) * p.n)));
            } else {
                const int r = min(k0 + 8 * g + e, p.k - 1);
                c.b[e] = stream_load(reinterpret_cast<const uint4*>(
                    p.B + static_cast<uint32_t>(r * p.n + col)));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // Column t + 1 is widened while column t's MFMAs run; the barriers pin
    // that order (left alone, the scheduler puts each widening right before
    // its MFMAs, which then wait on it).
    // RAW: low half non-zero once a lo term of this lane's A row 16 rb + j
    // dropped bits.
    uint32_t lost[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) lost[rb] = 0;
    auto multiply = [&](const Chunk<RB, RAW>& c) {
        uint4 aop[RB][3];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if constexpr (RAW && !WHOLE) {
                const floatx4 z{0.f, 0.f, 0.f, 0.f};
                split8(c.aok ? c.a[rb][0] : z, c.aok ? c.a[rb][1] : z, aop[rb], lost[rb]);
            } else if constexpr (RAW) {
                split8(c.a[rb][0], c.a[rb][1], aop[rb], lost[rb]);
            } else {
#pragma unroll
                for (int term = 0; term < 3; ++term) aop[rb][term] = c.a[rb][term];
            }
        }
        bf16x8 bop = column(c.b, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            bf16x8 next = bop;
            if (t + 1 < 16) next = column(c.b, t + 1);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int term = 0; term < 3; ++term)
                    acc[rb][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, aop[rb][term]), bop, acc[rb][t], 0, 0, 0);
            bop = next;
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // This wave's chunks: k0 + i * kStep for i < n, in a ring of kDepth
    // register sets (all in flight before the first multiply); past the last
    // chunk the ring re-reads it rather than branch around a load.
    const int k0 = kb + kChunk * w;
    const int n = k0 < ke ? (ke - k0 + kStep - 1) / kStep : 0;
    auto at = [&](int i) { return k0 + (i < n ? i : n - 1) * kStep; };
    if (n > 0) {
        Chunk<RB, RAW> ring[kDepth];
#pragma unroll
        for (int d = 0; d < kDepth; ++d) fetch(ring[d], at(d));
        for (int i = 0; i < n; i += kDepth) {
#pragma unroll
            for (int d = 0; d < kDepth; ++d) {
                if (i + d < n) multiply(ring[d]);
                fetch(ring[d], at(i + d + kDepth));
            }
        }
    }

    // Epilogue, one 16-row block at a time: wave sums into LDS by actual
    // column, then each thread adds the four waves for 16 consecutive
    // columns of one row and writes four float4. RAW: a block where a lo
    // term dropped bits (|a| below 2^-110) or a sum is not finite (an
    // infinite or NaN activation, or an overflow) is not written here but
    // computed again by fma_block once the others are out.
    //
    // The epilogue's loads come before its stores: a load placed after a
    // store that may alias it cannot be moved above it, and a wait for a
    // load is also a wait for every store issued before it on this target,
    // so loads between stores would make each store wait for the last. The
    // column scales and the rows' shifts were loaded before the chunks;
    // every block's prior C values (kAccumulate) or RoPE angles (kRope) are
    // loaded here, before any store, unconditionally (rows and columns
    // clamped into range, their values then unused), so that no merge of a
    // loaded and a constant value makes a later instruction wait.
    __shared__ int any_bad[4];
    uint32_t redo = 0;  // RAW: bit rb set for each block fma_block recomputes
    floatx4 extra[EPI == kStore ? 1 : RB][4];
    if constexpr (EPI != kStore) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int row = min(m0 + 16 * rb + orow, p.m - 1);
                const int c = min(c0 + ocol + 4 * q, p.n - 4);
                if constexpr (EPI == kRope)
                    extra[rb][q] = rope_angles_any(p.rope, rpos0 + row, c);
                else
                    extra[rb][q] = *reinterpret_cast<const floatx4*>(
                        p.out + static_cast<std::size_t>(row) * p.n + c);
            }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        if (rb > 0) __syncthreads();
        floatx4* mine = tile + w * 16 * (kTile / 4);
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                mine[(4 * g + r) * (kTile / 4) + granule(4 * j + q)] =
                    floatx4{acc[rb][4 * q][r], acc[rb][4 * q + 1][r], acc[rb][4 * q + 2][r],
                            acc[rb][4 * q + 3][r]};
        __syncthreads();
        if constexpr (PAIR) {
            // Eight gates of one row per thread and their ups 128 columns
            // on, each summed over the waves in order as below, scaled as C
            // would be written, then paired.
            const int prow = tid / 16;
            const int prow_m = m0 + 16 * rb + prow;
            floatx4 gv[2], uv[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int gq = granule(pp / 4 + q), uq = granule((pp + kTile / 2) / 4 + q);
                gv[q] = tile[prow * (kTile / 4) + gq];
                uv[q] = tile[prow * (kTile / 4) + uq];
#pragma unroll
                for (int ww = 1; ww < 4; ++ww) {
                    gv[q] += tile[(ww * 16 + prow) * (kTile / 4) + gq];
                    uv[q] += tile[(ww * 16 + prow) * (kTile / 4) + uq];
                }
            }
            if (prow_m < p.m) {
                const int sh = esh[rb];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int c = c0 + pp + 4 * q;
                    if (c >= p.pair) break;
                    const floatx4 gx = gv[q] * esc[q];
                    const floatx4 ux = uv[q] * esc[2 + q];
                    floatx4 y;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        y[e] = silu_mul(__builtin_ldexpf(gx[e], sh), __builtin_ldexpf(ux[e], sh));
                    *reinterpret_cast<floatx4*>(p.out + static_cast<std::size_t>(prow_m) * p.pair + c) = y;
                }
            }
            continue;
        }
        const int row = m0 + 16 * rb + orow;
        floatx4 v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            // (Columns past n are in the tile too; their sums go nowhere.)
            const int gq = granule(ocol / 4 + q);
            v[q] = tile[orow * (kTile / 4) + gq];
#pragma unroll
            for (int ww = 1; ww < 4; ++ww) v[q] += tile[(ww * 16 + orow) * (kTile / 4) + gq];
        }
        if constexpr (RAW) {
            bool bad = (lost[rb] & 0xffffu) != 0;
            if (row < p.m) {
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        bad |= c0 + ocol + 4 * q < p.n && !(fabsf(v[q][e]) < __builtin_inff());
            }
            const bool wave_bad = __ballot(bad) != 0;
            if (lane == 0) any_bad[w] = wave_bad;
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(any_bad[0] | any_bad[1] | any_bad[2] | any_bad[3])) {
                redo |= 1u << rb;
                continue;
            }
        }
        if (row < p.m) {
            // Pre-split planes: the row's scale undone, after the column
            // scale into C, before it into the partials (reduce_slices
            // applies it).
            const int sh = esh[rb];
            auto unshift = [&](floatx4 x) {
                if constexpr (!RAW) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) x[e] = __builtin_ldexpf(x[e], sh);
                }
                return x;
            };
            if (EPI == kStore && !p.direct) {
                // A k slice's sums into the partials.
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int c = c0 + ocol + 4 * q;
                    if (c >= p.n) break;
                    *reinterpret_cast<floatx4*>(
                        p.out + (static_cast<std::size_t>(place.slice) * p.m + row) * p.n + c) = unshift(v[q]);
                }
                continue;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int c = c0 + ocol + 4 * q;
                if (c >= p.n) break;
                const floatx4 x = unshift(v[q] * esc[q]);
                if constexpr (EPI == kRope) {
                    rope_put(p, row, rpos0 + row, c, x, extra[rb][q]);
                } else {
                    floatx4* o = reinterpret_cast<floatx4*>(p.out + static_cast<std::size_t>(row) * p.n + c);
                    if constexpr (EPI == kAccumulate)
                        *o = extra[rb][q] + x;
                    else
                        *o = x;
                }
            }
        }
    }
    if constexpr (RAW) {
        while (redo) {
            const int rb = __builtin_ctz(redo);
            redo &= redo - 1;
            fma_block(p, c0, m0 + 16 * rb, kb, ke, place.slice);
        }
    }
}

template <int RB, int EPI>
void launch_epi(const SbParams& p, int blocks, bool raw, bool whole, hipStream_t s) {
    const dim3 grid(blocks), block(kThreads);
    if constexpr (EPI != kRope) {  // the RoPE epilogue only follows a pre-pass
        if (raw) {
            if (whole)
                hipLaunchKernelGGL((split_bf16_kernel<RB, true, true, false, EPI>), grid, block, 0, s, p);
            else
                hipLaunchKernelGGL((split_bf16_kernel<RB, true, false, false, EPI>), grid, block, 0, s, p);
            return;
        }
    }
    if (whole)
        hipLaunchKernelGGL((split_bf16_kernel<RB, false, true, false, EPI>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((split_bf16_kernel<RB, false, false, false, EPI>), grid, block, 0, s, p);
}

template <int RB>
void launch(const SbParams& p, int blocks, bool raw, hipStream_t s) {
    const bool whole = p.k % kChunk == 0;
    if (p.pair) {
        if (whole)
            hipLaunchKernelGGL((split_bf16_kernel<RB, false, true, true>), dim3(blocks), dim3(kThreads), 0, s, p);
        else
            hipLaunchKernelGGL((split_bf16_kernel<RB, false, false, true>), dim3(blocks), dim3(kThreads), 0, s, p);
        return;
    }
    if (p.rope.pos)  // direct, pre-split (split_run fuses RoPE only then)
        return launch_epi<RB, kRope>(p, blocks, raw, whole, s);
    if (p.accumulate)  // direct (the partials of a k split are added by reduce_slices)
        return launch_epi<RB, kAccumulate>(p, blocks, raw, whole, s);
    launch_epi<RB, kStore>(p, blocks, raw, whole, s);
}

}  // namespace

bool split_bf16_supports(const MatmulArgs& a) {
    return a.n % 16 == 0 && reinterpret_cast<uintptr_t>(a.B) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(a.scale) % 16 == 0;
}

// The GEMV's cost grows with m (its multiply-adds, and from 5 rows an
// 8-row kernel whose slices are half as deep), while this kernel pays for a
// whole 16-row block at any m. Measured per call in HIP graphs, GEMV against
// exact-split (us):
//   4096 x 4096:   m 2  7.5 /  9.6, m 4  9.1 /  9.6, m 5 11.7 /  9.7, m 8 12.5 / 10.0
//   4096 x 11008:  m 2 12.9 / 13.8, m 3 15.6 / 14.6, m 5 27.7 / 14.2, m 8 31.6 / 14.5
//   11008 x 4096:  m 2 12.9 / 14.4, m 3 15.3 / 14.4, m 5 25.1 / 14.5, m 8 28.2 / 14.9
//   4096 x 32000:  m 2 27.6 / 26.2, m 3 32.4 / 26.0, m 5 59.6 / 26.3, m 8 67.3 / 26.7
// So: from 5 rows always; from 3 rows for 2^25 weights or more; from 2 rows
// for 2^26 or more.
bool split_bf16_preferred(int m, int n, int k) {
    const long long w = static_cast<long long>(n) * k;
    return m >= 5 || (m >= 3 && w >= (1LL << 25)) || (m >= 2 && w >= (1LL << 26));
}

namespace {

// The product, or with pair > 0 the SwiGLU pair (out = a.C, m x pair);
// false when pair is asked for and the product would need a k split (then
// nothing is launched). *fused: RoPE was fused.
bool split_run(const MatmulArgs& a, const RopeFuse* rope, int pair, bool* fused) {
    // Without a norm, the kernel splits A itself, chunk by chunk (needs whole
    // 8-value groups and 16-byte rows); otherwise a pre-pass writes the three
    // planes with the norm fused. The SwiGLU pair always reads the planes.
    const bool raw = !pair && !a.rms_weight && a.k % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(a.A) % 16 == 0;

    // More 16-row blocks per workgroup cut how often each weight is widened
    // (the VALU work that paces this kernel); fewer keep more workgroups in
    // flight without a k split and its reduce, and round the grid better
    // (one workgroup per CU at a time). The largest of 4 / 2 / 1 whose tile
    // grid, weighted by k / 4096 (deeper k holds more work per workgroup),
    // reaches 160 workgroups and, past one per CU, leaves its last round at
    // least 80 % full (70 % with A pre-split into planes, where a workgroup
    // splits nothing itself and widening weighs more). Over sweeps of
    // m = 128..1024 and 15 shapes (widths 4096..32000, k 4096 and 11008,
    // with and without the norm) it averaged 0.6 % above the best of the
    // three, at most 8 %. At m = 512: 4096^2 takes 2 (55 vs 64 us for 4),
    // 4096 x 11008 2 (162 vs 177), 4096 x 22016 4 (266 vs 294), 4096 x 32000
    // 4 (362 vs 408).
    const int col_tiles = ceil_div(a.n, kTile);
    const double kf = std::max(1.0, a.k / 4096.0);
    auto fits = [&](int rb) {
        if (16 * rb > a.m + 15) return false;
        const double grid = static_cast<double>(ceil_div(a.m, 16 * rb)) * col_tiles;
        if (grid * kf < 160.0) return false;
        const double rounds = grid / cu_count();
        return rounds <= 1.0 || rounds / std::ceil(rounds) >= (raw ? 0.8 : 0.7);
    };
    auto tiles = [&](int rb) {
        return static_cast<long long>(ceil_div(a.m, 16 * rb)) * col_tiles;
    };
    int RB = fits(4) ? 4 : fits(2) ? 2 : 1;
    // Four-block tiles whose last round is at most half full also win when
    // that round runs as two-block tiles (the tail below), though the rounds
    // rule above turns them down: 4096 x 11008 at m = 512 131.9 against
    // 136.9 us (146.3 / 154.2 with the norm; from HBM, 144.9 / 154.6), m =
    // 1024 244.7 / 249.5; the same bits either way.
    if (RB != 4 && 64 <= a.m + 15 && tiles(4) >= cu_count()) {
        const long long cu = cu_count(), g4 = tiles(4), rest = g4 % cu;
        if (rest > 0 && 2 * rest <= cu && (g4 - rest) % ceil_div(a.m, 64) == 0) RB = 4;
    }
    const int row_tiles = ceil_div(a.m, 16 * RB);
    const int m_pad = row_tiles * 16 * RB;
    const int k_pad = ceil_div(a.k, kChunk) * kChunk;

    // k slices up to one workgroup per CU, each at least 256 rows deep.
    const long long blocks = static_cast<long long>(row_tiles) * col_tiles;
    const int want = static_cast<int>(std::max(1LL, cu_count() / blocks));
    int slices = std::max(1, std::min(want, ceil_div(a.k, 256)));
    const int span = ceil_div(ceil_div(a.k, slices), kStep) * kStep;
    slices = ceil_div(a.k, span);

    if (pair && slices > 1) return false;

    uint16_t* A3 = nullptr;
    int* shifts = nullptr;
    if (!raw) {
        // The planes, then one int per row: its power-of-two shift.
        const std::size_t plane_floats = (static_cast<std::size_t>(3) * m_pad * k_pad + 1) / 2;
        float* base = scratch(kSplitA, plane_floats + m_pad);
        A3 = reinterpret_cast<uint16_t*>(base);
        shifts = reinterpret_cast<int*>(base + plane_floats);
        const int steps = ceil_div(k_pad, 8 * kThreads);
        // Rows (and the norm weight) read as float4 where 16-byte aligned.
        const int vec4 = a.k % 4 == 0 && reinterpret_cast<uintptr_t>(a.A) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(a.rms_weight) % 16 == 0;
        auto row = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(m_pad), dim3(kThreads), 0, a.stream, a.m, a.k, m_pad,
                               k_pad, vec4, a.A, a.rms_weight, A3, shifts);
        };
        if (steps <= 1) {
            row(split_a_row_kernel<1>);
        } else if (steps <= 2) {
            row(split_a_row_kernel<2>);
        } else if (steps <= 4) {
            row(split_a_row_kernel<4>);
        } else {
            hipLaunchKernelGGL(split_a_kernel, dim3(m_pad), dim3(kThreads), 0, a.stream, a.m, a.k,
                               m_pad, k_pad, a.A, a.rms_weight, A3, shifts);
        }
    }

    SbParams p{};
    p.m = a.m;
    p.n = a.n;
    p.k = a.k;
    p.k_span = span;
    p.m_pad = m_pad;
    p.k_pad = k_pad;
    p.A3 = A3;
    p.shifts = shifts;
    p.A = a.A;
    p.B = static_cast<const int8_t*>(a.B);
    p.scale = a.scale;
    p.direct = slices == 1;
    p.pair = pair;
    p.accumulate = a.accumulate && p.direct;
    p.out = p.direct ? a.C : scratch(kPartial, static_cast<std::size_t>(slices) * a.m * a.n);
    p.row_tiles = row_tiles;
    p.col_tiles = col_tiles;
    // One row tile over a multiple of 8 column tiles: plain order puts every
    // k slice of column tile t on XCD t mod 8, where the reduce workgroup for
    // those columns also runs, so the partials stay in one L2 (m = 16:
    // 4096^2 11.7 -> 9.9 us, 11008 x 4096 16.4 -> 15.1). Otherwise the
    // XCD-grouped order, which gives each XCD a contiguous run of B (4096 x
    // 32000, m = 5: 26.6 against 28.6 us in plain order).
    p.xcd_order = row_tiles == 1 && col_tiles % 8 == 0 ? 0 : 1;
    const bool fuse = rope && p.direct && !raw && !a.accumulate && rope->head_size % 4 == 0 &&
                      rope->dim % 4 == 0 && rope->kv_dim % 4 == 0 &&
                      a.n == rope->dim + 2 * rope->kv_dim;
    if (fuse) p.rope = *rope;
    // A product in one slice whose four-block tiles leave a last round at
    // most half full runs that round's column tiles as two-block tiles: one
    // round of twice the workgroups, each about 0.7 of a four-block tile's
    // time (widening shared by half the rows), rather than one of half the
    // CUs at a full tile's time. Same arithmetic per element, so the same
    // bits. qkv of a 512-row Llama-7B prefill: 384 tiles, 128 of them the
    // last round.
    int tail_cols = 0;
    if (RB == 4 && slices == 1) {
        const long long cu = cu_count();
        const long long full = blocks / cu * cu, rest = blocks - full;
        if (full > 0 && rest > 0 && 2 * rest <= cu && full % row_tiles == 0)
            tail_cols = col_tiles - static_cast<int>(full / row_tiles);
    }
    if (tail_cols > 0) {
        p.col_tiles = col_tiles - tail_cols;
        launch<4>(p, row_tiles * p.col_tiles, raw, a.stream);
        SbParams t = p;
        t.row_tiles = ceil_div(a.m, 32);  // within m_pad: a multiple of 64
        t.col_tiles = tail_cols;
        t.col_base = col_tiles - tail_cols;
        t.xcd_order = 1;
        launch<2>(t, t.row_tiles * tail_cols, raw, a.stream);
        *fused = fuse;
        return true;
    }
    const int total = static_cast<int>(blocks) * slices;
    switch (RB) {
        case 1: launch<1>(p, total, raw, a.stream); break;
        case 4: launch<4>(p, total, raw, a.stream); break;
        default: launch<2>(p, total, raw, a.stream); break;
    }
    if (!p.direct) run_reduce_slices(a.m, a.n, slices, p.out, a.scale, a.C, a.accumulate, a.stream);
    *fused = fuse;
    return true;
}

}  // namespace

bool run_split_bf16(const MatmulArgs& a, const RopeFuse* rope) {
    bool fused = false;
    split_run(a, rope, 0, &fused);
    return fused;
}

bool split_bf16_swiglu_supported(const MatmulArgs& a, int hidden) {
    return hidden > 0 && hidden % 16 == 0 && a.n == 2 * hidden && !a.accumulate &&
           split_bf16_supports(a) && reinterpret_cast<uintptr_t>(a.C) % 16 == 0;
}

bool run_split_bf16_swiglu(const MatmulArgs& a, int hidden) {
    if (!split_bf16_swiglu_supported(a, hidden)) return false;
    bool fused = false;
    return split_run(a, nullptr, hidden, &fused);
}

}  // namespace em
