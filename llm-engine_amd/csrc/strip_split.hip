// Decode batches of 9 .. 16 rows over registered int8 weights, in one
// launch: the exact bf16 split of split_bf16.hip run over the library's
// strip-layout copy of B (gemv_packed.hip), with k split across workgroups
// and the slices added inside the same launch. It replaces, for these
// shapes, the reference's tiled_split product followed by sum_slices
// (/root/reference/src/cuda_matmul.cu:333-363, 245-254), which is a
// row-major product plus a second launch.
//
// Tile. A workgroup owns 64 columns (four strips) and a slice of k. Lane
// (g, j) of a wave, g = lane / 16, j = lane % 16, reads unit j % 4 of strip
// j / 4: for a 32-row chunk it loads the units of quads g and g + 4 (rows
// 4g .. 4g + 3 and 16 + 4g .. 16 + 4g + 3), 16 bytes each, each holding four
// rows of four columns. v_mfma_f32_16x16x32_bf16 takes from lane (g, j) the
// 8 k-values 8g .. 8g + 7 of B's column j and of A's row j; here those k
// positions are the lane's eight rows, in the same order for A and B, and
// MFMA u (0..3) takes byte u of each row, i.e. column 4(j % 4) + u of strip
// j / 4. So MFMA u's output column j is tile column 4j + u, and lane (g, j)
// ends up holding columns 4j .. 4j + 3 of rows 4g .. 4g + 3: one float4 per
// row, stored without any transpose. Each weight byte is widened once (a
// sign-extending byte convert and half a byte permute) and feeds 3 x RB
// MFMAs; each A value is split once per tile (split8 of split_bf16.hip's
// arithmetic, in registers).
//
// Slices. k is cut into slices so the grid covers the CUs (4096^2: 64
// tiles x 4 slices). Within a workgroup the four waves take interleaved
// 32-row chunks and are added through LDS in wave order. Each workgroup
// then stores its slice's sums as device-coherent (sc1) buffer stores (no
// cache write-back), waits for them, and counts itself in at its tile's
// counter (one relaxed agent-scope atomic add). The workgroup that counts
// in last adds the tile's slices in slice order (its own from registers,
// the others by sc1 buffer loads), applies the scale, norm and
// accumulation, stores C and sets the counter back to zero for the next
// call. The sum order is fixed, so repeated calls give the same bits,
// whichever workgroup arrives last. Counters are library memory, zero when
// allocated and zero again after every call; the partials live in the
// library's scratch. As with every product here, calls that overlap on one
// device race on that memory.
//
// Range. As in split_bf16.hip: a 16-row block whose lo terms dropped bits
// (|a| below 2^-110) or whose slice sums are not finite (an infinite or NaN
// activation, or an overflow) has that slice computed again by fp32
// multiply-adds, so infinities and NaN propagate as fp32 arithmetic gives.
//
// Norm. With a fused RMSNorm each lane multiplies its A values by the norm
// weight before splitting and sums their squares on the way; the slices'
// sums of squares are added in slice order like the products, and the row's
// RMS scale multiplies each finished sum once.
#include <algorithm>

#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kCols = 64;        // columns per workgroup: four strips
constexpr int kStripCols = 16;
constexpr int kRows32 = 32;      // k rows per chunk
constexpr int kNT = 256;                 // threads per workgroup
constexpr int kWaves = kNT / kWave;
constexpr int kStep = kWaves * kRows32;  // k rows the waves take per round
constexpr int kMaxSlices = 8;            // k slices of one tile, at most

struct SsParams {
    int m, n, k;
    int span;    // k rows per slice (a multiple of kStep)
    int slices;
    int tiles;   // column tiles
    int xcd;     // slices of a tile spread over XCDs (slice = XCD mod slices)
    const float* A;
    const float* w;     // norm weight, or null
    const int8_t* P;    // strip layout
    const float* scale;
    float* C;
    int accumulate;
    float* part;        // [tile][slice][16 RB][64] slice sums
    float* part_ssq;    // [tile][slice][16 RB] sums of squares (norm)
    unsigned* count;    // [tile] arrival counters, zero between calls
};

__device__ __forceinline__ uint32_t bits(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ float from_bits(uint32_t u) { return __builtin_bit_cast(float, u); }

// Eight fp32 values -> three bf16 terms, packed as MFMA A operands (the
// arithmetic of split_bf16.hip's split8): hi = the value's top half, mid =
// the top half of the exact remainder, lo = the top half of what is left.
// lo's low half is ORed into `lost`: non-zero iff bits were dropped.
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

// MFMA u's B operand: byte u of each of the lane's eight rows (the four
// words of unit b0, then of unit b1), widened to bf16 (exact: |q| <= 127).
template <int U>
__device__ __forceinline__ bf16x8 widen_column(const uint4& b0, const uint4& b1) {
    const uint32_t w[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    uint32_t f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = bits(static_cast<float>(static_cast<int8_t>(w[e] >> (8 * U))));
    uint4 packed;
    packed.x = __builtin_amdgcn_perm(f[1], f[0], 0x07060302u);
    packed.y = __builtin_amdgcn_perm(f[3], f[2], 0x07060302u);
    packed.z = __builtin_amdgcn_perm(f[5], f[4], 0x07060302u);
    packed.w = __builtin_amdgcn_perm(f[7], f[6], 0x07060302u);
    return __builtin_bit_cast(bf16x8, packed);
}

template <int RB, bool NORM>
struct SsChunk {
    uint4 b0, b1;           // units of quads g and g + 4 of the chunk
    floatx4 a[RB][2];       // A[row][k0 + 4g ..], A[row][k0 + 16 + 4g ..]
    floatx4 w[NORM ? 2 : 1];  // norm weights at the same k
    bool ok0, ok1;          // the two float4 groups lie inside k (EXACT: always)
};

// Columns c .. c + 3 (one unit of one strip) of rows `row`, summed over k in
// [kb, ke) by fp32 multiply-adds of (a (* w)) * q: the recomputation of a
// slice whose split could not hold A exactly.
template <bool NORM>
__device__ floatx4 fma_slice(const SsParams& p, int row, int c, int kb, int ke) {
    const int strip = c / kStripCols, unit = (c % kStripCols) / 4;
    const int8_t* base = p.P + static_cast<std::size_t>(strip) * p.k * kStripCols + 16 * unit;
    const float* a = p.A + static_cast<std::size_t>(row) * p.k;
    floatx4 acc{0.f, 0.f, 0.f, 0.f};
    for (int kk = kb; kk < ke; ++kk) {
        float x = a[kk];
        if constexpr (NORM) x *= p.w[kk];
        // Row kk of columns 4 unit .. 4 unit + 3: quad kk / 4, word kk % 4
        // of the unit.
        const uint32_t q4 = *reinterpret_cast<const uint32_t*>(
            base + static_cast<std::size_t>(kk / 4) * 64 + 4 * (kk % 4));
        float qv[4];
        widen4(q4, qv);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = fmaf(x, qv[e], acc[e]);
    }
    return acc;
}

// RB: 16-row blocks (m <= 16 RB). D: chunks per wave in flight (a ring).
// EXACT: every chunk lies inside k (k % 32 == 0), no masks. SB: the k
// slices of a tile are at most SB (1: one slice, no partials).
template <int RB, int D, bool NORM, bool EXACT, int SB>
__global__ __launch_bounds__(kNT) void strip_split_kernel(SsParams p) {
    constexpr int MR = 16 * RB;  // rows of the tile
    constexpr int NI = (MR * 16 + kNT - 1) / kNT;  // output items per thread
    __shared__ __attribute__((aligned(16))) floatx4 red[kWaves][MR][16];
    __shared__ float ssq_red[kWaves][NORM ? MR : 1];
    // Per wave and row block: a lo term dropped bits, a slice sum is not
    // finite (each entry written by its own wave only).
    __shared__ int lost_w[kWaves][RB], nonfinite_w[kWaves][RB];
    __shared__ unsigned arrived;

    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int g = lane >> 4, j = lane & 15;

    int tile, slice;
    if (p.xcd) {
        // Workgroups go to the eight XCDs in turn: XCD x runs slice x mod
        // slices of its tiles, so each XCD reads one k range of A.
        const int x = blockIdx.x & 7, q = blockIdx.x >> 3, per = 8 / p.slices;
        slice = x % p.slices;
        tile = q * per + x / p.slices;
    } else {
        tile = blockIdx.x / p.slices;
        slice = blockIdx.x % p.slices;
    }

    const int strips = p.n / kStripCols;
    const int strip = min(tile * 4 + (j >> 2), strips - 1);  // past n: read, never stored
    const int8_t* unit0 = p.P + static_cast<std::size_t>(strip) * p.k * kStripCols + 16 * (j & 3);
    const int k4 = p.k / 4;
    const int kb = slice * p.span;
    const int ke = min(p.k, kb + p.span);
    const float* a_row[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
        a_row[rb] = p.A + static_cast<std::size_t>(min(16 * rb + j, p.m - 1)) * p.k;

    // Chunk loads are issued unconditionally, so the compiler's wait counts
    // stay exact (a load behind a branch makes every later wait a wait for
    // all loads). A chunk past the wave's last (`real` false) reads one
    // 64-byte line that every lane shares, the first column scales (hot in
    // L2, one request per instruction), and is never multiplied.
    const floatx4* dummy = reinterpret_cast<const floatx4*>(p.scale);
    auto fetch = [&](SsChunk<RB, NORM>& c, int k0, bool real) {
        int qa0 = k0 / 4 + g, qa1 = k0 / 4 + 4 + g;
        int ka0 = k0 + 4 * g, ka1 = k0 + 16 + 4 * g;
        if constexpr (!EXACT) {
            c.ok0 = ka0 < p.k;
            c.ok1 = ka1 < p.k;
            qa0 = min(qa0, k4 - 1);
            qa1 = min(qa1, k4 - 1);
            ka0 = min(ka0, p.k - 4);
            ka1 = min(ka1, p.k - 4);
        }
        const uint4* b0 = real ? reinterpret_cast<const uint4*>(unit0 + static_cast<std::size_t>(qa0) * 64)
                               : reinterpret_cast<const uint4*>(dummy);
        const uint4* b1 = real ? reinterpret_cast<const uint4*>(unit0 + static_cast<std::size_t>(qa1) * 64)
                               : reinterpret_cast<const uint4*>(dummy);
        c.b0 = stream_load(b0);
        c.b1 = stream_load(b1);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            c.a[rb][0] = *(real ? reinterpret_cast<const floatx4*>(a_row[rb] + ka0) : dummy);
            c.a[rb][1] = *(real ? reinterpret_cast<const floatx4*>(a_row[rb] + ka1) : dummy);
        }
        if constexpr (NORM) {
            c.w[0] = *(real ? reinterpret_cast<const floatx4*>(p.w + ka0) : dummy);
            c.w[1] = *(real ? reinterpret_cast<const floatx4*>(p.w + ka1) : dummy);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    floatx4 acc[RB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[rb][u] = floatx4{0.f, 0.f, 0.f, 0.f};
    uint32_t lost[RB];
    float ss[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        lost[rb] = 0;
        ss[rb] = 0.0f;
    }

    auto multiply = [&](const SsChunk<RB, NORM>& c) {
        uint4 aop[RB][3];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            floatx4 x0 = c.a[rb][0], x1 = c.a[rb][1];
            if constexpr (!EXACT) {
                const floatx4 z{0.f, 0.f, 0.f, 0.f};
                x0 = c.ok0 ? x0 : z;
                x1 = c.ok1 ? x1 : z;
            }
            if constexpr (NORM) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ss[rb] = fmaf(x0[e], x0[e], ss[rb]);
                    ss[rb] = fmaf(x1[e], x1[e], ss[rb]);
                }
                x0 *= c.w[0];
                x1 *= c.w[1];
            }
            split8(x0, x1, aop[rb], lost[rb]);
        }
        const bf16x8 b[4] = {widen_column<0>(c.b0, c.b1), widen_column<1>(c.b0, c.b1),
                             widen_column<2>(c.b0, c.b1), widen_column<3>(c.b0, c.b1)};
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int term = 0; term < 3; ++term)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc[rb][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, aop[rb][term]), b[u], acc[rb][u], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    };

    // This wave's chunks: k0 + i * kStep, i < nc, in a ring of D register
    // sets; past the last chunk the ring re-reads it (never multiplied).
    const int k0 = kb + kRows32 * w;
    const int nc = k0 < ke ? (ke - k0 + kStep - 1) / kStep : 0;
    auto at = [&](int i) { return k0 + (i < nc ? i : nc - 1) * kStep; };
    if (nc > 0) {
        SsChunk<RB, NORM> ring[D];
#pragma unroll
        for (int d = 0; d < D; ++d) fetch(ring[d], at(d), d < nc);
        for (int i = 0; i < nc; i += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                if (i + d < nc) multiply(ring[d]);
                fetch(ring[d], at(i + d + D), i + d + D < nc);
            }
        }
    }

    // Item i of this thread: row it / 16 of the tile, columns 4 (it % 16) ..
    // 4 (it % 16) + 3, for it = tid + kNT i below 16 MR.
    auto item = [&](int i, int& row, int& q) {
        const int it = tid + kNT * i;
        row = it >> 4;
        q = it & 15;
        return it < MR * 16;
    };
    // The epilogue's column scales, issued here so that their latency passes
    // behind the wave sums' staging and the slice exchange, not after the
    // last workgroup's sums (n is a multiple of 16, so c < n covers c + 3).
    // Without k slices the prior C (accumulate) comes with them; with slices
    // only the last workgroup of the tile loads it, beside the others' sums.
    floatx4 esc[NI], eprior[NI];
    auto load_prior = [&](int i, int row, int c) {
        if (p.accumulate)
            eprior[i] = *reinterpret_cast<const floatx4*>(p.C + static_cast<std::size_t>(row) * p.n + c);
    };
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        int row, q;
        esc[i] = eprior[i] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (!item(i, row, q)) continue;
        const int c = tile * kCols + 4 * q;
        if (row >= p.m || c >= p.n) continue;
        esc[i] = *reinterpret_cast<const floatx4*>(p.scale + c);
        if constexpr (SB == 1) load_prior(i, row, c);
    }

    // Wave sums into LDS: lane (g, j) holds rows 4g + r, columns 4j .. 4j + 3.
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            red[w][16 * rb + 4 * g + r][j] =
                floatx4{acc[rb][0][r], acc[rb][1][r], acc[rb][2][r], acc[rb][3][r]};
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        if constexpr (NORM) {
            // Row 16 rb + j: this lane's squares, then the four lane groups.
            float v = ss[rb];
            v += __shfl_xor(v, 16, kWave);
            v += __shfl_xor(v, 32, kWave);
            if (g == 0) ssq_red[w][16 * rb + j] = v;
        }
        const bool any_lost = __ballot((lost[rb] & 0xffffu) != 0) != 0;
        if (lane == 0) lost_w[w][rb] = any_lost;
    }
    __syncthreads();

    floatx4 v[NI];
    float sq[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        int row, q;
        v[i] = floatx4{0.f, 0.f, 0.f, 0.f};
        sq[i] = 0.0f;
        if (!item(i, row, q)) continue;
        v[i] = red[0][row][q];
#pragma unroll
        for (int ww = 1; ww < kWaves; ++ww) v[i] += red[ww][row][q];
        if constexpr (NORM) {
            sq[i] = ssq_red[0][row];
#pragma unroll
            for (int ww = 1; ww < kWaves; ++ww) sq[i] += ssq_red[ww][row];
        }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        bool nonfinite = false;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            int row, q;
            if (!item(i, row, q) || (row >> 4) != rb) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) nonfinite |= !(fabsf(v[i][e]) < __builtin_inff());
        }
        const bool any = __ballot(nonfinite) != 0;
        if (lane == 0) nonfinite_w[w][rb] = any;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        int row, q;
        if (!item(i, row, q)) continue;
        bool bad = false;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) bad |= lost_w[ww][row >> 4] || nonfinite_w[ww][row >> 4];
        const int c = tile * kCols + 4 * q;
        if (bad && row < p.m && c < p.n) v[i] = fma_slice<NORM>(p, row, c, kb, ke);
    }

    if constexpr (SB > 1) {
        // This slice's sums as device-coherent (sc1) 16-byte buffer stores,
        // visible device-wide once the wait returns. Byte offsets fit 32
        // bits (the host keeps the partials under 2 GiB).
        const __amdgpu_buffer_rsrc_t prs =
            __builtin_amdgcn_make_buffer_rsrc(p.part, 0, 0x7fffffff, 0x00020000);
        const __amdgpu_buffer_rsrc_t qrs =
            __builtin_amdgcn_make_buffer_rsrc(p.part_ssq, 0, 0x7fffffff, 0x00020000);
        constexpr int kSc1 = 16;  // the cache-policy operand's sc1 bit
        const uint32_t base = static_cast<uint32_t>((tile * p.slices + slice) * MR);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            int row, q;
            if (!item(i, row, q)) continue;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[i]), prs,
                                                   ((base + row) * kCols + 4 * q) * 4, 0, kSc1);
            if (NORM && q == 0)
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sq[i]), qrs,
                                                      (base + row) * 4, 0, kSc1);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0)
            arrived = __hip_atomic_fetch_add(p.count + tile, 1u, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (arrived != static_cast<unsigned>(p.slices - 1)) return;
        // Last of the tile: every other slice's sums loaded at once (sc1,
        // so from the device-coherent level, not a stale cache line; slots
        // past the slice count read offset 0, one shared line), then added
        // in slice order with this slice's own from registers.
        const uint32_t tile0 = static_cast<uint32_t>(tile * p.slices * MR);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            int row, q;
            if (!item(i, row, q)) continue;
            const int c = tile * kCols + 4 * q;
            if (row < p.m && c < p.n) load_prior(i, row, c);
        }
        floatx4 xs[NI][SB];
        float ys[NI][SB];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            int row, q;
            const bool live = item(i, row, q);
#pragma unroll
            for (int s2 = 0; s2 < SB; ++s2) {
                const bool real = live && s2 < p.slices && s2 != slice;
                const uint32_t r = tile0 + s2 * MR + row;
                xs[i][s2] = __builtin_bit_cast(
                    floatx4, __builtin_amdgcn_raw_buffer_load_b128(prs, real ? (r * kCols + 4 * q) * 4 : 0,
                                                                   0, kSc1));
                ys[i][s2] = 0.0f;
                if constexpr (NORM)
                    ys[i][s2] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(qrs, real ? r * 4 : 0, 0, kSc1));
            }
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            floatx4 total = slice == 0 ? v[i] : xs[i][0];
            float sqt = slice == 0 ? sq[i] : ys[i][0];
#pragma unroll
            for (int s2 = 1; s2 < SB; ++s2) {
                if (s2 >= p.slices) break;
                total += s2 == slice ? v[i] : xs[i][s2];
                sqt += s2 == slice ? sq[i] : ys[i][s2];
            }
            v[i] = total;
            sq[i] = sqt;
        }
        if (tid == 0)
            __hip_atomic_store(p.count + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

#pragma unroll
    for (int i = 0; i < NI; ++i) {
        int row, q;
        if (!item(i, row, q)) continue;
        const int c = tile * kCols + 4 * q;
        if (row >= p.m || c >= p.n) continue;
        floatx4 x = v[i];
        if constexpr (NORM) x *= 1.0f / sqrtf(sq[i] / static_cast<float>(p.k) + kRmsEps);
        x *= esc[i];
        floatx4* o = reinterpret_cast<floatx4*>(p.C + static_cast<std::size_t>(row) * p.n + c);
        *o = p.accumulate ? eprior[i] + x : x;
    }
}

template <int RB, int D, bool NORM, int SB>
void launch_sb(const SsParams& p, int blocks, hipStream_t s) {
    if (p.k % kRows32 == 0)
        hipLaunchKernelGGL((strip_split_kernel<RB, D, NORM, true, SB>), dim3(blocks), dim3(kNT), 0, s, p);
    else
        hipLaunchKernelGGL((strip_split_kernel<RB, D, NORM, false, SB>), dim3(blocks), dim3(kNT), 0, s, p);
}

template <int RB, int D, bool NORM>
void launch_rb(const SsParams& p, int blocks, hipStream_t s) {
    if (p.slices == 1) return launch_sb<RB, D, NORM, 1>(p, blocks, s);
    if (p.slices <= 4) return launch_sb<RB, D, NORM, 4>(p, blocks, s);
    return launch_sb<RB, D, NORM, kMaxSlices>(p, blocks, s);
}

template <bool NORM>
void launch_norm(const SsParams& p, int blocks, hipStream_t s) {
    launch_rb<1, 4, NORM>(p, blocks, s);
}

}  // namespace

bool strip_split_supported(const MatmulArgs& a) {
    auto a16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
    // n <= 2^18: the partials of 4096 tiles x 8 slices stay far under 2 GiB,
    // so the kernel's 32-bit byte offsets cannot wrap.
    return a.m >= 9 && a.m <= 16 && a.n % kStripCols == 0 && a.n <= (1 << 18) &&
           a.k % 4 == 0 && a.k > 0 && a16(a.A) && a16(a.scale) && a16(a.C) &&
           (!a.rms_weight || a16(a.rms_weight));
}

// Where automatic takes this kernel over the row-major exact split (per
// call, us, registered against unregistered weights, graph replay over
// pools past the Infinity Cache where they fit):
//   k x n          m = 9         m = 16
//   4096 x 4096    9.6 / 9.8     9.5 / 10.6
//   4096 x 11008   15.6 / 15.5   16.2 / 16.8
//   4096 x 12288   15.8 / 16.4   16.5 / 17.5
//   288 x 864      5.4 / 8.0     5.5 / 8.3   (288 x 288, 288 x 1536, 768 x
//   288 x 32000    6.2 / 10.1    6.7 / 11.1   288 alike)
// and where it does not:
//   11008 x 4096   15.1 / 14.6   16.3 / 15.2  (22 rounds a wave)
//   4096 x 22016   25.4 / 23.1   29.3 / 24.8  (one slice, 344 tiles)
//   4096 x 32000   27.6 / 27.2   32.0 / 28.4
//   1024 x 2048     8.2 / 7.9     8.3 / 8.1
// Above 16 rows (two or more 16-row blocks per tile) it lost at every
// shape but the smallest: each block re-reads and re-splits the tile's A,
// which the row-major kernel's 256-column tiles share four times more
// (4096^2 at m = 32 / 64: 13.2 / 19.6 against 13.3 / 16.3).
bool strip_split_preferred(int m, int n, int k) {
    const long long w = static_cast<long long>(n) * k;
    return m <= 16 && (k <= 768 || (k <= 4096 && n <= 12288 && w >= (1LL << 24)));
}

void run_strip_split(const MatmulArgs& a, const int8_t* packed) {
    SsParams p{};
    p.m = a.m;
    p.n = a.n;
    p.k = a.k;
    p.A = a.A;
    p.w = a.rms_weight;
    p.P = packed;
    p.scale = a.scale;
    p.C = a.C;
    p.accumulate = a.accumulate ? 1 : 0;
    p.tiles = ceil_div(a.n, kCols);
    // Slices until the grid covers the CUs, each a whole number of rounds
    // of the four waves' chunks.
    const int rounds = ceil_div(a.k, kStep);
    int slices = std::max(1, std::min({cu_count() / p.tiles, rounds, kMaxSlices}));
    p.span = ceil_div(rounds, slices) * kStep;
    slices = ceil_div(a.k, p.span);
    p.slices = slices;
    p.xcd = (8 % slices == 0 && p.tiles % (8 / slices) == 0) ? 1 : 0;
    const int RB = (a.m + 15) / 16;
    if (slices > 1) {
        const std::size_t part = static_cast<std::size_t>(p.tiles) * slices * 16 * RB * kCols;
        const std::size_t ssq = static_cast<std::size_t>(p.tiles) * slices * 16 * RB;
        p.part = scratch(kPartial, part + ssq);
        p.part_ssq = p.part + part;
        p.count = tile_counters(p.tiles);
    }
    const int blocks = p.tiles * slices;
    if (a.rms_weight)
        launch_norm<true>(p, blocks, a.stream);
    else
        launch_norm<false>(p, blocks, a.stream);
}

}  // namespace em
