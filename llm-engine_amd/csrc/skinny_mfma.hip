// Medium-m products (9..64 rows of A, and any m when asked for):
// GpuKernel::tiled_split (reference sgemm_tiled<32|64,...,Split> +
// run_tiled_split, /root/reference/src/cuda_matmul.cu:350-363).
//
// At these m the weights are still the bulk of the traffic (m = 16 and
// m = 64 against a 4096^2 int8 matrix move ~17-19 MB but need 0.5-2.1
// GFLOP), so B is streamed from HBM straight into MFMA operands, read once
// per row tile, without an LDS round trip:
//
//  * v_mfma_f32_16x16x4_f32 takes, in lane l (group g = l / 16, j = l % 16),
//    A[row j][k_g] and B[k_g][col j] and adds into D[row 4g + r][col j].
//    The "column j" of an MFMA need not be a fixed column of C: in MFMA
//    number t, lane j supplies column c0 + col(j, t), where every lane with
//    the same j uses the same col(j, t). A lane can therefore load 16
//    consecutive bytes of one B row (16 int8 columns, or four float4 of fp32
//    columns 64 apart), widen them and feed them to 16 different MFMAs that
//    accumulate into 16 different 16 x 16 blocks. 16 lanes cover a run of
//    256 columns of one row; the four lane groups cover four rows.
//  * A workgroup owns a 256-column tile, a 16 * RB row tile and a k slice.
//    Its four waves take interleaved 16-row chunks of the slice
//    (rows k0 + 4g + u, u = 0..3, so a lane's A operands for one chunk are
//    one float4), prefetching the next chunk while the current one is
//    multiplied. The waves' sums are added in LDS in wave order.
//  * int8 sums stay unscaled; the column scale is applied to the reduced
//    sum (direct) or after the slices are added (reduce_slices).
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

constexpr int kTile = 256;   // columns per workgroup
constexpr int kChunk = 16;   // k rows per wave step
constexpr int kDepth = 2;    // chunks in flight per wave
constexpr int kTileStride = kTile + 4;  // LDS row stride of the epilogue tile

template <class BT>
struct SkParams {
    int m, n, k;
    int k_span;  // multiple of 4 * kChunk
    const float* A;
    const BT* B;
    const float* scale;
    float* out;  // C (direct) or partials [slice][m][n]
    int accumulate;
    int direct;
    int row_tiles, col_tiles;  // grid = row_tiles * col_tiles * slices workgroups
    int xcd_order;
};


// One chunk's B operands for one lane: four rows (u), 16 columns each.
//
// No load is predicated and no loaded value is selected: a lane whose
// columns lie past n reads column 0 instead (its outputs are never stored),
// and in the tail chunk of a slice a row past the slice end reads the
// chunk's first row, whose product is cancelled by a zero A operand. The
// main loop therefore has no branch or select between a load and its use,
// so the wait before each multiply covers only that chunk's loads.
template <class BT>
struct BChunk;

template <>
struct BChunk<int8_t> {
    uint4 v[4];
    // Column of C (relative to the tile) that MFMA t reads in lane column j.
    static __device__ __forceinline__ int col(int j, int t) { return 16 * j + t; }
    template <bool TAIL>
    __device__ __forceinline__ void load(const int8_t* B, int n, int k0row, int ke, int c0, int j,
                                         int g) {
        int c = c0 + 16 * j;
        c = c < n ? c : 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            int r = k0row + 4 * g + u;
            if constexpr (TAIL) r = r < ke ? r : k0row;
            // k * n < 2^31, so the offset fits 32 bits: base in SGPRs + VGPR offset.
            v[u] = stream_load(reinterpret_cast<const uint4*>(B + static_cast<uint32_t>(r * n + c)));
        }
    }
    __device__ __forceinline__ void widen(int u, float* b) const {
        widen4(v[u].x, b);
        widen4(v[u].y, b + 4);
        widen4(v[u].z, b + 8);
        widen4(v[u].w, b + 12);
    }
};

template <>
struct BChunk<float> {
    float4 v[4][4];
    static __device__ __forceinline__ int col(int j, int t) { return 64 * (t >> 2) + 4 * j + (t & 3); }
    template <bool TAIL>
    __device__ __forceinline__ void load(const float* B, int n, int k0row, int ke, int c0, int j,
                                         int g) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            int r = k0row + 4 * g + u;
            if constexpr (TAIL) r = r < ke ? r : k0row;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                int c = c0 + 64 * q + 4 * j;
                c = c < n ? c : 0;
                v[u][q] = stream_load(reinterpret_cast<const float4*>(B + static_cast<uint32_t>(r * n + c)));
            }
        }
    }
    __device__ __forceinline__ void widen(int u, float* b) const {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            b[4 * q + 0] = v[u][q].x;
            b[4 * q + 1] = v[u][q].y;
            b[4 * q + 2] = v[u][q].z;
            b[4 * q + 3] = v[u][q].w;
        }
    }
};

// A operands of one chunk: lane (g, j) holds A[m0 + 16 rb + j][k0 + 4g + u]
// for u = 0..3, one float4 when AVEC (k % 4 == 0 and A 16-byte aligned).
// Rows past m read row 0 (their outputs are never stored). In the tail
// chunk, k past the slice end gives 0, which also cancels the clamped B rows.
template <class BT, int RB, bool AVEC, bool TAIL>
__device__ __forceinline__ void load_a(const float* A, int m, int k, int m0, int k0row, int ke,
                                       int j, int g, floatx4 (&a)[RB]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        int row = m0 + 16 * rb + j;
        row = row < m ? row : 0;
        const int kk = k0row + 4 * g;
        const float* src = A + static_cast<uint32_t>(row * k);
        if constexpr (AVEC && !TAIL) {
            a[rb] = *reinterpret_cast<const floatx4*>(src + kk);
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const bool ok = !TAIL || kk + u < ke;
                const float x = src[ok ? kk + u : k0row];
                a[rb][u] = ok ? x : 0.0f;
            }
        }
    }
}

template <class BT, int RB, bool AVEC>
__global__ __launch_bounds__(kThreads) void skinny_mfma_kernel(SkParams<BT> p) {
    constexpr bool kQ8 = std::is_same<BT, int8_t>::value;
    // Each wave's sums for one 16-row block, row-major by actual column.
    __shared__ __attribute__((aligned(16))) float tile[4 * 16 * kTileStride];

    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    // The wave index is uniform across the wave; saying so keeps every loop
    // test below a scalar branch.
    const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int g = lane >> 4, j = lane & 15;
    const int total = gridDim.x;
    const TileId place = tile_of(blockIdx.x, total, p.row_tiles, p.col_tiles, p.xcd_order != 0);
    const int c0 = place.col * kTile;
    const int m0 = place.row * 16 * RB;
    const int kb = place.slice * p.k_span;
    const int ke = min(p.k, kb + p.k_span);

    floatx4 acc[RB][16];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int t = 0; t < 16; ++t) acc[rb][t] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Row u + 1 of a chunk is widened while row u's MFMAs run. Each MFMA is
    // paired with one conversion for the next row and a scheduling barrier
    // pins that order: left to itself the scheduler puts every conversion
    // right before the MFMA that reads it, and each MFMA then waits on it
    // (measured 1.2x slower at m = 16).
    auto multiply = [&](const BChunk<BT>& bc, const floatx4 (&a)[RB]) {
        float bx[2][16];
        bc.widen(0, bx[0]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float next[16];
            if (u + 1 < 4) bc.widen(u + 1, next);
#pragma unroll
            for (int t = 0; t < 16; ++t) {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
                    acc[rb][t] = mfma16x16x4(a[rb][u], bx[u & 1][t], acc[rb][t]);
                if (u + 1 < 4) bx[(u + 1) & 1][t] = next[t];
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    constexpr int kStep = 4 * kChunk;  // the four waves' chunks
    int k0 = kb + kChunk * w;
    // The scheduling barrier keeps the compiler from sinking a prefetch
    // down to its use (which it does to lower register pressure).
    auto fetch = [&](BChunk<BT>& bc, floatx4 (&a)[RB], int at) {
        load_a<BT, RB, AVEC, false>(p.A, p.m, p.k, m0, at, ke, j, g, a);
        bc.template load<false>(p.B, p.n, at, ke, c0, j, g);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Full chunks of this wave are k0 + i * kStep for i < nfull, kept in a
    // ring of kDepth register sets: all kDepth are in flight before the
    // first multiply, and each multiply is followed by the load of the
    // chunk kDepth ahead into the set it frees. Past the last chunk the
    // ring re-reads it (a cache hit) rather than branch around a load, so
    // every multiply waits only for its own chunk's loads. Then at most
    // one partial chunk at the end of the slice.
    const int nfull = ke - k0 >= kChunk ? (ke - k0 - kChunk) / kStep + 1 : 0;
    auto at = [&](int i) { return k0 + (i < nfull ? i : nfull - 1) * kStep; };
    BChunk<BT> b[kDepth];
    floatx4 a[kDepth][RB];
    if (nfull > 0) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) fetch(b[d], a[d], at(d));
        for (int i = 0; i < nfull; i += kDepth) {
#pragma unroll
            for (int d = 0; d < kDepth; ++d) {
                if (i + d < nfull) multiply(b[d], a[d]);
                fetch(b[d], a[d], at(i + d + kDepth));
            }
        }
    }
    k0 += nfull * kStep;
    if (k0 < ke) {  // the slice's last, partial chunk
        load_a<BT, RB, AVEC, true>(p.A, p.m, p.k, m0, k0, ke, j, g, a[0]);
        b[0].template load<true>(p.B, p.n, k0, ke, c0, j, g);
        multiply(b[0], a[0]);
    }

    // Epilogue, one 16-row block at a time: every wave stores its sums in
    // LDS as a row-major 16 x 256 tile (by actual column), then each thread
    // takes 16 consecutive columns of one row, adds the four waves in wave
    // order and writes four float4: consecutive threads write consecutive
    // 64-byte runs. (Writing straight from the MFMA layout would scatter
    // 4-byte stores 64 bytes apart.)
    const int orow = tid / 16, ocol = (tid % 16) * 16;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        if (rb > 0) __syncthreads();  // the previous block's tile has been read
        float* mine = tile + w * 16 * kTileStride;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int c = BChunk<BT>::col(j, t);
#pragma unroll
            for (int r = 0; r < 4; ++r) mine[(4 * g + r) * kTileStride + c] = acc[rb][t][r];
        }
        __syncthreads();
        const int row = m0 + 16 * rb + orow;
        if (row < p.m) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int c = c0 + ocol + 4 * q;
                if (c >= p.n) break;
                floatx4 v = *reinterpret_cast<const floatx4*>(&tile[orow * kTileStride + ocol + 4 * q]);
#pragma unroll
                for (int ww = 1; ww < 4; ++ww)
                    v += *reinterpret_cast<const floatx4*>(
                        &tile[(ww * 16 + orow) * kTileStride + ocol + 4 * q]);
                if (p.direct) {
                    if constexpr (kQ8) v *= *reinterpret_cast<const floatx4*>(p.scale + c);
                    floatx4* o = reinterpret_cast<floatx4*>(p.out + static_cast<size_t>(row) * p.n + c);
                    *o = p.accumulate ? *o + v : v;
                } else {
                    *reinterpret_cast<floatx4*>(
                        p.out + (static_cast<size_t>(place.slice) * p.m + row) * p.n + c) = v;
                }
            }
        }
    }
}

template <class BT, int RB>
void launch(const SkParams<BT>& p, dim3 grid, bool avec, hipStream_t s) {
    if (avec) {
        hipLaunchKernelGGL((skinny_mfma_kernel<BT, RB, true>), grid, dim3(kThreads), 0, s, p);
    } else {
        hipLaunchKernelGGL((skinny_mfma_kernel<BT, RB, false>), grid, dim3(kThreads), 0, s, p);
    }
}

}  // namespace

template <class BT>
bool tiled_split_supports(const MatmulArgs& a) {
    const uintptr_t b = reinterpret_cast<uintptr_t>(a.B);
    if (std::is_same<BT, int8_t>::value) return a.n % 16 == 0 && b % 16 == 0;
    return a.n % 4 == 0 && b % 16 == 0;
}

template bool tiled_split_supports<float>(const MatmulArgs&);
template bool tiled_split_supports<int8_t>(const MatmulArgs&);

template <class BT>
void run_tiled_split(const MatmulArgs& a) {
    // Row tile: 16 or 32 rows, the smallest m fits in; larger m takes several
    // 32-row tiles (grid.z), each streaming B again (mostly from L2/MALL, as
    // the tiles of one column run at the same time). 64-row tiles would need
    // 256 accumulator registers and spill.
    const int RB = a.m <= 16 ? 1 : 2;
    const int row_tiles = ceil_div(a.m, 16 * RB);
    const int col_tiles = ceil_div(a.n, kTile);
    // Split k until the grid has up to one workgroup per CU, keeping every
    // slice at least 256 rows deep (four 16-row chunks per wave). More
    // slices measured slower: each adds m x n partials to write and re-read
    // (at m = 64, 16 slices move as many partial bytes as the int8 weights).
    // Rounding down keeps a grid just past the CU count from running a
    // second, mostly idle round (m = 96: 288 workgroups took 1.25x as long
    // as 240).
    const long long blocks = static_cast<long long>(row_tiles) * col_tiles;
    const int want = static_cast<int>(std::max(1LL, cu_count() / blocks));
    int slices = std::max(1, std::min(want, ceil_div(a.k, 256)));
    const int span = ceil_div(ceil_div(a.k, slices), 4 * kChunk) * 4 * kChunk;
    slices = ceil_div(a.k, span);

    SkParams<BT> p{};
    p.m = a.m;
    p.n = a.n;
    p.k = a.k;
    p.k_span = span;
    p.A = a.A;
    p.B = static_cast<const BT*>(a.B);
    p.scale = a.scale;
    p.direct = slices == 1;
    p.accumulate = a.accumulate && p.direct;
    p.out = p.direct ? a.C : scratch(kPartial, static_cast<size_t>(slices) * a.m * a.n);
    p.row_tiles = row_tiles;
    p.col_tiles = col_tiles;
    p.xcd_order = 1;
    const dim3 grid(col_tiles * slices * row_tiles);
    const bool avec = a.k % 4 == 0 && reinterpret_cast<uintptr_t>(a.A) % 16 == 0;
    if (RB == 1) {
        launch<BT, 1>(p, grid, avec, a.stream);
    } else {
        launch<BT, 2>(p, grid, avec, a.stream);
    }
    if (!p.direct)
        run_reduce_slices(a.m, a.n, slices, p.out,
                          std::is_same<BT, int8_t>::value ? a.scale : nullptr, a.C, a.accumulate,
                          a.stream);
}

template void run_tiled_split<float>(const MatmulArgs&);
template void run_tiled_split<int8_t>(const MatmulArgs&);

}  // namespace em
