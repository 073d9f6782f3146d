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
#include <type_traits>

#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

constexpr int kTile = 256;   // columns per workgroup
constexpr int kChunk = 16;   // k rows per wave step

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
};

// One chunk's B operands for one lane: four rows (u), 16 columns each.
template <class BT>
struct BChunk;

template <>
struct BChunk<int8_t> {
    uint4 v[4];
    // Column of C (relative to the tile) that MFMA t reads in lane column j.
    static __device__ __forceinline__ int col(int j, int t) { return 16 * j + t; }
    __device__ __forceinline__ void load(const int8_t* B, int n, int k0row, int ke, int c0, int j,
                                         int g) {
        const int c = c0 + 16 * j;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = k0row + 4 * g + u;
            v[u] = (r < ke && c < n)
                       ? *reinterpret_cast<const uint4*>(B + static_cast<size_t>(r) * n + c)
                       : make_uint4(0, 0, 0, 0);
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
    __device__ __forceinline__ void load(const float* B, int n, int k0row, int ke, int c0, int j,
                                         int g) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = k0row + 4 * g + u;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int c = c0 + 64 * q + 4 * j;
                v[u][q] = (r < ke && c < n)
                              ? *reinterpret_cast<const float4*>(B + static_cast<size_t>(r) * n + c)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
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

// AVEC: k % 4 == 0 and A 16-byte aligned, so a lane's four A values of a
// chunk are one float4.
template <class BT, int RB, bool AVEC>
__device__ __forceinline__ void load_a(const float* A, int m, int k, int m0, int k0row, int j,
                                       int g, floatx4 (&a)[RB]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int row = m0 + 16 * rb + j;
        const int kk = k0row + 4 * g;
        if constexpr (AVEC) {
            a[rb] = (row < m && kk < k)
                        ? *reinterpret_cast<const floatx4*>(A + static_cast<size_t>(row) * k + kk)
                        : floatx4{0.f, 0.f, 0.f, 0.f};
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                a[rb][u] = (row < m && kk + u < k) ? A[static_cast<size_t>(row) * k + kk + u] : 0.0f;
        }
    }
}

template <class BT, int RB, bool AVEC>
__global__ __launch_bounds__(kThreads) void skinny_mfma_kernel(SkParams<BT> p) {
    constexpr bool kQ8 = std::is_same<BT, int8_t>::value;
    // Waves 1..3 leave one row block's sums here: [wave-1][t][r][lane].
    __shared__ float red[3 * 16 * 4 * kWave];

    const int tid = threadIdx.x;
    const int lane = tid % kWave, w = tid / kWave;
    const int g = lane >> 4, j = lane & 15;
    const int c0 = blockIdx.x * kTile;
    const int m0 = blockIdx.z * 16 * RB;
    const int kb = blockIdx.y * p.k_span;
    const int ke = min(p.k, kb + p.k_span);

    floatx4 acc[RB][16];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int t = 0; t < 16; ++t) acc[rb][t] = floatx4{0.f, 0.f, 0.f, 0.f};

    int k0 = kb + kChunk * w;
    BChunk<BT> bc;
    floatx4 a[RB];
    if (k0 < ke) {
        bc.load(p.B, p.n, k0, ke, c0, j, g);
        load_a<BT, RB, AVEC>(p.A, p.m, p.k, m0, k0, j, g, a);
    }
    for (; k0 < ke; k0 += 4 * kChunk) {
        BChunk<BT> bn;
        floatx4 an[RB];
        const int k1 = k0 + 4 * kChunk;
        if (k1 < ke) {
            bn.load(p.B, p.n, k1, ke, c0, j, g);
            load_a<BT, RB, AVEC>(p.A, p.m, p.k, m0, k1, j, g, an);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float b[16];
            bc.widen(u, b);
#pragma unroll
            for (int t = 0; t < 16; ++t)
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) acc[rb][t] = mfma16x16x4(a[rb][u], b[t], acc[rb][t]);
        }
        bc = bn;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) a[rb] = an[rb];
    }

    // Wave sums, added in wave order: acc(0) + acc(1) + acc(2) + acc(3).
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        if (w > 0) {
#pragma unroll
            for (int t = 0; t < 16; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) red[(((w - 1) * 16 + t) * 4 + r) * kWave + lane] = acc[rb][t][r];
        }
        __syncthreads();
        if (w == 0) {
#pragma unroll
            for (int ww = 0; ww < 3; ++ww)
#pragma unroll
                for (int t = 0; t < 16; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[rb][t][r] += red[((ww * 16 + t) * 4 + r) * kWave + lane];
        }
        __syncthreads();
    }
    if (w != 0) return;

    // Lane (g, j) holds rows m0 + 16 rb + 4g + r and columns c0 + col(j, t).
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        const int c = c0 + BChunk<BT>::col(j, t);
        if (c >= p.n) continue;
        float s = 1.0f;
        if constexpr (kQ8) {
            if (p.direct) s = p.scale[c];
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + 16 * rb + 4 * g + r;
                if (row >= p.m) continue;
                const float v = acc[rb][t][r] * s;
                if (p.direct) {
                    float* o = p.out + static_cast<size_t>(row) * p.n + c;
                    *o = p.accumulate ? *o + v : v;
                } else {
                    p.out[(static_cast<size_t>(blockIdx.y) * p.m + row) * p.n + c] = v;
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
    // Split k until the grid has about two workgroups per CU, keeping every
    // slice at least 256 rows deep (four 16-row chunks per wave).
    const long long blocks = static_cast<long long>(row_tiles) * col_tiles;
    const int want = std::max(1, ceil_div(2LL * cu_count(), blocks));
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
    const dim3 grid(col_tiles, slices, row_tiles);
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
