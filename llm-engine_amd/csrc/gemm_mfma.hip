// Prefill-shaped and square products: GpuKernel::tiled (reference
// sgemm_tiled<128,8> + run_tiled, /root/reference/src/cuda_matmul.cu:49-125,
// 333-348), rebuilt around CDNA4's fp32 matrix cores.
//
//  * A workgroup (four wave64s) computes a 128 x 128 tile of C, each wave a
//    64 x 64 quadrant as 4 x 4 blocks of v_mfma_f32_16x16x4_f32. gfx950 has
//    no xf32, and bf16/tf32 inputs would miss the 1e-4 * sum|a||b| bound, so
//    the contraction is true fp32.
//  * k advances 16 at a time. The next 128 x 16 slab of A and 16 x 128 slab
//    of B are fetched into registers while the current slab is multiplied
//    out of LDS, then written to the other half of a double buffer: one
//    barrier per step.
//  * LDS layout. A is kept row-major with rows padded to 20 floats: in MFMA
//    step s of a 16-deep slab, lane l (group g = l / 16) supplies
//    A[row l % 16][4g + s], so one ds_read_b128 per 16-row block feeds all
//    four steps. B is kept k-major with rows padded to 132 floats, so the
//    four lane groups of a ds_read_b32 land on disjoint banks. The k order
//    inside a slab (4g + s) is the same for A and B, so the sum is exact.
//  * int8 B is widened and multiplied by its column scale on the way into
//    LDS, exactly as the reference's pack_b dequantises (matmul.cpp:73-90),
//    so the MFMAs only see fp32.
//  * With split, blockIdx.z takes one k slice and writes partials; the
//    caller adds them in slice order.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int AST = BK + 4;   // A row stride in LDS (floats)
constexpr int BST = BN + 4;   // B row stride in LDS (floats)

template <class BT>
struct TiledParams {
    int m, n, k;
    int k_span;  // rows of k per z slice, a multiple of BK
    const float* A;
    const BT* B;
    const float* scale;
    float* out;  // C, or partials [slice][m][n] when split
    int accumulate;
    int split;
};

// VEC: k % 4 == 0, n % 4 == 0 and both operands aligned for 16-byte (fp32 B)
// or 4-byte (int8 B) vector loads. Otherwise every element is loaded alone.
// Four workgroups per CU (at most 128 registers): the 1024 tiles of an
// N = 4096 product are then all resident at once, with no tail wave.
template <class BT, bool VEC>
__global__ __launch_bounds__(kThreads, 4) void gemm_tiled_kernel(TiledParams<BT> p) {
    constexpr bool kQ8 = std::is_same<BT, int8_t>::value;
    __shared__ __attribute__((aligned(16))) float As[2][BM * AST];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * BST];

    const int tid = threadIdx.x;
    const int lane = tid % kWave, wave = tid / kWave;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, j = lane & 15;

    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kb = blockIdx.z * p.k_span;
    const int ke = min(p.k, kb + p.k_span);
    const int steps = (ke - kb + BK - 1) / BK;

    // Global -> register roles: two float4 of A and two 4-column pieces of B
    // per thread. A: row f / 4, k offset 4 (f % 4). B: row f / 32, column 4 (f % 32).
    int a_row[2], a_kq[2], b_row[2], b_cq[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int f = tid + h * kThreads;
        a_row[h] = f >> 2;
        a_kq[h] = (f & 3) * 4;
        b_row[h] = f >> 5;
        b_cq[h] = (f & 31) * 4;
    }

    floatx4 ra[2], rb[2];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int gr = m0 + a_row[h], gk = k0 + a_kq[h];
            if constexpr (VEC) {
                ra[h] = (gr < p.m && gk < ke)
                            ? *reinterpret_cast<const floatx4*>(p.A + static_cast<size_t>(gr) * p.k + gk)
                            : floatx4{0.f, 0.f, 0.f, 0.f};
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    ra[h][e] = (gr < p.m && gk + e < ke) ? p.A[static_cast<size_t>(gr) * p.k + gk + e]
                                                         : 0.0f;
            }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int gk = k0 + b_row[h], gc = n0 + b_cq[h];
            const bool row_ok = gk < ke;
            if constexpr (VEC) {
                const bool ok = row_ok && gc < p.n;
                if constexpr (kQ8) {
                    // Column scales are re-read per slab (an L1 hit) rather than
                    // held in registers, to stay within 128 registers.
                    const uint32_t w =
                        ok ? *reinterpret_cast<const uint32_t*>(p.B + static_cast<size_t>(gk) * p.n + gc)
                           : 0u;
                    const floatx4 sc = gc < p.n ? *reinterpret_cast<const floatx4*>(p.scale + gc)
                                                : floatx4{0.f, 0.f, 0.f, 0.f};
                    float v[4];
                    widen4(w, v);
#pragma unroll
                    for (int e = 0; e < 4; ++e) rb[h][e] = v[e] * sc[e];
                } else {
                    rb[h] = ok ? *reinterpret_cast<const floatx4*>(p.B + static_cast<size_t>(gk) * p.n + gc)
                               : floatx4{0.f, 0.f, 0.f, 0.f};
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool ok = row_ok && gc + e < p.n;
                    const size_t idx = static_cast<size_t>(gk) * p.n + gc + e;
                    if constexpr (kQ8) {
                        rb[h][e] = ok ? static_cast<float>(p.B[idx]) * p.scale[gc + e] : 0.0f;
                    } else {
                        rb[h][e] = ok ? p.B[idx] : 0.0f;
                    }
                }
            }
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            *reinterpret_cast<floatx4*>(&As[buf][a_row[h] * AST + a_kq[h]]) = ra[h];
            *reinterpret_cast<floatx4*>(&Bs[buf][b_row[h] * BST + b_cq[h]]) = rb[h];
        }
    };

    floatx4 acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = floatx4{0.f, 0.f, 0.f, 0.f};

    if (steps > 0) {
        fetch(kb);
        stash(0);
    }
    __syncthreads();
    for (int t = 0; t < steps; ++t) {
        const int cur = t & 1;
        if (t + 1 < steps) fetch(kb + (t + 1) * BK);
        const float* as = As[cur];
        const float* bs = Bs[cur];
        floatx4 a4[4];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
            a4[mi] = *reinterpret_cast<const floatx4*>(&as[(wm * 64 + mi * 16 + j) * AST + 4 * g]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            float b[4];
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) b[ni] = bs[(4 * g + s) * BST + wn * 64 + ni * 16 + j];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma16x16x4(a4[mi][s], b[ni], acc[mi][ni]);
        }
        if (t + 1 < steps) stash(cur ^ 1);
        __syncthreads();
    }

    // acc[mi][ni][r] is C[row 4g + r][col j] of block (mi, ni).
    float* out = p.split ? p.out + static_cast<size_t>(blockIdx.z) * p.m * p.n : p.out;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = m0 + wm * 64 + mi * 16 + 4 * g + r;
            if (row >= p.m) continue;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const int col = n0 + wn * 64 + ni * 16 + j;
                if (col >= p.n) continue;
                float* o = out + static_cast<size_t>(row) * p.n + col;
                const float v = acc[mi][ni][r];
                *o = (!p.split && p.accumulate) ? *o + v : v;
            }
        }
}

bool vec_ok(const MatmulArgs& a, size_t b_align) {
    return a.k % 4 == 0 && a.n % 4 == 0 && reinterpret_cast<uintptr_t>(a.A) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(a.B) % b_align == 0 &&
           (a.scale == nullptr || reinterpret_cast<uintptr_t>(a.scale) % 16 == 0);
}

}  // namespace

template <class BT>
void run_tiled(const MatmulArgs& a) {
    const int tiles_n = ceil_div(a.n, BN), tiles_m = ceil_div(a.m, BM);
    const long long tiles = static_cast<long long>(tiles_n) * tiles_m;
    // Split k when the tile grid gives fewer than two workgroups per CU and
    // k is deep enough for each slice to keep 256+ rows (two per CU measured
    // 1.2-1.3x faster than one on the Llama-7B m = 512 projections, and four
    // no better). EM_TILED_BLOCKS_PER_CU overrides the target (tuning sweeps).
    static const int per_cu = [] {
        const char* v = std::getenv("EM_TILED_BLOCKS_PER_CU");
        const int x = v ? std::atoi(v) : 0;
        return x > 0 ? x : 2;
    }();
    int slices = 1;
    const long long target = static_cast<long long>(per_cu) * cu_count();
    if (tiles < target) {
        const int want = ceil_div(target, tiles);
        slices = std::max(1, std::min(want, a.k / 256));
    }
    const int span = ceil_div(ceil_div(a.k, slices), BK) * BK;
    slices = ceil_div(a.k, span);

    TiledParams<BT> p{};
    p.m = a.m;
    p.n = a.n;
    p.k = a.k;
    p.k_span = span;
    p.A = a.A;
    p.B = static_cast<const BT*>(a.B);
    p.scale = a.scale;
    p.split = slices > 1;
    p.accumulate = a.accumulate ? 1 : 0;
    p.out = p.split ? scratch(kPartial, static_cast<size_t>(slices) * a.m * a.n) : a.C;
    const dim3 grid(tiles_n, tiles_m, slices);
    const bool vec = vec_ok(a, std::is_same<BT, int8_t>::value ? 4 : 16);
    if (vec) {
        hipLaunchKernelGGL((gemm_tiled_kernel<BT, true>), grid, dim3(kThreads), 0, a.stream, p);
    } else {
        hipLaunchKernelGGL((gemm_tiled_kernel<BT, false>), grid, dim3(kThreads), 0, a.stream, p);
    }
    if (p.split) run_reduce_slices(a.m, a.n, slices, p.out, nullptr, a.C, a.accumulate, a.stream);
}

template void run_tiled<float>(const MatmulArgs&);
template void run_tiled<int8_t>(const MatmulArgs&);

}  // namespace em
