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
// fp32 B with k % 32 == 0, n % 4 == 0 and 16-byte aligned operands takes
// gemm_fast_kernel instead (below): the same true-fp32 MFMAs, with buffer
// loads, k-packed A and untransposed B in LDS, and an explicit software
// pipeline.
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

// --- fp32 B with k % 32 == 0 and n % 4 == 0: the streamlined kernel --------
//
// Tiles of T x T (T = 32 WB: 64, or 128), four waves in 2 x 2, each wave
// WB x WB blocks of v_mfma_f32_16x16x4_f32. The
// per-step work is the MFMAs, the loads and the LDS traffic only:
//  * k advances 32 at a time (64 WB^2 MFMAs per wave between barriers);
//  * global loads are buffer loads from a descriptor whose base moves by a
//    scalar add per step; each thread's offsets are fixed, and rows past m or
//    columns past n get an offset past the descriptor's range, so the
//    hardware returns zeros there (no compare or select per load);
//  * A is stored k-packed in LDS, As[k / 4][row][4], each k/4 plane padded
//    by one 16-byte granule: a lane's four k values of one row are one
//    ds_read_b128, the 16 lanes of a group read 16 consecutive granules, and
//    the eight lanes storing the eight planes of one row hit distinct banks;
//  * B is stored as it is in memory, Bs[k][column] (rows padded by 4
//    floats), and lane j of a wave takes columns WB j .. WB j + WB - 1 of its
//    half, one per column block: one ds_read of WB floats per k row feeds
//    all WB column blocks, B goes to LDS without a transpose, and each lane
//    ends with WB consecutive columns of every row to store;
//  * each 16-deep group's MFMAs run while the next group's operands load;
//    before the last group the next step's slab goes to the other LDS stage,
//    and the barrier comes kTail MFMAs before the end of the step, so the
//    next step's first operands load under those last MFMAs. Both stages'
//    addresses are immediates (the loop is unrolled over the two stages);
//  * the tile order keeps each XCD on a compact block of tiles: XCD x takes
//    the x-th eighth of the tile sequence, which walks 8 row bands per
//    column, so the tiles an XCD holds at once share their A rows and B
//    columns in its L2.
constexpr int FK = 32;             // k per step
constexpr int kGroupRows = 8;      // row bands walked per column
constexpr uint32_t kOutOfRange = 0x80000000u;  // a buffer offset past the descriptor
// s_waitcnt immediate with lgkmcnt 0 and vmcnt / expcnt at their maxima (no
// wait on those): vmcnt[3:0] = 15, expcnt[6:4] = 7, lgkmcnt[11:8] = 0,
// vmcnt[15:14] = 3.
constexpr int kLgkmZero = 0xC07F;

struct FastParams {
    int m, n, k;
    int k_span;        // k per slice, a multiple of FK
    int tiles_m, tiles_n, slices;
    const float* A;
    const float* B;
    float* out;        // C, or partials [slice][m][n]
    int accumulate;
    int split;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t fp32_rsrc(const float* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, 0x7fffffff, 0x00020000);
}

__device__ __forceinline__ floatx4 buffer_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

template <int W>
struct FloatVec;
template <>
struct FloatVec<4> {
    typedef float type __attribute__((ext_vector_type(4)));
};
template <>
struct FloatVec<2> {
    typedef float type __attribute__((ext_vector_type(2)));
};

template <int WB, int OCC>
__global__ __launch_bounds__(kThreads, OCC) void gemm_fast_kernel(FastParams p) {
    typedef typename FloatVec<WB>::type bvec;
    constexpr int T = 32 * WB;            // tile side
    constexpr int PL = FK / 4;            // k/4 planes of an A stage
    constexpr int kPlane = T * 4 + 4;     // floats of one plane
    constexpr int kAStage = PL * kPlane;  // floats of one A stage
    constexpr int kBRow = T + 4;          // floats of one k row of a B stage
    constexpr int kBStage = FK * kBRow;   // floats of one B stage
    constexpr int RA = kThreads / PL;     // A rows per load pass (32)
    constexpr int NA = T / RA;            // A loads per thread
    constexpr int C4 = T / 4;             // float4s per B row
    constexpr int RB = kThreads / C4;     // B rows per load pass
    constexpr int NB = FK / RB;           // B loads per thread
    __shared__ __attribute__((aligned(16))) float As[2 * kAStage];
    __shared__ __attribute__((aligned(16))) float Bs[2 * kBStage];

    const int tid = threadIdx.x;
    const int lane = tid % kWave, wave = tid / kWave;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, j = lane & 15;

    // Tile order: XCD-compact (see above) when the grid divides by 8.
    const int tiles = p.tiles_m * p.tiles_n;
    const int total = tiles * p.slices;
    int id = blockIdx.x;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
    const int slice = id / tiles;
    int t = id - slice * tiles;
    const int band = t / (kGroupRows * p.tiles_n);
    const int first = band * kGroupRows;
    const int rows_here = min(kGroupRows, p.tiles_m - first);
    t -= band * kGroupRows * p.tiles_n;
    const int m0 = (first + t % rows_here) * T;
    const int n0 = (t / rows_here) * T;
    const int kb = slice * p.k_span;
    const int steps = (min(p.k, kb + p.k_span) - kb) / FK;

    // Loads: thread tid takes plane q = tid % PL of A rows tid / PL + RA i
    // (four k values each), and columns 4 (tid % C4) .. + 3 of B rows
    // tid / C4 + RB i.
    const int q = tid % PL, a_row = tid / PL;
    const int b_row = tid / C4, b_col = (tid % C4) * 4;
    uint32_t a_off[NA], b_off[NB];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int row = a_row + RA * i;
        a_off[i] = m0 + row < p.m ? static_cast<uint32_t>((row * p.k + 4 * q) * 4) : kOutOfRange;
    }
#pragma unroll
    for (int i = 0; i < NB; ++i)
        b_off[i] = n0 + b_col < p.n ? static_cast<uint32_t>(((b_row + RB * i) * p.n + b_col) * 4)
                                    : kOutOfRange;
    const float* a_base = p.A + static_cast<size_t>(m0) * p.k + kb;
    const float* b_base = p.B + static_cast<size_t>(kb) * p.n + n0;

    floatx4 ra[NA], rb[NB];
    auto fetch = [&](int step) {
        const __amdgpu_buffer_rsrc_t sa = fp32_rsrc(a_base + step * FK);
        const __amdgpu_buffer_rsrc_t sb = fp32_rsrc(b_base + static_cast<size_t>(step) * FK * p.n);
#pragma unroll
        for (int i = 0; i < NA; ++i) ra[i] = buffer_load4(sa, a_off[i]);
#pragma unroll
        for (int i = 0; i < NB; ++i) rb[i] = buffer_load4(sb, b_off[i]);
    };
    const int a_st = q * kPlane + a_row * 4;
    const int b_st = b_row * kBRow + b_col;
    auto stash = [&](float* as, float* bs) {
#pragma unroll
        for (int i = 0; i < NA; ++i)
            *reinterpret_cast<floatx4*>(as + a_st + RA * 4 * i) = ra[i];
#pragma unroll
        for (int i = 0; i < NB; ++i)
            *reinterpret_cast<floatx4*>(bs + b_st + RB * i * kBRow) = rb[i];
    };
    // Reads: lane (g, j) takes plane 4h + g of A row wm T/2 + 16 mi + j, and
    // B row 16h + 4g + s at columns wn T/2 + WB j .. + WB - 1.
    const int a_rd = g * kPlane + (wm * (T / 2) + j) * 4;
    const int b_rd = 4 * g * kBRow + wn * (T / 2) + WB * j;

    floatx4 acc[WB][WB];
#pragma unroll
    for (int mi = 0; mi < WB; ++mi)
#pragma unroll
        for (int ni = 0; ni < WB; ++ni) acc[mi][ni] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Operand registers of one 16-deep group: a[mi] holds k 4g .. 4g + 3 of
    // the lane's A row in block mi (MFMA s takes element s); b[s] holds k row
    // 4g + s of the lane's WB B columns (column block ni takes element ni).
    struct Ops {
        floatx4 a[WB];
        bvec b[4];
    };
    Ops op[2];
    auto read = [&](Ops& o, const float* as, const float* bs, int h) {
#pragma unroll
        for (int mi = 0; mi < WB; ++mi)
            o.a[mi] = *reinterpret_cast<const floatx4*>(as + a_rd + 4 * h * kPlane + mi * 64);
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
            o.b[s4] = *reinterpret_cast<const bvec*>(bs + b_rd + (16 * h + s4) * kBRow);
    };
    // MFMAs lo .. hi - 1 of a group's 4 WB^2, in the order s, mi, ni (WB^2
    // independent accumulators between two updates of one).
    constexpr int kGroup = 4 * WB * WB;
    auto mma = [&](const Ops& o, int lo, int hi) {
#pragma unroll
        for (int x = 0; x < kGroup; ++x) {
            if (x < lo || x >= hi) continue;
            const int s4 = x / (WB * WB), mi = (x / WB) % WB, ni = x % WB;
            acc[mi][ni] = mfma16x16x4(o.a[mi][s4], o.b[s4][ni], acc[mi][ni]);
        }
    };
    constexpr int H = FK / 16;
    constexpr int kTail = kGroup / 8;
    // The compiler's scheduler would move loads next to their first use;
    // these fences keep each phase where it is written.
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
    // One k step out of stage (as, bs); op[0] already holds its first group.
    auto step = [&](auto more_c, const float* as, const float* bs, float* as_n, float* bs_n) {
        constexpr bool more = decltype(more_c)::value;
#pragma unroll
        for (int h = 0; h < H; ++h) {
            Ops& cur = op[h & 1];
            if (h + 1 < H) {
                read(op[(h + 1) & 1], as, bs, h + 1);
                fence();
                mma(cur, 0, kGroup);
                fence();
            } else {
                if constexpr (more) stash(as_n, bs_n);
                fence();
                mma(cur, 0, kGroup - kTail);
                fence();
                __syncthreads();
                fence();
                if constexpr (more) read(op[0], as_n, bs_n, 0);
                fence();
                mma(cur, kGroup - kTail, kGroup);
                fence();
                // The next group's operands have had kTail MFMAs to arrive;
                // waiting here leaves no LDS read pending across the loop's
                // back edge, where the wait-count pass would wait for all.
                __builtin_amdgcn_s_waitcnt(kLgkmZero);
                fence();
            }
        }
    };
    using Yes = std::integral_constant<bool, true>;
    using No = std::integral_constant<bool, false>;

    if (steps > 0) {
        fetch(0);
        stash(As, Bs);
    }
    __syncthreads();
    if (steps > 0) read(op[0], As, Bs, 0);
    __builtin_amdgcn_s_waitcnt(kLgkmZero);
    // Pairs of steps, one per LDS stage; the last one or two are peeled.
    int ks = 0;
    for (; ks + 2 < steps; ks += 2) {
        fetch(ks + 1);
        fence();
        step(Yes{}, As, Bs, As + kAStage, Bs + kBStage);
        fetch(ks + 2);
        fence();
        step(Yes{}, As + kAStage, Bs + kBStage, As, Bs);
    }
    if (ks + 1 < steps) {
        fetch(ks + 1);
        fence();
        step(Yes{}, As, Bs, As + kAStage, Bs + kBStage);
        step(No{}, As + kAStage, Bs + kBStage, As, Bs);
    } else if (ks < steps) {
        step(No{}, As, Bs, As + kAStage, Bs + kBStage);
    }

    // acc[mi][ni][r] is C[row 4g + r][column WB j + ni] of the wave's 16-row
    // block mi: each lane holds WB consecutive columns of each row.
    float* out = p.split ? p.out + static_cast<size_t>(slice) * p.m * p.n : p.out;
    const int col = n0 + wn * (T / 2) + WB * j;
    if (col < p.n) {
#pragma unroll
        for (int mi = 0; mi < WB; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm * (T / 2) + mi * 16 + 4 * g + r;
                if (row >= p.m) continue;
                bvec v;
#pragma unroll
                for (int ni = 0; ni < WB; ++ni) v[ni] = acc[mi][ni][r];
                bvec* o = reinterpret_cast<bvec*>(out + static_cast<size_t>(row) * p.n + col);
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

// The streamlined kernel's conditions: fp32 B, whole 32-deep k steps, rows of
// whole float4s, 16-byte aligned operands, and per-tile offsets within the
// buffer descriptors' 31-bit range.
bool fast_ok(const MatmulArgs& a) {
    return a.k % FK == 0 && a.n % 4 == 0 &&
           reinterpret_cast<uintptr_t>(a.A) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(a.B) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(a.C) % 16 == 0 &&
           static_cast<long long>(128) * a.k < (1LL << 29) &&
           static_cast<long long>(FK) * a.n < (1LL << 29);
}

template <int WB>
void launch_fast(const MatmulArgs& a, int per_cu) {
    constexpr int T = 32 * WB;
    const int tiles_n = ceil_div(a.n, T), tiles_m = ceil_div(a.m, T);
    const long long tiles = static_cast<long long>(tiles_n) * tiles_m;
    int slices = 1;
    const long long target = static_cast<long long>(per_cu) * cu_count();
    if (tiles < target) {
        const int want = ceil_div(target, tiles);
        slices = std::max(1, std::min(want, a.k / 256));
    }
    const int span = ceil_div(ceil_div(a.k, slices), FK) * FK;
    slices = ceil_div(a.k, span);

    FastParams p{};
    p.m = a.m;
    p.n = a.n;
    p.k = a.k;
    p.k_span = span;
    p.tiles_m = tiles_m;
    p.tiles_n = tiles_n;
    p.slices = slices;
    p.A = a.A;
    p.B = static_cast<const float*>(a.B);
    p.split = slices > 1;
    p.accumulate = a.accumulate ? 1 : 0;
    p.out = p.split ? scratch(kPartial, static_cast<size_t>(slices) * a.m * a.n) : a.C;
    hipLaunchKernelGGL((gemm_fast_kernel<WB, 2>), dim3(static_cast<unsigned>(tiles * slices)),
                       dim3(kThreads), 0, a.stream, p);
    if (p.split) run_reduce_slices(a.m, a.n, slices, p.out, nullptr, a.C, a.accumulate, a.stream);
}

// 64 x 64 tiles by default: at 97 registers and 34 KB of LDS four
// workgroups share a CU and cover each other's barriers and loads, which
// measured faster than 128 x 128 tiles at every size tried (fp32 N = 1024 /
// 2048 / 4096: 97.6 / 133.1 / 143.9 against 66.9 / 123.7 / 142.9 TFLOP/s).
// k is split until the grid holds one workgroup per CU.
void run_fast(const MatmulArgs& a) { launch_fast<2>(a, 1); }

bool tiled_preferred(const MatmulArgs& a) {
    if (a.m <= 8 || !fast_ok(a)) return false;
    const long long kn = static_cast<long long>(a.k) * a.n;
    return a.m >= 1024 || kn <= (1LL << 20) || (a.m >= 256 && a.n >= 2 * a.k);
}

template <class BT>
void run_tiled(const MatmulArgs& a) {
    if (std::is_same<BT, float>::value && fast_ok(a)) {
        run_fast(a);
        return;
    }
    const int tiles_n = ceil_div(a.n, BN), tiles_m = ceil_div(a.m, BM);
    const long long tiles = static_cast<long long>(tiles_n) * tiles_m;
    // Split k when the tile grid gives fewer than two workgroups per CU and
    // k is deep enough for each slice to keep 256+ rows (two per CU measured
    // 1.2-1.3x faster than one on the Llama-7B m = 512 projections, and four
    // no better).
    constexpr int per_cu = 2;
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
