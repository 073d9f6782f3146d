// Decode-batch products (2 .. 8 rows of A) over int8 weights in the strip
// layout (gemv_packed.hip), one launch, on fp32 MFMA: the counterpart of the
// reference's skinny GEMV plus sum_slices (cuda_matmul.cu:189-254, 365-397)
// for a few rows, reading the library's strip copy of B instead of the
// row-major matrix.
//
// Why MFMA. A GEMV lane that widens 16 weights and multiplies them into m
// rows issues 1 + m VALU ops per weight byte: 2.1 us per SIMD at m = 4 over
// 4096^2 and 3.8 us at m = 8, more than the ~2.4 us the weights take to
// stream. v_mfma_f32_4x4x1_16b_f32 multiplies 64 weights (one per lane) into
// four rows of A in 8 cycles, so the same work costs one conversion per
// weight plus one MFMA per four rows.
//
// The instruction computes 16 independent 4x4 blocks: lane 4b + i supplies
// row i of block b's A column, lane 4b + j column j of block b's B row, and
// lane 4b + j receives D_b[i][j] in register i (checked on the device).
// Block b is one k row, so a block's four lanes must hold the same rows of
// B, which is what the strip layout's quads give:
//  * lane 4b + c of wave w loads unit c of quad Q = 16 (round * waves + w) +
//    b: rows 4Q .. 4Q + 3, columns 4c .. 4c + 3 of the strip. A wave's load
//    is 1 KiB of consecutive units;
//  * MFMA (t, u) takes row 4Q + t, byte u: column 4c + u goes to
//    accumulator u, and lane 4b + i supplies A[4g + i][4Q + t] for row group
//    g (one float4 of A per quad and group);
//  * each lane's accumulators hold its quads' share of each output; the sum
//    over a wave's 16 quads is lane_reduce16, the sum over waves goes
//    through LDS in wave order, so repeated calls give the same bits.
//
// A is staged in LDS once per workgroup in the lanes' order ([group][quad]
// [c][4]: a wave's read is 1 KiB contiguous), zero past k and m, so the
// padding quads (their weight loads clamped to the last quad) add zeros; a
// fused norm weight is staged beside it and multiplied in as A is read. Its loads are issued before the
// weights: loads complete in issue order, and the staging must not wait for
// the weight stream. The row's RMS scale multiplies each output once, from
// the sums of squares formed while staging.
#include <algorithm>
#include <cstdlib>

#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

constexpr int kStrip = 16;     // columns per strip
constexpr int kDecodeMaxQuads = 1024;  // k <= 4096

struct DecodeParams {
    int m, n, k;
    int k4;      // quads of the strip (k / 4)
    int k4p;     // quads covered: rounds x 16 x waves
    int rounds;  // 16-byte loads per lane (a power of two, padded)
    const float* A;
    const float* rms_weight;
    const int8_t* P;  // strip layout
    const float* scale;
    float* C;
    int accumulate;
};

typedef float f4v __attribute__((ext_vector_type(4)));

// NT threads, G groups of four rows of A; R rounds of loads (k4p = R x 16
// x waves quads), LB of them in flight; EXACT: k4 == k4p (no padding quads
// to zero).
template <int NT, int G, int R, int LB, bool NORM, bool EXACT>
__global__ __launch_bounds__(NT) void decode_mfma_kernel(DecodeParams p) {
    constexpr int NW = NT / kWave;
    constexpr int NV = 16 * G;                  // accumulator values per lane
    constexpr int K4P = R * 16 * NW;            // quads covered (p.k4p)
    constexpr int QB = (K4P + NT - 1) / NT;     // norm-weight quads per thread
    __shared__ float red[NW][4 * G][kStrip];
    __shared__ float ssq[NW][4 * G];
    extern __shared__ float4 wq[];  // [K4P] norm weights (NORM only)
    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int b = lane >> 2, c = lane & 3;
    const int strip = blockIdx.x;
    const uint4* base = reinterpret_cast<const uint4*>(p.P + static_cast<size_t>(strip) * p.k * kStrip);

    // Norm weights first (staged in LDS; loads complete in issue order, so
    // they must not queue behind the weight stream).
    if constexpr (NORM) {
        float4 wn[QB];
#pragma unroll
        for (int q = 0; q < QB; ++q) {
            const float* w = p.rms_weight + 4 * min(q * NT + tid, p.k4 - 1);
            wn[q] = make_float4(w[0], w[1], w[2], w[3]);
        }
#pragma unroll
        for (int q = 0; q < QB; ++q) {
            const int Q = q * NT + tid;
            if (Q < K4P) wq[Q] = Q < p.k4 ? wn[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __syncthreads();
    }

    // Round i: lane 4b + c loads unit c of quad Q (16 bytes of weights) and,
    // per group g, A[4g + c][4Q .. 4Q + 3] straight from A (rows past m read
    // row m - 1: their outputs are never stored). Issued in round order, LB
    // rounds ahead, so waiting for round i waits for nothing later.
    const int arow[G > 1 ? G : 1] = {};
    uint4 wt[R];
    float4 av[R][G];
    // Workgroups start at different rounds (strip mod R) and wrap around, so
    // the 32 workgroups of an XCD do not all read the same lines of A at the
    // same time; each output's order is still fixed.
    const int rot = strip & (R - 1);
    auto quad = [&](int i) { return (((i + rot) & (R - 1)) * NW + wave) * 16 + b; };
    auto issue = [&](int i) {
        const int Q = quad(i);
        const int Qc = EXACT ? Q : min(Q, p.k4 - 1);
        wt[i] = stream_load(base + 4 * Qc + c);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int row = min(4 * g + c, p.m - 1);
            av[i][g] = *reinterpret_cast<const float4*>(p.A + static_cast<size_t>(row) * p.k + 4 * Qc);
        }
    };
    (void)arow;
#pragma unroll
    for (int i = 0; i < (LB < R ? LB : R); ++i) issue(i);
    __builtin_amdgcn_sched_barrier(0);
    // The epilogue's scale and prior C, behind the first loads.
    const int er = tid / kStrip, ej = tid % kStrip, ec = strip * kStrip + ej;
    const bool eout = tid < 4 * G * kStrip && er < p.m;
    const float esc = p.scale[ec];
    const float eprior = p.accumulate ? p.C[static_cast<size_t>(min(er, p.m - 1)) * p.n + ec] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);

    f4v acc[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[g][u] = f4v{0.f, 0.f, 0.f, 0.f};
    float ss[G];  // sums of squares of this lane's A values, row 4g + c
#pragma unroll
    for (int g = 0; g < G; ++g) ss[g] = 0.0f;

#pragma unroll
    for (int i = 0; i < R; ++i) {
        if (i + LB < R) issue(i + LB);
        const int Q = quad(i);
        float4 a4[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            a4[g] = av[i][g];
            if (!EXACT && Q >= p.k4) a4[g] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if constexpr (NORM) {
            const float4 w4 = wq[Q];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                ss[g] = fmaf(a4[g].x, a4[g].x, ss[g]);
                ss[g] = fmaf(a4[g].y, a4[g].y, ss[g]);
                ss[g] = fmaf(a4[g].z, a4[g].z, ss[g]);
                ss[g] = fmaf(a4[g].w, a4[g].w, ss[g]);
                a4[g].x *= w4.x;
                a4[g].y *= w4.y;
                a4[g].z *= w4.z;
                a4[g].w *= w4.w;
            }
        }
        float bv[4][4];  // [row t of the quad][column 4c + u]
        widen4(wt[i].x, bv[0]);
        widen4(wt[i].y, bv[1]);
        widen4(wt[i].z, bv[2]);
        widen4(wt[i].w, bv[3]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float a = t == 0 ? a4[g].x : t == 1 ? a4[g].y : t == 2 ? a4[g].z : a4[g].w;
                    acc[g][u] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, bv[t][u], acc[g][u], 0, 0, 0);
                }
            }
        }
    }

    // Item (u * 4 + i) * G + g is row 4g + i, column 4c + u.
    float v[NV], o[G];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int g = 0; g < G; ++g) v[(u * 4 + i) * G + g] = acc[g][u][i];
    lane_reduce16<NV>(v, o);
#pragma unroll
    for (int s2 = 0; s2 < G; ++s2) {
        const int t = lane_item<NV>(lane, s2);
        const int g = t % G, ui = t / G;
        red[wave][4 * g + (ui & 3)][4 * c + (ui >> 2)] = o[s2];
    }
    if constexpr (NORM) {
        // Row 4g + c's sum of squares over the wave's 16 lanes with this c.
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float one[1] = {ss[g]}, o1[1];
            lane_reduce16<1>(one, o1);
            if (lane < 4) ssq[wave][4 * g + lane] = o1[0];
        }
    }
    __syncthreads();
    if (eout) {
        float total = red[0][er][ej];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) total += red[w2][er][ej];
        if constexpr (NORM) {
            float sq = ssq[0][er];
#pragma unroll
            for (int w2 = 1; w2 < NW; ++w2) sq += ssq[w2][er];
            total *= 1.0f / sqrtf(sq / static_cast<float>(p.k) + kRmsEps);
        }
        total *= esc;
        p.C[static_cast<size_t>(er) * p.n + ec] = p.accumulate ? eprior + total : total;
    }
}

int decode_groups(int m) { return m <= 4 ? 1 : 2; }

// Threads per workgroup: 1024 (four waves per SIMD, so one wave's MFMAs
// run while another waits for its weights: 4096^2 at m = 4 took 7.8 us at
// 256 threads, 6.3 at 1024).
constexpr int kDecodeThreads = 1024;

template <int NT, int G, int R, bool NORM, bool EXACT>
void launch_decode(const DecodeParams& p, hipStream_t s) {
    constexpr int LB = G == 1 ? 16 : 8;
    auto kern = decode_mfma_kernel<NT, G, R, LB, NORM, EXACT>;
    const size_t lds = NORM ? static_cast<size_t>(p.k4p) * 16 : 0;
    hipLaunchKernelGGL(kern, dim3(p.n / kStrip), dim3(NT), lds, s, p);
}

// Rounds padded to a power of two R (k4p = R x 16 x waves quads).
template <int NT, int G, bool NORM>
void launch_decode_rounds(DecodeParams p, hipStream_t s) {
    constexpr int QPR = 16 * (NT / kWave);
    int R = 1;
    while (R * QPR < p.k4) R *= 2;
    p.rounds = R;
    p.k4p = R * QPR;
    const bool exact = p.k4 == p.k4p;
    constexpr int RMAX = kDecodeMaxQuads / QPR;
    switch (R) {
        case 1: return exact ? launch_decode<NT, G, 1, NORM, true>(p, s) : launch_decode<NT, G, 1, NORM, false>(p, s);
        case 2: return exact ? launch_decode<NT, G, 2, NORM, true>(p, s) : launch_decode<NT, G, 2, NORM, false>(p, s);
        case 4: return exact ? launch_decode<NT, G, 4, NORM, true>(p, s) : launch_decode<NT, G, 4, NORM, false>(p, s);
        default:
            if constexpr (RMAX >= 8) {
                if (R == 8) return exact ? launch_decode<NT, G, 8, NORM, true>(p, s) : launch_decode<NT, G, 8, NORM, false>(p, s);
            }
            if constexpr (RMAX >= 16) {
                return exact ? launch_decode<NT, G, 16, NORM, true>(p, s) : launch_decode<NT, G, 16, NORM, false>(p, s);
            }
    }
}

template <int G, bool NORM>
void launch_decode_threads(const DecodeParams& p, hipStream_t s) {
    launch_decode_rounds<kDecodeThreads, G, NORM>(p, s);
}

}  // namespace

// Where the kernel wins against the row-major products (registered 4096 x n
// weights, per call, us):
//   n        4096       11008        12288        22016        32000
//   m = 2    5.5 / 7.4  11.6 / 12.9  11.8 / 12.8  19.3 / 22.6  26.1 / 26.8
//   m = 4    6.3 / 8.7  12.5 / 15.0  13.5 / 16.0  21.6 / 22.9  29.0 / 27.1
//   m = 8    8.1 / 9.7  20.5 / 15.5  21.7 / 16.4  38.1 / 23.3  50.3 / 27.4
// So 2 rows at any width, 3 - 4 up to n = 24576, 5 - 8 only up to 4096:
// every workgroup reads all of A, and wider B means more workgroups than
// CUs. (Fetching A once for several strips per workgroup, 512 threads,
// was slower at every one of these shapes: 4096 x 22016 at m = 4, 37.8
// against 21.6 us.) k is at most 4096 (all loads of a lane in flight at
// once).
bool decode_mfma_supported(const MatmulArgs& a) {
    if (a.m < 2 || a.m > 8 || a.n % kStrip != 0 || a.k % 4 != 0 || a.k <= 0 ||
        a.k > kDecodeMaxQuads * 4 || reinterpret_cast<uintptr_t>(a.A) % 16 != 0)
        return false;
    return a.m <= 2 || (a.m <= 4 && a.n <= 24576) || a.n <= 4096;
}

void run_decode_mfma(const MatmulArgs& a, const int8_t* packed) {
    DecodeParams p{};
    p.m = a.m;
    p.n = a.n;
    p.k = a.k;
    p.k4 = a.k / 4;
    p.A = a.A;
    p.rms_weight = a.rms_weight;
    p.P = packed;
    p.scale = a.scale;
    p.C = a.C;
    p.accumulate = a.accumulate ? 1 : 0;
    const bool norm = a.rms_weight != nullptr;
    if (decode_groups(a.m) == 1)
        norm ? launch_decode_threads<1, true>(p, a.stream) : launch_decode_threads<1, false>(p, a.stream);
    else
        norm ? launch_decode_threads<2, true>(p, a.stream) : launch_decode_threads<2, false>(p, a.stream);
}

}  // namespace em
