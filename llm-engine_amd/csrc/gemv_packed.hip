// Decode-shaped products over int8 weights held in the strip layout, one
// launch per product: an explicit opt-in weight format behind the boundary
// (the reference keeps QTensor row-major, tensor.h:23-28, and its decode
// product is sgemm_skinny + sum_slices, cuda_matmul.cu:189-254, 365-397).
// This file holds the layout and the VALU products over it: one row of A
// up to k = 12288 (8192 with a fused norm) in gemv_row_kernel (A loaded
// beside each weight unit), and in gemv_packed_kernel (A staged in LDS per
// batch) deeper k, A not
// 16-byte aligned, and the 2 .. 8 row shapes that the MFMA kernel over the
// same layout (decode_mfma.hip) does not take.
//
// Strip layout. A k x n int8 matrix (n % 16 == 0, k % 4 == 0) is stored as
// n / 16 strips of 16 columns; strip j holds rows 0 .. k - 1 of columns
// 16j .. 16j + 15 contiguously, in quads of four rows (64 bytes each), and a
// quad in four 16-byte units, unit c holding columns 4c .. 4c + 3 of the
// quad's rows, row by row:
//     packed[(j * k + 4q) * 16 + 16c + 4t + u] = B[(4q + t) * n + 16j + 4c + u].
// The bytes are the quantised bytes, only reordered, and the column scales
// are unchanged.
//
// Why. In row-major order a contiguous run of a row holds many columns, so
// spreading one m = 1 product over the chip means splitting k across
// workgroups, writing partials and adding them in a second launch. On gfx950
// a dependent launch costs ~1.6 us, about 70 % of the 2.4 us the 16 MiB of a
// 4096^2 int8 matrix take to stream once a launch is running. In the strip
// layout one workgroup reads all of k for its 16 columns as one contiguous
// run, so no partial leaves the workgroup and the product is one launch.
// The quads give every 16-byte load four rows of four columns: the four
// lanes of a quad hold the same rows, which is what the 4x4 blocks of
// v_mfma_f32_4x4x1_16b_f32 need (decode_mfma.hip), and a one-row lane reads
// its four A values as one float4.
//
//  * Workgroup = one strip (256 or 512 threads). Thread t takes 16-byte
//    units t, t + NT, ... of the strip: each load instruction of a wave
//    reads 1 KiB of consecutive units. All loads of a batch (L units per
//    lane) are in flight before any is used; with more than one batch the
//    next batch loads while this one is summed.
//  * int8 is widened in registers and summed unscaled; the column scale is
//    applied once to the reduced sum.
//  * A lane's four column sums are reduced over the 16 lanes holding the
//    same columns by a fixed reduce-scatter (lane_reduce16), the waves in
//    LDS in wave order. Every order is fixed, so repeated calls give the
//    same bits.
//  * gemv_row_kernel: each unit comes with its own float4 of A, loaded just
//    before it; a fused norm weight is loaded the same way and the row's RMS
//    scale, from sums of squares formed on the way, multiplies each output.
//  * gemv_packed_kernel: A is staged in LDS per batch (float4 loads issued
//    before the weights, so waiting for them does not wait for the weight
//    stream). With a norm weight, the workgroup forms the row's RMS scale
//    from a pass over A (fixed order) while its first weights are in
//    flight, and normalises each A value as it uses it, as rmsnorm_rows
//    does.
#include <algorithm>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

constexpr int kStrip = 16;  // columns per strip

struct PackedParams {
    int m, n, k;
    const float* A;
    const float* rms_weight;
    const int8_t* P;  // strip layout
    const float* scale;
    float* C;
    int accumulate;
};

// Thread i writes 16-byte unit i of the packed matrix: strip j, quad q,
// unit c with i = (j * k/4 + q) * 4 + c, from four 4-byte words of B (rows
// 4q .. 4q + 3, columns 16j + 4c .. + 3). Threads walk q slowest, so
// neighbours read neighbouring columns of the same rows.
__global__ __launch_bounds__(kThreads) void pack_strips_kernel(int k, int n, const int8_t* B,
                                                               int8_t* P) {
    const long long strips = n / kStrip, quads = k / 4;
    const long long total = strips * quads * 4;
    for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * kThreads) {
        const long long q = i / (strips * 4), rest = i - q * strips * 4;
        const long long j = rest / 4, c = rest % 4;
        const uint32_t* src = reinterpret_cast<const uint32_t*>(B + 4 * q * n + j * kStrip + 4 * c);
        uint4 v;
        v.x = src[0];
        v.y = src[n / 4];
        v.z = src[2 * (n / 4)];
        v.w = src[3 * (n / 4)];
        *reinterpret_cast<uint4*>(P + ((j * quads + q) * 4 + c) * 16) = v;
    }
}

__global__ __launch_bounds__(kThreads) void unpack_strips_kernel(int k, int n, const int8_t* P,
                                                                 int8_t* B) {
    const long long strips = n / kStrip, quads = k / 4;
    const long long total = strips * quads * 4;
    for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * kThreads) {
        const long long q = i / (strips * 4), rest = i - q * strips * 4;
        const long long j = rest / 4, c = rest % 4;
        const uint4 v = *reinterpret_cast<const uint4*>(P + ((j * quads + q) * 4 + c) * 16);
        uint32_t* dst = reinterpret_cast<uint32_t*>(B + 4 * q * n + j * kStrip + 4 * c);
        dst[0] = v.x;
        dst[n / 4] = v.y;
        dst[2 * (n / 4)] = v.z;
        dst[3 * (n / 4)] = v.w;
    }
}

// Sum over the workgroup's NW waves, every thread gets the result: wave
// sums by a fixed butterfly, then added in wave order. `part` holds NW
// floats of LDS; the leading barrier lets a previous use finish.
template <int NW>
__device__ __forceinline__ float group_sum(float v, float* part) {
    v = wave_sum(v);
    __syncthreads();
    if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = v;
    __syncthreads();
    float t = part[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) t += part[w];
    return t;
}

// NT threads per workgroup (one strip), L units per lane per batch (a
// batch covers NT * L rows). VEC: A 16-byte aligned (k % 4 == 0 always).
// MULTI: k is more than one batch (the next batch loads while this one is
// summed).
template <int NT, int MM, int L, bool NORM, bool VEC, bool MULTI>
__global__ __launch_bounds__(NT) void gemv_packed_kernel(PackedParams p) {
    constexpr int NW = NT / kWave;
    constexpr int RB = NT * L;              // rows of the strip per batch
    constexpr int NF = MM * RB / 4 / NT;    // A float4s per thread per batch
    static_assert(NF >= 1 && MM * RB % (4 * NT) == 0, "whole float4 slots per thread");
    constexpr int NV = 4 * MM;              // column sums per lane: 4 columns x MM rows
    constexpr int NO = NV >= 16 ? NV / 16 : 1;
    __shared__ float4 a_s4[MM * RB / 4];
    __shared__ float red[NW][MM][kStrip];
    __shared__ float part[NW];
    const int tid = threadIdx.x;
    const int c = tid & 3;  // the unit's column group
    const int strip = blockIdx.x;
    const int8_t* base = p.P + static_cast<size_t>(strip) * p.k * kStrip;
    const int batches = MULTI ? (p.k + RB - 1) / RB : 1;

    // This thread's output in the epilogue (row er, column ec).
    const int er = tid / kStrip, ej = tid % kStrip;
    const int ec = strip * kStrip + ej;
    const bool eout = tid < MM * kStrip && er < p.m;

    // A of batch b, raw: slot s = tid + NT t holds row r = s / (RB / 4) of
    // A, values b * RB + 4 (s % (RB / 4)) .. + 3. Loads are unconditional
    // (indices clamped into A); what lies past k or m is zeroed when the
    // slot is written to LDS.
    auto load_a = [&](int b, float4 (&av)[NF]) {
#pragma unroll
        for (int t = 0; t < NF; ++t) {
            const int sl = tid + t * NT;
            const int r = min(sl / (RB / 4), p.m - 1);
            const int j = b * RB + 4 * (sl % (RB / 4));
            const float* row = p.A + static_cast<size_t>(r) * p.k;
            if constexpr (VEC) {
                av[t] = *reinterpret_cast<const float4*>(row + min(j, p.k - 4));
            } else {
                av[t] = make_float4(row[min(j, p.k - 1)], row[min(j + 1, p.k - 1)],
                                    row[min(j + 2, p.k - 1)], row[min(j + 3, p.k - 1)]);
            }
        }
    };
    auto store_a = [&](int b, const float4 (&av)[NF]) {
#pragma unroll
        for (int t = 0; t < NF; ++t) {
            const int sl = tid + t * NT;
            const int r = sl / (RB / 4);
            const int j = b * RB + 4 * (sl % (RB / 4));
            const bool rin = r < p.m;
            float4 v = av[t];
            v.x = rin && j < p.k ? v.x : 0.0f;
            v.y = rin && j + 1 < p.k ? v.y : 0.0f;
            v.z = rin && j + 2 < p.k ? v.z : 0.0f;
            v.w = rin && j + 3 < p.k ? v.w : 0.0f;
            a_s4[sl] = v;
        }
    };
    // Weights of batch b: units b * RB + tid + NT i of the strip (rows
    // b * RB + NT i + (tid & ~3) .. + 3); past k the last quad's unit c,
    // whose A values are zero.
    auto load_w = [&](int b, uint4 (&w)[L]) {
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int unit = min(b * RB + tid + i * NT, p.k - 4 + c);
            w[i] = stream_load(reinterpret_cast<const uint4*>(base + static_cast<size_t>(unit) * kStrip));
        }
    };

    // One accumulator per (row of A, row of the quad, column) for one row of
    // A, so a unit's 16 multiply-adds are independent; with more rows of A
    // the quad's rows share one (the registers go to the rows).
    constexpr int AT = MM == 1 ? 4 : 1;
    float acc[MM][AT][4];
#pragma unroll
    for (int r = 0; r < MM; ++r)
#pragma unroll
        for (int t = 0; t < AT; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[r][t][u] = 0.0f;
    auto fma_batch = [&](const uint4 (&w)[L], const float (&rs)[MM], int b) {
        // One row of A: every A value of the batch read from LDS up front
        // (16 bytes per unit), so no multiply-add waits on an LDS read.
        float4 apre[MM == 1 ? L : 1];
        if constexpr (MM == 1) {
#pragma unroll
            for (int i = 0; i < L; ++i) apre[i] = a_s4[(i * NT + (tid & ~3)) / 4];
        }
#pragma unroll
        for (int i = 0; i < L; ++i) {
            float bv[4][4];  // [row t of the quad][column 4c + u]
            widen4(w[i].x, bv[0]);
            widen4(w[i].y, bv[1]);
            widen4(w[i].z, bv[2]);
            widen4(w[i].w, bv[3]);
            const int pl = i * NT + (tid & ~3);  // the quad's first row in the batch
#pragma unroll
            for (int r = 0; r < MM; ++r) {
                float4 a4 = MM == 1 ? apre[i % (MM == 1 ? L : 1)] : a_s4[(r * RB + pl) / 4];
                float a[4] = {a4.x, a4.y, a4.z, a4.w};
                if constexpr (NORM) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int row = b * RB + pl + t;
                        a[t] = row < p.k ? a[t] * rs[r] * p.rms_weight[row] : 0.0f;
                    }
                }
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        acc[r][t % AT][u] = fmaf(a[t], bv[t][u], acc[r][t % AT][u]);
            }
            if constexpr (MM > 1) __builtin_amdgcn_sched_barrier(0);
        }
    };

    // With a norm, the row's RMS scale comes first: a pass over A summing
    // squares in a fixed order (per thread, then the workgroup), as
    // rmsnorm_rows. It runs while the first weights are in flight.
    float rs[MM];
    float4 av[NF];
    uint4 w[L];
    load_a(0, av);
    load_w(0, w);
    __builtin_amdgcn_sched_barrier(0);
    // The epilogue's scale (and prior C) behind the weights: in flight with
    // them, and waited for only at the end. (Issued before the weights, the
    // scales, cold like the weights, held up the A staging's wait, which
    // counts loads in issue order: 5.9 against 5.5 us at 4096^2.)
    const float esc = p.scale[ec];
    const float eprior = p.accumulate ? p.C[static_cast<size_t>(min(er, p.m - 1)) * p.n + ec] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < MM; ++r) rs[r] = 1.0f;
    if constexpr (NORM) {
#pragma unroll
        for (int r = 0; r < MM; ++r) {
            float ss = 0.0f;
            if (r < p.m)
                for (int j = tid; j < p.k; j += NT) {
                    const float v = p.A[static_cast<size_t>(r) * p.k + j];
                    ss = fmaf(v, v, ss);
                }
            rs[r] = 1.0f / sqrtf(group_sum<NW>(ss, part) / static_cast<float>(p.k) + kRmsEps);
        }
    }
    store_a(0, av);
    __syncthreads();
    if constexpr (!MULTI) {
        fma_batch(w, rs, 0);
    } else {
        for (int b = 0; b < batches; ++b) {
            uint4 wn[L];
            const bool more = b + 1 < batches;
            if (more) {
                load_a(b + 1, av);
                load_w(b + 1, wn);
            }
            fma_batch(w, rs, b);
            __syncthreads();
            if (more) {
                store_a(b + 1, av);
#pragma unroll
                for (int i = 0; i < L; ++i) w[i] = wn[i];
            }
            __syncthreads();
        }
    }

    // Item u * MM + r is column 4c + u of row r; lane_reduce16 sums it over
    // the wave's 16 lanes with the same c.
    const int wave = tid / kWave, lane = tid % kWave;
    float v[NV], o[NO];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 0; r < MM; ++r) {
            float x = acc[r][0][u];
#pragma unroll
            for (int t = 1; t < AT; ++t) x += acc[r][t][u];
            v[u * MM + r] = x;
        }
    lane_reduce16<NV>(v, o);
    if (lane_writes<NV>(lane)) {
#pragma unroll
        for (int s = 0; s < NO; ++s) {
            const int t = lane_item<NV>(lane, s);
            red[wave][t % MM][4 * c + t / MM] = o[s];
        }
    }
    __syncthreads();
    if (eout) {
        float total = red[0][er][ej];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) total += red[w2][er][ej];
        total *= esc;
        p.C[static_cast<size_t>(er) * p.n + ec] = p.accumulate ? eprior + total : total;
    }
}

// One row of A, all of k in one pass, nothing staged in LDS: unit i of a
// lane (u = tid + i * NT) is loaded together with its own float4 of A (the
// quad's rows u & ~3 .. + 3), issued just before the unit's weights. A
// lane's first multiply-adds then wait for one A vector and one weight unit
// instead of all of A and a barrier. (With A staged in LDS first, the wait
// for A ended 1.4-1.8 us into a 3.6 us kernel at 4096^2, when most of the
// weights had arrived, so the widening and multiply-adds ran after the
// stream instead of beside it.) Units past k (TAIL) read the last quad's
// unit c again with A zeroed. With a norm weight, the weight is loaded
// beside A and multiplied in; the row's sum of squares is formed on the
// way (counted from the c == 0 lanes, which between them hold each A value
// once) and its RMS scale multiplies each reduced sum once.
// PAIR (one row of A over a matrix of 2h columns, h % 16 == 0, whose
// first h columns are gates and last h ups, as the forward pass's w13):
// workgroup j takes strips j and j + h / 16 with the same A values and
// writes silu(gate) * up for columns 16j .. 16j + 15 of an h-wide output,
// not the product. Each half is summed in the order the unpaired kernel
// sums it, so the result has the bits of the product followed by the
// SwiGLU, one launch fewer.
template <int NT, int L, bool NORM, bool TAIL, bool PAIR = false>
__global__ __launch_bounds__(NT) void gemv_row_kernel(PackedParams p) {
    constexpr int NW = NT / kWave;
    constexpr int NH = PAIR ? 2 : 1;  // strips per workgroup
    __shared__ float red[NW][NH * kStrip + 1];
    const int tid = threadIdx.x;
    const int c = tid & 3;
    const int strip = blockIdx.x;
    const int pair_off = PAIR ? p.n / (2 * kStrip) : 0;  // the up strip, strips after the gate
    const int8_t* base = p.P + static_cast<size_t>(strip) * p.k * kStrip;
    float4 av[L];
    float4 nv[NORM ? L : 1];
    uint4 w[NH][L];
#pragma unroll
    for (int i = 0; i < L; ++i) {
        const int u = tid + i * NT;
        const int uc = TAIL ? min(u, p.k - 4 + c) : u;
        av[i] = *reinterpret_cast<const float4*>(p.A + (uc & ~3));
        if constexpr (NORM) nv[i] = *reinterpret_cast<const float4*>(p.rms_weight + (uc & ~3));
        w[0][i] = stream_load(reinterpret_cast<const uint4*>(base + static_cast<size_t>(uc) * kStrip));
        if constexpr (PAIR)
            w[NH - 1][i] = stream_load(reinterpret_cast<const uint4*>(
                base + (static_cast<size_t>(pair_off) * p.k + uc) * kStrip));
    }
    // The epilogue's scale (and prior C) behind the weights, waited for at
    // the end.
    __builtin_amdgcn_sched_barrier(0);
    const int ec = strip * kStrip + tid % kStrip;
    const float esc = p.scale[ec];
    const float esc_up = PAIR ? p.scale[ec + pair_off * kStrip] : 0.0f;
    const float eprior = !PAIR && p.accumulate ? p.C[ec] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);

    float acc[NH][4][4];
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[h][t][u] = 0.0f;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < L; ++i) {
        float a[4] = {av[i].x, av[i].y, av[i].z, av[i].w};
        if constexpr (TAIL) {
            const bool in = tid + i * NT < p.k;
#pragma unroll
            for (int t = 0; t < 4; ++t) a[t] = in ? a[t] : 0.0f;
        }
        if constexpr (NORM) {
            const float g[4] = {nv[i].x, nv[i].y, nv[i].z, nv[i].w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                ss = fmaf(a[t], a[t], ss);
                a[t] *= g[t];
            }
        }
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            float bv[4][4];  // [row t of the quad][column 4c + u]
            widen4(w[h][i].x, bv[0]);
            widen4(w[h][i].y, bv[1]);
            widen4(w[h][i].z, bv[2]);
            widen4(w[h][i].w, bv[3]);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int u = 0; u < 4; ++u) acc[h][t][u] = fmaf(a[t], bv[t][u], acc[h][t][u]);
        }
    }

    // Column 4c + u summed over the quad's rows, then over the wave's 16
    // lanes with the same c (lane_reduce16), then over the waves in order.
    const int wave = tid / kWave, lane = tid % kWave;
    float v[4 * NH], o[1];
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int u = 0; u < 4; ++u)
            v[4 * h + u] = ((acc[h][0][u] + acc[h][1][u]) + acc[h][2][u]) + acc[h][3][u];
    lane_reduce16<4 * NH>(v, o);
    if (lane_writes<4 * NH>(lane)) {
        const int item = lane_item<4 * NH>(lane, 0);  // half item / 4, column 4c + item % 4
        red[wave][(item / 4) * kStrip + 4 * c + item % 4] = o[0];
    }
    if constexpr (NORM) {
        const float sw = wave_sum(c == 0 ? ss : 0.0f);
        if (lane == 0) red[wave][NH * kStrip] = sw;
    }
    __syncthreads();
    if (tid < kStrip) {
        float total[NH];
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            total[h] = red[0][h * kStrip + tid];
#pragma unroll
            for (int w2 = 1; w2 < NW; ++w2) total[h] += red[w2][h * kStrip + tid];
        }
        if constexpr (NORM) {
            float sq = red[0][NH * kStrip];
#pragma unroll
            for (int w2 = 1; w2 < NW; ++w2) sq += red[w2][NH * kStrip];
            const float rs = 1.0f / sqrtf(sq / static_cast<float>(p.k) + kRmsEps);
#pragma unroll
            for (int h = 0; h < NH; ++h) total[h] *= rs;
        }
        total[0] *= esc;
        if constexpr (PAIR) {
            total[NH - 1] *= esc_up;
            p.C[ec] = silu_mul(total[0], total[NH - 1]);
        } else {
            p.C[ec] = p.accumulate ? eprior + total[0] : total[0];
        }
    }
}

// Rows per lane L for MM rows of A: capped at LMAX (more rows of A hold
// more accumulators and A values per lane). One batch holds NT x L rows.
template <int NT, int MM, bool NORM, bool VEC, int LMAX>
void launch_depth(int L, const PackedParams& p, hipStream_t s) {
    const dim3 grid(p.n / kStrip);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(NT), 0, s, p); };
    if (L > LMAX) L = LMAX;
    if (NT * L < p.k) {
        // Several batches, half as deep (at most 8 rows a lane from 512
        // threads up), so the next batch's loads fit beside this one's.
        constexpr int LH = LMAX >= 8 ? LMAX / 2 : LMAX;
        constexpr int LM = NT >= 512 && LH > 8 ? 8 : LH;
        return go(gemv_packed_kernel<NT, MM, LM, NORM, VEC, true>);
    }
    if (L <= 4) return go(gemv_packed_kernel<NT, MM, 4, NORM, VEC, false>);
    if constexpr (LMAX >= 8) {
        if (L <= 8) return go(gemv_packed_kernel<NT, MM, 8, NORM, VEC, false>);
    }
    if constexpr (LMAX >= 16) {
        if (L <= 16) return go(gemv_packed_kernel<NT, MM, 16, NORM, VEC, false>);
    }
    if constexpr (LMAX >= 32) go(gemv_packed_kernel<NT, MM, 32, NORM, VEC, false>);
}

// The shallowest L (4 .. LMAX) whose batch holds all of k.
int packed_depth(int nt, int k, int lmax) {
    int L = 4;
    while (L < lmax && nt * L < k) L *= 2;
    return L;
}

// Rows of A -> rows per lane cap at 256 threads (32, 16, 8, 4 for 1, 2, 4,
// 8 rows: accumulators and A values per lane grow with the rows). One row
// may also run 512 or 1024 threads per strip, with 8192 / NT rows per lane
// at most (the same rows per batch, the register budget per lane shrinking
// with the waves per SIMD).
// gemv_row_kernel at NT threads: the shallowest L (4, 8, 16, then 24 at 512
// threads without a norm; at most 8 for PAIR) whose NT x L units hold all
// of k; false when k is deeper than that.
template <int NT, bool NORM, bool PAIR = false>
bool launch_row(const PackedParams& p, hipStream_t s) {
    // Deeper lanes spill: 32 units to AGPRs, 24 with the norm weight's
    // registers (or 8 at 1024 threads, or 16 of each half of a pair) to
    // scratch.
    constexpr int LMAX = NT == 1024 ? 4 : PAIR ? 8 : NT == 512 && !NORM ? 24 : 16;
    int L = 4;
    while (L < LMAX && NT * L < p.k) L = L < 16 ? 2 * L : L + 8;
    if (NT * L < p.k) return false;
    const dim3 grid(p.n / (PAIR ? 2 * kStrip : kStrip));
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(NT), 0, s, p); };
    auto pick = [&](auto tail) {
        constexpr bool T = decltype(tail)::value;
        switch (L) {
            case 4: return go(gemv_row_kernel<NT, 4, NORM, T, PAIR>);
            case 8:
                if constexpr (LMAX >= 8) return go(gemv_row_kernel<NT, 8, NORM, T, PAIR>);
                break;
            case 16:
                if constexpr (LMAX >= 16) return go(gemv_row_kernel<NT, 16, NORM, T, PAIR>);
                break;
            default:
                if constexpr (LMAX >= 24) return go(gemv_row_kernel<NT, 24, NORM, T, PAIR>);
                break;
        }
    };
    if (NT * L == p.k) pick(std::false_type{});
    else pick(std::true_type{});
    return true;
}

// Threads per workgroup of gemv_row_kernel: 512 above 2048 rows of k and
// 256 up to it.
int row_threads(int k) { return k > 2048 ? 512 : 256; }

template <bool NORM, bool VEC>
void launch_threads(const PackedParams& p, hipStream_t s) {
    if (p.m == 1 && VEC) {
        // 512 threads (two waves per SIMD, one multiplying while the other
        // waits for its loads) above 2048 rows of k, 256 up to it (4096^2:
        // 4.7 against 4.9 us; 2048 x 8192: 4.8 against 4.7); at most 4096
        // rows at 256 threads, 8192 at 512 (12288 without a norm). Deeper k
        // loops in gemv_packed_kernel.
        const int nt = row_threads(p.k);
        if (nt == 256 && launch_row<256, NORM>(p, s)) return;
        if (launch_row<512, NORM>(p, s)) return;
    }
    if (p.m <= 1) {
        // Past 8192 rows a 256-thread workgroup would loop over batches;
        // 512 threads hold up to 16384 rows in one batch.
        if (p.k > kThreads * 32 && p.k <= 512 * 32)
            return launch_depth<512, 1, NORM, VEC, 32>(packed_depth(512, p.k, 32), p, s);
        return launch_depth<256, 1, NORM, VEC, 32>(packed_depth(256, p.k, 32), p, s);
    }
    if (p.m <= 2) return launch_depth<256, 2, NORM, VEC, 16>(packed_depth(256, p.k, 16), p, s);
    if (p.m <= 4) return launch_depth<256, 4, NORM, VEC, 8>(packed_depth(256, p.k, 8), p, s);
    launch_depth<256, 8, NORM, VEC, 4>(4, p, s);
}

}  // namespace

void run_pack_strips(int k, int n, const int8_t* B, int8_t* P, hipStream_t stream) {
    const long long total = static_cast<long long>(n / kStrip) * k;
    const int blocks = static_cast<int>(std::min<long long>((total + kThreads - 1) / kThreads,
                                                            static_cast<long long>(cu_count()) * 16));
    hipLaunchKernelGGL(pack_strips_kernel, dim3(blocks > 0 ? blocks : 1), dim3(kThreads), 0, stream,
                       k, n, B, P);
}

bool gemv_swiglu_supported(const MatmulArgs& a) {
    const int half = a.n / 2;
    const int nt = row_threads(a.k);
    const int deepest = nt == 1024 ? 1024 * 4 : nt * 8;
    return a.m == 1 && a.n % (2 * kStrip) == 0 && a.k % 4 == 0 && half > 0 && a.k <= deepest &&
           reinterpret_cast<uintptr_t>(a.A) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(a.rms_weight) % 16 == 0 && !a.accumulate;
}

void run_gemv_swiglu(const MatmulArgs& a, const int8_t* packed) {
    PackedParams p{};
    p.m = 1;
    p.n = a.n;
    p.k = a.k;
    p.A = a.A;
    p.rms_weight = a.rms_weight;
    p.P = packed;
    p.scale = a.scale;
    p.C = a.C;
    p.accumulate = 0;
    bool done = false;
    const int nt = row_threads(a.k);
    if (a.rms_weight) {
        done = nt == 1024 ? launch_row<1024, true, true>(p, a.stream)
               : nt == 256 ? launch_row<256, true, true>(p, a.stream)
                           : launch_row<512, true, true>(p, a.stream);
    } else {
        done = nt == 1024 ? launch_row<1024, false, true>(p, a.stream)
               : nt == 256 ? launch_row<256, false, true>(p, a.stream)
                           : launch_row<512, false, true>(p, a.stream);
    }
    if (!done) throw DeviceError("gemv_swiglu: k too deep for one pass");
}

void run_unpack_strips(int k, int n, const int8_t* P, int8_t* B, hipStream_t stream) {
    const long long total = static_cast<long long>(n / kStrip) * k;
    const int blocks = static_cast<int>(std::min<long long>((total + kThreads - 1) / kThreads,
                                                            static_cast<long long>(cu_count()) * 16));
    hipLaunchKernelGGL(unpack_strips_kernel, dim3(blocks > 0 ? blocks : 1), dim3(kThreads), 0,
                       stream, k, n, P, B);
}

// One batch when k fits NT x L rows, at the shallowest depth that holds
// it (L capped by the rows of A: 32, 16, 8, 4 for 1, 2, 4, 8 rows); deeper
// k loops over batches with the next batch in flight.
void run_gemv_packed(const MatmulArgs& a, const int8_t* packed) {
    PackedParams p{};
    p.m = a.m;
    p.n = a.n;
    p.k = a.k;
    p.A = a.A;
    p.rms_weight = a.rms_weight;
    p.P = packed;
    p.scale = a.scale;
    p.C = a.C;
    p.accumulate = a.accumulate ? 1 : 0;
    // The float4 kernels load A and the norm weight four values at a time.
    const bool vec = a.k % 4 == 0 && reinterpret_cast<uintptr_t>(a.A) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(a.rms_weight) % 16 == 0;
    if (a.rms_weight) {
        if (vec) launch_threads<true, true>(p, a.stream);
        else launch_threads<true, false>(p, a.stream);
    } else {
        if (vec) launch_threads<false, true>(p, a.stream);
        else launch_threads<false, false>(p, a.stream);
    }
}

}  // namespace em
