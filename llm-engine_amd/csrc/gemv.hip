// Decode-shaped products, m <= 8 rows of A against a k x n weight matrix:
// GpuKernel::skinny (reference: sgemm_skinny + run_skinny,
// /root/reference/src/cuda_matmul.cu:127-243,365-397).
//
// The product is bound by reading B once, so the kernel is laid out for HBM:
//
//  * A workgroup (256 threads, four wave64s) owns a 256-column tile of C and
//    a slice of R = E * L rows of B. Each lane loads E consecutive columns of
//    a row as one 16-byte vector (E = 16 int8 or 4 fp32; 4-byte and scalar
//    variants cover widths that are not a multiple of 16 bytes), so the
//    256 / E lanes of a row group read one contiguous 256-column run of a row
//    (256 B int8, 1 KB fp32) per instruction.
//  * The tile has E row groups; lane rows are rg, rg + E, ..., so every
//    lane issues all L of its loads before it uses any: 16 B x L in flight
//    per lane, and the whole matrix is in flight across the grid at 4096^2.
//  * int8 is widened in registers (one SDWA convert per byte) and summed
//    unscaled; the column scale is applied once to the reduced sum, as the
//    reference's 4-column path and CPU streaming path do
//    (cuda_matmul.cu:148-153,234-242; matmul.cpp:273-281).
//  * The E row groups are added in LDS in a fixed order. k slices across
//    workgroups go to a partial buffer [slice][m][n] and are added in slice
//    order by reduce_slices, so repeated calls give the same bits
//    (tests/test_cuda.cpp:221-275 of the reference).
//  * With a norm weight, each workgroup computes its rows' RMS scales over
//    all of k and normalises its slice of A as it stages it in LDS
//    (cuda_matmul.cu:159-170,197,213).
#include <cstdlib>
#include <type_traits>

#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

// E elements of BT per lane and row, loaded as one vector and widened to fp32.
template <class BT, int E>
struct Lane;

template <>
struct Lane<int8_t, 16> {
    using V = uint4;
    static __device__ __forceinline__ V load(const int8_t* p) {
        return stream_load(reinterpret_cast<const uint4*>(p));
    }
    static __device__ __forceinline__ V zero() { return make_uint4(0, 0, 0, 0); }
    static __device__ __forceinline__ void widen(const V& v, float* b) {
        widen4(v.x, b);
        widen4(v.y, b + 4);
        widen4(v.z, b + 8);
        widen4(v.w, b + 12);
    }
};

template <>
struct Lane<int8_t, 4> {
    using V = uint32_t;
    static __device__ __forceinline__ V load(const int8_t* p) {
        return stream_load(reinterpret_cast<const uint32_t*>(p));
    }
    static __device__ __forceinline__ V zero() { return 0u; }
    static __device__ __forceinline__ void widen(const V& v, float* b) { widen4(v, b); }
};

template <>
struct Lane<int8_t, 1> {
    using V = int8_t;
    static __device__ __forceinline__ V load(const int8_t* p) { return stream_load(p); }
    static __device__ __forceinline__ V zero() { return 0; }
    static __device__ __forceinline__ void widen(const V& v, float* b) {
        b[0] = static_cast<float>(v);
    }
};

template <>
struct Lane<float, 4> {
    using V = float4;
    static __device__ __forceinline__ V load(const float* p) {
        return stream_load(reinterpret_cast<const float4*>(p));
    }
    static __device__ __forceinline__ V zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
    static __device__ __forceinline__ void widen(const V& v, float* b) {
        b[0] = v.x;
        b[1] = v.y;
        b[2] = v.z;
        b[3] = v.w;
    }
};

template <>
struct Lane<float, 1> {
    using V = float;
    static __device__ __forceinline__ V load(const float* p) { return stream_load(p); }
    static __device__ __forceinline__ V zero() { return 0.f; }
    static __device__ __forceinline__ void widen(const V& v, float* b) { b[0] = v; }
};

template <class BT>
struct GemvParams {
    int m, n, k;
    const float* A;
    const float* rms_weight;
    const BT* B;
    const float* scale;  // int8 only
    float* out;          // C when direct, else partials [slice][m][n]
    int accumulate;
    int direct;
    int a_vec4;          // k % 4 == 0 and A 16-byte aligned: the norm reads float4
    Summed gu;           // SWI: the w13 product A is formed from
    int hidden;          // SWI: its gate | up split
    const float* ssq;    // NORM 2: sums of squares of A, one per 64 values
    int ssq_parts;       // NORM 2: their count, ceil(k / 64) <= kSsqParts
    SplitRow att;        // merged source: the attention chunks A is merged from
};

// Where A comes from: read (kSrcA), or formed in the A staging from a
// gate | up product (kSrcSwiGLU) or from split attention chunks (kSrcMerge).
constexpr int kSrcA = 0, kSrcSwiGLU = 1, kSrcMerge = 2;

// Slices a SwiGLU source may have: its values are loaded into registers.
constexpr int kSwiSlices = 16;
// Sums of squares a NORM 2 row may have: four per lane of one wave.
constexpr int kSsqParts = 4 * kWave;

// MM: rows of A the kernel is compiled for (m <= MM; extra rows are zero).
// E: columns per lane. L: rows per lane. NORM: fused RMSNorm of A, 0 none,
// 1 with the sum of squares formed here over all of A's row, 2 (one row)
// with it formed from the sums of squares the producer of A left, one per
// 64 values (p.ssq): each wave adds them with a fixed butterfly, so every
// lane and workgroup gets the same bits without a barrier, and no
// workgroup reads more of A than its own slice.
// SRC: formed sources take one row and at most 256 rows of k per
// workgroup, one A value per thread. kSrcSwiGLU: A[j] = silu_mul(gate[j],
// up[j]) of a product given as a Summed (p.gu, gate | up at p.hidden): the
// arithmetic of the forward pass's SwiGLU kernel, so the result is the same
// as running that kernel first. kSrcMerge: A[h * hs + d] is the merge of
// head h's attention chunks (p.att) in the merge kernel's slots and order,
// so the result is the same as merging first; a row of one chunk, or of
// more than kMergeInGemv, is read from p.att.out.
template <class BT, int MM, int E, int L, int NORM, int SRC = kSrcA>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvParams<BT> p) {
    constexpr bool SWI = SRC == kSrcSwiGLU, MRG = SRC == kSrcMerge;
    using LT = Lane<BT, E>;
    using V = typename LT::V;
    constexpr int LPR = kThreads / E;  // lanes across one 256-column run
    constexpr int R = E * L;           // rows of B per workgroup
    constexpr int AREG = (MM * R + kThreads - 1) / kThreads;
    constexpr int RS = LPR + 1;  // padded stride of the reduction buffer
    constexpr bool kQ8 = std::is_same<BT, int8_t>::value;

    __shared__ float a_s[MM * R];
    // E == 16: the four waves' column sums (after the in-wave fold), else
    // every row group's sums.
    __shared__ float red[E == 16 ? MM * 4 * kThreads : E * E * RS];
    __shared__ float part[4];
    __shared__ float rs_s[MM];

    const int tid = threadIdx.x;
    const int cg = tid % LPR;
    const int rg = tid / LPR;
    const int col = blockIdx.x * kThreads + cg * E;
    const bool active = col < p.n;
    const int p0 = blockIdx.y * R;

    // With a norm: the first NP values of each row this thread sums squares
    // of (k = tid, tid + 256, ...), loaded before the weight loads. A loop
    // of loads after them would wait for the whole weight stream at its
    // first s_waitcnt and then take one L2 round trip per step.
    static_assert(NORM != 2 || (MM == 1 && SRC == kSrcA), "producer sums of squares: one row");
    constexpr int NP = NORM != 1 ? 1 : MM == 1 ? 32 : MM == 2 ? 16 : MM <= 4 ? 4 : 2;
    // Loads are unconditional (addresses clamped into A; k >= 1 here) so
    // that no branch separates them; values past m or k are masked at use.
    // With a_vec4 the thread takes float4 f = tid, tid + 256, ... (values
    // 4f .. 4f + 3): a quarter of the load instructions.
    constexpr int NP4 = NP / 4;
    float npre[MM][NP];
    if constexpr (NORM == 1) {
#pragma unroll
        for (int r = 0; r < MM; ++r) {
            const int rr = r < p.m ? r : p.m - 1;
            if (NP4 > 0 && p.a_vec4) {
                const floatx4* row4 = reinterpret_cast<const floatx4*>(p.A + rr * p.k);
#pragma unroll
                for (int i = 0; i < NP4; ++i) {
                    const floatx4 v = row4[min(tid + i * kThreads, p.k / 4 - 1)];
                    npre[r][4 * i] = v.x;
                    npre[r][4 * i + 1] = v.y;
                    npre[r][4 * i + 2] = v.z;
                    npre[r][4 * i + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < NP; ++i)
                    npre[r][i] = p.A[rr * p.k + min(tid + i * kThreads, p.k - 1)];
            }
        }
    }

    // This workgroup's slice of A, raw, into registers: issued before the
    // weight loads so its wait does not include them.
    float a_reg[AREG];
    float sg[SWI ? kSwiSlices : 1], su[SWI ? kSwiSlices : 1];
    float mo[MRG ? kMergeInGemv : 1], mout = 0.0f;
    float2 mml[MRG ? kMergeInGemv : 1];
    if constexpr (MRG) {
        static_assert(MM == 1 && AREG == 1 && !NORM, "merged source: one row, one value per thread");
        // This thread's column of the first kMergeInGemv chunks its head
        // may have (clamped past splits; only the row's chunks are used) and
        // of out, which holds the row when it has one chunk or more than
        // kMergeInGemv (merged by the merge kernel): nothing waits for *pos.
        const int col = min(p0 + tid % R, p.k - 1);
        const int h = col / p.att.head_size, d = col - h * p.att.head_size;
        mout = p.att.out[col];
#pragma unroll
        for (int c = 0; c < kMergeInGemv; ++c) {
            const int b = h * p.att.splits + min(c, p.att.splits - 1);
            mml[c] = p.att.ml[b];
            mo[c] = p.att.o[static_cast<size_t>(b) * p.att.head_size + d];
        }
    } else if constexpr (SWI) {
        static_assert(MM == 1 && AREG == 1 && !NORM, "SwiGLU source: one row, one value per thread");
        // Gate and up of this thread's k index, every slice (clamped past
        // the last; only the first gu.slices are added).
        const int col = min(p0 + tid % R, p.k - 1);
        if (p.gu.slices == 1) {
            sg[0] = p.gu.c[col];
            su[0] = p.gu.c[p.hidden + col];
        } else {
#pragma unroll
            for (int sl = 0; sl < kSwiSlices; ++sl) {
                const size_t off = static_cast<size_t>(min(sl, p.gu.slices - 1)) * p.gu.mn + col;
                sg[sl] = p.gu.partial[off];
                su[sl] = p.gu.partial[off + p.hidden];
            }
        }
    } else {
#pragma unroll
        for (int t = 0; t < AREG; ++t) {
            const int idx = tid + t * kThreads;
            const int r = idx / R, pp = p0 + idx % R;
            a_reg[t] = (idx < MM * R && r < p.m && pp < p.k) ? p.A[r * p.k + pp] : 0.0f;
        }
    }
    // NORM 2: this lane's share of the sums of squares (parts lane, lane +
    // 64, ...) and the norm weights of its slice values, before the weights.
    float sq[NORM == 2 ? kSsqParts / kWave : 1];
    float gain[NORM == 2 ? AREG : 1];
    if constexpr (NORM == 2) {
        const int lane = tid % kWave;
#pragma unroll
        for (int j = 0; j < kSsqParts / kWave; ++j)
            sq[j] = p.ssq[min(lane + j * kWave, p.ssq_parts - 1)];
#pragma unroll
        for (int t = 0; t < AREG; ++t)
            gain[t] = p.rms_weight[min(p0 + (tid + t * kThreads) % R, p.k - 1)];
    }

    // All L weight vectors of this lane in flight at once. No load is
    // predicated and no loaded value is selected, so nothing sits between a
    // load and its use: a row past k reads row k - 1 (its A operand is
    // staged as zero), and a lane past n reads column 0 (its sums are never
    // stored). k * n < 2^31, so offsets are 32-bit from the uniform base.
    const int lcol = active ? col : 0;
    V w[L];
#pragma unroll
    for (int i = 0; i < L; ++i) {
        const int pp = min(p0 + rg + i * E, p.k - 1);
        w[i] = LT::load(p.B + static_cast<uint32_t>(pp * p.n + lcol));
    }
    // Nothing that uses a loaded value is moved above the loads.
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (SWI) {
        // summed(): C as is, or the slices added in order, then the scale.
        const int col = min(p0 + tid % R, p.k - 1);
        float g = sg[0], u = su[0];
        if (p.gu.slices > 1) {
            g = 0.0f;
            u = 0.0f;
#pragma unroll
            for (int sl = 0; sl < kSwiSlices; ++sl) {
                if (sl < p.gu.slices) {
                    g += sg[sl];
                    u += su[sl];
                }
            }
            if (p.gu.scale) {
                g *= p.gu.scale[col];
                u *= p.gu.scale[p.hidden + col];
            }
        }
        a_reg[0] = (tid < R && p0 + tid % R < p.k) ? silu_mul(g, u) : 0.0f;
    }
    if constexpr (MRG) {
        const int n_ctx = *p.att.pos + 1;
        const int chunk = split_chunk(n_ctx, p.att.splits, p.att.min_chunk);
        const int n = (n_ctx + chunk - 1) / chunk;
        float v = mout;
        float2 ml8[8];
        float o8[8];
        if (n > 1 && n <= 8) {
            // One slot over chunks 0 .. n - 1.
            float m = -INFINITY, l = 0.0f, acc = 0.0f;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                ml8[u] = mml[u];
                o8[u] = mo[u];
            }
            merge_batch8(m, l, acc, ml8, o8, 0, 1, n);
            const float2 s0 = make_float2(m, l);
            v = merge_combine(1, 0.0f, [&](int) { return s0; }, [&](int) { return acc; });
        } else if (n > 8 && n <= kMergeInGemv) {
            // Two slots: chunks 0, 2, 4, ... and 1, 3, 5, ...
            float2 sm[2];
            float sa[2];
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                float m = -INFINITY, l = 0.0f, acc = 0.0f;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    ml8[u] = mml[2 * u + r];
                    o8[u] = mo[2 * u + r];
                }
                merge_batch8(m, l, acc, ml8, o8, r, 2, n);
                sm[r] = make_float2(m, l);
                sa[r] = acc;
            }
            v = merge_combine(2, 0.0f, [&](int r) { return sm[r]; }, [&](int r) { return sa[r]; });
        }
        a_reg[0] = (tid < R && p0 + tid % R < p.k) ? v : 0.0f;
    }
    if constexpr (NORM == 1) {
#pragma unroll
        for (int r = 0; r < MM; ++r) {
            // One fixed sequence of fmaf per thread: the preloaded values
            // (zero past k adds exactly nothing), then any rest of the row.
            float ss = 0.0f;
            if (NP4 > 0 && p.a_vec4) {
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const bool ok = r < p.m && tid + (i / 4) * kThreads < p.k / 4;
                    const float v = ok ? npre[r][i] : 0.0f;
                    ss = fmaf(v, v, ss);
                }
                if (r < p.m)
                    for (int j = 4 * (tid + NP4 * kThreads); j < p.k; j += 4 * kThreads)
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const float v = p.A[r * p.k + j + c];
                            ss = fmaf(v, v, ss);
                        }
            } else {
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const float v = (r < p.m && tid + i * kThreads < p.k) ? npre[r][i] : 0.0f;
                    ss = fmaf(v, v, ss);
                }
                if (r < p.m)
                    for (int j = tid + NP * kThreads; j < p.k; j += kThreads) {
                        const float v = p.A[r * p.k + j];
                        ss = fmaf(v, v, ss);
                    }
            }
            const float total = block_sum(ss, part);
            if (tid == 0) rs_s[r] = 1.0f / sqrtf(total / static_cast<float>(p.k) + kRmsEps);
        }
        __syncthreads();
    }
    float rs2 = 0.0f;
    if constexpr (NORM == 2) {
        // Parts past ssq_parts add +0: a sum of squares is never -0.
        const int lane = tid % kWave;
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < kSsqParts / kWave; ++j)
            v += lane + j * kWave < p.ssq_parts ? sq[j] : 0.0f;
        rs2 = 1.0f / sqrtf(wave_sum(v) / static_cast<float>(p.k) + kRmsEps);
    }
#pragma unroll
    for (int t = 0; t < AREG; ++t) {
        const int idx = tid + t * kThreads;
        if (idx < MM * R) {
            float v = a_reg[t];
            if constexpr (NORM == 1) {
                const int r = idx / R, pp = p0 + idx % R;
                if (r < p.m && pp < p.k) v = v * rs_s[r] * p.rms_weight[pp];
            } else if constexpr (NORM == 2) {
                if (p0 + idx % R < p.k) v = v * rs2 * gain[t];
            }
            a_s[idx] = v;
        }
    }
    __syncthreads();

    float acc[MM][E];
#pragma unroll
    for (int r = 0; r < MM; ++r)
#pragma unroll
        for (int j = 0; j < E; ++j) acc[r][j] = 0.0f;

#pragma unroll
    for (int i = 0; i < L; ++i) {
        float b[E];
        LT::widen(w[i], b);
        const int pl = rg + i * E;
#pragma unroll
        for (int r = 0; r < MM; ++r) {
            const float a = a_s[r * R + pl];
#pragma unroll
            for (int j = 0; j < E; ++j) acc[r][j] = fmaf(a, b[j], acc[r][j]);
        }
    }

    // Add the E row groups in order, one row of C at a time. Thread t then
    // owns local column t of the tile. Rows past m hold zeros and go through
    // the same steps with their stores skipped: a branch on m around the
    // barriers measured 0.6 us slower per 16 MiB GEMV.
    //
    // With 16 columns per lane (16 lanes a row), the four row groups of a
    // wave are lanes l, l ^ 16, l ^ 32, l ^ 48: two lane-swap folds leave
    // each lane four sums of consecutive columns (16 cg + 4 b4 + 8 b5 + i,
    // b4 and b5 the lane's bits 4 and 5), written as one 16-byte store; one
    // barrier, then thread t adds the four waves' sums of column t in wave
    // order. Other widths add every row group's sums through LDS.
    const int ccg = tid / E, cj = tid % E;
    const int c = blockIdx.x * kThreads + tid;
    if constexpr (E == 16) {
        const int lane = tid % kWave, wave = tid / kWave;
#pragma unroll
        for (int r = 0; r < MM; ++r) {
            float a8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) a8[i] = fold32(acc[r][i], acc[r][i + 8]);
            float4 a4;
            a4.x = fold16(a8[0], a8[4]);
            a4.y = fold16(a8[1], a8[5]);
            a4.z = fold16(a8[2], a8[6]);
            a4.w = fold16(a8[3], a8[7]);
            const int col = 16 * cg + 4 * ((lane >> 4) & 1) + 8 * ((lane >> 5) & 1);
            *reinterpret_cast<float4*>(&red[(r * 4 + wave) * kThreads + col]) = a4;
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < MM; ++r) {
        float total = 0.0f;
        if constexpr (E == 16) {
            total = red[(r * 4) * kThreads + tid];
#pragma unroll
            for (int w = 1; w < 4; ++w) total += red[(r * 4 + w) * kThreads + tid];
        } else {
#pragma unroll
            for (int j = 0; j < E; ++j) red[(rg * E + j) * RS + cg] = acc[r][j];
            __syncthreads();
#pragma unroll
            for (int g = 0; g < E; ++g) total += red[(g * E + cj) * RS + ccg];
        }
        if (r < p.m && c < p.n) {
            if (p.direct) {
                float v = total;
                if constexpr (kQ8) v *= p.scale[c];
                float* o = p.out + static_cast<size_t>(r) * p.n + c;
                *o = p.accumulate ? *o + v : v;
            } else {
                p.out[(static_cast<size_t>(blockIdx.y) * p.m + r) * p.n + c] = total;
            }
        }
        if constexpr (E != 16) __syncthreads();
    }
}

// Deepest rows-per-lane that fits the register file without spilling: with
// 16 int8 columns per lane, eight rows of A hold 128 accumulators and 16
// loads in flight would pass 256 VGPRs (four rows: 155). One row of A leaves
// room for 32 loads in flight (128 VGPRs).
constexpr int max_depth(int E, int MM) { return MM == 1 ? 32 : (E == 16 ? (MM <= 4 ? 16 : 8) : 16); }

template <class BT, int MM, int E, int L, int NORM>
void launch(const GemvParams<BT>& p, dim3 grid, hipStream_t s) {
    hipLaunchKernelGGL((gemv_kernel<BT, MM, E, L, NORM>), grid, dim3(kThreads), 0, s, p);
}

template <class BT, int E, int L, int NORM>
void pick_rows(const GemvParams<BT>& p, dim3 grid, hipStream_t s) {
    if constexpr (NORM == 2) {
        launch<BT, 1, E, L, 2>(p, grid, s);  // one row (run_skinny_partials checks)
    } else if (p.m <= 1) {
        launch<BT, 1, E, L, NORM>(p, grid, s);
    } else if (p.m <= 2) {
        launch<BT, 2, E, (L < max_depth(E, 2) ? L : max_depth(E, 2)), NORM>(p, grid, s);
    } else if (p.m <= 4) {
        launch<BT, 4, E, (L < max_depth(E, 4) ? L : max_depth(E, 4)), NORM>(p, grid, s);
    } else {
        launch<BT, 8, E, (L < max_depth(E, 8) ? L : max_depth(E, 8)), NORM>(p, grid, s);
    }
}

template <class BT, int E, int NORM>
void pick_depth(int L, const GemvParams<BT>& p, dim3 grid, hipStream_t s) {
    if constexpr (E == 1) {
        pick_rows<BT, 1, 16, NORM>(p, grid, s);
    } else {
        switch (L) {
            case 4: pick_rows<BT, E, 4, NORM>(p, grid, s); break;
            case 8: pick_rows<BT, E, 8, NORM>(p, grid, s); break;
            case 32: pick_rows<BT, E, 32, NORM>(p, grid, s); break;
            default: pick_rows<BT, E, 16, NORM>(p, grid, s); break;
        }
    }
}

template <class BT, int NORM>
void pick_width(int E, int L, const GemvParams<BT>& p, dim3 grid, hipStream_t s) {
    if constexpr (std::is_same<BT, int8_t>::value) {
        if (E == 16) return pick_depth<BT, 16, NORM>(L, p, grid, s);
    }
    if (E == 4) return pick_depth<BT, 4, NORM>(L, p, grid, s);
    pick_depth<BT, 1, NORM>(L, p, grid, s);
}

bool aligned(const void* ptr, size_t bytes) {
    return reinterpret_cast<uintptr_t>(ptr) % bytes == 0;
}

// Rows per lane: if all of k fits one slice and n is wide, the shallowest
// depth that holds it. Otherwise the deepest of 16 / 8 / 4 that still gives the grid
// half a workgroup per CU or more. Deep slices mean fewer partials to reduce; with
// nontemporal weight loads one 16-row-deep workgroup per CU streams a
// 4096^2 int8 matrix faster than two 8-deep ones, and sweeps over the
// Llama-7B and stories15M shapes put the cut near CUs / 2.
// The result is what the launched kernel uses: capped by max_depth as
// pick_rows caps it.
int rows_per_lane(int E, int m, int n, int k) {
    if (E == 1) return 16;
    const int mm = m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
    const int cap = max_depth(E, mm);
    // Too few columns and rows for half a workgroup per CU: fp32 lanes still
    // take 8 rows (4 would make 16-row slices, 18 of them at k = 288: the
    // stories15M fp32 decode ran 0.217 ms/token against 0.198 at 8).
    int L = E == 4 ? 8 : 4;
    if (k <= E * cap && ceil_div(n, kThreads) >= cu_count() / 4) {
        // All of k in one slice when the columns alone give a quarter of a
        // workgroup per CU: no partials and no second launch (the stories15M
        // classifier, k = 288, n = 32000). Narrower products still split k,
        // since a handful of workgroups cannot keep enough loads in flight.
        while (E * L < k) L *= 2;
    } else {
        // Half a workgroup per CU. Two to four rows of int8 (each lane also
        // holds 2-4x the accumulators; 16-deep only since four rows fit in
        // 155 registers): 1.5 per CU, which took m = 4 x 4096x11008 from
        // 18.5 to 16.4 us and leaves 4096^2 (1 per CU at depth 16) at 8.
        const long long tiles = ceil_div(n, kThreads);
        const bool few_rows = E == 16 && (mm == 2 || mm == 4);
        const long long target = few_rows ? cu_count() + cu_count() / 2 : cu_count() / 2;
        for (int depth : {16, 8}) {
            if (tiles * ceil_div(k, static_cast<long long>(E) * depth) >= target) {
                L = depth;
                break;
            }
        }
    }
    return L < cap ? L : cap;
}

// The GEMV's lane width E (16 int8 or 4 fp32 columns per 16-byte load, 1
// for widths or alignments that rule those out), rows per lane L and k
// slices for a product.
struct SkinnyLayout {
    int E, L, slices;
};

template <class BT>
SkinnyLayout skinny_layout(const MatmulArgs& a) {
    const BT* B = static_cast<const BT*>(a.B);
    int E = 1;
    if (std::is_same<BT, int8_t>::value && a.n % 16 == 0 && aligned(B, 16)) {
        E = 16;
    } else if (a.n % 4 == 0 && aligned(B, 4 * sizeof(BT))) {
        E = 4;
    }
    const int L = rows_per_lane(E, a.m, a.n, a.k);
    const int rows_per_block = E * (E == 1 ? 16 : L);
    return {E, L, ceil_div(a.k, rows_per_block)};
}

}  // namespace

template <class BT>
std::size_t skinny_partial_floats(const MatmulArgs& a) {
    const int slices = skinny_layout<BT>(a).slices;
    return slices > 1 ? static_cast<std::size_t>(slices) * a.m * a.n : 0;
}

template <class BT>
int run_skinny_partials(const MatmulArgs& a, const float** partial) {
    const BT* B = static_cast<const BT*>(a.B);
    const SkinnyLayout lay = skinny_layout<BT>(a);
    const int E = lay.E, L = lay.L, slices = lay.slices;
    const dim3 grid(ceil_div(a.n, kThreads), slices);

    GemvParams<BT> p{};
    p.m = a.m;
    p.n = a.n;
    p.k = a.k;
    p.A = a.A;
    p.rms_weight = a.rms_weight;
    p.B = B;
    p.scale = a.scale;
    p.direct = slices == 1;
    p.a_vec4 = a.k % 4 == 0 && aligned(a.A, 16);
    p.accumulate = a.accumulate && p.direct;
    p.out = p.direct      ? a.C
            : a.partials ? a.partials
                         : scratch(kPartial, static_cast<size_t>(slices) * a.m * a.n);
    p.ssq = a.ssq;
    p.ssq_parts = ceil_div(a.k, kSsqChunk);
    if (a.rms_weight && a.ssq && a.m == 1 && p.ssq_parts <= kSsqParts) {
        pick_width<BT, 2>(E, L, p, grid, a.stream);
    } else if (a.rms_weight) {
        pick_width<BT, 1>(E, L, p, grid, a.stream);
    } else {
        pick_width<BT, 0>(E, L, p, grid, a.stream);
    }
    *partial = p.direct ? nullptr : p.out;
    return slices;
}

namespace {

// One row whose A the kernel forms (SRC), p carrying the source's fields:
// the launch and its k slices, 0 if the shape has no 4- or 16-wide lanes.
template <class BT, int SRC>
int run_formed_partials(const MatmulArgs& a, GemvParams<BT> p, const float** partial) {
    const BT* B = static_cast<const BT*>(a.B);
    int E = 1;
    if (std::is_same<BT, int8_t>::value && a.n % 16 == 0 && aligned(B, 16)) {
        E = 16;
    } else if (a.n % 4 == 0 && aligned(B, 4 * sizeof(BT))) {
        E = 4;
    }
    if (E == 1) return 0;
    // One A value per thread: at most 256 rows of B per workgroup.
    int L = rows_per_lane(E, a.m, a.n, a.k);
    while (E * L > kThreads) L /= 2;
    const int slices = ceil_div(a.k, E * L);
    const dim3 grid(ceil_div(a.n, kThreads), slices);
    p.m = 1;
    p.n = a.n;
    p.k = a.k;
    p.B = B;
    p.scale = a.scale;
    p.direct = slices == 1;
    p.accumulate = a.accumulate && p.direct;
    // A SwiGLU source reads the w13 GEMV's partials in slot 0.
    p.out = p.direct ? a.C
                     : scratch(SRC == kSrcSwiGLU ? kPartialFromPartial : kPartial,
                               static_cast<size_t>(slices) * a.n);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, a.stream, p); };
    if constexpr (std::is_same<BT, int8_t>::value) {
        if (E == 16) {
            switch (L) {
                case 4: go(gemv_kernel<BT, 1, 16, 4, 0, SRC>); break;
                case 8: go(gemv_kernel<BT, 1, 16, 8, 0, SRC>); break;
                default: go(gemv_kernel<BT, 1, 16, 16, 0, SRC>); break;
            }
            *partial = p.direct ? nullptr : p.out;
            return slices;
        }
    }
    switch (L) {
        case 4: go(gemv_kernel<BT, 1, 4, 4, 0, SRC>); break;
        case 8: go(gemv_kernel<BT, 1, 4, 8, 0, SRC>); break;
        case 16: go(gemv_kernel<BT, 1, 4, 16, 0, SRC>); break;
        default: go(gemv_kernel<BT, 1, 4, 32, 0, SRC>); break;
    }
    *partial = p.direct ? nullptr : p.out;
    return slices;
}

// The slice sum after a formed-source GEMV, as run_skinny's.
template <class BT>
int finish_formed(const MatmulArgs& a, int slices, const float* partial, float* ssq) {
    if (slices > 1)
        run_reduce_slices(1, a.n, slices, partial,
                          std::is_same<BT, int8_t>::value ? a.scale : nullptr, a.C,
                          a.accumulate, a.stream, ssq);
    return slices;
}

}  // namespace

// x (k = hidden) = silu_mul of a Summed w13 product, times W (hidden x n),
// one row: the forward pass's SwiGLU and w2 product in one GEMV.
template <class BT>
int run_skinny_swiglu(const MatmulArgs& a, const Summed& gu, int hidden, float* ssq) {
    if (a.m != 1 || gu.slices > kSwiSlices || a.rms_weight) return 0;
    GemvParams<BT> p{};
    p.gu = gu;
    p.hidden = hidden;
    const float* partial = nullptr;
    const int slices = run_formed_partials<BT, kSrcSwiGLU>(a, p, &partial);
    return finish_formed<BT>(a, slices, partial, ssq);
}

// Attention output (k = heads x head_size) merged from its chunks, times W,
// one row: the merge kernel's work inside the wo GEMV.
template <class BT>
int run_skinny_merged(const MatmulArgs& a, const SplitRow& att, float* ssq) {
    if (a.m != 1 || a.rms_weight || att.splits < 1 ||
        static_cast<long long>(att.n_heads) * att.head_size != a.k)
        return 0;
    GemvParams<BT> p{};
    p.att = att;
    const float* partial = nullptr;
    const int slices = run_formed_partials<BT, kSrcMerge>(a, p, &partial);
    return finish_formed<BT>(a, slices, partial, ssq);
}

template int run_skinny_swiglu<float>(const MatmulArgs&, const Summed&, int, float*);
template int run_skinny_swiglu<int8_t>(const MatmulArgs&, const Summed&, int, float*);
template int run_skinny_merged<float>(const MatmulArgs&, const SplitRow&, float*);
template int run_skinny_merged<int8_t>(const MatmulArgs&, const SplitRow&, float*);

template <class BT>
void run_skinny(const MatmulArgs& a) {
    const float* partial = nullptr;
    const int slices = run_skinny_partials<BT>(a, &partial);
    if (slices > 1)
        run_reduce_slices(a.m, a.n, slices, partial,
                          std::is_same<BT, int8_t>::value ? a.scale : nullptr, a.C,
                          a.accumulate, a.stream);
}

template std::size_t skinny_partial_floats<float>(const MatmulArgs&);
template std::size_t skinny_partial_floats<int8_t>(const MatmulArgs&);
template int run_skinny_partials<float>(const MatmulArgs&, const float**);
template int run_skinny_partials<int8_t>(const MatmulArgs&, const float**);
template void run_skinny<float>(const MatmulArgs&);
template void run_skinny<int8_t>(const MatmulArgs&);

}  // namespace em
