// One-launch decode GEMV for int8 B: k split in two halves across
// workgroups, the halves combined through one 64-bit atomic exchange per
// output, with no fence and no second launch (the skinny path's reference
// is sgemm_skinny + sum_slices, /root/reference/src/cuda_matmul.cu:189-254,
// 365-397).
//
// Why this shape. At m = 1 a 4096^2 int8 product needs the whole chip to
// stream its 16 MiB, so k has to be split across workgroups, and the split
// has to be summed. A second launch costs a full dependent-launch floor; an
// in-kernel "last workgroup adds the slices" needs an agent-scope release by
// every workgroup and an acquire by the last, and on gfx950 those fences
// cost more than the launch. A single atomic location per output needs
// neither: every atomic read-modify-write of one location is ordered, so of
// the two halves' exchanges the second always reads the first's word.
//
//  * Workgroup (tile, half): 256 threads over 32 columns and half of k. Two
//    lanes share a row (16 int8 columns each, one 16-byte nontemporal load),
//    so a wave reads 32 rows x 32 bytes per instruction; each lane issues all
//    of its L loads (rows rg, rg + 128, ...) before it uses any.
//  * Sums are unscaled, in fp32. The 32 lanes of a wave that hold the same
//    columns are added by a xor butterfly (every lane ends with the same
//    bits), then the four waves in LDS in wave order.
//  * Thread j < 32 exchanges (1 << 32 | bits(sum)) into word[column] with
//    relaxed agent-scope atomics. If it reads back a word with the flag set
//    it arrived second: it adds the two halves in half order from +0, scales,
//    accumulates and stores C exactly as reduce_slices does for two slices,
//    then stores 0 back so the word is clear for the next call. The first
//    arrival does nothing more. A later call is a later kernel, which sees
//    the cleared word.
#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

constexpr int kPairCols = 32;        // columns per workgroup
constexpr int kPairRows = kThreads / 2;  // rows per pass: two lanes per row

struct PairParams {
    int m, n, k;
    int ks;  // rows per half
    const float* A;
    const int8_t* B;
    const float* scale;
    float* C;
    int accumulate;
    unsigned long long* word;  // m x n exchange words, zero between calls
};

template <int MM, int L>
__global__ __launch_bounds__(kThreads) void gemv_pair_kernel(PairParams p) {
    constexpr int R = kPairRows * L;  // rows of B per workgroup
    constexpr int AREG = (MM * R + kThreads - 1) / kThreads;
    __shared__ float a_s[MM * R];
    __shared__ float red[4][MM][kPairCols];

    const int tid = threadIdx.x;
    const int cg = tid & 1, rg = tid >> 1;
    const int col = blockIdx.x * kPairCols + cg * 16;
    const int lcol = col < p.n ? col : 0;
    const int half = blockIdx.y;
    const int r0 = half * p.ks;
    const int r1 = min(p.k, r0 + p.ks);

    // This half's A, raw, into registers before the weights (its wait then
    // does not include them); rows past the half or past m stage as zero.
    float a_reg[AREG];
#pragma unroll
    for (int t = 0; t < AREG; ++t) {
        const int idx = tid + t * kThreads;
        const int r = idx / R, pp = r0 + idx % R;
        a_reg[t] = (idx < MM * R && r < p.m && pp < r1) ? p.A[r * p.k + pp] : 0.0f;
    }
    // All L weight vectors in flight; rows past k read row k - 1 (their A is
    // zero) and lanes past n read column 0 (their sums are never used).
    uint4 w[L];
#pragma unroll
    for (int i = 0; i < L; ++i) {
        const int pp = min(r0 + rg + i * kPairRows, p.k - 1);
        w[i] = stream_load(reinterpret_cast<const uint4*>(p.B + static_cast<uint32_t>(pp * p.n + lcol)));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < AREG; ++t) {
        const int idx = tid + t * kThreads;
        if (idx < MM * R) a_s[idx] = a_reg[t];
    }
    __syncthreads();

    float acc[MM][16];
#pragma unroll
    for (int r = 0; r < MM; ++r)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[r][j] = 0.0f;
#pragma unroll
    for (int i = 0; i < L; ++i) {
        float b[16];
        widen4(w[i].x, b);
        widen4(w[i].y, b + 4);
        widen4(w[i].z, b + 8);
        widen4(w[i].w, b + 12);
        const int pl = rg + i * kPairRows;
#pragma unroll
        for (int r = 0; r < MM; ++r) {
            const float a = a_s[r * R + pl];
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[r][j] = fmaf(a, b[j], acc[r][j]);
        }
    }

    // Lanes of one parity in a wave hold the same 16 columns for 32 rows.
#pragma unroll
    for (int r = 0; r < MM; ++r)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            float v = acc[r][j];
#pragma unroll
            for (int o = 2; o < kWave; o <<= 1) v += __shfl_xor(v, o, kWave);
            acc[r][j] = v;
        }
    const int wave = tid / kWave, lane = tid % kWave;
    if (lane < 2) {
#pragma unroll
        for (int r = 0; r < MM; ++r)
#pragma unroll
            for (int j = 0; j < 16; ++j) red[wave][r][lane * 16 + j] = acc[r][j];
    }
    __syncthreads();

    if (tid < MM * kPairCols) {
        const int r = tid / kPairCols, j = tid % kPairCols;
        const int c = blockIdx.x * kPairCols + j;
        if (r < p.m && c < p.n) {
            const float mine = ((red[0][r][j] + red[1][r][j]) + red[2][r][j]) + red[3][r][j];
            const size_t i = static_cast<size_t>(r) * p.n + c;
            const unsigned long long put = (1ull << 32) | __float_as_uint(mine);
            const unsigned long long got =
                __hip_atomic_exchange(p.word + i, put, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (got >> 32) {
                const float other = __uint_as_float(static_cast<uint32_t>(got));
                const float p0 = half == 0 ? mine : other;
                const float p1 = half == 0 ? other : mine;
                float total = 0.0f;
                total += p0;
                total += p1;
                total *= p.scale[c];
                float* o = p.C + i;
                *o = p.accumulate ? *o + total : total;
                __hip_atomic_store(p.word + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

template <int MM>
void launch_pair(int L, const PairParams& p, dim3 grid, hipStream_t s) {
    switch (L) {
        case 4: hipLaunchKernelGGL((gemv_pair_kernel<MM, 4>), grid, dim3(kThreads), 0, s, p); break;
        case 8: hipLaunchKernelGGL((gemv_pair_kernel<MM, 8>), grid, dim3(kThreads), 0, s, p); break;
        case 16: hipLaunchKernelGGL((gemv_pair_kernel<MM, 16>), grid, dim3(kThreads), 0, s, p); break;
        default: hipLaunchKernelGGL((gemv_pair_kernel<MM, 32>), grid, dim3(kThreads), 0, s, p); break;
    }
}

}  // namespace

bool gemv_pair_supports(const MatmulArgs& a) {
    return a.m == 1 && !a.rms_weight && a.n % 16 == 0 &&
           reinterpret_cast<uintptr_t>(a.B) % 16 == 0 && a.k >= 2 &&
           a.k <= 2 * kPairRows * 32;
}

void run_gemv_pair(const MatmulArgs& a) {
    PairParams p{};
    p.m = a.m;
    p.n = a.n;
    p.k = a.k;
    p.ks = ceil_div(a.k, 2);
    p.A = a.A;
    p.B = static_cast<const int8_t*>(a.B);
    p.scale = a.scale;
    p.C = a.C;
    p.accumulate = a.accumulate ? 1 : 0;
    p.word = exchange_words(static_cast<std::size_t>(a.m) * a.n);
    int L = 4;
    while (kPairRows * L < p.ks) L *= 2;
    const dim3 grid(ceil_div(a.n, kPairCols), 2);
    launch_pair<1>(L, p, grid, a.stream);
}

}  // namespace em
