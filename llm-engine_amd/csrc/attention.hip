// Causal attention over a KV cache, the step after the qkv projection of a
// decode or prefill pass (reference: cuda_attention.h:8-39, attention_single
// and attention_split in cuda_attention.cu:39-285, attention_cuda :339-362).
//
// Row i of a call sits at position *pos + i and attends to cached positions
// [0, *pos + i]; query head h reads kv head h / (n_heads / n_kv_heads).
// out[i][h*hs + d] = sum_t softmax_t(q . k_t / sqrt(hs)) v_t[d]. The position
// is read on the device, so one captured graph serves every position.
//
// Two kernels, both for 256-thread workgroups of four wave64s:
//
//  * split (decode, few rows): workgroup (head group, row, chunk) covers one
//    chunk of the context for the G query heads that share a kv head, so a
//    key or value row is loaded once for all G. A position's key and value
//    are read by a power-of-two group of lanes, float4 each, contiguous
//    across the group; every key and value of a 64-position round is loaded
//    before any is used, and the dot products are finished with xor shuffles
//    inside the wave. Each lane group keeps an online softmax of its
//    positions in registers; the groups are merged in LDS in a fixed order.
//    The chunk's softmax is left unnormalised (max m, sum l, exp-weighted
//    values o) in scratch, and a second kernel merges the chunks of each
//    (row, head) in chunk order. The merge is a separate launch rather than a
//    "last workgroup merges" arrival: on gfx950 every cross-workgroup arrival
//    measured slower than a second launch, and the fixed merge order keeps
//    results bit-identical across calls. A context that fits one chunk is
//    normalised and written by the first kernel; the merge kernel then exits.
//    With more rows (prefill), automatic runs the tile kernel (16
//    query rows per wave on fp32 MFMA), split over the context as well when
//    its grid is small; for head sizes it is not built for, the same split
//    kernel with one chunk per row: the whole context in rounds, no merge.
//  * single_block (on request): workgroup (head, row) holds the query and
//    the scores of the whole context in LDS; any head size.
//
// The grid is sized for seq_len, never for the position: chunks past the end
// of a row's context return at once.
#include <algorithm>
#include <cmath>
#include <string>

#include "common.hpp"
#include "internal.hpp"

namespace em {
namespace {

// Chunks per (row, head group), at most: past 128 the merge's extra chunks
// cost more than the shorter chunks save (context 16384, 32 heads / 8 kv
// heads: 105.4 / 39.3 us at 256, 103.5 / 36.5 at 128; shorter contexts
// never reach the cap).
constexpr int kMaxSplits = 128;
constexpr std::size_t kSplitMaxRows = 12;  // automatic: split up to this many rows, at most
constexpr std::size_t kMaxLds = 64 * 1024;  // dynamic LDS per workgroup

// Query heads per split workgroup: the most of 8, 4, 2, 1 that divides the
// heads sharing a kv head.
int heads_per_block(const AttnShape& s) {
    const int group = s.n_heads / s.n_kv_heads;
    for (int g : {8, 4, 2})
        if (group % g == 0) return g;
    return 1;
}

// Positions per split workgroup, at least (split_chunk).
int min_chunk(const AttnShape& s) {
    return heads_per_block(s) > 1 ? kSplitMinChunkGrouped : kSplitMinChunk;
}

int split_count(const AttnShape& s) {
    const int mc = min_chunk(s);
    const int n = (s.seq_len + mc - 1) / mc;
    return n < kMaxSplits ? n : kMaxSplits;
}

int split_chunk_cap(const AttnShape& s) {
    return split_chunk(s.seq_len, split_count(s), min_chunk(s));
}

std::size_t single_lds(const AttnShape& s) {
    return (static_cast<std::size_t>(s.head_size) + s.seq_len + kThreads) * sizeof(float);
}

// Lanes per position of the split kernel: head_size / 4 rounded up to a
// power of two in [4, 64]; F float4 columns per lane.
int split_lanes(const AttnShape& s) {
    const int hs4 = s.head_size / 4;
    int l = 4;
    while (l < hs4 && l < kWave) l <<= 1;
    return l;
}
int split_f(const AttnShape& s) { return (s.head_size / 4 + split_lanes(s) - 1) / split_lanes(s); }

// LDS of the in-kernel merge (merge_chunks): one float4 and one (max, sum)
// pair per thread.
constexpr std::size_t kMergeLds = kThreads * (sizeof(floatx4) + sizeof(float2));

// Slot merge buffers, plus with RoPE fused the G queries, key and value (and
// at least the in-kernel merge's buffers when it merges its own chunks).
std::size_t split_lds(const AttnShape& s, bool rope = false, bool merge_inside = false) {
    const std::size_t G = heads_per_block(s), hs = s.head_size;
    const std::size_t ns = kThreads / split_lanes(s);
    const std::size_t lds = (G * ns * hs + 2 * G * ns + (rope ? (G + 2) * hs : 0)) * sizeof(float);
    return merge_inside && lds < kMergeLds ? kMergeLds : lds;
}

struct SplitScratch {
    std::size_t o, ml, total;  // offsets and size in floats
};

SplitScratch split_scratch(const AttnShape& s, std::size_t rows) {
    const std::size_t blocks = rows * s.n_heads * split_count(s);
    auto up4 = [](std::size_t x) { return (x + 3) / 4 * 4; };
    SplitScratch l{};
    l.o = 0;
    l.ml = up4(blocks * s.head_size);
    l.total = l.ml + up4(2 * blocks);
    return l;
}

// automatic: the split kernel with chunks across workgroups for few rows,
// beyond that the tile kernel (16 query rows per wave on fp32 MFMA, each key
// and value row loaded once per 16 rows, split over the context when its
// grid is small) for head sizes it is built for; other head sizes run the
// split kernel with one chunk per row (the whole context, in rounds of 64
// positions, no merge) from 13 rows. The split kernel's cost grows with the
// rows (each reads its chunks' keys and values); the split tile kernel's
// hardly does below 16. Measured at 7B shapes (MHA / 8 kv heads), split
// against split tile, us:
//   context  256, 2-12 rows: 10.0-14.5 / 15.4-15.7, 12.0-14.8 / 14.2-15.4
//   context 1024, 4 rows:    18.2 / 18.5, 14.9 / 17.4; 8 rows: 25.1 / 19.0, 20.9 / 17.9
//   context 4096, 4 rows:    48.4 / 41.0, 31.6 / 33.7; 8 rows: 75.4 / 41.1, 51.8 / 33.9
// The context is read on the device, so the cut goes by seq_len: up to 5
// rows split when seq_len exceeds 512, up to 12 otherwise (and for head
// sizes the tile kernel does not take).
constexpr int kAttnWhole = 3;
constexpr int kAttnTile = 4;
constexpr int kTileRows = 16;        // query rows per tile wave
constexpr int kTileMaxHeadSize = 128;

bool tile_supports(const AttnShape& s) {
    return s.head_size % 16 == 0 && s.head_size <= kTileMaxHeadSize;
}

// A tile grid of a few row tiles has one workgroup per (head, 16 rows): 32
// workgroups for 16 rows of a 32-head model, which took 108-114 us at
// context 4096 whatever the row count. Such a grid is split over the
// context as well, into chunks of at least kTileChunkMin positions, enough
// to bring it near kTileTargetGroups workgroups; each chunk leaves its
// unnormalised softmax for the merge kernel, as the split kernel's do.
// Grids of 512 workgroups or more are not split.
constexpr int kTileChunkMin = 256;
constexpr long long kTileTargetGroups = 1024;

int tile_splits(const AttnShape& s, std::size_t rows) {
    const long long tiles = static_cast<long long>(s.n_heads) *
                            static_cast<long long>((rows + kTileRows - 1) / kTileRows);
    if (tiles >= kTileTargetGroups / 2) return 1;
    const long long want = (kTileTargetGroups + tiles - 1) / tiles;
    const long long cap = (s.seq_len + kTileChunkMin - 1) / kTileChunkMin;
    return static_cast<int>(std::max(1LL, std::min(want, cap)));
}

// Positions per chunk: a multiple of 64, so chunks are whole 16-position
// blocks, and splits chunks cover seq_len.
int tile_chunk(const AttnShape& s, int splits) {
    const int c = (s.seq_len + splits - 1) / splits;
    return (c + 63) / 64 * 64;
}

SplitScratch tile_scratch(const AttnShape& s, std::size_t rows, int splits) {
    const std::size_t blocks = rows * s.n_heads * static_cast<std::size_t>(splits);
    auto up4 = [](std::size_t x) { return (x + 3) / 4 * 4; };
    SplitScratch l{};
    l.o = 0;
    l.ml = up4(blocks * s.head_size);
    l.total = l.ml + up4(2 * blocks);
    return l;
}

std::size_t split_max_rows(const AttnShape& s) {
    return tile_supports(s) && s.seq_len > 512 ? 5 : kSplitMaxRows;
}

int resolve(int kernel, std::size_t rows, const AttnShape& s) {
    if (kernel != kAttnAutomatic) return kernel;
    if (rows <= split_max_rows(s)) return kAttnSplit;
    return tile_supports(s) ? kAttnTile : kAttnWhole;
}

struct AttnArgs {
    int n_heads, head_size, group, seq_len, splits, chunk_cap, rows;
    int min_chunk;   // split_chunk's least chunk for this shape
    int merge_from;  // the merge kernel takes rows of at least this many chunks (>= 2)
    int tile_chunk;  // tile kernel split over the context: positions per chunk (0: no split)
    int q_stride, kv_stride, out_stride;
    const int* pos;
    const float* q;
    const float* kc;
    const float* vc;
    float* part_o;
    float2* part_ml;
    float* out;
    // One-row decode with RoPE fused (attn_split_kernel<..., true>): the qkv
    // product as its consumers read it (q at column 0, k at dim, v at
    // dim + kv_dim), the rotation tables, and the caches to write.
    Summed src;
    int dim, kv_dim;
    const float* cos_t;
    const float* sin_t;
    float* kc_w;
    float* vc_w;
    // Non-null: a row split over several chunks is merged by the last of
    // its chunks' workgroups to finish (one counter per row and head group,
    // zero between calls), not by a merge launch.
    unsigned* merge_count;
};

// Lanes per key row: hs4 rounded up to a power of two, at most one wave.
__device__ __forceinline__ int lanes_per_row(int n) {
    int l = 1;
    while (l < n && l < kWave) l <<= 1;
    return l;
}

// Positions a lane group loads per round, at most: all of a round's key and
// value loads are issued before any is used.
constexpr int kRoundPerSlot = 8;

constexpr int kMergeDims = 8;
constexpr int kSc1 = 16;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));  // the cache-policy operand's sc1 bit (device-coherent access)

// The merge of the n chunks of heads h0 .. h0 + G - 1 of row i, inside the
// split launch by the last of the row's chunk workgroups: the arithmetic of
// attn_merge_kernel (below), which a merge launch would run, in the same
// slots and order, so the result has its bits. Each (head, group of dpw
// float4 columns) the merge kernel gives a workgroup is given a team of
// used x dpw threads here, as many teams at once as 256 threads hold. The
// chunks' partials, stored by other workgroups of this launch, are read with
// device-coherent (sc1) loads.
__device__ void merge_chunks(const AttnArgs& a, int i, int h0, int G, int n, float* lds) {
    const int hs4 = a.head_size / 4;
    const int dpw = hs4 < kMergeDims ? hs4 : kMergeDims, groups = (hs4 + dpw - 1) / dpw;
    const int slots = kThreads / dpw, used = min(slots, (n + 7) / 8);
    const int T = used * dpw, teams = kThreads / T, combos = G * groups;
    floatx4* red4 = reinterpret_cast<floatx4*>(lds);
    float2* red_ml = reinterpret_cast<float2*>(red4 + kThreads);
    const __amdgpu_buffer_rsrc_t ors =
        __builtin_amdgcn_make_buffer_rsrc(a.part_o, 0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t mrs =
        __builtin_amdgcn_make_buffer_rsrc(a.part_ml, 0, 0x7fffffff, 0x00020000);
    const int tid = threadIdx.x, team = tid / T, w = tid % T, r = w / dpw, dd = w % dpw;
    for (int base = 0; base < combos; base += teams) {
        const int combo = base + team;
        const bool active = team < teams && combo < combos;
        const int g = active ? combo / groups : 0;
        const int d = (active ? combo % groups : 0) * dpw + dd;
        const bool dok = d < hs4;
        const int dl = dok ? d : hs4 - 1;  // past the head: computed, not stored
        const uint32_t b = static_cast<uint32_t>((i * a.n_heads + h0 + g) * a.splits);
        if (active) {
            float m = -INFINITY, l = 0.0f;
            floatx4 acc{0.f, 0.f, 0.f, 0.f};
            for (int c0 = r; c0 < n; c0 += 8 * used) {
                float2 ml[8];
                floatx4 o[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint32_t c = b + min(c0 + u * used, n - 1);
                    ml[u] = __builtin_bit_cast(
                        float2, __builtin_amdgcn_raw_buffer_load_b64(mrs, c * 8, 0, kSc1));
                    o[u] = __builtin_bit_cast(
                        floatx4, __builtin_amdgcn_raw_buffer_load_b128(ors, (c * hs4 + dl) * 16, 0, kSc1));
                }
                merge_batch8(m, l, acc, ml, o, c0, used, n);
            }
            red4[team * T + r * dpw + dd] = acc;
            if (dd == 0) red_ml[team * used + r] = make_float2(m, l);
        }
        __syncthreads();
        if (active && w < dpw && dok) {
            reinterpret_cast<floatx4*>(a.out + static_cast<std::size_t>(i) * a.out_stride +
                                       static_cast<std::size_t>(h0 + g) * a.head_size)[d] =
                merge_combine(used, floatx4{0.f, 0.f, 0.f, 0.f},
                              [&](int rr) { return red_ml[team * used + rr]; },
                              [&](int rr) { return red4[team * T + rr * dpw + w]; });
        }
        __syncthreads();
    }
}

// Split workgroup: (head group hg, row i, chunk s). Thread = (slot, sub): the
// LPP lanes of a slot share a position and hold float4 columns
// d = sub + f * LPP of it (F per lane). Each slot keeps an online softmax of
// its positions in registers (running max m, sum l, weighted values o) for
// the G heads; the NS = 256 / LPP slots are then merged in LDS in slot order.
//
// ROPE (one row, the forward pass's decode step): the query is not read
// from a.q but formed here from the qkv product (a.src): summed, rotated as
// rope_cache_kernel rotates it (rope_pair), into LDS. The last chunk also
// forms the current position's key and value, writes them to the caches
// (the workgroup of the first head group of each kv head) and takes that
// position in slot 0 after its loop, from LDS: no workgroup reads a cache
// row written in the same launch.
template <int G, int LPP, int F, bool ROPE = false>
__global__ __launch_bounds__(kThreads) void attn_split_kernel(AttnArgs a) {
    constexpr int NS = kThreads / LPP;
    constexpr int MC = G > 1 ? kSplitMinChunkGrouped : kSplitMinChunk;  // min_chunk of the shape
    constexpr int PP = MC / NS < kRoundPerSlot ? (MC / NS > 0 ? MC / NS : 1) : kRoundPerSlot;
    constexpr int ROUND = NS * PP;
    extern __shared__ float lds[];

    const int hs = a.head_size, hs4 = hs / 4;
    const int hg = blockIdx.x, i = blockIdx.y, s = blockIdx.z;
    const int n_ctx = *a.pos + i + 1;
    const int chunk = split_chunk(n_ctx, a.splits, a.min_chunk);
    const int t0 = s * chunk;
    if (t0 >= n_ctx) return;  // uniform across the workgroup
    const int len = min(chunk, n_ctx - t0);
    const int nchunks = (n_ctx + chunk - 1) / chunk;
    const int h0 = hg * G;
    const int kv_off = (h0 / a.group) * hs;
    const int tid = threadIdx.x, sub = tid % LPP, slot = tid / LPP;
    // With ROPE the last position (the current one) is not in the cache yet.
    const bool own_pos = ROPE && s == nchunks - 1;
    const int loop_len = own_pos ? len - 1 : len;
    float* rq = lds + G * NS * hs + 2 * G * NS;  // ROPE: G rotated queries, key, value

    // This lane's columns; lanes past hs4 read the last column with a zero
    // query and store nothing.
    int dcol[F];
    bool dok[F];
#pragma unroll
    for (int f = 0; f < F; ++f) {
        const int d = sub + f * LPP;
        dok[f] = d < hs4;
        dcol[f] = dok[f] ? d : hs4 - 1;
    }
    const float* kbase = a.kc + static_cast<std::size_t>(t0) * a.kv_stride + kv_off;
    const float* vbase = a.vc + static_cast<std::size_t>(t0) * a.kv_stride + kv_off;
    // Every key and value of a round in flight; positions past the chunk
    // re-read its last position and are masked. (Issuing the first round
    // before the ROPE query is formed measured 1 us slower at ctx 512: the
    // query's loads then wait behind the whole chunk's.)
    floatx4 kv[PP][F], vv[PP][F];
    auto load_round = [&](int b0) {
#pragma unroll
        for (int pp = 0; pp < PP; ++pp) {
            const int t = min(b0 + slot + pp * NS, loop_len - 1);
            const floatx4* kr = reinterpret_cast<const floatx4*>(kbase + static_cast<std::size_t>(t) * a.kv_stride);
            const floatx4* vr = reinterpret_cast<const floatx4*>(vbase + static_cast<std::size_t>(t) * a.kv_stride);
#pragma unroll
            for (int f = 0; f < F; ++f) {
                kv[pp][f] = kr[dcol[f]];
                vv[pp][f] = vr[dcol[f]];
            }
        }
    };

    if constexpr (ROPE) {
        const int pos = n_ctx - 1, half = hs / 2;
        const float* cs = a.cos_t + static_cast<std::size_t>(pos) * half;
        const float* sn = a.sin_t + static_cast<std::size_t>(pos) * half;
        const bool writer = h0 % a.group == 0;
        const int nq = G * hs4, total = nq + (own_pos ? 2 * hs4 : 0);
        for (int j = tid; j < total; j += kThreads) {
            int col, d;
            bool rot = true;
            if (j < nq) {
                d = j % hs4;
                col = h0 * hs + 4 * j;
            } else if (j < nq + hs4) {
                d = j - nq;
                col = a.dim + kv_off + 4 * d;
            } else {
                d = j - nq - hs4;
                col = a.dim + a.kv_dim + kv_off + 4 * d;
                rot = false;
            }
            // The angles are loaded for values too (d < hs4, so in range) and
            // before the product's slices: one wait covers every load here
            // and the first round of keys and values.
            const float c0 = cs[2 * d], s0 = sn[2 * d], c1 = cs[2 * d + 1], s1 = sn[2 * d + 1];
            const floatx4 x = summed4(a.src, 0, col);
            floatx4 y = x;
            if (rot) {
                const float2 r0 = rope_pair(x.x, x.y, c0, s0);
                const float2 r1 = rope_pair(x.z, x.w, c1, s1);
                y = floatx4{r0.x, r0.y, r1.x, r1.y};
            }
            reinterpret_cast<floatx4*>(rq)[j] = y;
            if (j >= nq && writer) {
                float* cache = j < nq + hs4 ? a.kc_w : a.vc_w;
                reinterpret_cast<floatx4*>(cache + static_cast<std::size_t>(pos) * a.kv_stride +
                                           kv_off)[d] = y;
            }
        }
        __syncthreads();
    }

    floatx4 q[G][F];
    const float* qrow = ROPE ? rq : a.q + static_cast<std::size_t>(i) * a.q_stride +
                                        static_cast<std::size_t>(h0) * hs;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int f = 0; f < F; ++f)
            q[g][f] = dok[f] ? reinterpret_cast<const floatx4*>(qrow + g * hs)[dcol[f]]
                             : floatx4{0.f, 0.f, 0.f, 0.f};

    const float scale = 1.0f / sqrtf(static_cast<float>(hs));
    float m[G], l[G];
    floatx4 o[G][F];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int f = 0; f < F; ++f) o[g][f] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

    for (int b0 = 0; b0 < loop_len; b0 += ROUND) {
        load_round(b0);
        float sc[G][PP];
#pragma unroll
        for (int pp = 0; pp < PP; ++pp) {
            const bool valid = b0 + slot + pp * NS < loop_len;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float dot = 0.0f;
#pragma unroll
                for (int f = 0; f < F; ++f) {
                    const floatx4 x = q[g][f] * kv[pp][f];
                    dot += (x.x + x.y) + (x.z + x.w);
                }
#pragma unroll
                for (int off = LPP / 2; off > 0; off >>= 1) dot += __shfl_xor(dot, off, kWave);
                sc[g][pp] = valid ? dot * scale : -INFINITY;
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mb = sc[g][0];
#pragma unroll
            for (int pp = 1; pp < PP; ++pp) mb = fmaxf(mb, sc[g][pp]);
            const float mn = fmaxf(m[g], mb);
            if (mn == -INFINITY) continue;  // no position of this slot yet
            const float alpha = expf(m[g] - mn);
            l[g] *= alpha;
#pragma unroll
            for (int f = 0; f < F; ++f) o[g][f] *= alpha;
#pragma unroll
            for (int pp = 0; pp < PP; ++pp) {
                const float e = expf(sc[g][pp] - mn);
                l[g] += e;
#pragma unroll
                for (int f = 0; f < F; ++f) o[g][f] += e * vv[pp][f];
            }
            m[g] = mn;
        }
    }

    if (own_pos && slot == 0) {
        // The current position, in slot 0: its key and value from LDS.
        floatx4 kx[F], vx[F];
#pragma unroll
        for (int f = 0; f < F; ++f) {
            kx[f] = reinterpret_cast<const floatx4*>(rq + G * hs)[dcol[f]];
            vx[f] = reinterpret_cast<const floatx4*>(rq + G * hs + hs)[dcol[f]];
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float dot = 0.0f;
#pragma unroll
            for (int f = 0; f < F; ++f) {
                const floatx4 x = q[g][f] * kx[f];
                dot += (x.x + x.y) + (x.z + x.w);
            }
#pragma unroll
            for (int off = LPP / 2; off > 0; off >>= 1) dot += __shfl_xor(dot, off, kWave);
            const float sc = dot * scale;
            const float mn = fmaxf(m[g], sc);
            const float alpha = expf(m[g] - mn);
            const float e = expf(sc - mn);
            l[g] = l[g] * alpha + e;
#pragma unroll
            for (int f = 0; f < F; ++f) o[g][f] = o[g][f] * alpha + e * vx[f];
            m[g] = mn;
        }
    }

    // Merge the slots in slot order: o_s[g][slot][hs], ml_s[g][slot][2].
    float* o_s = lds;
    float* ml_s = lds + G * NS * hs;
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int f = 0; f < F; ++f)
            if (dok[f])
                reinterpret_cast<floatx4*>(o_s + (g * NS + slot) * hs)[dcol[f]] = o[g][f];
        if (sub == 0) {
            ml_s[(g * NS + slot) * 2] = m[g];
            ml_s[(g * NS + slot) * 2 + 1] = l[g];
        }
    }
    __syncthreads();

    const std::size_t head_row = static_cast<std::size_t>(i) * a.n_heads + h0;
    for (int j = tid; j < G * hs4; j += kThreads) {
        const int g = j / hs4, d = j % hs4;
        const float* mlg = ml_s + g * NS * 2;
        float M = -INFINITY;
        for (int sl = 0; sl < NS; ++sl) M = fmaxf(M, mlg[2 * sl]);
        float L = 0.0f;
        floatx4 O{0.f, 0.f, 0.f, 0.f};
        for (int sl = 0; sl < NS; ++sl) {
            const float w = expf(mlg[2 * sl] - M);  // 0 for a slot with no position
            L += w * mlg[2 * sl + 1];
            O += w * reinterpret_cast<const floatx4*>(o_s + (g * NS + sl) * hs)[d];
        }
        if (nchunks == 1) {
            reinterpret_cast<floatx4*>(a.out + static_cast<std::size_t>(i) * a.out_stride +
                                       static_cast<std::size_t>(h0 + g) * hs)[d] = O * (1.0f / L);
        } else if (a.merge_count) {
            // Device-coherent stores: the row's last workgroup reads them.
            const uint32_t c = static_cast<uint32_t>((head_row + g) * a.splits + s);
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4, O),
                __builtin_amdgcn_make_buffer_rsrc(a.part_o, 0, 0x7fffffff, 0x00020000),
                (c * hs4 + d) * 16, 0, kSc1);
            if (d == 0)
                __builtin_amdgcn_raw_buffer_store_b64(
                    __builtin_bit_cast(u32x2, make_float2(M, L)),
                    __builtin_amdgcn_make_buffer_rsrc(a.part_ml, 0, 0x7fffffff, 0x00020000),
                    c * 8, 0, kSc1);
        } else {
            reinterpret_cast<floatx4*>(a.part_o)[((head_row + g) * a.splits + s) * hs4 + d] = O;
            if (d == 0) a.part_ml[(head_row + g) * a.splits + s] = make_float2(M, L);
        }
    }
    if (nchunks == 1 || !a.merge_count) return;
    // Counted in once every partial store above has landed; the last of the
    // row's chunks merges them and sets the counter back to zero.
    __shared__ unsigned arrived;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    unsigned* counter = a.merge_count + static_cast<std::size_t>(i) * gridDim.x + hg;
    if (tid == 0) arrived = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != static_cast<unsigned>(nchunks - 1)) return;
    merge_chunks(a, i, h0, G, nchunks, lds);
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merges the chunks of one (head, row): m = max m_c,
// l = sum e^(m_c - m) l_c, out = sum e^(m_c - m) o_c / l. A workgroup takes
// kMergeDims float4s of the head's columns (blockIdx.x = head * groups +
// group), so a long context's chunks spread over more workgroups. As many
// slots work as eight chunks each need (up to 256 / dpw): the dpw threads of
// slot r take chunks r, r + used, ..., loaded in one batch, and keep their
// own max, sum and output over them; the slots are then combined in slot
// order, each scaled by e^(its max - m), after one barrier. The result is
// the same on every call. (One workgroup per head took 8.7 us for 32 heads
// x 256 chunks: four dependent batches in each of 32 workgroups; always
// using every slot made 64 chunks slower, a 32-step combine.)

__global__ __launch_bounds__(kThreads) void attn_merge_kernel(AttnArgs a) {
    extern __shared__ floatx4 red4[];  // slots x dpw outputs, then slots x (max, sum)
    const int hs4 = a.head_size / 4;
    const int dpw = hs4 < kMergeDims ? hs4 : kMergeDims, groups = (hs4 + dpw - 1) / dpw;
    const int h = blockIdx.x / groups, d0 = (blockIdx.x % groups) * dpw;
    const int i = blockIdx.y;
    const int n_ctx = *a.pos + i + 1;
    const int chunk = a.tile_chunk ? a.tile_chunk : split_chunk(n_ctx, a.splits, a.min_chunk);
    const int n = (n_ctx + chunk - 1) / chunk;
    if (n < a.merge_from) return;  // one chunk: written by the split kernel; few: by their consumer
    const std::size_t b = (static_cast<std::size_t>(i) * a.n_heads + h) * a.splits;
    const int tid = threadIdx.x;
    const int slots = kThreads / dpw, r = tid / dpw, dd = tid % dpw, d = d0 + dd;
    const bool dok = d < hs4;
    const int dl = dok ? d : hs4 - 1;  // past the head: computed, not stored
    const floatx4* po = reinterpret_cast<const floatx4*>(a.part_o);
    float2* red_ml = reinterpret_cast<float2*>(red4 + slots * dpw);
    const int used = min(slots, (n + 7) / 8);  // slots that take chunks

    if (r < used) {
        float m = -INFINITY, l = 0.0f;
        floatx4 acc{0.f, 0.f, 0.f, 0.f};
        for (int c0 = r; c0 < n; c0 += 8 * used) {
            float2 ml[8];
            floatx4 o[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int c = min(c0 + u * used, n - 1);
                ml[u] = a.part_ml[b + c];
                o[u] = po[(b + c) * hs4 + dl];
            }
            merge_batch8(m, l, acc, ml, o, c0, used, n);
        }
        red4[r * dpw + dd] = acc;
        if (dd == 0) red_ml[r] = make_float2(m, l);
    }
    __syncthreads();
    if (tid < dpw && dok) {
        reinterpret_cast<floatx4*>(a.out + static_cast<std::size_t>(i) * a.out_stride +
                                   static_cast<std::size_t>(h) * a.head_size)[d] =
            merge_combine(used, floatx4{0.f, 0.f, 0.f, 0.f},
                          [&](int rr) { return red_ml[rr]; },
                          [&](int rr) { return red4[rr * dpw + tid]; });
    }
}

// One workgroup per (head, row): query and scores in LDS, scalar loads, so
// any head size works.
__global__ __launch_bounds__(kThreads) void attn_single_kernel(AttnArgs a) {
    extern __shared__ float lds[];
    __shared__ float part[4];
    const int hs = a.head_size;
    float* q_s = lds;               // hs
    float* sc = lds + hs;           // seq_len
    float* red = sc + a.seq_len;    // kThreads
    const int h = blockIdx.x, i = blockIdx.y;
    const int n_ctx = *a.pos + i + 1;
    const int kv_off = (h / a.group) * hs;
    const int tid = threadIdx.x;

    const float* qg = a.q + static_cast<std::size_t>(i) * a.q_stride + static_cast<std::size_t>(h) * hs;
    for (int d = tid; d < hs; d += kThreads) q_s[d] = qg[d];
    __syncthreads();

    const int lpp = lanes_per_row(hs);
    const int sub = tid % lpp, slot = tid / lpp, nslots = kThreads / lpp;
    const float scale = 1.0f / sqrtf(static_cast<float>(hs));
    for (int base = 0; base < n_ctx; base += nslots) {
        const int t = base + slot;
        float dot = 0.0f;
        if (t < n_ctx) {
            const float* k = a.kc + static_cast<std::size_t>(t) * a.kv_stride + kv_off;
            for (int d = sub; d < hs; d += lpp) dot += q_s[d] * k[d];
        }
        for (int o = lpp / 2; o > 0; o >>= 1) dot += __shfl_xor(dot, o, kWave);
        if (t < n_ctx && sub == 0) sc[t] = dot * scale;
    }
    __syncthreads();

    float m = -INFINITY;
    for (int t = tid; t < n_ctx; t += kThreads) m = fmaxf(m, sc[t]);
    m = block_max(m, part);
    float l = 0.0f;
    for (int t = tid; t < n_ctx; t += kThreads) {
        const float e = expf(sc[t] - m);
        sc[t] = e;
        l += e;
    }
    l = block_sum(l, part);  // its barriers also publish the exponentials
    const float inv = 1.0f / l;

    float* oh = a.out + static_cast<std::size_t>(i) * a.out_stride + static_cast<std::size_t>(h) * hs;
    const float* vb = a.vc + kv_off;
    if (hs <= kThreads) {
        const int d = tid % hs, r = tid / hs, slots = kThreads / hs;
        if (r < slots) {
            float acc = 0.0f;
            for (int t = r; t < n_ctx; t += slots)
                acc += sc[t] * vb[static_cast<std::size_t>(t) * a.kv_stride + d];
            red[r * hs + d] = acc;
        }
        __syncthreads();
        if (tid < hs) {
            float o = red[tid];
            for (int rr = 1; rr < slots; ++rr) o += red[rr * hs + tid];
            oh[tid] = o * inv;
        }
    } else {
        for (int d = tid; d < hs; d += kThreads) {
            float acc = 0.0f;
            for (int t = 0; t < n_ctx; ++t)
                acc += sc[t] * vb[static_cast<std::size_t>(t) * a.kv_stride + d];
            oh[d] = acc * inv;
        }
    }
}

// --- prefill rows: tiles of 16 queries on fp32 MFMA ------------------------
//
// One wave per (query head, 16 consecutive rows). For each block of 16
// cached positions it forms S^T = K Q^T (positions x queries) with
// v_mfma_f32_16x16x4_f32, then O^T += V^T P^T. In lane l (g = l / 16,
// j = l % 16):
//  * S^T: the lane supplies K[position j][d] and Q[query j][d] for the head
//    dims d of its lane group's quarter (4E contiguous floats, E = hs / 16),
//    so its key and query loads are float4 runs; both operands take the
//    head dims in the same order.
//  * S^T's output layout leaves in the lane the scores of query j at
//    positions 4g + r (r = 0..3) of the block: exactly the B operand
//    P^T[position 4g + r][query j] of k-step r of the V product, so scores
//    never leave the lane's registers.
//  * V^T: lane j supplies rows d = E j + c (c = 0..E-1, one MFMA each), E
//    contiguous floats of a value row; output block c then holds
//    O[query j][E (4g + r) + c], so the lane ends with 4E contiguous head
//    dims of its query.
//  * Every accumulator of a lane belongs to query j: the online softmax
//    rescale is one factor per lane. The block max takes two xor shuffles
//    (the four lane groups of a query); the sum is combined once, at the end.
// Positions past a query's own are masked, and blocks past the tile's last
// row are never read; the next block's keys and values are loaded while
// this one is used (two register sets, alternating; a 32-position block
// measured no faster and needs twice the registers).
//
// A workgroup is four such waves on one (head, 16-row tile): wave w takes
// the w-th quarter of the tile's blocks, keeping its own online softmax, and
// the four are merged in LDS in wave order at the end. Causal tiles differ
// in length up to 32-fold at 512 rows, and with one wave per tile the
// longest set the kernel's time. A query with no position in a wave's
// quarter leaves that wave's m = -inf, l = 0, O = 0.
template <int E>
struct TileBlock {
    floatx4 k[E];   // K[t0 + j][4E g .. 4E g + 4E)
    float v[4][E];  // per r: V[t0 + 4g + r][E j .. E j + E)
};

template <int E>
__device__ __forceinline__ void load_run(const float* src, float* dst) {
    if constexpr (E % 4 == 0) {
#pragma unroll
        for (int u = 0; u < E / 4; ++u) {
            const floatx4 x = reinterpret_cast<const floatx4*>(src)[u];
            dst[4 * u] = x.x;
            dst[4 * u + 1] = x.y;
            dst[4 * u + 2] = x.z;
            dst[4 * u + 3] = x.w;
        }
    } else if constexpr (E % 2 == 0) {
#pragma unroll
        for (int u = 0; u < E / 2; ++u) {
            const float2 x = reinterpret_cast<const float2*>(src)[u];
            dst[2 * u] = x.x;
            dst[2 * u + 1] = x.y;
        }
    } else {
#pragma unroll
        for (int u = 0; u < E; ++u) dst[u] = src[u];
    }
}

constexpr int kTileWaves = 4;

template <int E>
__global__ __launch_bounds__(kTileWaves * kWave) void attn_tile_kernel(AttnArgs a) {
    constexpr int HS = 16 * E, Q4 = 4 * E;
    constexpr int KB = 16;  // positions per block
    __shared__ float ms[kTileWaves][kWave], ls[kTileWaves][kWave];
    __shared__ floatx4 os[kTileWaves][E][kWave];
    const int lane = threadIdx.x % kWave, g = lane >> 4, j = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    // Row tiles in reverse: the longest (causal) start first and the short
    // ones fill in behind them.
    const int h = blockIdx.x, r0 = (gridDim.y - 1 - blockIdx.y) * kTileRows;
    const int pos0 = *a.pos;
    const int row = min(r0 + j, a.rows - 1);  // rows past the call: computed, not stored
    const int pq = pos0 + row;                // this lane's query position
    const int last = pos0 + min(r0 + kTileRows - 1, a.rows - 1);  // the wave's last position
    // Split over the context: this workgroup takes positions [lo, hi] of
    // chunk blockIdx.z (none past last: the grid is sized for seq_len).
    const int cz = blockIdx.z;
    const int lo = cz * a.tile_chunk;
    if (lo > last) return;
    const int hi = a.tile_chunk ? min(last, lo + a.tile_chunk - 1) : last;
    const float* kbase = a.kc + static_cast<std::size_t>((h / a.group) * HS);
    const float* vbase = a.vc + static_cast<std::size_t>((h / a.group) * HS);

    float q[Q4];
    load_run<Q4>(a.q + static_cast<std::size_t>(row) * a.q_stride + static_cast<std::size_t>(h) * HS + Q4 * g, q);

    // Positions past `last` re-read position `last` (in the cache: the
    // caller keeps *pos + rows <= seq_len) and are masked.
    auto load = [&](TileBlock<E>& b, int t0) {
        const int tk = min(t0 + j, last);
        const floatx4* kr = reinterpret_cast<const floatx4*>(
            kbase + static_cast<std::size_t>(tk) * a.kv_stride + Q4 * g);
#pragma unroll
        for (int u = 0; u < E; ++u) b.k[u] = kr[u];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tv = min(t0 + 4 * g + r, last);
            load_run<E>(vbase + static_cast<std::size_t>(tv) * a.kv_stride + E * j, b.v[r]);
        }
    };

    const float scale = 1.0f / sqrtf(static_cast<float>(HS));
    float m = -INFINITY, l = 0.0f;
    floatx4 o[E];
#pragma unroll
    for (int c = 0; c < E; ++c) o[c] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto use = [&](const TileBlock<E>& b, int t0) {
        // S^T in four accumulators (head-dim steps u mod 4), so consecutive
        // MFMAs are independent, added pairwise at the end.
        floatx4 sacc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) sacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < Q4; ++u) sacc[u & 3] = mfma16x16x4(b.k[u / 4][u % 4], q[u], sacc[u & 3]);
        float sv[4];
        float mb = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + 4 * g + r;
            const float x = ((sacc[0][r] + sacc[1][r]) + (sacc[2][r] + sacc[3][r])) * scale;
            sv[r] = t <= pq ? x : -INFINITY;
            mb = fmaxf(mb, sv[r]);
        }
        mb = fmaxf(mb, __shfl_xor(mb, 16, kWave));
        mb = fmaxf(mb, __shfl_xor(mb, 32, kWave));
        // mn = -inf: no position of this query yet (its position precedes
        // the wave's blocks so far); everything stays as it is.
        const float mn = fmaxf(m, mb);
        const bool none = mn == -INFINITY;
        const float alpha = none ? 1.0f : expf(m - mn);
        l *= alpha;
#pragma unroll
        for (int c = 0; c < E; ++c) o[c] *= alpha;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float p = none ? 0.0f : expf(sv[r] - mn);
            l += p;
#pragma unroll
            for (int c = 0; c < E; ++c) o[c] = mfma16x16x4(b.v[r][c], p, o[c]);
        }
        m = mn;
    };

    // This wave's blocks: [nb * w / 4, nb * (w + 1) / 4) of the nb blocks
    // from lo (a multiple of 16) through hi.
    const int b0i = lo / KB, nb = hi / KB + 1 - b0i;
    const int first = KB * (b0i + nb * wave / kTileWaves);
    const int wlast = KB * (b0i + nb * (wave + 1) / kTileWaves) - 1;  // < first: no blocks
    if (first <= wlast) {
        TileBlock<E> b0, b1;
        load(b0, first);
        for (int t0 = first; t0 <= wlast; t0 += 2 * KB) {
            if (t0 + KB <= wlast) load(b1, t0 + KB);
            use(b0, t0);
            if (t0 + KB > wlast) break;
            if (t0 + 2 * KB <= wlast) load(b0, t0 + 2 * KB);
            use(b1, t0 + KB);
        }
    }

    // Merge the waves in order: lane l of every wave holds query j's state.
    ms[wave][lane] = m;
    ls[wave][lane] = l;
#pragma unroll
    for (int c = 0; c < E; ++c) os[wave][c][lane] = o[c];
    __syncthreads();
    if (wave != 0) return;
    // M is finite for every query with a position in [lo, hi] (the others
    // are not stored): some wave holds that position.
    float M = ms[0][lane];
#pragma unroll
    for (int w = 1; w < kTileWaves; ++w) M = fmaxf(M, ms[w][lane]);
    l = 0.0f;
#pragma unroll
    for (int c = 0; c < E; ++c) o[c] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kTileWaves; ++w) {
        const float mw = ms[w][lane];
        const float f = mw == -INFINITY ? 0.0f : expf(mw - M);
        l += f * ls[w][lane];
#pragma unroll
        for (int c = 0; c < E; ++c) o[c] += f * os[w][c][lane];
    }

    // The four lane groups of query j hold partial sums of its denominator;
    // the xor pairs add them in the same order in every lane.
    l += __shfl_xor(l, 16, kWave);
    l += __shfl_xor(l, 32, kWave);
    // Split: a query whose context spans more than one chunk leaves this
    // chunk's (max, sum, unnormalised output) for the merge kernel; one whose
    // context fits chunk 0 is written here, as the split kernel writes it.
    if (r0 + j < a.rows && a.tile_chunk && pq >= a.tile_chunk && lo <= pq) {
        const std::size_t b = (static_cast<std::size_t>(r0 + j) * a.n_heads + h) * a.splits + cz;
        floatx4* dst = reinterpret_cast<floatx4*>(a.part_o + b * HS + Q4 * g);
        float run[Q4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int c = 0; c < E; ++c) run[E * r + c] = o[c][r];
#pragma unroll
        for (int u = 0; u < E; ++u)
            dst[u] = floatx4{run[4 * u], run[4 * u + 1], run[4 * u + 2], run[4 * u + 3]};
        if (g == 0) a.part_ml[b] = make_float2(M, l);
    } else if (r0 + j < a.rows && cz == 0 && (a.tile_chunk == 0 || pq < a.tile_chunk)) {
        const float inv = 1.0f / l;
        floatx4* dst = reinterpret_cast<floatx4*>(a.out + static_cast<std::size_t>(r0 + j) * a.out_stride +
                                                  static_cast<std::size_t>(h) * HS + Q4 * g);
        float run[Q4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int c = 0; c < E; ++c) run[E * r + c] = o[c][r] * inv;
#pragma unroll
        for (int u = 0; u < E; ++u)
            dst[u] = floatx4{run[4 * u], run[4 * u + 1], run[4 * u + 2], run[4 * u + 3]};
    }
}

void launch_tile(const AttnShape& s, const AttnArgs& a, int rows, hipStream_t stream) {
    const dim3 grid(s.n_heads, (rows + kTileRows - 1) / kTileRows, a.tile_chunk ? a.splits : 1);
    const dim3 block(kTileWaves * kWave);
    switch (s.head_size / 16) {
        case 1: hipLaunchKernelGGL(attn_tile_kernel<1>, grid, block, 0, stream, a); break;
        case 2: hipLaunchKernelGGL(attn_tile_kernel<2>, grid, block, 0, stream, a); break;
        case 3: hipLaunchKernelGGL(attn_tile_kernel<3>, grid, block, 0, stream, a); break;
        case 4: hipLaunchKernelGGL(attn_tile_kernel<4>, grid, block, 0, stream, a); break;
        case 5: hipLaunchKernelGGL(attn_tile_kernel<5>, grid, block, 0, stream, a); break;
        case 6: hipLaunchKernelGGL(attn_tile_kernel<6>, grid, block, 0, stream, a); break;
        case 7: hipLaunchKernelGGL(attn_tile_kernel<7>, grid, block, 0, stream, a); break;
        default: hipLaunchKernelGGL(attn_tile_kernel<8>, grid, block, 0, stream, a); break;
    }
}

void launch_merge(const AttnShape& s, const AttnArgs& a, int rows, hipStream_t stream) {
    const int hs4 = s.head_size / 4;
    const int dpw = hs4 < kMergeDims ? hs4 : kMergeDims, groups = (hs4 + dpw - 1) / dpw;
    const std::size_t slots = kThreads / dpw;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(s.n_heads * groups, rows), dim3(kThreads),
                       (slots * dpw * 4 + 2 * slots) * sizeof(float), stream, a);
}

// Rows of fewer than a.merge_from chunks are left for the caller to merge;
// no merge launches when no row can have that many.
template <int G, int LPP, int F, bool ROPE>
void launch_split(const AttnShape& s, const AttnArgs& a, int rows, hipStream_t stream) {
    const dim3 grid(s.n_heads / G, rows, a.splits);
    hipLaunchKernelGGL((attn_split_kernel<G, LPP, F, ROPE>), grid, dim3(kThreads),
                       split_lds(s, ROPE, a.merge_count != nullptr), stream, a);
    if (a.merge_count) return;  // the kernel merges its own rows
    if (a.splits < a.merge_from) return;  // e.g. one chunk per row: written directly
    launch_merge(s, a, rows, stream);
}

template <int G, bool ROPE = false>
void launch_split_g(const AttnShape& s, const AttnArgs& a, int rows, hipStream_t stream) {
    switch (split_lanes(s) * 10 + split_f(s)) {
        case 41: launch_split<G, 4, 1, ROPE>(s, a, rows, stream); break;
        case 81: launch_split<G, 8, 1, ROPE>(s, a, rows, stream); break;
        case 161: launch_split<G, 16, 1, ROPE>(s, a, rows, stream); break;
        case 321: launch_split<G, 32, 1, ROPE>(s, a, rows, stream); break;
        case 641: launch_split<G, 64, 1, ROPE>(s, a, rows, stream); break;
        default: launch_split<G, 64, 2, ROPE>(s, a, rows, stream); break;
    }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

std::string attention_reject(const AttnShape& s, int kernel) {
    if (kernel < kAttnAutomatic || kernel > kAttnSplit) return "attention: unknown kernel";
    if (s.n_heads <= 0 || s.n_kv_heads <= 0 || s.head_size <= 0 || s.seq_len <= 0 ||
        s.n_heads % s.n_kv_heads != 0)
        return "attention: bad shape";
    if (static_cast<std::size_t>(s.seq_len) * s.kv_stride >= (std::size_t{1} << 31) ||
        s.q_stride >= (std::size_t{1} << 31) || s.out_stride >= (std::size_t{1} << 31))
        return "attention: cache past 32-bit indexing";
    const bool single = kernel == kAttnSingle;
    // split loads float4s.
    if (!single && (s.head_size % 4 || s.head_size > 512 || s.q_stride % 4 ||
                    s.kv_stride % 4 || s.out_stride % 4))
        return "attention: split needs head_size and strides divisible by 4";
    const std::size_t need = single ? single_lds(s) : split_lds(s);
    if (need > kMaxLds)
        return "attention: seq_len " + std::to_string(s.seq_len) + " needs " +
               std::to_string(need) + " bytes of LDS, more than " + std::to_string(kMaxLds);
    return "";
}

// Enough for any call of up to `rows` rows, so that a buffer sized once for
// the most rows serves every smaller call: a split tile grid's chunk count
// grows as its row tiles shrink.
std::size_t attention_scratch_floats(const AttnShape& s, std::size_t rows, int kernel) {
    if (kernel == kAttnSingle) return 0;
    if (kernel != kAttnAutomatic) return split_scratch(s, rows).total;
    const std::size_t cut = split_max_rows(s);
    std::size_t need = split_scratch(s, rows < cut ? rows : cut).total;
    if (rows > cut && tile_supports(s)) {
        const std::size_t tiles = (rows + kTileRows - 1) / kTileRows;
        for (std::size_t rt = 1; rt <= tiles; ++rt) {
            const std::size_t m = std::min(rows, rt * kTileRows);
            if (m <= cut) continue;
            const int S = tile_splits(s, m);
            if (S == 1) break;  // more row tiles split no further
            need = std::max(need, tile_scratch(s, m, S).total);
        }
    }
    return need;
}

bool attention_uses_split(const AttnShape& s, std::size_t rows, int kernel) {
    return resolve(kernel, rows, s) != kAttnSingle;
}

bool attention_needs_scratch(const AttnShape& s, std::size_t rows, int kernel) {
    return resolve(kernel, rows, s) == kAttnSplit;
}

namespace {

AttnArgs base_args(const AttnShape& s, int rows, const int* pos, const float* q, const float* kc,
                   const float* vc, float* out) {
    AttnArgs a{};
    a.n_heads = s.n_heads;
    a.head_size = s.head_size;
    a.group = s.n_heads / s.n_kv_heads;
    a.seq_len = s.seq_len;
    a.q_stride = static_cast<int>(s.q_stride);
    a.kv_stride = static_cast<int>(s.kv_stride);
    a.out_stride = static_cast<int>(s.out_stride);
    a.pos = pos;
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.out = out;
    a.rows = rows;
    a.merge_from = 2;
    a.min_chunk = min_chunk(s);
    return a;
}

void set_split(const AttnShape& s, int rows, float* scratch, AttnArgs& a) {
    const SplitScratch l = split_scratch(s, rows);
    a.splits = split_count(s);
    a.chunk_cap = split_chunk_cap(s);
    a.part_o = scratch + l.o;
    a.part_ml = reinterpret_cast<float2*>(scratch + l.ml);
}

}  // namespace

void run_attention(const AttnShape& s, int rows, const int* pos, const float* q, const float* kc,
                   const float* vc, float* out, float* scratch, int kernel, hipStream_t stream) {
    kernel = resolve(kernel, rows, s);
    AttnArgs a = base_args(s, rows, pos, q, kc, vc, out);
    if (kernel == kAttnTile) {
        // The context split needs the caller's scratch (sized by
        // attention_scratch_floats); without it the grid stays whole.
        const int S = scratch && reinterpret_cast<uintptr_t>(scratch) % 16 == 0
                          ? tile_splits(s, static_cast<std::size_t>(rows))
                          : 1;
        if (S > 1) {
            const SplitScratch l = tile_scratch(s, static_cast<std::size_t>(rows), S);
            a.splits = S;
            a.tile_chunk = tile_chunk(s, S);
            a.part_o = scratch + l.o;
            a.part_ml = reinterpret_cast<float2*>(scratch + l.ml);
        }
        launch_tile(s, a, rows, stream);
        if (S > 1) launch_merge(s, a, rows, stream);
        return;
    }
    if (kernel == kAttnSingle) {
        hipLaunchKernelGGL(attn_single_kernel, dim3(s.n_heads, rows), dim3(kThreads),
                           single_lds(s), stream, a);
        return;
    }
    if (kernel == kAttnWhole) {
        a.splits = 1;
        a.chunk_cap = s.seq_len;
    } else {
        set_split(s, rows, scratch, a);
    }
    switch (heads_per_block(s)) {
        case 8: launch_split_g<8>(s, a, rows, stream); break;
        case 4: launch_split_g<4>(s, a, rows, stream); break;
        case 2: launch_split_g<2>(s, a, rows, stream); break;
        default: launch_split_g<1>(s, a, rows, stream); break;
    }
}

bool run_attention_rope(const AttnShape& s, const int* pos, const Summed& src, int dim,
                        int kv_dim, const float* cos_t, const float* sin_t, float* kc, float* vc,
                        float* out, float* scratch, hipStream_t stream, SplitRow* defer,
                        bool merge_inside) {
    if (resolve(kAttnAutomatic, 1, s) != kAttnSplit || split_lds(s, true, true) > kMaxLds)
        return false;
    if (src.n % 4 || src.mn % 4 || dim % 4 || kv_dim % 4) return false;
    if (!aligned16(src.slices == 1 ? src.c : src.partial) || (src.scale && !aligned16(src.scale)))
        return false;
    AttnArgs a = base_args(s, 1, pos, nullptr, kc, vc, out);
    set_split(s, 1, scratch, a);
    a.src = src;
    a.dim = dim;
    a.kv_dim = kv_dim;
    a.cos_t = cos_t;
    a.sin_t = sin_t;
    a.kc_w = kc;
    a.vc_w = vc;
    // Deferred: rows of up to kMergeInGemv chunks are merged by the consumer,
    // longer ones (a shape with more splits) by the merge kernel, into out.
    const bool hold = defer && a.splits > 1;
    if (hold) a.merge_from = kMergeInGemv + 1;
    if (!defer && merge_inside && a.splits > 1)
        a.merge_count = tile_counters(static_cast<std::size_t>(s.n_heads / heads_per_block(s)));
    switch (heads_per_block(s)) {
        case 8: launch_split_g<8, true>(s, a, 1, stream); break;
        case 4: launch_split_g<4, true>(s, a, 1, stream); break;
        case 2: launch_split_g<2, true>(s, a, 1, stream); break;
        default: launch_split_g<1, true>(s, a, 1, stream); break;
    }
    if (defer) {
        *defer = SplitRow{};
        if (hold) *defer = SplitRow{a.part_o, a.part_ml, out, pos, a.splits, s.n_heads, s.head_size, a.min_chunk};
    }
    return true;
}

bool attention_merge_inside_preferred(const AttnShape& s) { return heads_per_block(s) == 1; }

void run_attention_merge(const AttnShape& s, const SplitRow& r, float* out, hipStream_t stream) {
    AttnArgs a = base_args(s, 1, r.pos, nullptr, nullptr, nullptr, out);
    a.splits = r.splits;
    a.part_o = const_cast<float*>(r.o);
    a.part_ml = const_cast<float2*>(r.ml);
    launch_merge(s, a, 1, stream);
}

}  // namespace em
