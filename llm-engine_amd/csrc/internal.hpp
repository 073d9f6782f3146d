// Host-side interface between the C ABI (api.hip) and the kernel files.
// Every launcher takes already-validated arguments: shapes below 2^31
// elements, non-null pointers where the shape needs them, and m, n, k > 0.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "common.hpp"

namespace em {

// A HIP runtime failure; api.hip turns it into EM_EDEVICE with this text.
struct DeviceError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline void hip_check(hipError_t err, const char* what) {
    if (err != hipSuccess)
        throw DeviceError(std::string("hip: ") + what + ": " + hipGetErrorString(err));
}

// Library-owned, grow-only device scratch (split-K partials, the normed copy
// of A, quantiser column maxima). Growing waits for the device, frees the old
// buffer and bumps scratch_generation(). Slot 0 holds partials, slot 1 the
// norm buffer, slot 2 quantiser work space, slot 3 the bf16 planes of A,
// slot 4 the partials of a GEMV whose A is formed from slot 0's partials
// (run_skinny_swiglu), which it must not overwrite while reading them.
enum ScratchSlot { kPartial = 0, kNorm = 1, kQuant = 2, kSplitA = 3, kPartialFromPartial = 4,
                   kSlots = 5 };
float* scratch(ScratchSlot slot, std::size_t floats);
std::size_t scratch_generation();
// Library-owned arrival counters for one-launch split-K products: `count`
// 32-bit words, zero. Grow-only like scratch() (growth bumps
// scratch_generation()); zeroed when allocated, and every call leaves the
// counters it used zero.
unsigned* tile_counters(std::size_t count);

// Compute units of the current device (cached).
int cu_count();

// Values per sum of squares that a producer of a GEMV's A may leave for the
// GEMV's norm (embed and the residual reduce, in the forward pass).
constexpr int kSsqChunk = 64;

struct MatmulArgs {
    int m, n, k;
    const float* A;
    const void* B;         // float* or int8_t*
    const float* scale;    // int8 column scales, null for fp32
    float* C;
    bool accumulate;
    const float* rms_weight;  // null: no norm
    hipStream_t stream;
    // With rms_weight and m == 1 (GEMV only): the sums of squares of A's
    // values [64j, 64j + 64), j < ceil(k / 64), that A's producer left; the
    // norm is formed from them instead of from all of A in every workgroup.
    const float* ssq;
    // GEMV only: the caller's buffer for the split-K partials (at least
    // skinny_partial_floats() floats) in place of the library's scratch.
    float* partials;
};

// em_matmul_f32 / em_matmul_q8 (api.hip): validation, dispatch, errors as
// EM_* codes. `workspace`, when given (em_matmul_q8_noalloc), supplies the
// buffer for the GEMV's split-K partials and its size in floats, or returns
// null with the error message set.
using Workspace = float* (*)(std::size_t* floats);
template <class BT>
int matmul_entry(std::size_t m, std::size_t n, std::size_t k, const float* A, const BT* B,
                 const float* scale, float* C, int kernel, int accumulate,
                 const float* rms_weight, void* stream, Workspace workspace = nullptr);

// Decode-shaped GEMV, m <= 8 (GpuKernel::skinny). Fuses the norm.
template <class BT>
void run_skinny(const MatmulArgs& a);
// The same GEMV without its slice sum: returns the number of k slices. With
// one slice C is written (scaled, accumulated) as run_skinny writes it;
// with more, *partial holds [slice][m][n] unscaled sums (library scratch)
// that the caller must add in slice order, scale and store exactly as
// reduce_slices does (a consumer kernel that fuses the sum).
template <class BT>
int run_skinny_partials(const MatmulArgs& a, const float** partial);
// The floats of split-K partials run_skinny_partials(a) writes (0 when it
// needs one k slice and writes C itself).
template <class BT>
std::size_t skinny_partial_floats(const MatmulArgs& a);
// One row of silu_mul(gate, up) x B, the gate | up product (split at
// `hidden` = k) given as a Summed with at most 16 slices: the forward pass's
// SwiGLU formed inside the GEMV's A staging, C (+)= as run_skinny writes
// it. Returns its k slices; 0 (nothing launched) for a shape it does not
// take. With more than one slice the reduce also writes ssq (as
// run_reduce_slices does) when ssq is given and n % 64 == 0.
template <class BT>
int run_skinny_swiglu(const MatmulArgs& a, const Summed& gu, int hidden, float* ssq = nullptr);
// One row of attention output x B with A merged inside the GEMV's A
// staging from the split chunks att (k = heads x head_size) when the row
// has 2 .. kMergeInGemv of them, as the merge kernel merges them, and read
// from att.out otherwise: the same bits as run_attention_merge followed by
// run_skinny. Returns the k slices and
// writes ssq as run_skinny_swiglu does; 0 (nothing launched) for a shape
// it does not take.
constexpr int kMergeInGemv = 16;
template <class BT>
int run_skinny_merged(const MatmulArgs& a, const SplitRow& att, float* ssq = nullptr);

// MFMA over 16/32/64-row tiles with B streamed once and k split across
// blocks (GpuKernel::tiled_split). A must already be normed.
template <class BT>
void run_tiled_split(const MatmulArgs& a);

// LDS-tiled MFMA GEMM (GpuKernel::tiled). A must already be normed.
template <class BT>
void run_tiled(const MatmulArgs& a);

// True where automatic should run an fp32 product of more than 8 rows on the
// tiled kernel rather than tiled_split: the streamlined tiled kernel takes
// the shape and m >= 1024, or B has at most 2^20 values, or m >= 256 with
// n >= 2k. Measured (us, tiled_split against tiled): 4096^2 at m = 1024
// 267 / 253, m = 512 136 / 140; 4096 x 11008 at m = 256 263 / 197, m = 128
// 135 / 140; 11008 x 4096 at m = 512 355 / 374, m = 1024 706 / 676;
// 288 x 768 at m = 9 .. 1024 12-18 / 8.5; 768 x 288 at m = 32 16.2 / 11.8.
bool tiled_preferred(const MatmulArgs& a);

// One thread per element (GpuKernel::naive). A must already be normed.
template <class BT>
void run_naive(const MatmulArgs& a);

// int8 B at m > 8 on bf16 MFMA with A split exactly into three bf16 terms
// (split_bf16.hip). Fuses the norm. Needs n % 16 == 0 and 16-byte aligned B
// and scales.
bool split_bf16_supports(const MatmulArgs& a);
// The forward pass's RoPE and cache write for a qkv product (columns: q at
// 0, k at dim, v at dim + kv_dim), rows at positions *pos + i.
struct RopeFuse {
    const int* pos;
    const float* cos_t;
    const float* sin_t;
    float* kc;
    float* vc;
    int dim, kv_dim, head_size;
};
// With rope, and when the product needs no k split (it writes C directly):
// q is stored rotated, k rotated into kc and v into vc (not into C), with
// rope_cache_kernel's arithmetic; returns true. Otherwise C as usual, false.
bool run_split_bf16(const MatmulArgs& a, const RopeFuse* rope = nullptr);
// The forward pass's w13 with its SwiGLU: B (k x 2 hidden) holds gates then
// ups, a.C is hidden wide and gets silu(gate) * up, the bits of the product
// followed by swiglu_kernel. False, nothing launched, when the shape is not
// supported (hidden % 16, alignment, accumulate) or the product would need
// a k split.
bool split_bf16_swiglu_supported(const MatmulArgs& a, int hidden);
bool run_split_bf16_swiglu(const MatmulArgs& a, int hidden);
// True if automatic sends an int8 product of m rows (k x n weights) to the
// exact-split kernel rather than the GEMV.
bool split_bf16_preferred(int m, int n, int k);

// True if run_tiled_split can take this shape (vector loads of B rows).
template <class BT>
bool tiled_split_supports(const MatmulArgs& a);

// out[m x k] = rmsnorm(A) * w, one workgroup per row.
void run_rmsnorm_rows(int m, int k, const float* A, const float* w, float* out,
                      hipStream_t stream);

// C[i] = (accumulate ? C[i] : 0) + scale[i % n] * sum_s partial[s][i], s in order.
// With ssq (n % 64 == 0): also ssq[j] = the sum of squares of the new
// C[64j .. 64j + 63], for a GEMV norm over C's rows (MatmulArgs::ssq).
void run_reduce_slices(int m, int n, int slices, const float* partial, const float* scale,
                       float* C, bool accumulate, hipStream_t stream, float* ssq = nullptr);

// Zero `count` floats with a kernel (not hipMemsetAsync, so graph capture is safe).
void run_fill_zero(float* p, std::size_t count, hipStream_t stream);
// Reads bytes (a multiple of 16) of buf once, 16-byte aligned.
void run_stream_read(const void* buf, std::size_t bytes, uint32_t* sink, hipStream_t stream);

// Measurement kernels (probes.hip): an empty launch of `blocks`
// workgroups; one read of `bytes` (a multiple of 16) by `blocks` workgroups
// with `depth` (4, 8, 16) loads in flight per thread, contiguous chunks per
// workgroup or a grid stride (false for another depth).
void run_probe_empty(int blocks, hipStream_t stream);
bool run_probe_read(const void* buf, std::size_t bytes, int blocks, int depth, bool contig,
                    uint32_t* sink, hipStream_t stream);
// One read of a rows x row_bytes matrix, workgroup (group, slice) taking the
// seg_bytes-wide column run `group` (64 .. 1024, a power of two dividing
// row_bytes) of rows [slice * span, ...), span = ceil(rows / slices); depth
// 8 or 16 (false for another seg_bytes or depth). xcd: each XCD's
// workgroups own consecutive (group, slice) pairs.
bool run_probe_read_columns(const void* buf, int rows, int row_bytes, int seg_bytes, int slices,
                            int depth, bool xcd, uint32_t* sink, hipStream_t stream);

// The strip layout of int8 weights (gemv_packed.hip): n / 16 strips of 16
// columns, strip j holding rows 0 .. k - 1 of columns 16j .. 16j + 15
// contiguously. n % 16 == 0, both buffers 16-byte aligned.
void run_pack_strips(int k, int n, const int8_t* B, int8_t* P, hipStream_t stream);
void run_unpack_strips(int k, int n, const int8_t* P, int8_t* B, hipStream_t stream);
// C (+)= rmsnorm?(A) x B for m <= 8 rows, B in the strip layout, one launch.
void run_gemv_packed(const MatmulArgs& a, const int8_t* packed);
// One row, B of 2h columns (gates, then ups) in the strip layout:
// C[j] = silu(P[j]) * P[h + j] for j < h, P = rmsnorm?(A) x B, one launch,
// the bits of run_gemv_packed followed by the SwiGLU. Supported: n a
// multiple of 32, k % 4 == 0, k within one pass (4096 rows at 512 threads),
// A 16-byte aligned, no accumulate.
bool gemv_swiglu_supported(const MatmulArgs& a);
void run_gemv_swiglu(const MatmulArgs& a, const int8_t* packed);
// The strip-layout copy of registered int8 weights B (k x n), or null.
const int8_t* registered_strip(const void* B, std::size_t k, std::size_t n);
// 2 .. 8 rows over a strip-layout copy, fp32 MFMA, one launch
// (decode_mfma.hip): n % 16 == 0, k % 4 == 0, k <= 4096, A 16-byte aligned.
bool decode_mfma_supported(const MatmulArgs& a);
void run_decode_mfma(const MatmulArgs& a, const int8_t* packed);
// 9 .. 16 rows over a strip-layout copy, exact bf16 split, k slices added
// inside the launch (strip_split.hip): n % 16 == 0, k % 4 == 0, A, C,
// scales and the norm weight 16-byte aligned. strip_split_preferred: where
// automatic takes it over the row-major exact split for registered weights.
bool strip_split_supported(const MatmulArgs& a);
bool strip_split_preferred(int m, int n, int k);
void run_strip_split(const MatmulArgs& a, const int8_t* packed);

void run_quantize_q8(int rows, int cols, const float* B, int8_t* q, float* scale,
                     hipStream_t stream);
void run_dequantize_q8(int rows, int cols, const int8_t* q, const float* scale, float* out,
                       hipStream_t stream);

inline int ceil_div(long long x, long long d) { return static_cast<int>((x + d - 1) / d); }

// Records `msg` for em_last_error() on this thread and returns `code`.
int fail(int code, const std::string& msg);
bool device_present();

// --- attention (attention.hip) ----------------------------------------------

struct AttnShape {
    int n_heads, n_kv_heads, head_size, seq_len;
    std::size_t q_stride, kv_stride, out_stride;  // floats between rows / positions
};
enum AttnKernel { kAttnAutomatic = 0, kAttnSingle = 1, kAttnSplit = 2 };

// "" if `kernel` can run shape `s`, else the reason.
std::string attention_reject(const AttnShape& s, int kernel);
std::size_t attention_scratch_floats(const AttnShape& s, std::size_t rows, int kernel);
// True if the call runs a float4 kernel, split or tile (16-byte alignment
// needed); attention_needs_scratch: true if it also writes per-chunk partials.
bool attention_uses_split(const AttnShape& s, std::size_t rows, int kernel);
bool attention_needs_scratch(const AttnShape& s, std::size_t rows, int kernel);
// Rows [0, rows) at positions *pos + i; the caller guarantees *pos + rows <= seq_len.
void run_attention(const AttnShape& s, int rows, const int* pos, const float* q, const float* kc,
                   const float* vc, float* out, float* scratch, int kernel, hipStream_t stream);
// One row at position *pos with the forward pass's RoPE and cache write
// fused in: q, k, v are the columns [0, dim), [dim, dim + kv_dim) and
// [dim + kv_dim, dim + 2 kv_dim) of the qkv product `src` (one row); q and k
// are rotated with the tables' row *pos as rope_cache_kernel rotates them,
// k and v are written to the caches at *pos, and out receives attention over
// positions 0 .. *pos. Scratch as run_attention's for one row. False
// (nothing launched) for a shape or alignment it does not take.
// With merge_inside (and no defer), a row split over several chunks is
// merged inside the same launch by the last of its chunks to finish (the
// merge kernel's arithmetic, so the same bits), not by a merge launch.
// With defer, a row split over up to kMergeInGemv chunks is not merged:
// *defer describes the chunks for the consumer to merge, run_skinny_merged
// or run_attention_merge. `out` holds the row when it has one chunk, or
// (a shape with more splits) more than kMergeInGemv, merged by the merge
// kernel. defer->o is null when the shape has one chunk per row.
bool run_attention_rope(const AttnShape& s, const int* pos, const Summed& src, int dim,
                        int kv_dim, const float* cos_t, const float* sin_t, float* kc, float* vc,
                        float* out, float* scratch, hipStream_t stream,
                        SplitRow* defer = nullptr, bool merge_inside = false);
// True where the split attention launch should merge a row's chunks itself
// (merge_inside) rather than leave them to the merge kernel: where one
// workgroup serves one head. With a group of heads per workgroup the last
// chunk's merge covers every head of the group, a longer tail than the
// merge launch (Llama-7B, 8 kv heads, 32 layers at context 512: 1.79
// against 1.75 ms per decode token; 32 kv heads: 1.83 against 1.88).
bool attention_merge_inside_preferred(const AttnShape& s);
// The merge run_attention_rope left for its consumer, written to out.
void run_attention_merge(const AttnShape& s, const SplitRow& r, float* out, hipStream_t stream);

}  // namespace em
