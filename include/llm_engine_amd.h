/*
 * llm_engine_amd.h -- C ABI of the MI355X (gfx950) matmul hot path.
 *
 * Plain pointers and sizes only. Every entry point validates its arguments on
 * the host before it touches the GPU, returns EM_OK or an error code, and
 * leaves a message for em_last_error(). Device pointers are plain HIP device
 * allocations (em_malloc, hipMalloc or a torch tensor's data_ptr()).
 *
 * Streams: `stream` is a hipStream_t passed through as is. NULL is HIP's
 * legacy null stream; EM_STREAM_PER_THREAD is the calling thread's default
 * stream, which is what the reference's library uses (it is compiled with
 * --default-stream per-thread, /root/reference/CMakeLists.txt:100-105), and
 * what the C++ layer in cuda_matmul.h passes. Calls are queued and return
 * before the GPU finishes. Calls that use split-K share one library-owned
 * scratch buffer: concurrent calls on different streams race, as in the
 * reference (cuda_matmul.h:7-12).
 *
 * Layout (cuda_matmul.h:94-107): A is m x k, B is k x n, C is m x n, all
 * dense row-major fp32 with no leading dimensions; int8 B carries n fp32
 * column scales. rms_weight, when not NULL, holds k floats.
 */
#ifndef LLM_ENGINE_AMD_H
#define LLM_ENGINE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define EM_OK 0
#define EM_EINVAL 1  /* bad arguments: shapes, kernel choice, sizes (std::invalid_argument) */
#define EM_EDEVICE 2 /* a HIP runtime error (std::runtime_error "cuda: <op>: <err>") */
#define EM_ENODEV 3  /* no usable GPU */
#define EM_ERANGE 4  /* a token or position outside the model's range (std::out_of_range) */
#define EM_EIO 5     /* a checkpoint that cannot be opened or read, or whose header or size is
                        bad (std::runtime_error from load_checkpoint) */

/* Kernel choice; replaces enum class GpuKernel, cuda_matmul.h:61-67. */
#define EM_KERNEL_AUTOMATIC 0   /* fp32 B: skinny for m <= 8 (m <= 3 for 2^25 weights or more),
                                   else tiled_split (tiled if B is unaligned); int8 B: skinny
                                   for 1 row, and for 2-4 rows of small weights, else the
                                   exact-split bf16 MFMA kernel */
#define EM_KERNEL_NAIVE 1       /* one thread per element of C; the reference kernel */
#define EM_KERNEL_TILED 2       /* LDS-tiled fp32 MFMA GEMM, 128 x 128 tiles */
#define EM_KERNEL_TILED_SPLIT 3 /* MFMA over 16/32-row tiles, B streamed from HBM/L2, k split */
#define EM_KERNEL_SKINNY 4      /* m <= 8 only: wave64 GEMV, k split across waves and blocks */

#define EM_STREAM_PER_THREAD ((void*)2) /* hipStreamPerThread */

/* Message of the last failed call on this thread ("" if none). */
const char* em_last_error(void);

/* 1 if a usable GPU is present; replaces cuda_available(), cuda_matmul.h:121-122. */
int em_available(void);

/* Waits for all queued GPU work; replaces cuda_synchronize(), cuda_matmul.h:118-119. */
int em_synchronize(void);

/* Bumped whenever the library reallocates its split-K / norm scratch; a HIP
 * graph captured before the bump must be captured again. Replaces
 * cuda_scratch_generation(), cuda_matmul.h:109-112, cuda_matmul.cu:268-297,567. */
size_t em_scratch_generation(void);

/* Device memory, for DeviceTensor / DeviceQTensor (cuda_matmul.cu:452-525):
 * allocation, free, and the synchronous copies of upload() / download().
 * em_free also drops the strip copies registered (em_q8_register) for
 * buffers inside the freed allocation. */
int em_malloc(void** ptr, size_t bytes);
int em_free(void* ptr);
int em_memcpy_h2d(void* dst, const void* src, size_t bytes);
int em_memcpy_d2h(void* dst, const void* src, size_t bytes);

/* C = A x B (C += A x B if accumulate), A optionally replaced by
 * rmsnorm(A) * rms_weight (eps 1e-5). Replaces
 *   void matmul_cuda(size_t m, size_t n, size_t k, const float* A, const float* B,
 *                    float* C, GpuKernel, const MatmulFusion&)   cuda_matmul.h:94-99
 * Errors (before any launch): skinny with m > 8; m*k, k*n or m*n >= 2^31;
 * a NULL pointer where the shape needs one; an unknown kernel. m == 0 or
 * n == 0 does nothing; k == 0 zeroes C unless accumulating
 * (cuda_matmul.cu:406-422). Results are bit-identical across repeats. */
int em_matmul_f32(size_t m, size_t n, size_t k, const float* A, const float* B, float* C,
                  int kernel, int accumulate, const float* rms_weight, void* stream);

/* Same with int8 B and n column scales: C = A x dequantize(B). Replaces
 *   void matmul_cuda(size_t m, size_t n, size_t k, const float* A, const int8_t* B,
 *                    const float* scale, float* C, GpuKernel, const MatmulFusion&)
 *                                                                 cuda_matmul.h:101-107 */
int em_matmul_q8(size_t m, size_t n, size_t k, const float* A, const int8_t* B,
                 const float* scale, float* C, int kernel, int accumulate,
                 const float* rms_weight, void* stream);

/* em_matmul_q8 with EM_KERNEL_SKINNY (m <= 8), allocating nothing: for
 * callers that cannot call hipMalloc (code under HIP graph capture, tight
 * serving loops, harnesses that forbid it). The GEMV's split-K partials go
 * to a 32 MiB device array the library holds on each GPU until the process
 * ends, instead of grow-only scratch; results are the same bits as
 * em_matmul_q8 with EM_KERNEL_SKINNY (registered weights included), and
 * em_scratch_generation() does not move. EM_EINVAL, before any launch, for
 * what em_matmul_q8 rejects and for a shape whose partials need more than
 * 32 MiB (every Llama-7B-shaped product up to 8 rows fits: 8 rows of the
 * 4096 x 32000 classifier need 31.25 MiB). Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU (other streams, other
 * host threads) race; calls on one stream are ordered. No counterpart in
 * the reference. */
int em_matmul_q8_noalloc(size_t m, size_t n, size_t k, const float* A, const int8_t* B,
                         const float* scale, float* C, int accumulate, const float* rms_weight,
                         void* stream);

/* ---- Strip layout of int8 weights (explicit opt-in) ------------------------
 * The reference keeps int8 weights row-major (QTensor, tensor.h:23-28); the
 * entry points above take that layout. The strip layout is an opt-in copy for
 * decode-shaped products: n / 16 strips of 16 columns, strip j holding rows
 * 0 .. k - 1 of columns 16j .. 16j + 15 contiguously in quads of four rows,
 * each quad as four 16-byte units, unit c holding columns 4c .. 4c + 3 of the
 * quad's four rows, row by row:
 *     packed[(j * k + 4q) * 16 + 16c + 4t + u] = B[(4q + t) * n + 16j + 4c + u],
 * the same bytes reordered (scales unchanged). An m <= 8 product over it is
 * one launch with no split-K partials. Needs n % 16 == 0, k % 4 == 0 and
 * 16-byte aligned buffers of k * n bytes. No counterpart in the reference. */
int em_pack_q8(size_t k, size_t n, const int8_t* B, int8_t* packed, void* stream);
int em_unpack_q8(size_t k, size_t n, const int8_t* packed, int8_t* B, void* stream);
/* Registers row-major int8 weights B (k x n, device memory) for em_matmul_q8:
 * the library keeps a strip-layout copy, packed from B's bytes on `stream`
 * (then drained), and em_matmul_q8 runs decode-shaped products over that
 * copy in one launch: one row (m == 1, k <= 8192, or k <= 12288 without a
 * norm weight when n >= 4096) with EM_KERNEL_AUTOMATIC
 * or EM_KERNEL_SKINNY, and, with EM_KERNEL_AUTOMATIC, 2 - 8 rows at
 * k <= 4096 (3 - 4 rows up to n = 24576, 5 - 8 up to n = 4096; A 16-byte
 * aligned) and 9 - 16 rows where that kernel beats the row-major one (k <=
 * 768, or k <= 4096 with n <= 12288 and k x n >= 2^24; A, C, scales and the
 * norm weight 16-byte aligned). Same
 * semantics, results within the same tolerance of the row-major path,
 * bit-identical across repeats. B's bytes must not change while it is
 * registered (register again after changing them). Unregister, or free
 * with em_free (which drops the copy), before the memory is used for other
 * bytes: a buffer freed another way and allocated again at the same address
 * would find the stale copy. Registering again replaces the copy. Shapes the layout cannot
 * hold (n % 16 != 0, k % 4 != 0, misaligned B) and EM_STRIP_COPY=0 in the
 * environment leave B unregistered (EM_OK); EM_DECODE_MFMA=0 keeps 2 - 8
 * rows on the row-major kernels. The C++ DeviceQTensor registers its buffer
 * on construction and unregisters it on destruction, so the reference's
 * callers (cuda_model.cu:112,167; bench_cuda.cpp:123,139) get the one-launch
 * products unchanged. No counterpart in the reference. */
int em_q8_register(const int8_t* B, size_t k, size_t n, void* stream);
int em_q8_unregister(const int8_t* B);
/* 1 if B has a strip copy of shape k x n, else 0. */
int em_q8_registered(const int8_t* B, size_t k, size_t n);
/* C = A x dequantize(B) (C += if accumulate; A replaced by rmsnorm(A) *
 * rms_weight when given), B in the strip layout: the semantics of
 * em_matmul_q8 for m <= 16 rows, in one launch, bit-identical across
 * repeats (the same kernels and bits as a registered em_matmul_q8 call where
 * that runs over the copy). EM_EINVAL for m > 16, n % 16 != 0, k % 4 != 0, a
 * misaligned B, more than 2^31 elements, and at 9 to 16 rows for A, C, the
 * scales or the norm weight off a 16-byte boundary; m == 0 or n == 0 does
 * nothing; k == 0 zeroes C unless accumulating. */
int em_matmul_q8_packed(size_t m, size_t n, size_t k, const float* A, const int8_t* packed,
                        const float* scale, float* C, int accumulate, const float* rms_weight,
                        void* stream);

/* Symmetric per-column int8 quantisation on the GPU, bit-exact with
 *   QTensor quantize_q8(const Tensor& B)   quant.h:7, quant.cpp:6-28
 * B is rows x cols fp32 on the device; q receives rows x cols int8 and scale
 * cols floats: scale = max|B[:,c]| / 127, inv = 1 / scale (0 for a zero
 * column), q = clamp(lround(B * inv), -127, 127), rounding half away from zero. */
int em_quantize_q8(size_t rows, size_t cols, const float* B, int8_t* q, float* scale,
                   void* stream);

/* out = q * scale[c] on the GPU; replaces Tensor dequantize(const QTensor&),
 * quant.h:9, quant.cpp:30-36. */
int em_dequantize_q8(size_t rows, size_t cols, const int8_t* q, const float* scale, float* out,
                     void* stream);

/* Reads `bytes` of device memory at `buf` once (both multiples of 16), the
 * read-only HBM ceiling that bench.py reports beside the GEMV. No counterpart
 * in the reference, whose bench times a device-to-device copy as its ceiling
 * (bench_cuda.cpp:79-88); it is for callers that measure the matmul path.
 * `sink` is 4 bytes of device memory the kernel may write (almost never). */
int em_stream_read(const void* buf, size_t bytes, uint32_t* sink, void* stream);

/* Measurement entry points for bench.py's floor study (no counterpart in the
 * reference; not part of the matmul interface). em_probe_empty launches an
 * empty kernel of `blocks` 256-thread workgroups. em_probe_read reads `bytes`
 * at `buf` once with `blocks` workgroups and `depth` (4, 8 or 16) 16-byte
 * loads in flight per thread, each workgroup on one contiguous chunk
 * (contiguous != 0) or the grid striding over the buffer. */
int em_probe_empty(unsigned blocks, void* stream);
int em_probe_read(const void* buf, size_t bytes, uint32_t* sink, unsigned blocks, unsigned depth,
                  int contiguous, void* stream);
/* em_probe_read_columns reads a rows x row_bytes row-major matrix once (under
 * 2^31 bytes, 16-byte aligned) the way a GEMV over row-major weights could
 * split it: workgroup (g, s) reads bytes [g * seg_bytes, (g + 1) * seg_bytes)
 * of every row of k slice s (slices of ceil(rows / slices) rows), seg_bytes
 * 64, 128, 256, 512 or 1024, `depth` (8 or 16) 16-byte loads in flight per
 * thread; with xcd != 0 (and a grid of a multiple of 8 workgroups) the
 * workgroups one XCD runs own consecutive (g, s) pairs. */
int em_probe_read_columns(const void* buf, unsigned rows, unsigned row_bytes, unsigned seg_bytes,
                          unsigned slices, unsigned depth, int xcd, uint32_t* sink, void* stream);

/* ---- Causal attention over a KV cache (cuda_attention.h) ------------------ */

/* Replaces struct AttentionShape, cuda_attention.h:8-13. */
typedef struct {
    int n_heads, n_kv_heads, head_size, seq_len;
    size_t q_stride;   /* floats between rows of q; head h starts at h * head_size */
    size_t kv_stride;  /* floats between positions of the caches (kv_dim) */
    size_t out_stride; /* floats between rows of out */
} em_attention_shape;

/* Replaces enum class AttentionKernel, cuda_attention.h:15-19. */
#define EM_ATTN_AUTOMATIC 0    /* split for up to 5 rows (12 when seq_len <= 512); more rows:
                                  16-row fp32 MFMA tiles, also split over the context when
                                  their grid is small (head_size a multiple of 16, at most
                                  128), else split for up to 12 rows and then one chunk per
                                  row, no merge. Scratch for rows serves fewer rows too. */
#define EM_ATTN_SINGLE_BLOCK 1 /* one workgroup per (head, row), scores in LDS */
#define EM_ATTN_SPLIT 2        /* positions split across workgroups, merged in chunk order */

/* EM_OK if `kernel` can run shape s, else EM_EINVAL with the reason; replaces
 * attention_check(), cuda_attention.h:23-26. Rejects a non-positive size,
 * n_heads not a multiple of n_kv_heads, caches past 32-bit indexing; for split
 * (and automatic) head_size or a stride not a multiple of 4; and a kernel whose
 * LDS need (single_block: head_size + seq_len + 256 floats) passes 64 KiB. */
int em_attention_check(const em_attention_shape* s, int kernel);

/* Floats of scratch em_attention needs for `rows` rows (0 for single_block);
 * replaces attention_scratch_floats(), cuda_attention.h:21-22. */
size_t em_attention_scratch_floats(const em_attention_shape* s, size_t rows, int kernel);

/* For each of `rows` rows and each query head h: row i sits at position
 * *pos_dev + i and attends to cached positions [0, *pos_dev + i], with kv head
 * h / (n_heads / n_kv_heads): out[i][h*head_size + d] =
 * sum_t softmax_t(q . k_t / sqrt(head_size)) v_t[d]. pos_dev is device memory,
 * so a captured graph serves every position; the caller keeps
 * *pos_dev + rows <= seq_len. Replaces attention_cuda(), cuda_attention.h:28-38.
 * Unlike the reference, scratch needs no zero fill (no counters), and results
 * are bit-identical across calls. */
int em_attention(const em_attention_shape* s, size_t rows, const int* pos_dev, const float* q,
                 const float* key_cache, const float* value_cache, float* out, float* scratch,
                 int kernel, void* stream);

/* ---- The device-resident forward pass (cuda_model.h) --------------------- */

/* Replaces struct Config, model.h:11-22: head_size = dim / n_heads,
 * kv_dim = n_kv_heads * head_size. */
typedef struct {
    size_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
} em_model_config;

/* One layer's weights in the CPU model's layout (struct LayerWeights,
 * model.h:29-36): projections stored in x out, row-major, host memory. */
typedef struct {
    const float* rms_att; /* dim */
    const float* wqkv;    /* dim x (dim + 2 kv_dim): q | k | v */
    const float* wo;      /* dim x dim */
    const float* rms_ffn; /* dim */
    const float* w13;     /* dim x 2 hidden_dim: gate (w1) | up (w3) */
    const float* w2;      /* hidden_dim x dim */
} em_layer_weights;

/* Replaces enum class WeightType, model.h:60. q8 quantises every projection
 * and the classifier with quantize_q8 (bit-exact with quant.cpp); the
 * embedding stays fp32. */
#define EM_WEIGHTS_F32 0
#define EM_WEIGHTS_Q8 1

typedef struct em_model em_model;

/* Copies the weights to the GPU (quantising them there for q8) and allocates
 * the KV cache. Replaces CudaTransformer(const Checkpoint&, WeightType),
 * cuda_model.h:29-31. token_embedding is vocab_size x dim, rms_final dim,
 * wcls dim x vocab_size (the CPU model's Weights, model.h:38-43); `layers`
 * holds n_layers entries. EM_EINVAL for a shape the attention kernels cannot
 * run (as the reference's constructor rejects one) or a NULL weight. */
int em_model_create(const em_model_config* cfg, const float* token_embedding,
                    const em_layer_weights* layers, const float* rms_final, const float* wcls,
                    int weight_type, em_model** out);

/* Loads a llama2.c v0 checkpoint from `path` straight into a model: replaces
 *   Checkpoint load_checkpoint(const std::string& path)     model.h:69-71,
 *                                                           model.cpp:115-163
 * followed by CudaTransformer(ckpt, type). The 7-int header is checked as the
 * reference checks it (every field non-zero, all but the vocabulary
 * positive; dim split into even-sized heads, whole kv groups) and the file
 * size against the header; each failure is EM_EIO with the reference's
 * message ("cannot open checkpoint P", "checkpoint P: bad header field i =
 * v", "checkpoint P: dim must split ...", "checkpoint P is N bytes, header
 * implies M", "checkpoint P ended early"). The file streams through pinned
 * memory to the GPU, which transposes each projection (stored out x in) into
 * the CPU model's layout, fuses q | k | v and w1 | w3, takes the classifier
 * from the embedding when the vocabulary is positive, and for EM_WEIGHTS_Q8
 * quantises with quantize_q8 on the GPU. EM_EINVAL for a shape the forward
 * pass cannot run (as em_model_create). */
int em_model_load(const char* path, int weight_type, em_model** out);

/* The model's config (for one from em_model_load, the checkpoint header's). */
int em_model_config_get(const em_model* m, em_model_config* out);

/* Copies one weight array back to host memory, as stored: "token_embedding",
 * "rms_final", "wcls", and per layer "rms_att", "wqkv", "wo", "rms_ffn",
 * "w13", "w2" (the CPU model's Weights / LayerWeights, model.h:29-43) as fp32;
 * in an int8 model the projections ("wqkv", "wo", "w13", "w2", "wcls") are
 * their int8 bytes and "<name>.scale" their column scales. `bytes` must be
 * the array's size (EM_EINVAL otherwise, or for an unknown name). No
 * counterpart in the reference; for checking a load against the CPU loader. */
int em_model_read_weight(em_model* m, const char* name, size_t layer, void* dst, size_t bytes);

int em_model_destroy(em_model* m);

/* Feeds tokens[0:n] at positions [pos, pos + n) and writes the logits of the
 * token after the last (vocab_size floats, host memory). n == 1 is
 * CudaTransformer::forward, n > 1 prefill (cuda_model.h:37-39); both wait for
 * the GPU. EM_ERANGE (check_feed, model.cpp:165-177) for a token outside the
 * vocabulary, pos + n > seq_len, or pos past the positions already fed;
 * EM_EINVAL for n == 0. A rejected call leaves the cache as it was. The first
 * one-token call is captured into a HIP graph that later ones replay. Not
 * safe from several host threads at once. */
int em_model_forward(em_model* m, const int* tokens, size_t n, size_t pos, float* logits);

#ifdef __cplusplus
}
#endif

#endif /* LLM_ENGINE_AMD_H */
