// The device-resident forward pass: the caller of the matmul path
// (reference: CudaTransformer, cuda_model.h:24-89, cuda_model.cu:99-270;
// the CPU Transformer it must agree with is model.cpp:194-322).
//
// Weights, the KV cache and every activation stay in HBM. A call uploads its
// position and token ids ("the feed", from pinned host memory) and downloads
// the last row's logits. Per layer:
//   qkv = rmsnorm(x) Wqkv            one product, norm fused (skinny at m <= 8)
//   rotate q, k; write k, v to the caches          rope_cache_kernel
//   att = attention(q, caches)                      attention.hip
//   x += att Wo                                     product, residual fused
//   gu = rmsnorm(x) W13                             product, norm fused
//   x += swiglu(gu) W2                              swiglu_kernel, product
// then logits = rmsnorm(x[last]) Wcls. The products are this library's
// matmul entry, so they pick the same kernels a caller of em_matmul_* gets.
// At decode sizes (m <= 8) the qkv and w13 GEMVs leave their k-slice
// partials to rope_cache_kernel and swiglu_kernel, which add them in slice
// order and scale them exactly as reduce_slices would: the same bits, two
// dependent launches fewer per layer. An int8 model whose projections took
// strip-layout copies at load (em_q8_register) runs its one-token steps as
// one em_matmul_q8 call per product over them instead: each a single launch
// with the norm or the residual add inside, so no partials and no slice
// reduces; w13's launch also forms the SwiGLU (run_gemv_swiglu).
//
// Kernels read the position and tokens from the device feed, so the first
// one-token call is run eagerly and then captured into a HIP graph that
// later one-token calls replay with one launch; it is captured again when a
// buffer it points at has moved (own growth or the matmul scratch's).
// Everything runs on one stream the model owns, at default priority.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "common.hpp"
#include "internal.hpp"
#include "llm_engine_amd.h"

namespace em {
namespace {

// x[i] = table[feed[1 + i]] (the reference's embed, cuda_model.cu:26-31),
// row blockIdx.y. One float4 per thread when rows are 16-byte multiples, so
// a 4096-wide row is four workgroups with one load each; the restrict lets
// every load issue before the stores. With ssq (dim % 64 == 0, one row) it
// also writes the sum of squares of each 64 values, for the first layer's
// qkv GEMV norm: 16 lanes' float4s, added by a fixed butterfly. Token ids
// were range-checked on the host.
__global__ __launch_bounds__(kThreads) void embed_kernel(int dim, const int* __restrict__ feed,
                                                         const float* __restrict__ table,
                                                         float* __restrict__ x,
                                                         float* __restrict__ ssq) {
    const std::size_t src = static_cast<std::size_t>(feed[1 + blockIdx.y]) * dim;
    const std::size_t dst = static_cast<std::size_t>(blockIdx.y) * dim;
    const int j = blockIdx.x * kThreads + threadIdx.x;
    if (dim % 4 == 0) {
        const bool in = j < dim / 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (in) {
            v = reinterpret_cast<const float4*>(table + src)[j];
            reinterpret_cast<float4*>(x + dst)[j] = v;
        }
        if (ssq) {
            float sq = fmaf(v.w, v.w, fmaf(v.z, v.z, fmaf(v.y, v.y, v.x * v.x)));
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) sq += __shfl_xor(sq, o, kWave);
            if (in && j % 16 == 0) ssq[j / 16] = sq;
        }
    } else {
        for (int c = j; c < dim; c += gridDim.x * kThreads) x[dst + c] = table[src + c];
    }
}

// Row blockIdx.y, at position feed[0] + blockIdx.y: rotates each (even, odd)
// pair of q and k by the position's angles, as rope() does (model.cpp:93-103),
// then writes the rotated k and the v slice into the caches (model.cpp:297-
// 299). A thread takes one q pair, one k pair or one v element; src yields
// the qkv product (qkv_cols wide). Only the rotated q goes back into the qkv
// row: attention reads keys and values from the caches.
__global__ __launch_bounds__(kThreads) void rope_cache_kernel(Summed src, int qkv_cols, int dim,
                                                              int kv_dim, int head_size,
                                                              const int* feed, const float* cos_t,
                                                              const float* sin_t, float* qkv,
                                                              float* key_cache,
                                                              float* value_cache) {
    const int i = blockIdx.y, pos = feed[0] + i, half = head_size / 2;
    float* row = qkv + static_cast<std::size_t>(i) * qkv_cols;
    const int nq = dim / 2, nk = kv_dim / 2;
    const int j = blockIdx.x * kThreads + threadIdx.x;
    if (j < nq + nk) {
        const bool is_k = j >= nq;
        const int pair = is_k ? j - nq : j;
        const int col = (is_k ? dim : 0) + 2 * pair;
        const int a = pos * half + pair % half;
        const float c = cos_t[a], s = sin_t[a];
        const float x0 = summed(src, i, col), x1 = summed(src, i, col + 1);
        const float2 y = rope_pair(x0, x1, c, s);
        float* dst = is_k ? key_cache + static_cast<std::size_t>(pos) * kv_dim + 2 * pair
                          : row + col;
        dst[0] = y.x;
        dst[1] = y.y;
    } else if (j < nq + nk + kv_dim) {
        const int t = j - nq - nk;
        value_cache[static_cast<std::size_t>(pos) * kv_dim + t] =
            summed(src, i, dim + kv_dim + t);
    }
}

// hb[r][c] = silu(g) * u with g = gu[r][c], u = gu[r][hidden + c]
// (model.cpp:306-310); src yields the w13 product (2 * hidden wide).
__global__ __launch_bounds__(kThreads) void swiglu_kernel(int rows, int hidden, Summed src,
                                                          float* hb) {
    const int total = rows * hidden;
    for (int idx = blockIdx.x * kThreads + threadIdx.x; idx < total;
         idx += gridDim.x * kThreads) {
        const int r = idx / hidden, c = idx % hidden;
        hb[idx] = silu_mul(summed(src, r, c), summed(src, r, hidden + c));
    }
}

// dst[i * ld + col0 + r] = src[r * in + i] for r < rows, i < in: a block
// of `rows` rows of an (out x in) row-major matrix from a llama2.c file,
// written transposed into columns col0 .. col0 + rows of the (in x ld)
// destination (the CPU loader's read_transposed, model.cpp:43-53). 32 x 32
// tiles through LDS (padded against bank conflicts): both the reads and the
// writes are coalesced.
__global__ __launch_bounds__(kThreads) void transpose_kernel(const float* __restrict__ src,
                                                             std::size_t rows, std::size_t in,
                                                             float* __restrict__ dst,
                                                             std::size_t ld, std::size_t col0) {
    __shared__ float tile[32][33];
    const std::size_t r0 = static_cast<std::size_t>(blockIdx.y) * 32;
    const std::size_t i0 = static_cast<std::size_t>(blockIdx.x) * 32;
    const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;
    for (int k = ty; k < 32; k += kThreads / 32) {
        const std::size_t r = r0 + k, i = i0 + tx;
        if (r < rows && i < in) tile[k][tx] = src[r * in + i];
    }
    __syncthreads();
    for (int k = ty; k < 32; k += kThreads / 32) {
        const std::size_t i = i0 + k, r = r0 + tx;
        if (r < rows && i < in) dst[i * ld + col0 + r] = tile[tx][k];
    }
}

void check(hipError_t err, const char* what) { hip_check(err, what); }

// Device buffer of T, freed with the owner.
template <class T>
struct Buf {
    T* p = nullptr;
    std::size_t n = 0;
    Buf() = default;
    Buf(const Buf&) = delete;
    Buf& operator=(const Buf&) = delete;
    ~Buf() {
        if (p) (void)hipFree(p);
    }
    void alloc(std::size_t count) {
        if (p) check(hipFree(p), "free");
        p = nullptr;
        n = 0;
        if (count == 0) return;
        void* v = nullptr;
        check(hipMalloc(&v, count * sizeof(T)), "alloc");
        p = static_cast<T*>(v);
        n = count;
    }
};

// The model's stream (default priority), drained before it is destroyed.
struct Stream {
    hipStream_t s = nullptr;
    Stream() { check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "create stream"); }
    Stream(const Stream&) = delete;
    Stream& operator=(const Stream&) = delete;
    ~Stream() {
        (void)hipStreamSynchronize(s);
        (void)hipStreamDestroy(s);
    }
};

// Pinned host memory, so the feed and logits copies can be graph nodes.
template <class T>
struct Pinned {
    T* p = nullptr;
    explicit Pinned(std::size_t count) {
        check(hipHostMalloc(reinterpret_cast<void**>(&p), count * sizeof(T), hipHostMallocDefault),
              "alloc pinned");
    }
    Pinned(const Pinned&) = delete;
    Pinned& operator=(const Pinned&) = delete;
    ~Pinned() { (void)hipHostFree(p); }
};

struct GraphExec {
    hipGraphExec_t g = nullptr;
    GraphExec() = default;
    GraphExec(const GraphExec&) = delete;
    GraphExec& operator=(const GraphExec&) = delete;
    ~GraphExec() { reset(); }
    void reset() {
        if (g) (void)hipGraphExecDestroy(g);
        g = nullptr;
    }
};

}  // namespace

// One projection: fp32 (in x out) or int8 with per-column scales.
struct Proj {
    Buf<float> f32;
    Buf<int8_t> q8;
    Buf<float> scale;
    int rows = 0, cols = 0;
};

struct LayerDev {
    Buf<float> rms_att, rms_ffn, kcache, vcache;
    Proj wqkv, wo, w13, w2;
};

// A llama2.c v0 checkpoint's header and size (model.cpp:61-90): the
// reference's checks and messages.
struct CheckpointInfo {
    em_model_config cfg;
    bool shared;
};
CheckpointInfo read_checkpoint_header(const std::string& path);

class Model {
public:
    Model(const em_model_config& c, const float* emb, const em_layer_weights* layers,
          const float* rms_final, const float* wcls, bool q8);
    // Reads a llama2.c v0 checkpoint (load_checkpoint, model.cpp:115-163):
    // the file streams through pinned memory to the GPU, which transposes
    // and fuses the projections (q | k | v, gate | up) and quantises them.
    Model(const std::string& path, const CheckpointInfo& info, bool q8);
    const em_model_config& config() const { return cfg_; }
    // The stored bytes of one weight array (see em_model_read_weight).
    int read_weight(const std::string& name, std::size_t layer, void* dst, std::size_t bytes);
    ~Model();
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    // Returns EM_OK or an error code (message recorded with fail()).
    int run(const int* tokens, std::size_t n, std::size_t pos, float* logits);

private:
    void init_runtime();
    void quantize_proj(Proj& p);
    void upload(Buf<float>& b, const float* src, std::size_t count);
    void make_proj(Proj& p, const float* w, int rows, int cols, Buf<float>& staging);
    void project(int n, const float* in, const Proj& w, float* out, const float* rms,
                 bool accumulate);
    MatmulArgs gemv_args(int n, const float* in, const Proj& w, float* out, const float* rms,
                         bool accumulate, const float* ssq) const;
    Summed project_summed(int n, const float* in, const Proj& w, float* out, const float* rms,
                          const float* ssq);
    bool residual(int n, const float* in, const Proj& w);
    bool residual_merged(const SplitRow& att, const Proj& w);
    bool swiglu_pair(int n, const LayerDev& L);
    bool qkv_exact_split(int n, LayerDev& L, bool* roped);
    bool swiglu_w2(const Summed& gu, const Proj& w2, bool* wrote_ssq);
    void reserve_rows(std::size_t n);
    void enqueue(int n);
    std::size_t buffers_generation() const { return own_generation_ + scratch_generation(); }

    // Declared first, destroyed last: the buffers below are freed after the
    // stream has drained.
    Stream owned_stream_;
    hipStream_t stream_ = owned_stream_.s;
    em_model_config cfg_;
    bool q8_;
    AttnShape shape_;
    Buf<float> emb_, rms_final_, rope_cos_, rope_sin_, logits_dev_;
    Proj wcls_;
    std::vector<LayerDev> layers_;
    std::size_t filled_ = 0;

    std::size_t rows_ = 0, own_generation_ = 0;
    Buf<float> x_, qkv_, att_, gu_, hb_, attn_scratch_;
    // One-token steps: sums of squares of x per 64 values, left by the
    // kernel that last wrote x for the next norm GEMV (dim % 64 == 0).
    bool use_ssq_ = false;
    // EM_DECODE_MERGE_KERNEL=1 at creation: one-row steps merge the
    // attention chunks with the merge kernel, not in the wo GEMV (row-major
    // path) or inside the split attention launch (strip path) (tests).
    bool merge_kernel_ = false;
    // Strip path: the split attention launch merges its own chunks where a
    // workgroup serves one head (attention_merge_inside_preferred);
    // EM_DECODE_MERGE_KERNEL=0 at creation makes it do so for every shape
    // (tests).
    bool merge_inside_ = false;
    // EM_PREFILL_ROPE_FUSION=0 at creation: the exact-split qkv product of
    // prefill rows writes qkv_ and rope_cache_kernel follows, rather than
    // RoPE and the cache write in the product's epilogue (tests).
    bool rope_fusion_ = true;
    // int8 models whose five projections all took a strip-layout copy
    // (em_q8_register): one-token steps run every product as one
    // em_matmul_q8 call over it (norm fused, no k slices), the attention
    // merging its own chunks and swiglu_kernel between w13 and w2.
    // EM_MODEL_STRIPS=0 at creation keeps the row-major decode path.
    bool strips_ = false;
    // Over the strips, w13 and the SwiGLU are one launch (run_gemv_swiglu),
    // and so are they for int8 rows past 16 (swiglu_pair): the same bits;
    // EM_MODEL_SWIGLU_FUSION=0 at creation runs swiglu_kernel after the w13
    // product instead (tests).
    bool swiglu_fusion_ = true;
    void register_strips();
    Buf<float> ssq_;

    Pinned<int> feed_host_;  // [pos, tokens...]
    Buf<int> feed_dev_;
    Pinned<float> logits_host_;
    GraphExec graph_;
    std::size_t graph_generation_ = 0;
};

Model::Model(const em_model_config& c, const float* emb, const em_layer_weights* layers,
             const float* rms_final, const float* wcls, bool q8)
    : cfg_(c), q8_(q8), feed_host_(c.seq_len + 1), logits_host_(c.vocab_size) {
    const std::size_t D = c.dim, H = c.hidden_dim, hs = c.dim / c.n_heads;
    const std::size_t KV = c.n_kv_heads * hs, V = c.vocab_size;
    shape_ = {static_cast<int>(c.n_heads), static_cast<int>(c.n_kv_heads), static_cast<int>(hs),
              static_cast<int>(c.seq_len), D + 2 * KV, KV, D};

    Buf<float> staging;  // fp32 weights on their way to quantize_q8
    upload(emb_, emb, V * D);
    upload(rms_final_, rms_final, D);
    make_proj(wcls_, wcls, static_cast<int>(D), static_cast<int>(V), staging);
    layers_ = std::vector<LayerDev>(c.n_layers);
    for (std::size_t l = 0; l < c.n_layers; ++l) {
        LayerDev& L = layers_[l];
        const em_layer_weights& w = layers[l];
        upload(L.rms_att, w.rms_att, D);
        upload(L.rms_ffn, w.rms_ffn, D);
        make_proj(L.wqkv, w.wqkv, static_cast<int>(D), static_cast<int>(D + 2 * KV), staging);
        make_proj(L.wo, w.wo, static_cast<int>(D), static_cast<int>(D), staging);
        make_proj(L.w13, w.w13, static_cast<int>(D), static_cast<int>(2 * H), staging);
        make_proj(L.w2, w.w2, static_cast<int>(H), static_cast<int>(D), staging);
    }

    init_runtime();
}

// Everything but the weights: caches, RoPE tables, feed and logits buffers.
void Model::init_runtime() {
    const em_model_config& c = cfg_;
    const std::size_t D = c.dim, hs = c.dim / c.n_heads, V = c.vocab_size;
    const std::size_t KV = c.n_kv_heads * hs;
    for (LayerDev& L : layers_) {
        L.kcache.alloc(c.seq_len * KV);
        L.vcache.alloc(c.seq_len * KV);
    }
    // RoPE angles with the CPU model's float expressions (rope_tables,
    // model.cpp:179-192), so both models rotate by the same bits.
    const std::size_t half = hs / 2;
    std::vector<float> cs(c.seq_len * half), sn(c.seq_len * half);
    for (std::size_t pos = 0; pos < c.seq_len; ++pos) {
        for (std::size_t j = 0; j < half; ++j) {
            const float freq = 1.0f / std::pow(10000.0f, static_cast<float>(2 * j) /
                                                          static_cast<float>(hs));
            const float angle = static_cast<float>(pos) * freq;
            cs[pos * half + j] = std::cos(angle);
            sn[pos * half + j] = std::sin(angle);
        }
    }
    upload(rope_cos_, cs.data(), cs.size());
    upload(rope_sin_, sn.data(), sn.size());

    logits_dev_.alloc(V);
    feed_dev_.alloc(c.seq_len + 1);
    use_ssq_ = D % kSsqChunk == 0 && D / kSsqChunk <= 256;
    if (use_ssq_) ssq_.alloc(D / kSsqChunk);
    const char* mk = std::getenv("EM_DECODE_MERGE_KERNEL");
    merge_kernel_ = mk && std::atoi(mk) != 0;
    merge_inside_ = mk ? !merge_kernel_ : attention_merge_inside_preferred(shape_);
    const char* rf = std::getenv("EM_PREFILL_ROPE_FUSION");
    rope_fusion_ = !rf || std::atoi(rf) != 0;
    const char* sf = std::getenv("EM_MODEL_SWIGLU_FUSION");
    swiglu_fusion_ = !sf || std::atoi(sf) != 0;
    check(hipStreamSynchronize(stream_), "load weights");
    reserve_rows(1);
    register_strips();  // last: nothing after it can throw and skip the destructor
}

// Every int8 projection gets a strip-layout copy, or none does (a shape
// the layout cannot hold, or EM_MODEL_STRIPS=0 / EM_STRIP_COPY=0).
void Model::register_strips() {
    const char* env = std::getenv("EM_MODEL_STRIPS");
    if (!q8_ || (env && std::atoi(env) == 0)) return;
    std::vector<const Proj*> all{&wcls_};
    for (const LayerDev& L : layers_) {
        all.push_back(&L.wqkv);
        all.push_back(&L.wo);
        all.push_back(&L.w13);
        all.push_back(&L.w2);
    }
    // A copy left registered after its weights are freed could be found
    // again by a later allocation at the same address: on any failure every
    // registration made here is undone before the error propagates.
    bool every = true;
    for (const Proj* p : all) {
        if (em_q8_register(p->q8.p, p->rows, p->cols, stream_) != EM_OK) {
            const std::string msg = em_last_error();
            for (const Proj* q : all) (void)em_q8_unregister(q->q8.p);
            throw DeviceError(msg);
        }
        every = every && em_q8_registered(p->q8.p, p->rows, p->cols) == 1;
    }
    if (!every) {
        for (const Proj* p : all) (void)em_q8_unregister(p->q8.p);
        return;
    }
    strips_ = true;
}

// ---- llama2.c v0 checkpoint ---------------------------------------------

// A checkpoint that cannot be opened or read, or whose header or size is
// bad: EM_EIO (the reference's std::runtime_error from load_checkpoint).
struct CheckpointError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

namespace {

struct File {
    FILE* f = nullptr;
    explicit File(const std::string& path) : f(std::fopen(path.c_str(), "rb")) {}
    ~File() {
        if (f) std::fclose(f);
    }
};

}  // namespace

// parse_header and expected_size, model.cpp:61-90: every field non-zero and
// all but the vocabulary positive (a positive vocabulary means the classifier
// is the embedding); heads split evenly, even head size, whole kv groups; the
// file exactly as long as the header implies.
CheckpointInfo read_checkpoint_header(const std::string& path) {
    File in(path);
    if (!in.f) throw CheckpointError("cannot open checkpoint " + path);
    std::fseek(in.f, 0, SEEK_END);
    const std::uint64_t file_size = static_cast<std::uint64_t>(ftello(in.f));
    std::fseek(in.f, 0, SEEK_SET);
    std::int32_t h[7];
    if (std::fread(h, sizeof(std::int32_t), 7, in.f) != 7)
        throw CheckpointError("checkpoint " + path + " ended early");
    CheckpointInfo info{};
    info.shared = h[5] > 0;
    for (int i = 0; i < 7; ++i)
        if (h[i] == 0 || (i != 5 && h[i] < 0))
            throw CheckpointError("checkpoint " + path + ": bad header field " + std::to_string(i) +
                                  " = " + std::to_string(h[i]));
    auto u = [](std::int32_t v) { return static_cast<std::size_t>(v < 0 ? -std::int64_t{v} : v); };
    em_model_config& c = info.cfg;
    c = {u(h[0]), u(h[1]), u(h[2]), u(h[3]), u(h[4]), u(h[5]), u(h[6])};
    if (c.dim % c.n_heads != 0 || (c.dim / c.n_heads) % 2 != 0 || c.n_heads % c.n_kv_heads != 0)
        throw CheckpointError("checkpoint " + path +
                              ": dim must split into even-sized heads, and query heads into whole "
                              "groups per kv head");
    const std::uint64_t D = c.dim, H = c.hidden_dim, hs = c.dim / c.n_heads;
    const std::uint64_t KV = c.n_kv_heads * hs, V = c.vocab_size;
    const std::uint64_t per_layer = 2 * D + 2 * D * D + 2 * D * KV + 3 * D * H;
    std::uint64_t floats = V * D + c.n_layers * per_layer + D + std::uint64_t{c.seq_len} * hs;
    if (!info.shared) floats += V * D;
    const std::uint64_t want = 7 * sizeof(std::int32_t) + floats * sizeof(float);
    if (file_size != want)
        throw CheckpointError("checkpoint " + path + " is " + std::to_string(file_size) +
                              " bytes, header implies " + std::to_string(want));
    return info;
}

namespace {

// Streams a checkpoint's float sections to the GPU: two pinned chunks and
// two device staging chunks in turn, so reading one chunk from the file
// overlaps the copy and transpose of the previous one.
class Streamer {
public:
    static constexpr std::size_t kChunk = 64u << 20;  // bytes

    Streamer(const std::string& path, hipStream_t s) : path_(path), in_(path), s_(s) {
        if (!in_.f) throw CheckpointError("cannot open checkpoint " + path);
        std::fseek(in_.f, 7 * sizeof(std::int32_t), SEEK_SET);
        for (int b = 0; b < 2; ++b) {
            check(hipHostMalloc(&host_[b], kChunk, hipHostMallocDefault), "pinned staging");
            check(hipMalloc(&dev_[b], kChunk), "device staging");
            check(hipEventCreateWithFlags(&done_[b], hipEventDisableTiming), "event");
        }
    }
    ~Streamer() {
        (void)hipStreamSynchronize(s_);
        for (int b = 0; b < 2; ++b) {
            if (done_[b]) (void)hipEventDestroy(done_[b]);
            if (dev_[b]) (void)hipFree(dev_[b]);
            if (host_[b]) (void)hipHostFree(host_[b]);
        }
    }
    Streamer(const Streamer&) = delete;
    Streamer& operator=(const Streamer&) = delete;

    // `count` floats straight into dst.
    void plain(float* dst, std::size_t count) {
        const std::size_t per = kChunk / sizeof(float);
        for (std::size_t done = 0; done < count; done += per) {
            const std::size_t n = std::min(per, count - done);
            float* h = next(n);
            check(hipMemcpyAsync(dst + done, h, n * sizeof(float), hipMemcpyHostToDevice, s_),
                  "upload checkpoint");
            check(hipEventRecord(done_[cur_], s_), "event");
        }
    }

    // An (out x in) row-major matrix, transposed into columns col0 .. col0 +
    // out of dst (in x ld): read_transposed, model.cpp:43-53.
    void transposed(std::size_t out, std::size_t in, float* dst, std::size_t ld, std::size_t col0) {
        const std::size_t per = kChunk / sizeof(float);
        if (in > per) {
            // A row longer than a chunk (a wide w2): each row in chunk-sized
            // segments, segment [c, c + len) landing in rows c .. c + len - 1
            // of dst, column col0 + r.
            for (std::size_t r = 0; r < out; ++r) {
                for (std::size_t c = 0; c < in; c += per) {
                    const std::size_t len = std::min(per, in - c);
                    float* h = next(len);
                    float* d = dev_[cur_];
                    check(hipMemcpyAsync(d, h, len * sizeof(float), hipMemcpyHostToDevice, s_),
                          "upload checkpoint");
                    const dim3 grid(ceil_div(static_cast<long long>(len), 32), 1);
                    hipLaunchKernelGGL(transpose_kernel, grid, dim3(kThreads), 0, s_, d,
                                       std::size_t{1}, len, dst + c * ld, ld, col0 + r);
                    check(hipGetLastError(), "launch");
                    check(hipEventRecord(done_[cur_], s_), "event");
                }
            }
            return;
        }
        const std::size_t rows_per = per / in;
        for (std::size_t r = 0; r < out; r += rows_per) {
            const std::size_t rows = std::min(rows_per, out - r);
            float* h = next(rows * in);
            float* d = dev_[cur_];
            check(hipMemcpyAsync(d, h, rows * in * sizeof(float), hipMemcpyHostToDevice, s_),
                  "upload checkpoint");
            const dim3 grid(ceil_div(static_cast<long long>(in), 32),
                            ceil_div(static_cast<long long>(rows), 32));
            hipLaunchKernelGGL(transpose_kernel, grid, dim3(kThreads), 0, s_, d, rows, in, dst, ld,
                               col0 + r);
            check(hipGetLastError(), "launch");
            check(hipEventRecord(done_[cur_], s_), "event");
        }
    }

    void skip_floats(std::size_t n) {
        if (std::fseek(in_.f, static_cast<long>(n * sizeof(float)), SEEK_CUR) != 0)
            throw CheckpointError("checkpoint " + path_ + " ended early");
    }

private:
    // The next pinned chunk, filled with n floats from the file, once the
    // work that last used it (and its device twin) has finished.
    float* next(std::size_t n) {
        cur_ ^= 1;
        check(hipEventSynchronize(done_[cur_]), "staging reuse");
        float* h = static_cast<float*>(host_[cur_]);
        if (std::fread(h, sizeof(float), n, in_.f) != n)
            throw CheckpointError("checkpoint " + path_ + " ended early");
        return h;
    }

    std::string path_;
    File in_;
    hipStream_t s_;
    void* host_[2] = {};
    float* dev_[2] = {};
    hipEvent_t done_[2] = {};
    int cur_ = 1;
};

}  // namespace

// load_checkpoint's order (model.cpp:133-162): the file groups each weight
// across all layers (every layer's wq, then every wk, ...); projections are
// stored out x in and land transposed, q | k | v into wqkv and w1 | w3 into
// w13. The RoPE tables at the end are skipped (recomputed); a positive
// vocabulary makes the classifier the embedding's transpose. With q8 each
// projection is then quantised on the GPU (quantize_q8, bit-exact).
Model::Model(const std::string& path, const CheckpointInfo& info, bool q8)
    : cfg_(info.cfg), q8_(q8), feed_host_(info.cfg.seq_len + 1),
      logits_host_(info.cfg.vocab_size) {
    const em_model_config& c = cfg_;
    const std::size_t D = c.dim, H = c.hidden_dim, hs = c.dim / c.n_heads;
    const std::size_t KV = c.n_kv_heads * hs, V = c.vocab_size, QKV = D + 2 * KV;
    shape_ = {static_cast<int>(c.n_heads), static_cast<int>(c.n_kv_heads), static_cast<int>(hs),
              static_cast<int>(c.seq_len), QKV, KV, D};
    layers_ = std::vector<LayerDev>(c.n_layers);
    auto fp32 = [&](Proj& p, std::size_t rows, std::size_t cols) {
        p.rows = static_cast<int>(rows);
        p.cols = static_cast<int>(cols);
        p.f32.alloc(rows * cols);
    };
    emb_.alloc(V * D);
    rms_final_.alloc(D);
    fp32(wcls_, D, V);
    for (LayerDev& L : layers_) {
        L.rms_att.alloc(D);
        L.rms_ffn.alloc(D);
        fp32(L.wqkv, D, QKV);
        fp32(L.wo, D, D);
        fp32(L.w13, D, 2 * H);
        fp32(L.w2, H, D);
    }
    {
        Streamer r(path, stream_);
        r.plain(emb_.p, V * D);
        for (LayerDev& L : layers_) r.plain(L.rms_att.p, D);
        for (LayerDev& L : layers_) r.transposed(D, D, L.wqkv.f32.p, QKV, 0);
        for (LayerDev& L : layers_) r.transposed(KV, D, L.wqkv.f32.p, QKV, D);
        for (LayerDev& L : layers_) r.transposed(KV, D, L.wqkv.f32.p, QKV, D + KV);
        for (LayerDev& L : layers_) r.transposed(D, D, L.wo.f32.p, D, 0);
        for (LayerDev& L : layers_) r.plain(L.rms_ffn.p, D);
        for (LayerDev& L : layers_) r.transposed(H, D, L.w13.f32.p, 2 * H, 0);
        for (LayerDev& L : layers_) r.transposed(D, H, L.w2.f32.p, D, 0);
        for (LayerDev& L : layers_) r.transposed(H, D, L.w13.f32.p, 2 * H, H);
        r.plain(rms_final_.p, D);
        r.skip_floats(c.seq_len * hs);
        if (info.shared) {
            const dim3 grid(ceil_div(static_cast<long long>(D), 32),
                            ceil_div(static_cast<long long>(V), 32));
            hipLaunchKernelGGL(transpose_kernel, grid, dim3(kThreads), 0, stream_, emb_.p, V, D,
                               wcls_.f32.p, V, std::size_t{0});
            check(hipGetLastError(), "launch");
        } else {
            r.transposed(V, D, wcls_.f32.p, V, 0);
        }
        check(hipStreamSynchronize(stream_), "load checkpoint");
    }
    if (q8_) {
        quantize_proj(wcls_);
        for (LayerDev& L : layers_) {
            quantize_proj(L.wqkv);
            quantize_proj(L.wo);
            quantize_proj(L.w13);
            quantize_proj(L.w2);
        }
    }
    init_runtime();
}

// fp32 weights already on the device -> int8 + scales (quantize_q8), the
// fp32 copy freed once the stream has used it.
void Model::quantize_proj(Proj& p) {
    p.q8.alloc(static_cast<std::size_t>(p.rows) * p.cols);
    p.scale.alloc(p.cols);
    run_quantize_q8(p.rows, p.cols, p.f32.p, p.q8.p, p.scale.p, stream_);
    check(hipGetLastError(), "launch");
    check(hipStreamSynchronize(stream_), "quantize weights");
    p.f32.alloc(0);
}

// The array named like ref_ckpt_array / LayerWeights (model.h:29-43): fp32
// arrays as floats; an int8 model's projections as their int8 bytes, and
// "<name>.scale" as their column scales. bytes must be the array's size.
int Model::read_weight(const std::string& name, std::size_t layer, void* dst, std::size_t bytes) {
    const void* src = nullptr;
    std::size_t size = 0;
    auto from = [&](const void* p, std::size_t n) {
        src = p;
        size = n;
    };
    auto proj = [&](const Proj& w, const std::string& base) {
        const std::size_t count = static_cast<std::size_t>(w.rows) * w.cols;
        if (name == base) {
            if (q8_) from(w.q8.p, count);
            else from(w.f32.p, count * sizeof(float));
        } else if (q8_ && name == base + ".scale") {
            from(w.scale.p, w.cols * sizeof(float));
        }
    };
    const std::size_t D = cfg_.dim, V = cfg_.vocab_size;
    if (name == "token_embedding") from(emb_.p, V * D * sizeof(float));
    else if (name == "rms_final") from(rms_final_.p, D * sizeof(float));
    else if (name.rfind("wcls", 0) == 0) proj(wcls_, "wcls");
    else if (layer < layers_.size()) {
        const LayerDev& L = layers_[layer];
        if (name == "rms_att") from(L.rms_att.p, D * sizeof(float));
        else if (name == "rms_ffn") from(L.rms_ffn.p, D * sizeof(float));
        else if (name.rfind("wqkv", 0) == 0) proj(L.wqkv, "wqkv");
        else if (name.rfind("wo", 0) == 0) proj(L.wo, "wo");
        else if (name.rfind("w13", 0) == 0) proj(L.w13, "w13");
        else if (name.rfind("w2", 0) == 0) proj(L.w2, "w2");
    }
    if (!src) return fail(EM_EINVAL, "read_weight: no array " + name + " in layer " + std::to_string(layer));
    if (bytes != size)
        return fail(EM_EINVAL, "read_weight: " + name + " is " + std::to_string(size) +
                                   " bytes, not " + std::to_string(bytes));
    check(hipMemcpyAsync(dst, src, size, hipMemcpyDeviceToHost, stream_), "read weight");
    check(hipStreamSynchronize(stream_), "read weight");
    return EM_OK;
}

Model::~Model() {
    (void)hipStreamSynchronize(stream_);
    if (strips_) {
        (void)em_q8_unregister(wcls_.q8.p);
        for (const LayerDev& L : layers_) {
            (void)em_q8_unregister(L.wqkv.q8.p);
            (void)em_q8_unregister(L.wo.q8.p);
            (void)em_q8_unregister(L.w13.q8.p);
            (void)em_q8_unregister(L.w2.q8.p);
        }
    }
}

void Model::upload(Buf<float>& b, const float* src, std::size_t count) {
    b.alloc(count);
    if (count)
        check(hipMemcpyAsync(b.p, src, count * sizeof(float), hipMemcpyHostToDevice, stream_),
              "upload weights");
}

void Model::make_proj(Proj& p, const float* w, int rows, int cols, Buf<float>& staging) {
    p.rows = rows;
    p.cols = cols;
    const std::size_t count = static_cast<std::size_t>(rows) * cols;
    if (!q8_) {
        upload(p.f32, w, count);
        return;
    }
    // int8 as quant.cpp makes it, on the GPU (bit-exact, quantize_q8).
    if (staging.n < count) staging.alloc(count);
    check(hipMemcpyAsync(staging.p, w, count * sizeof(float), hipMemcpyHostToDevice, stream_),
          "upload weights");
    p.q8.alloc(count);
    p.scale.alloc(cols);
    run_quantize_q8(rows, cols, staging.p, p.q8.p, p.scale.p, stream_);
    check(hipGetLastError(), "launch");
    check(hipStreamSynchronize(stream_), "quantize weights");  // staging is reused
}

void Model::project(int n, const float* in, const Proj& w, float* out, const float* rms,
                    bool accumulate) {
    const int rc =
        q8_ ? em_matmul_q8(n, w.cols, w.rows, in, w.q8.p, w.scale.p, out, EM_KERNEL_AUTOMATIC,
                           accumulate ? 1 : 0, rms, stream_)
            : em_matmul_f32(n, w.cols, w.rows, in, w.f32.p, out, EM_KERNEL_AUTOMATIC,
                            accumulate ? 1 : 0, rms, stream_);
    if (rc != EM_OK) throw DeviceError(em_last_error());
}

MatmulArgs Model::gemv_args(int n, const float* in, const Proj& w, float* out, const float* rms,
                            bool accumulate, const float* ssq) const {
    MatmulArgs a{};
    a.m = n;
    a.n = w.cols;
    a.k = w.rows;
    a.A = in;
    a.B = q8_ ? static_cast<const void*>(w.q8.p) : static_cast<const void*>(w.f32.p);
    a.scale = q8_ ? w.scale.p : nullptr;
    a.C = out;
    a.accumulate = accumulate;
    a.rms_weight = rms;
    a.stream = stream_;
    a.ssq = ssq;
    return a;
}

// out = rmsnorm(in) W for a consumer that reads it through summed(): at
// decode sizes the skinny GEMV leaves its k-slice partials (no reduce
// launch), otherwise the product is written to out as project() does.
// ssq: the sums of squares of `in` that its producer left (one row), or null.
Summed Model::project_summed(int n, const float* in, const Proj& w, float* out,
                             const float* rms, const float* ssq) {
    Summed s{out, nullptr, nullptr, 1, w.cols, static_cast<std::size_t>(n) * w.cols};
    if (n > 8 || (q8_ && split_bf16_preferred(n, w.cols, w.rows))) {
        project(n, in, w, out, rms, false);
        return s;
    }
    const MatmulArgs a = gemv_args(n, in, w, out, rms, false, ssq);
    const float* partial = nullptr;
    s.slices = q8_ ? run_skinny_partials<int8_t>(a, &partial) : run_skinny_partials<float>(a, &partial);
    check(hipGetLastError(), "launch");
    if (s.slices > 1) {
        s.partial = partial;
        s.scale = a.scale;
    }
    return s;
}

// x += in W. For one row with the sums of squares in use, the GEMV's slice
// reduce also leaves those of the new x (true); otherwise as project().
bool Model::residual(int n, const float* in, const Proj& w) {
    if (n != 1 || !use_ssq_) {
        project(n, in, w, x_.p, nullptr, true);
        return false;
    }
    const MatmulArgs a = gemv_args(1, in, w, x_.p, nullptr, true, nullptr);
    const float* partial = nullptr;
    const int slices =
        q8_ ? run_skinny_partials<int8_t>(a, &partial) : run_skinny_partials<float>(a, &partial);
    if (slices > 1)
        run_reduce_slices(1, w.cols, slices, partial, a.scale, x_.p, true, stream_, ssq_.p);
    check(hipGetLastError(), "launch");
    return slices > 1;
}

// Prefill rows whose int8 qkv product goes to the exact-split kernel (as
// project() would send it): with RoPE and the cache write in the product's
// epilogue when it needs no k split (*roped; k and v then reach only the
// caches), else qkv_ as project() leaves it. The same bits either way as
// project() followed by rope_cache_kernel. False: not this path.
bool Model::qkv_exact_split(int n, LayerDev& L, bool* roped) {
    const MatmulArgs a = gemv_args(n, x_.p, L.wqkv, qkv_.p, L.rms_att.p, false, nullptr);
    if (!q8_ || n < 2 || !split_bf16_preferred(a.m, a.n, a.k) || !split_bf16_supports(a))
        return false;
    const RopeFuse r{feed_dev_.p, rope_cos_.p, rope_sin_.p, L.kcache.p, L.vcache.p,
                     static_cast<int>(cfg_.dim), static_cast<int>(shape_.kv_stride),
                     shape_.head_size};
    *roped = run_split_bf16(a, rope_fusion_ ? &r : nullptr);
    check(hipGetLastError(), "launch");
    return true;
}

// x += att W for one decode row whose attention chunks are not merged yet:
// the GEMV merges them in its A staging (run_skinny_merged), one launch
// fewer; for a shape it does not take, the merge kernel writes att first.
bool Model::residual_merged(const SplitRow& att, const Proj& w) {
    const MatmulArgs a = gemv_args(1, nullptr, w, x_.p, nullptr, true, nullptr);
    float* ssq = use_ssq_ ? ssq_.p : nullptr;
    const int slices = q8_ ? run_skinny_merged<int8_t>(a, att, ssq)
                           : run_skinny_merged<float>(a, att, ssq);
    if (slices) {
        check(hipGetLastError(), "launch");
        return ssq && slices > 1;
    }
    run_attention_merge(shape_, att, att_.p, stream_);
    return residual(1, att_.p, w);
}

// One decode row: x += silu_mul(gate, up) W2 with the SwiGLU formed inside
// the w2 GEMV (run_skinny_swiglu) rather than by swiglu_kernel first: one
// launch fewer, the same values. False if the GEMV does not take the shape.
// *wrote_ssq: whether the sums of squares of the new x were left.
bool Model::swiglu_w2(const Summed& gu, const Proj& w2, bool* wrote_ssq) {
    const MatmulArgs a = gemv_args(1, nullptr, w2, x_.p, nullptr, true, nullptr);
    float* ssq = use_ssq_ ? ssq_.p : nullptr;
    const int slices = q8_ ? run_skinny_swiglu<int8_t>(a, gu, w2.rows, ssq)
                           : run_skinny_swiglu<float>(a, gu, w2.rows, ssq);
    if (slices) check(hipGetLastError(), "launch");
    *wrote_ssq = ssq && slices > 1;
    return slices > 0;
}

// Rows past 16 of an int8 model: hb = silu(gate) * up straight from the
// exact-split w13 product (run_split_bf16_swiglu), which the product
// followed by swiglu_kernel gives bit for bit, with half the product's
// stores and one launch fewer. (Up to 16 rows `automatic` may run the
// strip-copy kernels instead, so those rows keep the two launches.) False,
// nothing launched, where it does not take the shape.
bool Model::swiglu_pair(int n, const LayerDev& L) {
    if (!q8_ || !swiglu_fusion_ || n <= 16) return false;
    const MatmulArgs a = gemv_args(n, x_.p, L.w13, hb_.p, L.rms_ffn.p, false, nullptr);
    if (!split_bf16_preferred(a.m, a.n, a.k) || !run_split_bf16_swiglu(a, cfg_.hidden_dim))
        return false;
    check(hipGetLastError(), "launch");
    return true;
}

void Model::reserve_rows(std::size_t n) {
    if (n <= rows_) return;
    check(hipStreamSynchronize(stream_), "synchronize before growth");
    const std::size_t D = cfg_.dim, H = cfg_.hidden_dim;
    x_.alloc(n * D);
    qkv_.alloc(n * shape_.q_stride);
    att_.alloc(n * D);
    gu_.alloc(n * 2 * H);
    hb_.alloc(n * H);
    const std::size_t sc = attention_scratch_floats(shape_, n, kAttnAutomatic);
    attn_scratch_.alloc(sc ? sc : 1);
    rows_ = n;
    ++own_generation_;
}

void Model::enqueue(int n) {
    const int D = static_cast<int>(cfg_.dim), H = static_cast<int>(cfg_.hidden_dim);
    const int KV = static_cast<int>(shape_.kv_stride), hs = shape_.head_size;
    const int qkv_cols = static_cast<int>(shape_.q_stride);
    check(hipMemcpyAsync(feed_dev_.p, feed_host_.p, (n + 1) * sizeof(int), hipMemcpyHostToDevice,
                         stream_),
          "upload feed");
    // One-token steps over strip copies: each product is one em_matmul_q8
    // call (the norm formed inside it). Other one-token steps hand the norm
    // GEMVs the sums of squares of x from whichever kernel last wrote x
    // (embed, or a residual reduce).
    const bool strip_step = n == 1 && strips_;
    bool have_ssq = n == 1 && use_ssq_ && !strip_step;
    hipLaunchKernelGGL(embed_kernel, dim3(ceil_div(ceil_div(D, 4), kThreads), n), dim3(kThreads), 0,
                       stream_, D, feed_dev_.p, emb_.p, x_.p, have_ssq ? ssq_.p : nullptr);
    const int rope_threads = D / 2 + KV / 2 + KV;
    const int swiglu_blocks = std::min(ceil_div(static_cast<long long>(n) * H, kThreads), 4096);
    for (LayerDev& L : layers_) {
        if (strip_step) {
            project(1, x_.p, L.wqkv, qkv_.p, L.rms_att.p, false);
            const Summed qkv{qkv_.p, nullptr, nullptr, 1, qkv_cols,
                             static_cast<std::size_t>(qkv_cols)};
            if (!run_attention_rope(shape_, feed_dev_.p, qkv, D, KV, rope_cos_.p, rope_sin_.p,
                                    L.kcache.p, L.vcache.p, att_.p, attn_scratch_.p, stream_,
                                    nullptr, merge_inside_)) {
                hipLaunchKernelGGL(rope_cache_kernel, dim3(ceil_div(rope_threads, kThreads), 1),
                                   dim3(kThreads), 0, stream_, qkv, qkv_cols, D, KV, hs,
                                   feed_dev_.p, rope_cos_.p, rope_sin_.p, qkv_.p, L.kcache.p,
                                   L.vcache.p);
                run_attention(shape_, 1, feed_dev_.p, qkv_.p, L.kcache.p, L.vcache.p, att_.p,
                              attn_scratch_.p, kAttnAutomatic, stream_);
            }
            project(1, att_.p, L.wo, x_.p, nullptr, true);
            const MatmulArgs a13 = gemv_args(1, x_.p, L.w13, hb_.p, L.rms_ffn.p, false, nullptr);
            const int8_t* p13 = registered_strip(L.w13.q8.p, L.w13.rows, L.w13.cols);
            if (swiglu_fusion_ && p13 && gemv_swiglu_supported(a13)) {
                run_gemv_swiglu(a13, p13);
                check(hipGetLastError(), "launch");
            } else {
                project(1, x_.p, L.w13, gu_.p, L.rms_ffn.p, false);
                const Summed gu{gu_.p, nullptr, nullptr, 1, 2 * H,
                                static_cast<std::size_t>(2 * H)};
                hipLaunchKernelGGL(swiglu_kernel, dim3(swiglu_blocks), dim3(kThreads), 0, stream_,
                                   1, H, gu, hb_.p);
            }
            project(1, hb_.p, L.w2, x_.p, nullptr, true);
            continue;
        }
        bool roped = false;
        Summed qkv{qkv_.p, nullptr, nullptr, 1, qkv_cols,
                   static_cast<std::size_t>(n) * qkv_cols};
        if (!(n > 1 && qkv_exact_split(n, L, &roped)))
            qkv = project_summed(n, x_.p, L.wqkv, qkv_.p, L.rms_att.p,
                                 have_ssq ? ssq_.p : nullptr);
        // One row: RoPE and the cache write inside the attention launch,
        // and the chunks' merge inside the wo GEMV.
        SplitRow chunks{};
        if (!(n == 1 && run_attention_rope(shape_, feed_dev_.p, qkv, D, KV, rope_cos_.p,
                                           rope_sin_.p, L.kcache.p, L.vcache.p, att_.p,
                                           attn_scratch_.p, stream_,
                                           merge_kernel_ ? nullptr : &chunks))) {
            if (!roped)
                hipLaunchKernelGGL(rope_cache_kernel, dim3(ceil_div(rope_threads, kThreads), n),
                                   dim3(kThreads), 0, stream_, qkv, qkv_cols, D, KV, hs,
                                   feed_dev_.p, rope_cos_.p, rope_sin_.p, qkv_.p, L.kcache.p,
                                   L.vcache.p);
            run_attention(shape_, n, feed_dev_.p, qkv_.p, L.kcache.p, L.vcache.p, att_.p,
                          attn_scratch_.p, kAttnAutomatic, stream_);
        }
        have_ssq = chunks.o ? residual_merged(chunks, L.wo) : residual(n, att_.p, L.wo);
        if (swiglu_pair(n, L)) {
            project(n, hb_.p, L.w2, x_.p, nullptr, true);
            have_ssq = false;
            continue;
        }
        const Summed gu = project_summed(n, x_.p, L.w13, gu_.p, L.rms_ffn.p,
                                         have_ssq ? ssq_.p : nullptr);
        if (!(n == 1 && swiglu_w2(gu, L.w2, &have_ssq))) {
            hipLaunchKernelGGL(swiglu_kernel, dim3(swiglu_blocks), dim3(kThreads), 0, stream_, n,
                               H, gu, hb_.p);
            project(n, hb_.p, L.w2, x_.p, nullptr, true);
            have_ssq = false;
        }
    }
    // Only the last row's logits are returned.
    const float* x_last = x_.p + static_cast<std::size_t>(n - 1) * D;
    if (have_ssq) {
        const MatmulArgs a =
            gemv_args(1, x_last, wcls_, logits_dev_.p, rms_final_.p, false, ssq_.p);
        if (q8_) {
            run_skinny<int8_t>(a);
        } else {
            run_skinny<float>(a);
        }
    } else {
        project(1, x_last, wcls_, logits_dev_.p, rms_final_.p, false);
    }
    check(hipMemcpyAsync(logits_host_.p, logits_dev_.p, cfg_.vocab_size * sizeof(float),
                         hipMemcpyDeviceToHost, stream_),
          "download logits");
    check(hipGetLastError(), "launch");
}

int Model::run(const int* tokens, std::size_t n, std::size_t pos, float* logits) {
    // check_feed, model.cpp:165-177: the CPU model's exact rules and messages.
    for (std::size_t i = 0; i < n; ++i) {
        if (tokens[i] < 0 || static_cast<std::size_t>(tokens[i]) >= cfg_.vocab_size)
            return fail(EM_ERANGE, "forward: token " + std::to_string(tokens[i]) + " outside vocab");
    }
    if (pos + n > cfg_.seq_len || pos > filled_)
        return fail(EM_ERANGE, "forward: positions " + std::to_string(pos) + ".." +
                                   std::to_string(pos + n - 1) + " with " +
                                   std::to_string(filled_) + " cached of " +
                                   std::to_string(cfg_.seq_len));
    reserve_rows(n);
    feed_host_.p[0] = static_cast<int>(pos);
    std::memcpy(feed_host_.p + 1, tokens, n * sizeof(int));

    const bool replay = n == 1 && graph_.g && graph_generation_ == buffers_generation();
    if (replay) {
        check(hipGraphLaunch(graph_.g, stream_), "graph launch");
    } else {
        enqueue(static_cast<int>(n));
    }
    check(hipStreamSynchronize(stream_), "forward");
    filled_ = pos + n;
    std::memcpy(logits, logits_host_.p, cfg_.vocab_size * sizeof(float));

    // After an eager one-token run every buffer the step needs has grown, so
    // capturing allocates nothing.
    if (n == 1 && !replay) {
        graph_.reset();
        hipGraph_t graph = nullptr;
        check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "begin capture");
        try {
            enqueue(1);
        } catch (...) {
            (void)hipStreamEndCapture(stream_, &graph);
            if (graph) (void)hipGraphDestroy(graph);
            throw;
        }
        check(hipStreamEndCapture(stream_, &graph), "end capture");
        hipGraphExec_t exec = nullptr;
        const hipError_t err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        check(err, "instantiate graph");
        graph_.g = exec;
        graph_generation_ = buffers_generation();
    }
    return EM_OK;
}

}  // namespace em

struct em_model {
    em::Model impl;
    em_model(const em_model_config& c, const float* emb, const em_layer_weights* layers,
             const float* rms_final, const float* wcls, bool q8)
        : impl(c, emb, layers, rms_final, wcls, q8) {}
    em_model(const std::string& path, const em::CheckpointInfo& info, bool q8)
        : impl(path, info, q8) {}
};

using em::fail;

namespace {

bool too_big(std::size_t a, std::size_t b) {
    constexpr std::size_t kLimit = (std::size_t{1} << 31) - 1;
    return a != 0 && b > kLimit / a;
}

// EM_OK if the forward pass can run config c (sizes, 32-bit indexing, a
// shape the attention kernels take), else EM_EINVAL with the reason.
int check_config(const em_model_config& c) {
    if (!c.dim || !c.hidden_dim || !c.n_layers || !c.n_heads || !c.n_kv_heads || !c.vocab_size ||
        !c.seq_len || c.dim % c.n_heads)
        return fail(EM_EINVAL, "CudaTransformer: bad config");
    const std::size_t hs = c.dim / c.n_heads, KV = c.n_kv_heads * hs;
    if (c.dim > (1u << 30) || c.seq_len > (1u << 30) || too_big(c.vocab_size, c.dim) ||
        too_big(c.dim, c.dim + 2 * KV) || too_big(c.dim, 2 * c.hidden_dim) ||
        too_big(c.seq_len, KV) || too_big(c.seq_len + 8, c.dim + 2 * KV) ||
        too_big(c.seq_len, 2 * c.hidden_dim))
        return fail(EM_EINVAL, "CudaTransformer: more than 2^31 elements");
    const em::AttnShape shape{static_cast<int>(c.n_heads), static_cast<int>(c.n_kv_heads),
                              static_cast<int>(hs), static_cast<int>(c.seq_len),
                              c.dim + 2 * KV, KV, c.dim};
    const std::string why = em::attention_reject(shape, em::kAttnAutomatic);
    if (!why.empty()) return fail(EM_EINVAL, "CudaTransformer: " + why);
    return EM_OK;
}

}  // namespace

extern "C" {

int em_model_create(const em_model_config* cfg, const float* token_embedding,
                    const em_layer_weights* layers, const float* rms_final, const float* wcls,
                    int weight_type, em_model** out) {
    if (!out) return fail(EM_EINVAL, "CudaTransformer: null output pointer");
    *out = nullptr;
    if (!cfg) return fail(EM_EINVAL, "CudaTransformer: null config");
    const em_model_config& c = *cfg;
    if (weight_type != EM_WEIGHTS_F32 && weight_type != EM_WEIGHTS_Q8)
        return fail(EM_EINVAL, "CudaTransformer: unknown weight type");
    if (const int rc = check_config(c)) return rc;
    if (!token_embedding || !layers || !rms_final || !wcls)
        return fail(EM_EINVAL, "CudaTransformer: null weights");
    for (std::size_t l = 0; l < c.n_layers; ++l) {
        const em_layer_weights& w = layers[l];
        if (!w.rms_att || !w.wqkv || !w.wo || !w.rms_ffn || !w.w13 || !w.w2)
            return fail(EM_EINVAL, "CudaTransformer: null weights in layer " + std::to_string(l));
    }
    if (!em::device_present()) return fail(EM_ENODEV, "CudaTransformer: no usable GPU");
    try {
        *out = new em_model(c, token_embedding, layers, rms_final, wcls,
                            weight_type == EM_WEIGHTS_Q8);
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, std::string("CudaTransformer: ") + e.what());
    }
    return EM_OK;
}

int em_model_load(const char* path, int weight_type, em_model** out) {
    if (!out) return fail(EM_EINVAL, "load_checkpoint: null output pointer");
    *out = nullptr;
    if (!path) return fail(EM_EINVAL, "load_checkpoint: null path");
    if (weight_type != EM_WEIGHTS_F32 && weight_type != EM_WEIGHTS_Q8)
        return fail(EM_EINVAL, "CudaTransformer: unknown weight type");
    em::CheckpointInfo info{};
    try {
        info = em::read_checkpoint_header(path);
    } catch (const std::exception& e) {
        return fail(EM_EIO, e.what());
    }
    if (const int rc = check_config(info.cfg)) return rc;
    if (!em::device_present()) return fail(EM_ENODEV, "CudaTransformer: no usable GPU");
    try {
        *out = new em_model(path, info, weight_type == EM_WEIGHTS_Q8);
    } catch (const em::CheckpointError& e) {
        return fail(EM_EIO, e.what());
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, std::string("CudaTransformer: ") + e.what());
    }
    return EM_OK;
}

int em_model_config_get(const em_model* m, em_model_config* out) {
    if (!m || !out) return fail(EM_EINVAL, "config: null pointer");
    *out = m->impl.config();
    return EM_OK;
}

int em_model_read_weight(em_model* m, const char* name, size_t layer, void* dst, size_t bytes) {
    if (!m || !name || !dst) return fail(EM_EINVAL, "read_weight: null pointer");
    try {
        return m->impl.read_weight(name, layer, dst, bytes);
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, e.what());
    }
}

int em_model_destroy(em_model* m) {
    delete m;
    return EM_OK;
}

int em_model_forward(em_model* m, const int* tokens, size_t n, size_t pos, float* logits) {
    if (!m) return fail(EM_EINVAL, "forward: null model");
    if (n == 0) return fail(EM_EINVAL, "prefill: no tokens");
    if (!tokens || !logits) return fail(EM_EINVAL, "forward: null pointer");
    try {
        return m->impl.run(tokens, n, pos, logits);
    } catch (const std::exception& e) {
        return fail(EM_EDEVICE, e.what());
    }
}

}  // extern "C"
