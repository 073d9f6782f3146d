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
// dependent launches fewer per layer.
//
// Kernels read the position and tokens from the device feed, so the first
// one-token call is run eagerly and then captured into a HIP graph that
// later one-token calls replay with one launch; it is captured again when a
// buffer it points at has moved (own growth or the matmul scratch's).
// Everything runs on one stream the model owns, at default priority.
#include <algorithm>
#include <cmath>
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

class Model {
public:
    Model(const em_model_config& c, const float* emb, const em_layer_weights* layers,
          const float* rms_final, const float* wcls, bool q8);
    ~Model();
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    // Returns EM_OK or an error code (message recorded with fail()).
    int run(const int* tokens, std::size_t n, std::size_t pos, float* logits);

private:
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
    // attention chunks with the merge kernel, not in the wo GEMV (tests).
    bool merge_kernel_ = false;
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
    check(hipStreamSynchronize(stream_), "load weights");
    reserve_rows(1);
}

Model::~Model() { (void)hipStreamSynchronize(stream_); }

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
    *roped = run_split_bf16(a, &r);
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
    // One-token steps hand the norm GEMVs the sums of squares of x from
    // whichever kernel last wrote x (embed, or a residual reduce).
    bool have_ssq = n == 1 && use_ssq_;
    hipLaunchKernelGGL(embed_kernel, dim3(ceil_div(ceil_div(D, 4), kThreads), n), dim3(kThreads), 0,
                       stream_, D, feed_dev_.p, emb_.p, x_.p, have_ssq ? ssq_.p : nullptr);
    const int rope_threads = D / 2 + KV / 2 + KV;
    const int swiglu_blocks = std::min(ceil_div(static_cast<long long>(n) * H, kThreads), 4096);
    for (LayerDev& L : layers_) {
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
};

using em::fail;

namespace {

bool too_big(std::size_t a, std::size_t b) {
    constexpr std::size_t kLimit = (std::size_t{1} << 31) - 1;
    return a != 0 && b > kLimit / a;
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
