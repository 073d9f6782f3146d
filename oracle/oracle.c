/*
 * CPU oracle for the matmul hot path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker. Nothing in the product library
 * (llm-engine_amd/) links or calls it.
 *
 * A plain-C restatement of the reference's arithmetic for this path.
 * Citations are to /root/reference:
 *   orc_quantize_q8      src/quant.cpp:6-28   (per-column absmax / 127, lround, clamp)
 *   orc_dequantize       src/quant.cpp:30-36
 *   orc_matmul_naive     src/matmul.cpp:205-217 (i-k-j, fp32 accumulate into C)
 *   orc_rmsnorm          src/ops.cpp:8-26     (double sum of squares)
 *   orc_matmul_fused     composition used by tests/test_cuda.cpp:126-213:
 *                        C = [C0 +] rmsnorm(A, w) x B, with B fp32 or dequantized int8
 *   orc_abs_bound        sum_k |a_ik| |b_kj| in double
 *                        1e-4 * sum|a||w| is built from it
 *   orc_matmul_f64       double-accumulated product, for error measurement
 *   orc_attention        causal attention over a KV cache in double:
 *                        src/cuda_attention.h:28-38 (contract) and the CPU
 *                        path Transformer::attention, src/model.cpp:217-254
 *
 * Built with -ffp-contract=off so every multiply and add rounds separately,
 * as the reference's C++ source reads.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   quantize_q8  bit-exact against oracle/_ref (the reference's quant.cpp
 *                compiled from source) on committed golden fixtures and
 *                SHA-256 digests at the 4096^2 and Llama-7B shapes; the
 *                invariants of tests/test_quant.cpp:33-51; hand-built ties.
 *   matmul_naive the known answer of tests/test_matmul.cpp:40-52; exact
 *                equality with the f64 product on small-integer inputs; the
 *                reference's matmul_parallel within 1e-5*k (golden fixtures).
 *   rmsnorm      the known values of tests/test_ops.cpp:30-50 and the
 *                reference's rmsnorm (golden fixtures).
 *   attention    closed forms: a one-position context returns v_0; equal keys
 *                return the mean of the values; a hand-computed two-position
 *                answer fixes the 1/sqrt(head_size) scale; constant per-kv-head
 *                values fix the h / (n_heads / n_kv_heads) head mapping. End to
 *                end, the forward-pass tests compare logits with the
 *                reference's compiled Transformer (oracle/_ref/libref_model.so).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* quant.cpp:6-28. scale[c] = max|B[:,c]| / 127, inv = 1/scale (0 for a zero
 * column), q = clamp(lround(B * inv), -127, 127). The absmax loop keeps the
 * running value when the new one compares unordered, as std::max does. */
void orc_quantize_q8(size_t rows, size_t cols, const float* B, int8_t* q, float* scale) {
    for (size_t c = 0; c < cols; ++c) scale[c] = 0.0f;
    for (size_t r = 0; r < rows; ++r) {
        for (size_t c = 0; c < cols; ++c) {
            const float v = fabsf(B[r * cols + c]);
            if (scale[c] < v) scale[c] = v;
        }
    }
    float* inv = (float*)malloc((cols ? cols : 1) * sizeof(float));
    for (size_t c = 0; c < cols; ++c) {
        scale[c] = scale[c] / 127.0f;
        inv[c] = scale[c] > 0.0f ? 1.0f / scale[c] : 0.0f;
    }
    for (size_t r = 0; r < rows; ++r) {
        for (size_t c = 0; c < cols; ++c) {
            const float x = B[r * cols + c] * inv[c];
            long v = lroundf(x);
            if (v < -127) v = -127;
            if (v > 127) v = 127;
            q[r * cols + c] = (int8_t)v;
        }
    }
    free(inv);
}

/* quant.cpp:30-36. */
void orc_dequantize(size_t rows, size_t cols, const int8_t* q, const float* scale, float* out) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) out[r * cols + c] = (float)q[r * cols + c] * scale[c];
}

/* matmul.cpp:205-217: C = 0, then for i, for p, a = A[i][p], C[i][:] += a * B[p][:]. */
void orc_matmul_naive(size_t m, size_t n, size_t k, const float* A, const float* B, float* C) {
    memset(C, 0, m * n * sizeof(float));
    for (size_t i = 0; i < m; ++i) {
        for (size_t p = 0; p < k; ++p) {
            const float a = A[i * k + p];
            float* c = C + i * n;
            const float* b = B + p * n;
            for (size_t j = 0; j < n; ++j) c[j] += a * b[j];
        }
    }
}

/* ops.cpp:8-26: ss in double, scale = (float)(1 / sqrt(ss / cols + eps)),
 * y = x * scale * w. */
void orc_rmsnorm(size_t rows, size_t cols, const float* x, const float* w, float eps, float* y) {
    if (cols == 0) return;
    for (size_t r = 0; r < rows; ++r) {
        const float* in = x + r * cols;
        float* out = y + r * cols;
        double ss = 0.0;
        for (size_t c = 0; c < cols; ++c) ss += (double)in[c] * (double)in[c];
        const float s = (float)(1.0 / sqrt(ss / (double)cols + (double)eps));
        for (size_t c = 0; c < cols; ++c) out[c] = in[c] * s * w[c];
    }
}

/* The MatmulFusion contract (cuda_matmul.h:85-92) as the reference's tests
 * state it (test_cuda.cpp:145-151, 201): C = [C +] rmsnorm(A, w) x B', where
 * B' is B (fp32) or dequantize(Bq, scale) (int8). Bq == NULL selects fp32.
 * w == NULL: no norm. C holds C0 on entry when accumulate != 0. */
void orc_matmul_fused(size_t m, size_t n, size_t k, const float* A, const float* B,
                      const int8_t* Bq, const float* scale, const float* w, int accumulate,
                      float* C) {
    float* a = (float*)malloc((m * k ? m * k : 1) * sizeof(float));
    float* b = (float*)malloc((k * n ? k * n : 1) * sizeof(float));
    float* prod = (float*)malloc((m * n ? m * n : 1) * sizeof(float));
    if (w) {
        orc_rmsnorm(m, k, A, w, 1e-5f, a);
    } else {
        memcpy(a, A, m * k * sizeof(float));
    }
    if (Bq) {
        orc_dequantize(k, n, Bq, scale, b);
    } else {
        memcpy(b, B, k * n * sizeof(float));
    }
    orc_matmul_naive(m, n, k, a, b, prod);
    for (size_t i = 0; i < m * n; ++i) C[i] = accumulate ? C[i] + prod[i] : prod[i];
    free(a);
    free(b);
    free(prod);
}

/* bound[i][j] = sum_p |A[i][p]| |B[p][j]| in double. */
void orc_abs_bound(size_t m, size_t n, size_t k, const float* A, const float* B, double* bound) {
    memset(bound, 0, m * n * sizeof(double));
    for (size_t i = 0; i < m; ++i)
        for (size_t p = 0; p < k; ++p) {
            const double a = fabs((double)A[i * k + p]);
            const float* b = B + p * n;
            double* o = bound + i * n;
            for (size_t j = 0; j < n; ++j) o[j] += a * fabs((double)b[j]);
        }
}

/* C = A x B accumulated in double. */
void orc_matmul_f64(size_t m, size_t n, size_t k, const float* A, const float* B, double* C) {
    memset(C, 0, m * n * sizeof(double));
    for (size_t i = 0; i < m; ++i)
        for (size_t p = 0; p < k; ++p) {
            const double a = (double)A[i * k + p];
            const float* b = B + p * n;
            double* o = C + i * n;
            for (size_t j = 0; j < n; ++j) o[j] += a * (double)b[j];
        }
}

/* Greedy pick, sampler.cpp:28-29: index of the first maximum. */
size_t orc_argmax(size_t n, const float* x) {
    size_t best = 0;
    for (size_t i = 1; i < n; ++i)
        if (x[i] > x[best]) best = i;
    return best;
}

/* Causal attention, accumulated in double. Row i of q sits at position
 * pos + i and attends to cache positions [0, pos + i]; query head h reads kv
 * head h / (n_heads / n_kv_heads); out[i][h*hs + d] =
 * sum_t softmax_t(q . k_t / sqrt(hs)) v_t[d] (cuda_attention.h:28-38,
 * model.cpp:217-254). */
void orc_attention(int n_heads, int n_kv_heads, int hs, size_t rows, size_t pos, const float* q,
                   size_t q_stride, const float* kc, const float* vc, size_t kv_stride,
                   double* out, size_t out_stride) {
    const int group = n_heads / n_kv_heads;
    double* sc = (double*)malloc((pos + rows) * sizeof(double));
    for (size_t i = 0; i < rows; ++i) {
        const size_t n_ctx = pos + i + 1;
        for (int h = 0; h < n_heads; ++h) {
            const size_t kv_off = (size_t)(h / group) * (size_t)hs;
            const float* qh = q + i * q_stride + (size_t)h * (size_t)hs;
            double mx = -INFINITY;
            for (size_t t = 0; t < n_ctx; ++t) {
                double dot = 0.0;
                for (int d = 0; d < hs; ++d) dot += (double)qh[d] * (double)kc[t * kv_stride + kv_off + d];
                sc[t] = dot / sqrt((double)hs);
                if (sc[t] > mx) mx = sc[t];
            }
            double sum = 0.0;
            for (size_t t = 0; t < n_ctx; ++t) {
                sc[t] = exp(sc[t] - mx);
                sum += sc[t];
            }
            double* oh = out + i * out_stride + (size_t)h * (size_t)hs;
            for (int d = 0; d < hs; ++d) {
                double acc = 0.0;
                for (size_t t = 0; t < n_ctx; ++t) acc += sc[t] * (double)vc[t * kv_stride + kv_off + d];
                oh[d] = acc / sum;
            }
        }
    }
    free(sc);
}
