// Drop-in for the reference's cuda_attention.h (/root/reference/src/
// cuda_attention.h:1-39): the same names, signatures, defaults and exception
// types, over the C ABI in llm_engine_amd.h. Calls queue on the calling
// thread's default stream (hipStreamPerThread) and return before the GPU
// finishes, like matmul_cuda().
//
// One difference the reference allows for: scratch needs no zero fill before
// its first use (the split kernel keeps no counters), and it is still fine to
// zero it.
#pragma once

#include <cstddef>
#include <stdexcept>
#include <string>

#include "llm_engine_amd.h"

// cuda_attention.h:8-13.
struct AttentionShape {
    int n_heads, n_kv_heads, head_size, seq_len;
    std::size_t q_stride;    // floats between rows of q; head h starts at h * head_size
    std::size_t kv_stride;   // floats between positions of the caches (kv_dim)
    std::size_t out_stride;  // floats between rows of out
};

// cuda_attention.h:15-19.
enum class AttentionKernel {
    automatic = EM_ATTN_AUTOMATIC,        // split for few rows; 16-row MFMA tiles for many
    single_block = EM_ATTN_SINGLE_BLOCK,  // one workgroup per (head, row), scores in LDS
    split = EM_ATTN_SPLIT,                // positions split across workgroups, then merged
};

namespace em_detail {

inline em_attention_shape to_c(const AttentionShape& s) {
    return {s.n_heads, s.n_kv_heads, s.head_size, s.seq_len, s.q_stride, s.kv_stride,
            s.out_stride};
}

inline void attention_throw(int rc) {
    if (rc == EM_OK) return;
    if (rc == EM_EINVAL) throw std::invalid_argument(em_last_error());
    throw std::runtime_error(std::string("cuda: ") + em_last_error());
}

}  // namespace em_detail

// cuda_attention.h:21-22.
inline std::size_t attention_scratch_floats(const AttentionShape& s, std::size_t rows,
                                            AttentionKernel kernel = AttentionKernel::automatic) {
    const em_attention_shape c = em_detail::to_c(s);
    return em_attention_scratch_floats(&c, rows, static_cast<int>(kernel));
}

// cuda_attention.h:24-26: throws std::invalid_argument if `kernel` cannot
// handle s.
inline void attention_check(const AttentionShape& s,
                            AttentionKernel kernel = AttentionKernel::automatic) {
    const em_attention_shape c = em_detail::to_c(s);
    em_detail::attention_throw(em_attention_check(&c, static_cast<int>(kernel)));
}

// cuda_attention.h:28-38.
inline void attention_cuda(const AttentionShape& s, std::size_t rows, const int* pos_dev,
                           const float* q, const float* key_cache, const float* value_cache,
                           float* out, float* scratch,
                           AttentionKernel kernel = AttentionKernel::automatic) {
    const em_attention_shape c = em_detail::to_c(s);
    em_detail::attention_throw(em_attention(&c, rows, pos_dev, q, key_cache, value_cache, out,
                                            scratch, static_cast<int>(kernel),
                                            EM_STREAM_PER_THREAD));
}
