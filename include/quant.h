// quantize_q8 / dequantize with the reference's signatures
// (/root/reference/src/quant.h:1-9), computed on the GPU by the C ABI's
// em_quantize_q8 / em_dequantize_q8. The result is bit-for-bit the
// reference's quant.cpp:6-36: scale[c] = max|B[:, c]| / 127, q =
// clamp(lround(B * (1 / scale)), -127, 127), an all-zero column gets scale 0.
#pragma once

#include "cuda_matmul.h"

inline QTensor quantize_q8(const Tensor& B) {
    QTensor q;
    q.rows = B.rows;
    q.cols = B.cols;
    q.data.resize(B.data.size());
    q.scale.assign(B.cols, 0.0f);
    if (B.cols == 0) return q;
    const DeviceTensor dB(B);
    void* dq = nullptr;
    void* ds = nullptr;
    try {
        em_detail::check(em_malloc(&dq, q.data.size()));
        em_detail::check(em_malloc(&ds, q.scale.size() * sizeof(float)));
        em_detail::check(em_quantize_q8(B.rows, B.cols, dB.data(), static_cast<std::int8_t*>(dq),
                                        static_cast<float*>(ds), EM_STREAM_PER_THREAD));
        if (!q.data.empty()) em_detail::check(em_memcpy_d2h(q.data.data(), dq, q.data.size()));
        em_detail::check(em_memcpy_d2h(q.scale.data(), ds, q.scale.size() * sizeof(float)));
    } catch (...) {
        em_free(dq);
        em_free(ds);
        throw;
    }
    em_free(dq);
    em_free(ds);
    return q;
}

inline Tensor dequantize(const QTensor& B) {
    const DeviceQTensor dB(B);
    DeviceTensor out(B.rows, B.cols);
    em_detail::check(em_dequantize_q8(B.rows, B.cols, dB.data(), dB.scale(), out.data(),
                                      EM_STREAM_PER_THREAD));
    return out.download();
}
