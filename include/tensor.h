// Host matrix types of the matmul path's C++ interface.
//
// Same members and layout as the reference's Tensor / QTensor
// (/root/reference/src/tensor.h:6-28), so code written against that header
// compiles unchanged: a row-major fp32 matrix, and an int8 matrix with one
// fp32 scale per column (weights are stored in x out, so a column is one
// output channel).
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

struct Tensor {
    std::size_t rows;
    std::size_t cols;
    std::vector<float> data;  // element (r, c) at r * cols + c

    Tensor() : rows(0), cols(0) {}
    Tensor(std::size_t r, std::size_t c) : rows(r), cols(c), data(r * c, 0.0f) {}

    float& at(std::size_t r, std::size_t c) { return data[r * cols + c]; }
    float at(std::size_t r, std::size_t c) const { return data[r * cols + c]; }
};

// Element (r, c) stands for data[r * cols + c] * scale[c].
struct QTensor {
    std::size_t rows = 0;
    std::size_t cols = 0;
    std::vector<std::int8_t> data;
    std::vector<float> scale;  // cols entries
};
