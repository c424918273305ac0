#pragma once
// Column sums: out[c] = sum over r of x[r, c] (the db of linear backward).

#include <cstdint>

namespace dl::kernels {

void colsum(const float* x, float* out, int64_t rows, int64_t cols);

}  // namespace dl::kernels
