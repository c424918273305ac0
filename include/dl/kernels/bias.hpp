#pragma once
// out[r, c] += bias[c] in place (reference include/dl/kernels/bias.hpp).

namespace dl::kernels {

void add_row_bias(float* output, const float* bias, int rows, int cols);

}  // namespace dl::kernels
