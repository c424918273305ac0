#pragma once
// param -= lr * grad (legacy/include/dl/optim/Optimizer.hpp:24-34 rule).

#include <cstdint>

namespace dl::kernels {

void sgd_update(float* param, const float* grad, float lr, int64_t n);

}  // namespace dl::kernels
