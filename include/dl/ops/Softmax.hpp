#pragma once
// Row softmax of a rank-2 float32 tensor (reference include/dl/ops/Softmax.hpp).

#include <cstddef>

#include <dl/tensor/Tensor.hpp>

namespace dl::ops {

Tensor softmax(const Tensor& input);

}  // namespace dl::ops
