#pragma once
// C = A . B for rank-2 float32 device tensors (reference include/dl/ops/Matmul.hpp).

#include <cstddef>

#include <dl/tensor/Tensor.hpp>

namespace dl::ops {

Tensor matmul(const Tensor& a, const Tensor& b);

}  // namespace dl::ops
