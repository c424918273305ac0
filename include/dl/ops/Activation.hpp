#pragma once
// Activations (reference include/dl/ops/Activation.hpp).  This build provides
// the ReLU on the GEMM path and its backward.

#include <cstddef>

#include <dl/tensor/Tensor.hpp>

namespace dl::ops {

Tensor relu(const Tensor& a);

// grad_input = activation > 0 ? grad_output : 0 (activation: ReLU input or output).
Tensor relu_backward(const Tensor& grad_output, const Tensor& activation);

}  // namespace dl::ops
