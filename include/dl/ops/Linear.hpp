#pragma once
// Linear layer ops (reference include/dl/ops/Linear.hpp), weight laid out
// [in_features, out_features] as in the reference's active API.

#include <dl/tensor/Tensor.hpp>

namespace dl::ops {

// Y = X W + b, computed by one GEMM with the bias fused into its epilogue.
Tensor linear(const Tensor& input, const Tensor& weight, const Tensor& bias);

// Y = max(0, X W + b) in one GEMM (bias and ReLU fused).
Tensor linear_relu(const Tensor& input, const Tensor& weight, const Tensor& bias);

// Gradients of Y = X W + b given dY (legacy/src/ops/Layers.cpp:24-45 restated
// for the [in, out] weight layout): dX = dY W^T (NT), dW = X^T dY (TN),
// db = column sums of dY.
struct LinearGrads {
    Tensor grad_input;
    Tensor grad_weight;
    Tensor grad_bias;
};

LinearGrads linear_backward(const Tensor& grad_output, const Tensor& input,
                            const Tensor& weight, bool need_grad_input = true);

}  // namespace dl::ops
