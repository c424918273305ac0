#pragma once
// Elementwise activation launcher (reference include/dl/kernels/activation.hpp).
// Only ReLU is on this build's path; the other enumerators are kept so code
// naming them compiles, and activation() throws std::runtime_error for them.

#include <cstddef>
#include <cstdint>

namespace dl::kernels {

enum class ActivationOp {
    ReLU,
    LeakyReLU,
    GELU,
    Sigmoid,
    Tanh
};

const char* to_string(ActivationOp op);

void activation(const float* a, float* b, int n, ActivationOp op, float alpha = 0.01f);

// grad_in = act > 0 ? grad_out : 0 (act: the ReLU input or output).
void relu_backward(const float* grad_out, const float* act, float* grad_in, int64_t n);

}  // namespace dl::kernels
