#pragma once
// Internal to libfastdl: how the ops of the MLP path record backward nodes.

#include <dl/autograd/Node.hpp>
#include <dl/tensor/Tensor.hpp>

#include <initializer_list>
#include <memory>

namespace dl::autograd {

// True when any of the tensors requires a gradient (the op must record).
bool any_requires_grad(std::initializer_list<const Tensor*> inputs);

// Makes `node` the producer of `output` and marks it as requiring a gradient.
void record(Tensor& output, std::shared_ptr<Node> node);

// Backward nodes of the recorded ops.  linear_relu's node keeps a weak
// reference to its output (for the ReLU mask) so that no ownership cycle
// output -> node -> output forms.
std::shared_ptr<Node> make_matmul_backward(const Tensor& a, const Tensor& b);
std::shared_ptr<Node> make_linear_backward(const Tensor& input, const Tensor& weight,
                                           const Tensor& bias);
std::shared_ptr<Node> make_linear_relu_backward(const Tensor& input, const Tensor& weight,
                                                const Tensor& bias, const Tensor& output);
std::shared_ptr<Node> make_relu_backward(const Tensor& input);
std::shared_ptr<Node> make_cross_entropy_backward(const Tensor& logits, const Tensor& labels);

}  // namespace dl::autograd
