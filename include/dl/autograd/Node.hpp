#pragma once
// Backward node of the autograd graph: the reference's planned abstract
// `Node` with `backward(grad_output)` (FUTURE_WORK.md:111-124).  The ops of
// the MLP path record one per call whose inputs require a gradient
// (MatmulBackward, LinearBackward, LinearReluBackward, ReluBackward,
// CrossEntropyBackward); Tensor::backward() runs them in reverse topological
// order.

#include <string>
#include <vector>

#include <dl/tensor/Tensor.hpp>

namespace dl::autograd {

class Node {
public:
    explicit Node(std::vector<Tensor> inputs) : inputs_(std::move(inputs)) {}
    virtual ~Node() = default;

    Node(const Node&) = delete;
    Node& operator=(const Node&) = delete;

    // Gradients with respect to inputs(), in order, given the gradient of the
    // node's output.  An entry is left undefined for an input that does not
    // require a gradient.  Every returned tensor is newly allocated.
    virtual std::vector<Tensor> backward(const Tensor& grad_output) = 0;
    virtual std::string name() const = 0;

    // The tensors the gradient flows to (the op's differentiable inputs).
    const std::vector<Tensor>& inputs() const { return inputs_; }

protected:
    std::vector<Tensor> inputs_;
};

}  // namespace dl::autograd
