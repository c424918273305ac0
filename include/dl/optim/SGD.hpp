#pragma once
// Plain SGD, p -= lr * g for each (parameter, gradient) pair
// (legacy/include/dl/optim/Optimizer.hpp:12-39).

#include <vector>

#include <dl/tensor/Tensor.hpp>

namespace dl::optim {

class SGD {
public:
    explicit SGD(float lr) : lr_(lr) {}

    // params[i] -= lr * grads[i]; shapes must match.
    void step(const std::vector<Tensor*>& params, const std::vector<const Tensor*>& grads) const;
    // params[i] -= lr * params[i]->grad(), the gradients accumulated by
    // Tensor::backward(); parameters without a gradient are skipped.
    void step(const std::vector<Tensor*>& params) const;
    // Drops the accumulated gradient of every parameter.
    static void zero_grad(const std::vector<Tensor*>& params);

    float learning_rate() const { return lr_; }

private:
    float lr_;
};

}  // namespace dl::optim
