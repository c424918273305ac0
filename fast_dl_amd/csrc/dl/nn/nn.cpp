// dl::nn modules (reference src/nn/Linear.cpp, ReLU.cpp, Sequential.cpp for
// behaviour: [in, out] weights, per-construction seeds counting up from 1234,
// zero bias, forward through the ops).
#include <dl/nn/Linear.hpp>
#include <dl/nn/ReLU.hpp>
#include <dl/nn/Sequential.hpp>
#include <dl/ops/Activation.hpp>
#include <dl/ops/Linear.hpp>

#include <atomic>
#include <stdexcept>
#include <utility>

namespace dl::nn {

namespace {

// Successive Linear modules draw successive seeds, starting at 1234.
uint64_t next_linear_seed() {
    static std::atomic<uint64_t> seed{1234};
    return seed.fetch_add(1);
}

}  // namespace

Linear::Linear(int in_features, int out_features, const Device& device, LinearInit init) {
    if (in_features <= 0 || out_features <= 0) {
        throw std::runtime_error("Linear features must be positive");
    }
    const Shape wshape({in_features, out_features});
    if (init == LinearInit::XavierUniform) {
        weight_ = Tensor::xavier_uniform(wshape, DType::Float32, device, next_linear_seed());
    } else {
        weight_ = Tensor::kaiming_uniform(wshape, DType::Float32, device, next_linear_seed());
    }
    bias_ = Tensor::zeros(Shape({out_features}), DType::Float32, device);
}

Tensor Linear::forward(const Tensor& input) { return ops::linear(input, weight_, bias_); }

std::vector<Tensor*> Linear::parameters() { return {&weight_, &bias_}; }

Tensor ReLU::forward(const Tensor& input) { return ops::relu(input); }

void Sequential::add(std::unique_ptr<Module> module) {
    if (!module) throw std::runtime_error("Sequential cannot add a null module");
    modules_.push_back(std::move(module));
    register_module(*modules_.back());
}

Tensor Sequential::forward(const Tensor& input) {
    Tensor x = input;
    for (auto& m : modules_) x = m->forward(x);
    return x;
}

}  // namespace dl::nn
