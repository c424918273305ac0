#pragma once
// ReLU module (reference include/dl/nn/ReLU.hpp).

#include <dl/nn/Module.hpp>
#include <dl/tensor/Tensor.hpp>

namespace dl::nn {

class ReLU : public Module {
public:
    Tensor forward(const Tensor& input) override;
};

}  // namespace dl::nn
