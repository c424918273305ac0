#pragma once
// Module base (reference include/dl/nn/Module.hpp): forward(), parameters()
// gathered from registered children in registration order, operator().

#include <dl/tensor/Tensor.hpp>

#include <vector>

namespace dl::nn {

class Module {
public:
    virtual ~Module() = default;

    virtual Tensor forward(const Tensor& input) = 0;

    virtual std::vector<Tensor*> parameters() {
        std::vector<Tensor*> all;
        for (Module* child : children_) {
            for (Tensor* p : child->parameters()) all.push_back(p);
        }
        return all;
    }

    Tensor operator()(const Tensor& input) { return forward(input); }

protected:
    void register_module(Module& module) { children_.push_back(&module); }

private:
    std::vector<Module*> children_;
};

}  // namespace dl::nn
