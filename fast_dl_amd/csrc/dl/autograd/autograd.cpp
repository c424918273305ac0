// Minimal reverse-mode autograd for the MLP path: the reference's planned
// Tensor::backward / grad / requires_grad and Node (FUTURE_WORK.md:94-127,
// 234-239).  Every backward node reuses the path's own kernels: NT/TN GEMMs,
// the ReLU mask, the softmax-CE gradient and the column sums of
// ops::linear_backward.  Gradients are accumulated with the SGD kernel at
// lr = -1 (a - (-1)*b = a + b, one rounding), so no extra kernel is needed.
#include "record.hpp"

#include <dl/core/HipUtils.hpp>
#include <dl/core/Stream.hpp>
#include <dl/kernels/gemm.hpp>
#include <dl/ops/Activation.hpp>
#include <dl/ops/CrossEntropy.hpp>
#include <dl/ops/Linear.hpp>
#include <dl/tensor/TensorImpl.hpp>

#include <fastdl_gemm.h>

#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

namespace dl::autograd {

struct TensorAccess {
    static const std::shared_ptr<TensorImpl>& impl(const Tensor& t) { return t.impl_; }
    static Tensor wrap(std::shared_ptr<TensorImpl> impl) {
        Tensor t;
        t.impl_ = std::move(impl);
        return t;
    }
};

namespace {

float* f32(Tensor& t) { return static_cast<float*>(t.data()); }
const float* f32(const Tensor& t) { return static_cast<const float*>(t.data()); }

// dst += src (same shape, float32, one device).
void add_into(Tensor& dst, const Tensor& src) {
    hip::check(hipSetDevice(dst.device().index), "cudaSetDevice failed");
    hip::check_fdl(fdl_sgd_update(f32(dst), f32(src), -1.0f, dst.numel(), current_stream()),
                   "autograd: gradient accumulation failed");
}

void accumulate(Tensor& slot, const Tensor& g) {
    if (!slot.defined()) {
        slot = g;  // nodes return new tensors, so the slot can own this one
    } else {
        add_into(slot, g);
    }
}

class MatmulBackward final : public Node {
public:
    MatmulBackward(const Tensor& a, const Tensor& b) : Node({a, b}) {}
    std::string name() const override { return "MatmulBackward"; }

    // C[M,N] = A[M,K] B[K,N]: dA = dC B^T (NT), dB = A^T dC (TN).
    std::vector<Tensor> backward(const Tensor& g) override {
        const Tensor& a = inputs_[0];
        const Tensor& b = inputs_[1];
        const int64_t m = a.shape()[0], k = a.shape()[1], n = b.shape()[1];
        std::vector<Tensor> out(2);
        hip::check(hipSetDevice(g.device().index), "cudaSetDevice failed");
        if (a.requires_grad()) {
            out[0] = Tensor(a.shape(), DType::Float32, a.device());
            kernels::gemm_ex(kernels::Transpose::No, kernels::Transpose::Yes, m, k, n, f32(g), n,
                             0, f32(b), n, 0, f32(out[0]), k, 0, 1, nullptr, nullptr,
                             kernels::Epilogue::None, kernels::GemmAlgo::Auto, current_stream());
        }
        if (b.requires_grad()) {
            out[1] = Tensor(b.shape(), DType::Float32, b.device());
            kernels::gemm_ex(kernels::Transpose::Yes, kernels::Transpose::No, k, n, m, f32(a), k,
                             0, f32(g), n, 0, f32(out[1]), n, 0, 1, nullptr, nullptr,
                             kernels::Epilogue::None, kernels::GemmAlgo::Auto, current_stream());
        }
        return out;
    }
};

std::vector<Tensor> linear_grads(const Tensor& g, const std::vector<Tensor>& in) {
    const ops::LinearGrads lg = ops::linear_backward(g, in[0], in[1], in[0].requires_grad());
    return {in[0].requires_grad() ? lg.grad_input : Tensor(),
            in[1].requires_grad() ? lg.grad_weight : Tensor(),
            in[2].requires_grad() ? lg.grad_bias : Tensor()};
}

class LinearBackward final : public Node {
public:
    LinearBackward(const Tensor& x, const Tensor& w, const Tensor& b) : Node({x, w, b}) {}
    std::string name() const override { return "LinearBackward"; }
    std::vector<Tensor> backward(const Tensor& g) override { return linear_grads(g, inputs_); }
};

class LinearReluBackward final : public Node {
public:
    LinearReluBackward(const Tensor& x, const Tensor& w, const Tensor& b, const Tensor& y)
        : Node({x, w, b}), output_(TensorAccess::impl(y)) {}
    std::string name() const override { return "LinearReluBackward"; }

    // Y = max(0, X W + b): the mask Y > 0 equals X W + b > 0.
    std::vector<Tensor> backward(const Tensor& g) override {
        std::shared_ptr<TensorImpl> y = output_.lock();
        if (!y) throw std::runtime_error("LinearReluBackward: the output no longer exists");
        return linear_grads(ops::relu_backward(g, TensorAccess::wrap(std::move(y))), inputs_);
    }

private:
    std::weak_ptr<TensorImpl> output_;
};

class ReluBackward final : public Node {
public:
    explicit ReluBackward(const Tensor& x) : Node({x}) {}
    std::string name() const override { return "ReluBackward"; }
    std::vector<Tensor> backward(const Tensor& g) override {
        return {ops::relu_backward(g, inputs_[0])};  // mask x > 0 equals relu(x) > 0
    }
};

class CrossEntropyBackward final : public Node {
public:
    CrossEntropyBackward(const Tensor& logits, const Tensor& labels)
        : Node({logits}), labels_(labels) {}
    std::string name() const override { return "CrossEntropyBackward"; }

    // d(loss)/d(logits) = (softmax - onehot) / batch, times the incoming
    // gradient g (one element on the device).  The product is a K = 1 GEMM
    // of the gradient as a column [B*C, 1] with g as [1, 1]: one rounded
    // multiply per element, so an incoming 1 leaves the bits unchanged.
    std::vector<Tensor> backward(const Tensor& g) override {
        const Tensor& logits = inputs_[0];
        Tensor grad = ops::cross_entropy_backward(logits, labels_);
        Tensor out(logits.shape(), DType::Float32, logits.device());
        const int64_t n = grad.numel();
        kernels::gemm_ex(kernels::Transpose::No, kernels::Transpose::No, n, 1, 1, f32(grad), 1, 0,
                         f32(g), 1, 0, f32(out), 1, 0, 1, nullptr, nullptr,
                         kernels::Epilogue::None, kernels::GemmAlgo::Auto, current_stream());
        return {out};
    }

private:
    Tensor labels_;
};

}  // namespace

bool any_requires_grad(std::initializer_list<const Tensor*> inputs) {
    for (const Tensor* t : inputs) {
        if (t->requires_grad()) return true;
    }
    return false;
}

void record(Tensor& output, std::shared_ptr<Node> node) {
    const std::shared_ptr<TensorImpl>& impl = TensorAccess::impl(output);
    impl->set_grad_fn(std::move(node));
    impl->set_requires_grad(true);
}

std::shared_ptr<Node> make_matmul_backward(const Tensor& a, const Tensor& b) {
    return std::make_shared<MatmulBackward>(a, b);
}

std::shared_ptr<Node> make_linear_backward(const Tensor& input, const Tensor& weight,
                                           const Tensor& bias) {
    return std::make_shared<LinearBackward>(input, weight, bias);
}

std::shared_ptr<Node> make_linear_relu_backward(const Tensor& input, const Tensor& weight,
                                                const Tensor& bias, const Tensor& output) {
    return std::make_shared<LinearReluBackward>(input, weight, bias, output);
}

std::shared_ptr<Node> make_relu_backward(const Tensor& input) {
    return std::make_shared<ReluBackward>(input);
}

std::shared_ptr<Node> make_cross_entropy_backward(const Tensor& logits, const Tensor& labels) {
    return std::make_shared<CrossEntropyBackward>(logits, labels);
}

}  // namespace dl::autograd

namespace dl {

bool Tensor::requires_grad() const { return impl_ && impl_->requires_grad(); }

Tensor& Tensor::set_requires_grad(bool requires_grad) {
    if (!impl_) throw std::runtime_error("set_requires_grad requires a defined tensor");
    if (impl_->grad_fn()) {
        throw std::runtime_error("set_requires_grad: only leaf tensors (not produced by a recorded op)");
    }
    if (requires_grad && dtype() != DType::Float32) {
        throw std::runtime_error("set_requires_grad: only float32 tensors can require gradients");
    }
    impl_->set_requires_grad(requires_grad);
    return *this;
}

Tensor Tensor::grad() const {
    if (!impl_ || !impl_->grad()) return Tensor();
    return autograd::TensorAccess::wrap(impl_->grad());
}

void Tensor::zero_grad() {
    if (impl_) impl_->set_grad(nullptr);
}

std::shared_ptr<autograd::Node> Tensor::grad_fn() const {
    return impl_ ? impl_->grad_fn() : nullptr;
}

void Tensor::backward() const {
    if (!defined() || numel() != 1 || dtype() != DType::Float32) {
        throw std::runtime_error("backward: needs a defined one-element float32 tensor (a loss)");
    }
    if (!requires_grad()) {
        throw std::runtime_error("backward: the tensor does not require a gradient");
    }
    // Post-order over the graph of tensors that require a gradient: every
    // tensor comes after the inputs of its node.
    std::vector<Tensor> order;
    std::unordered_set<const TensorImpl*> seen;
    std::vector<std::pair<Tensor, bool>> stack{{*this, false}};
    while (!stack.empty()) {
        auto [t, expanded] = stack.back();
        stack.pop_back();
        if (expanded) {
            order.push_back(t);
            continue;
        }
        if (!seen.insert(t.impl_.get()).second) continue;
        stack.push_back({t, true});
        if (const auto& fn = t.impl_->grad_fn()) {
            for (const Tensor& in : fn->inputs()) {
                if (in.requires_grad() && !seen.count(in.impl_.get())) stack.push_back({in, false});
            }
        }
    }
    // Outputs first: a tensor's gradient is complete once every node that
    // consumes it has run.
    std::unordered_map<const TensorImpl*, Tensor> grads;
    grads[impl_.get()] = Tensor::from_host(std::vector<float>{1.0f}, shape(), device());
    for (auto it = order.rbegin(); it != order.rend(); ++it) {
        const Tensor& t = *it;
        auto found = grads.find(t.impl_.get());
        if (found == grads.end()) continue;
        Tensor g = std::move(found->second);
        grads.erase(found);
        if (const auto& fn = t.impl_->grad_fn()) {
            std::vector<Tensor> in_grads = fn->backward(g);
            const std::vector<Tensor>& ins = fn->inputs();
            for (std::size_t i = 0; i < ins.size() && i < in_grads.size(); ++i) {
                if (ins[i].requires_grad() && in_grads[i].defined()) {
                    autograd::accumulate(grads[ins[i].impl_.get()], in_grads[i]);
                }
            }
        } else if (!t.impl_->grad()) {
            t.impl_->set_grad(autograd::TensorAccess::impl(g));
        } else {
            Tensor acc = autograd::TensorAccess::wrap(t.impl_->grad());
            autograd::add_into(acc, g);
        }
    }
}

}  // namespace dl
