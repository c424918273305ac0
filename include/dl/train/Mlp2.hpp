#pragma once
// Native training step of the two-layer MLP  in -> hidden (ReLU) -> classes
// with softmax cross-entropy and SGD, on preallocated device buffers (one
// call of fdl_mlp2_train_step per step: two fused forward GEMMs, the loss
// kernel, three backward GEMMs with the ReLU mask fused, two column sums and
// one SGD launch; no allocation per step).

#include <cstdint>

#include <dl/tensor/Tensor.hpp>

namespace dl::train {

class Mlp2 {
public:
    // Weights [in, hidden], [hidden, classes] Kaiming-uniform like nn::Linear, zero biases.
    Mlp2(int in_features, int hidden, int classes, int batch, const Device& device,
         uint64_t seed = 1234);

    // One step on x [batch, in] (float32) and labels [batch] (int64); returns
    // the pre-update loss when sync_loss is true (that reads it back, which
    // synchronises), else NaN.
    float step(const Tensor& x, const Tensor& labels, float lr, bool sync_loss = true);

    // Forward only: logits [batch, classes].
    Tensor forward(const Tensor& x);

    Tensor& w1() { return w1_; }
    Tensor& b1() { return b1_; }
    Tensor& w2() { return w2_; }
    Tensor& b2() { return b2_; }
    const Tensor& grad_input() const { return dx_; }

private:
    int in_, hidden_, classes_, batch_;
    Tensor w1_, b1_, w2_, b2_;
    Tensor h_, logits_, g2_, g1_, dw1_, db1_, dw2_, db2_, dx_, loss_;
};

}  // namespace dl::train
