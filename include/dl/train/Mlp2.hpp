#pragma once
// Native training step of the two-layer MLP  in -> hidden (ReLU) -> classes
// with softmax cross-entropy and SGD, on preallocated device buffers: one
// call of fdl_mlp2_train_step per step (four launches for the shapes the
// head kernel covers: layer 1 with bias+ReLU, the head with the loss and G1,
// the grouped backward jobs, the dW1 product with both weight steps), no
// allocation per step, on the calling thread's current stream.

#include <cstdint>
#include <memory>

#include <dl/tensor/Tensor.hpp>

struct fdl_mlp2_graph;  // include/fastdl_gemm.h

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
    // The same step on raw device pointers (the net's device): x holds
    // batch * in_features floats, row-major, and labels batch int64 values.
    float step(const float* x, const int64_t* labels, float lr, bool sync_loss = true);

    // Forward only: logits [batch, classes].
    Tensor forward(const Tensor& x);

    // The step captured once into a HIP graph on the current stream and then
    // replayed with one launch per step.  capture() records a step on x and
    // labels with learning rate lr (refill their buffers in place between
    // replays); nothing runs until replay().  Capturing again replaces the
    // graph.  replay() runs the captured steps on the current stream and
    // returns the last step's pre-update loss when sync_loss is true, else
    // NaN; it throws if nothing was captured.  With `steps` > 1 the graph
    // holds that many consecutive steps on the same batch, so one replay
    // costs one host launch for all of them.
    void capture(const Tensor& x, const Tensor& labels, float lr);
    void capture(const Tensor& x, const Tensor& labels, float lr, int steps);
    float replay(bool sync_loss = true);

    Tensor& w1() { return w1_; }
    Tensor& b1() { return b1_; }
    Tensor& w2() { return w2_; }
    Tensor& b2() { return b2_; }
    const Tensor& grad_input() const { return dx_; }
    // The last step's loss buffer [1] (written on the stream of that step).
    const Tensor& loss() const { return loss_; }
    int batch() const { return batch_; }
    int in_features() const { return in_; }

private:
    int in_, hidden_, classes_, batch_;
    Tensor w1_, b1_, w2_, b2_;
    Tensor h_, logits_, g2_, g1_, dw1_, db1_, dw2_, db2_, dx_, loss_;
    std::shared_ptr<fdl_mlp2_graph> graph_;
    Tensor graph_x_, graph_labels_;  // the captured step's inputs, kept alive

    void check_batch(const Tensor& x, const Tensor& labels, const char* what) const;
};

}  // namespace dl::train
