// Preallocated two-layer MLP trainer over fdl_mlp2_train_step.
#include <dl/core/HipUtils.hpp>
#include <dl/core/Stream.hpp>
#include <dl/train/Mlp2.hpp>

#include <fastdl_gemm.h>

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <limits>
#include <stdexcept>
#include <string>

namespace dl::train {

namespace {

float* fp(Tensor& t) { return static_cast<float*>(t.data()); }
const float* fp(const Tensor& t) { return static_cast<const float*>(t.data()); }

}  // namespace

Mlp2::Mlp2(int in_features, int hidden, int classes, int batch, const Device& device,
           uint64_t seed)
    : in_(in_features), hidden_(hidden), classes_(classes), batch_(batch) {
    if (in_features <= 0 || hidden <= 0 || classes <= 0 || batch <= 0) {
        throw std::runtime_error("Mlp2: sizes must be positive");
    }
    const DType f = DType::Float32;
    w1_ = Tensor::kaiming_uniform(Shape({in_features, hidden}), f, device, seed);
    w2_ = Tensor::kaiming_uniform(Shape({hidden, classes}), f, device, seed + 1);
    b1_ = Tensor::zeros(Shape({hidden}), f, device);
    b2_ = Tensor::zeros(Shape({classes}), f, device);
    h_ = Tensor(Shape({batch, hidden}), f, device);
    logits_ = Tensor(Shape({batch, classes}), f, device);
    g2_ = Tensor(Shape({batch, classes}), f, device);
    g1_ = Tensor(Shape({batch, hidden}), f, device);
    dw1_ = Tensor(Shape({in_features, hidden}), f, device);
    db1_ = Tensor(Shape({hidden}), f, device);
    dw2_ = Tensor(Shape({hidden, classes}), f, device);
    db2_ = Tensor(Shape({classes}), f, device);
    dx_ = Tensor(Shape({batch, in_features}), f, device);
    loss_ = Tensor(Shape({1}), f, device);
}

void Mlp2::check_batch(const Tensor& x, const Tensor& labels, const char* what) const {
    if (x.shape().rank() != 2 || x.shape()[0] != batch_ || x.shape()[1] != in_ ||
        x.dtype() != DType::Float32) {
        throw std::runtime_error(std::string(what) + ": x must be float32 [batch, in_features]");
    }
    if (labels.shape().rank() != 1 || labels.shape()[0] != batch_ || labels.dtype() != DType::Int64) {
        throw std::runtime_error(std::string(what) + ": labels must be int64 [batch]");
    }
}

float Mlp2::step(const Tensor& x, const Tensor& labels, float lr, bool sync_loss) {
    check_batch(x, labels, "Mlp2::step");
    return step(fp(x), static_cast<const int64_t*>(labels.data()), lr, sync_loss);
}

float Mlp2::step(const float* x, const int64_t* labels, float lr, bool sync_loss) {
    if (!x || !labels) throw std::runtime_error("Mlp2::step: null batch pointer");
    hip::check(hipSetDevice(w1_.device().index), "cudaSetDevice failed");
    hip::check_fdl(fdl_mlp2_train_step(x, labels, batch_, in_,
                                       hidden_, classes_, fp(w1_), fp(b1_), fp(w2_), fp(b2_), lr,
                                       fp(h_), fp(logits_), fp(g2_), fp(g1_), fp(dw1_), fp(db1_),
                                       fp(dw2_), fp(db2_), fp(dx_), fp(loss_), current_stream()),
                   "Mlp2::step failed");
    if (!sync_loss) return std::numeric_limits<float>::quiet_NaN();
    return loss_.to_host<float>()[0];
}

void Mlp2::capture(const Tensor& x, const Tensor& labels, float lr) { capture(x, labels, lr, 1); }

void Mlp2::capture(const Tensor& x, const Tensor& labels, float lr, int steps) {
    check_batch(x, labels, "Mlp2::capture");
    if (steps < 1) throw std::runtime_error("Mlp2::capture: steps must be at least 1");
    hip::check(hipSetDevice(x.device().index), "cudaSetDevice failed");
    fdl_mlp2_graph* g = nullptr;
    hip::check_fdl(fdl_mlp2_graph_create_steps(&g, steps, fp(x),
                                               static_cast<const int64_t*>(labels.data()), batch_,
                                               in_, hidden_, classes_, fp(w1_), fp(b1_), fp(w2_),
                                               fp(b2_), lr, fp(h_), fp(logits_), fp(g2_), fp(g1_),
                                               fp(dw1_), fp(db1_), fp(dw2_), fp(db2_), fp(dx_),
                                               fp(loss_), current_stream()),
                   "Mlp2::capture failed");
    graph_ = std::shared_ptr<fdl_mlp2_graph>(g, [](fdl_mlp2_graph* p) { (void)fdl_mlp2_graph_destroy(p); });
    graph_x_ = x;
    graph_labels_ = labels;
}

float Mlp2::replay(bool sync_loss) {
    if (!graph_) throw std::runtime_error("Mlp2::replay: no captured step");
    hip::check(hipSetDevice(graph_x_.device().index), "cudaSetDevice failed");
    hip::check_fdl(fdl_mlp2_graph_launch(graph_.get(), current_stream()), "Mlp2::replay failed");
    if (!sync_loss) return std::numeric_limits<float>::quiet_NaN();
    return loss_.to_host<float>()[0];
}

Tensor Mlp2::forward(const Tensor& x) {
    if (x.shape().rank() != 2 || x.shape()[1] != in_ || x.dtype() != DType::Float32) {
        throw std::runtime_error("Mlp2::forward: x must be float32 [rows, in_features]");
    }
    const int64_t rows = x.shape()[0];
    Tensor h(Shape({rows, hidden_}), DType::Float32, x.device());
    Tensor out(Shape({rows, classes_}), DType::Float32, x.device());
    hip::check(hipSetDevice(x.device().index), "cudaSetDevice failed");
    hip::check_fdl(fdl_sgemm_ex(FDL_OP_N, FDL_OP_N, rows, hidden_, in_, fp(x), in_, 0, fp(w1_),
                                hidden_, 0, fp(h), hidden_, 0, 1, fp(b1_), nullptr,
                                FDL_EPILOGUE_BIAS_RELU, current_stream()),
                   "Mlp2::forward failed");
    hip::check_fdl(fdl_sgemm_ex(FDL_OP_N, FDL_OP_N, rows, classes_, hidden_, fp(h), hidden_, 0,
                                fp(w2_), classes_, 0, fp(out), classes_, 0, 1, fp(b2_), nullptr,
                                FDL_EPILOGUE_BIAS, current_stream()),
                   "Mlp2::forward failed");
    return out;
}

}  // namespace dl::train
