// One Mlp2 training epoch from resident IDX bytes: the epoch's batches
// gathered in one launch, then one fused step per batch at a row offset.
#include <dl/train/Epoch.hpp>

#include <stdexcept>

namespace dl::train {

EpochResult train_epoch(Mlp2& net, data::DataLoader& loader, const Tensor& order, float lr,
                        bool whole_epoch) {
    const int64_t batch = net.batch();
    const int64_t pixels = int64_t(loader.getRows()) * loader.getCols();
    if (pixels != net.in_features()) {
        throw std::runtime_error("train_epoch: the loader's records do not match the net's input width");
    }
    if (order.dtype() != DType::Int64 || order.shape().rank() != 1 || !order.device().is_cuda()) {
        throw std::runtime_error("train_epoch: order must be an int64 vector on a GPU");
    }
    EpochResult result;
    const int64_t steps = order.numel() / batch;
    if (steps == 0) return result;
    const Device dev = order.device();
    const int64_t rows = whole_epoch ? steps * batch : batch;
    Tensor x(Shape({rows, pixels}), DType::Float32, dev);
    Tensor y(Shape({rows}), DType::Int64, dev);
    if (whole_epoch) loader.gather(order, 0, rows, x, y);
    for (int64_t i = 0; i < steps; ++i) {
        const int64_t row0 = whole_epoch ? i * batch : 0;
        if (!whole_epoch) loader.gather(order, i * batch, batch, x, y);
        net.step(static_cast<const float*>(x.data()) + row0 * pixels,
                 static_cast<const int64_t*>(y.data()) + row0, lr, false);
    }
    result.steps = steps;
    result.last_loss = net.loss().to_host<float>()[0];
    return result;
}

}  // namespace dl::train
