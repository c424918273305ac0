#pragma once
// Shared-ownership device tensor (reference include/dl/tensor/Tensor.hpp):
// same factories, accessors and host copy helpers.

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <vector>

#include <dl/core/DType.hpp>
#include <dl/core/Device.hpp>
#include <dl/core/Shape.hpp>

namespace dl {

class TensorImpl;

namespace autograd {
class Node;
struct TensorAccess;
}

template <typename T>
DType tensor_dtype();

template <>
inline DType tensor_dtype<float>() {
    return DType::Float32;
}

template <>
inline DType tensor_dtype<int32_t>() {
    return DType::Int32;
}

template <>
inline DType tensor_dtype<int64_t>() {
    return DType::Int64;
}

class Tensor {
public:
    Tensor() = default;
    Tensor(const Shape& shape, DType dtype = DType::Float32, Device device = Device());

    static Tensor empty(const Shape& shape, DType dtype = DType::Float32,
                        Device device = Device());
    static Tensor zeros(const Shape& shape, DType dtype = DType::Float32,
                        Device device = Device());
    // Counter-based Philox4x32-10 fills: same seed, same values; not the
    // reference's cuRAND stream.
    static Tensor randn(Shape shape, DType dtype, Device device, float mean, float stddev,
                        uint64_t seed = 1234);
    static Tensor uniform(Shape shape, DType dtype, Device device, float low, float high,
                          uint64_t seed = 1234);
    static Tensor xavier_uniform(Shape shape, DType dtype, Device device, uint64_t seed = 1234);
    static Tensor kaiming_uniform(Shape shape, DType dtype, Device device, uint64_t seed = 1234);

    static Tensor empty_like(const Tensor& other);
    static Tensor zeros_like(const Tensor& other);

    template <typename T>
    static Tensor from_host(const std::vector<T>& data, const Shape& shape,
                            Device device = Device());

    ~Tensor() = default;

    Tensor(const Tensor&) = default;
    Tensor& operator=(const Tensor&) = default;

    Tensor(Tensor&& other) noexcept = default;
    Tensor& operator=(Tensor&& other) noexcept = default;

    void* data();
    const void* data() const;
    const Shape& shape() const;
    DType dtype() const;
    Device device() const;

    int64_t numel() const;
    std::size_t nbytes() const;
    bool defined() const;

    void copy_from_host(const void* src, std::size_t bytes);
    void copy_to_host(void* dst, std::size_t bytes) const;
    void copy_from(const Tensor& src);
    void copy_to(Tensor& dst) const;
    void zero_();
    // Marks the memory as used by work on `stream` (a hipStream_t), so that
    // it is not reused before that work when this tensor dies.  data() and
    // every dl:: op record the calling thread's current stream by
    // themselves; this is for work queued on another stream through a raw
    // pointer.
    void record_stream(void* stream) const;

    template <typename T>
    std::vector<T> to_host() const;

    // Autograd: the reference's planned interface (FUTURE_WORK.md:94-127),
    // for the ops of the MLP path (matmul, linear, linear_relu, relu,
    // cross_entropy).  An op records its backward node when one of its
    // inputs requires a gradient; nothing is recorded otherwise, so code that
    // never sets requires_grad runs as before.  Copies of a Tensor share its
    // gradient, as they share its data.
    bool requires_grad() const;
    // Marks a leaf (a tensor no recorded op produced) as needing a gradient.
    Tensor& set_requires_grad(bool requires_grad = true);
    // The gradient accumulated into this leaf by backward() calls (float32,
    // this tensor's shape); not defined() before the first one reaches it.
    Tensor grad() const;
    void zero_grad();
    // The node that produced this tensor (null for leaves).
    std::shared_ptr<autograd::Node> grad_fn() const;
    // Back-propagates from this one-element float32 tensor (a loss), seeded
    // with 1, and adds d(this)/d(leaf) to grad() of every leaf that requires
    // a gradient.  Runs on the current stream; throws std::runtime_error if
    // this tensor has more than one element or does not require a gradient.
    void backward() const;

private:
    friend struct autograd::TensorAccess;  // the autograd engine's view of impl_
    std::shared_ptr<TensorImpl> impl_;
};

template <typename T>
Tensor Tensor::from_host(const std::vector<T>& data, const Shape& shape, Device device) {
    if (static_cast<int64_t>(data.size()) != shape.numel()) {
        throw std::runtime_error("from_host data size does not match shape");
    }
    Tensor out(shape, tensor_dtype<T>(), device);
    out.copy_from_host(data.data(), sizeof(T) * data.size());
    return out;
}

template <typename T>
std::vector<T> Tensor::to_host() const {
    if (tensor_dtype<T>() != dtype()) {
        throw std::runtime_error("to_host dtype does not match requested host type");
    }
    std::vector<T> out(static_cast<std::size_t>(numel()));
    copy_to_host(out.data(), sizeof(T) * out.size());
    return out;
}

}  // namespace dl

using Tensor = dl::Tensor;
using dl::tensor_dtype;
