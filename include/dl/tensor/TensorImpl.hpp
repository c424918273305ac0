#pragma once
// Owner of one device allocation (reference include/dl/tensor/TensorImpl.hpp).
// Memory comes from the HIP device allocator of this library (see
// dl::memory in TensorImpl.cpp): freed blocks are cached per device and size
// so steady-state op calls do not reach hipMalloc/hipFree.

#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

#include <dl/core/DType.hpp>
#include <dl/core/Device.hpp>
#include <dl/core/Shape.hpp>
#include <dl/tensor/StreamUseList.hpp>

namespace dl {

namespace autograd {
class Node;
}

class TensorImpl {
public:
    TensorImpl(const Shape& shape, DType dtype, Device device);
    ~TensorImpl();

    TensorImpl(const TensorImpl&) = delete;
    TensorImpl& operator=(const TensorImpl&) = delete;

    TensorImpl(TensorImpl&& other) noexcept;
    TensorImpl& operator=(TensorImpl&& other) noexcept;

    // The device pointer.  Also records the calling thread's current stream
    // as a stream this memory is used on (see record_stream).
    void* data();
    const void* data() const;
    // The pointer without recording a use.
    const void* data_ptr_raw() const { return data_; }

    const Shape& shape() const;
    DType dtype() const;
    Device device() const;

    int64_t numel() const;
    std::size_t nbytes() const;

    void copy_from_host(const void* src, std::size_t bytes);
    void copy_to_host(void* dst, std::size_t bytes) const;
    void copy_from(const TensorImpl& src);
    void zero_();

    // Autograd state, as the reference plans it (FUTURE_WORK.md:100-109:
    // grad_, requires_grad_, grad_fn_).  grad_ is the gradient accumulated by
    // backward passes; grad_fn_ is the node that produced this tensor.
    bool requires_grad() const { return requires_grad_; }
    void set_requires_grad(bool v) { requires_grad_ = v; }
    const std::shared_ptr<TensorImpl>& grad() const { return grad_; }
    void set_grad(std::shared_ptr<TensorImpl> g) { grad_ = std::move(g); }
    const std::shared_ptr<autograd::Node>& grad_fn() const { return grad_fn_; }
    void set_grad_fn(std::shared_ptr<autograd::Node> fn) { grad_fn_ = std::move(fn); }

    // The stream that was current when the memory was allocated: the block
    // returns to that stream's free list when this tensor dies, whichever
    // stream is current then.
    void* stream() const { return stream_; }
    // Records that the memory is used by work on `stream`.  When the tensor
    // dies, the block is not handed out again until every such stream other
    // than stream() has passed that point.
    void record_stream(void* stream) const;

private:
    void* data_ = nullptr;
    void* stream_ = nullptr;
    mutable detail::StreamUseList uses_;
    Shape shape_;
    DType dtype_ = DType::Float32;
    Device device_;
    bool requires_grad_ = false;
    std::shared_ptr<TensorImpl> grad_;
    std::shared_ptr<autograd::Node> grad_fn_;

    void allocate();
    void release();
    void note_use() const;
};

}  // namespace dl

using TensorImpl = dl::TensorImpl;
