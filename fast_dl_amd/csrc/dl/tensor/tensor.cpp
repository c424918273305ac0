// Tensor / TensorImpl on the HIP runtime (reference src/tensor/Tensor.cpp and
// TensorImpl.cpp for the API behaviour and error strings).
//
// Device memory comes from a small caching allocator: freed blocks are kept
// per (device, rounded size, stream) and handed out again, so the ops'
// per-call output allocation does not reach hipMalloc/hipFree in steady
// state.  A block freed while the calling thread's current stream is S goes
// only to later allocations made with S current: kernels still queued on S
// that use the old tensor run before any use of the new one, by stream
// order, while another stream would give no such order.  The cache is
// process-lifetime (never torn down at exit, when the HIP runtime may
// already be gone).
#include <dl/core/HipUtils.hpp>
#include <dl/core/Stream.hpp>
#include <dl/kernels/random.hpp>
#include <dl/tensor/Tensor.hpp>
#include <dl/tensor/TensorImpl.hpp>

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <functional>
#include <map>
#include <mutex>
#include <stdexcept>
#include <utility>
#include <vector>

namespace dl {

namespace {

class BlockCache {
public:
    static BlockCache& get() {
        static BlockCache* cache = new BlockCache();
        return *cache;
    }

    static std::size_t round(std::size_t bytes) {
        constexpr std::size_t kSmall = 512;
        constexpr std::size_t kLarge = std::size_t(2) << 20;
        const std::size_t g = bytes < kLarge ? kSmall : kLarge;
        return (bytes + g - 1) / g * g;
    }

    void* acquire(int device, std::size_t bytes) {
        const std::size_t sz = round(bytes);
        {
            std::lock_guard<std::mutex> lock(mu_);
            auto it = free_.find(Key{device, sz, current_stream()});
            if (it != free_.end() && !it->second.empty()) {
                void* p = it->second.back();
                it->second.pop_back();
                return p;
            }
        }
        void* p = nullptr;
        hipError_t err = hipMalloc(&p, sz);
        if (err != hipSuccess) {
            // Return every cached block of this device to HIP and retry once.
            release_all(device);
            hip::check(hipMalloc(&p, sz), "cudaMalloc failed");
        }
        return p;
    }

    void give_back(int device, std::size_t bytes, void* p) {
        std::lock_guard<std::mutex> lock(mu_);
        free_[Key{device, round(bytes), current_stream()}].push_back(p);
    }

    // hipFree waits for the device, so blocks still used by queued work are
    // freed only after it.
    void release_all(int device) {
        std::lock_guard<std::mutex> lock(mu_);
        for (auto& kv : free_) {
            if (kv.first.device != device) continue;
            for (void* p : kv.second) (void)hipFree(p);
            kv.second.clear();
        }
    }

private:
    struct Key {
        int device;
        std::size_t bytes;
        void* stream;
        bool operator<(const Key& o) const {
            if (device != o.device) return device < o.device;
            if (bytes != o.bytes) return bytes < o.bytes;
            return std::less<void*>()(stream, o.stream);
        }
    };
    std::mutex mu_;
    std::map<Key, std::vector<void*>> free_;
};

const Shape& no_shape() {
    static const Shape s;
    return s;
}

}  // namespace

// ---------------------------------------------------------------- TensorImpl

TensorImpl::TensorImpl(const Shape& shape, DType dtype, Device device)
    : shape_(shape), dtype_(dtype), device_(device) {
    allocate();
}

TensorImpl::~TensorImpl() { release(); }

TensorImpl::TensorImpl(TensorImpl&& o) noexcept
    : data_(o.data_), shape_(std::move(o.shape_)), dtype_(o.dtype_), device_(o.device_),
      requires_grad_(o.requires_grad_), grad_(std::move(o.grad_)),
      grad_fn_(std::move(o.grad_fn_)) {
    o.data_ = nullptr;
}

TensorImpl& TensorImpl::operator=(TensorImpl&& o) noexcept {
    if (this != &o) {
        release();
        data_ = o.data_;
        shape_ = std::move(o.shape_);
        dtype_ = o.dtype_;
        device_ = o.device_;
        requires_grad_ = o.requires_grad_;
        grad_ = std::move(o.grad_);
        grad_fn_ = std::move(o.grad_fn_);
        o.data_ = nullptr;
    }
    return *this;
}

void* TensorImpl::data() { return data_; }
const void* TensorImpl::data() const { return data_; }
const Shape& TensorImpl::shape() const { return shape_; }
DType TensorImpl::dtype() const { return dtype_; }
Device TensorImpl::device() const { return device_; }
int64_t TensorImpl::numel() const { return shape_.numel(); }
std::size_t TensorImpl::nbytes() const { return static_cast<std::size_t>(numel()) * dtype_size(dtype_); }

void TensorImpl::allocate() {
    const std::size_t bytes = nbytes();
    if (bytes == 0) return;
    if (!device_.is_cuda()) throw std::runtime_error("Tensor currently supports CUDA allocation only");
    hip::check(hipSetDevice(device_.index), "cudaSetDevice failed");
    data_ = BlockCache::get().acquire(device_.index, bytes);
}

void TensorImpl::release() {
    if (!data_) return;
    if (device_.is_cuda()) BlockCache::get().give_back(device_.index, nbytes(), data_);
    data_ = nullptr;
}

void TensorImpl::copy_from_host(const void* src, std::size_t bytes) {
    if (bytes > nbytes()) throw std::runtime_error("copy_from_host exceeds tensor size");
    if (bytes == 0) return;
    if (!device_.is_cuda()) throw std::runtime_error("copy_from_host currently supports CUDA tensors only");
    hip::check(hipSetDevice(device_.index), "cudaSetDevice failed");
    // Synchronous, as the reference's cudaMemcpy: the host buffer may be
    // reused as soon as this returns.
    const hipStream_t s = static_cast<hipStream_t>(current_stream());
    if (s) {
        hip::check(hipMemcpyAsync(data_, src, bytes, hipMemcpyHostToDevice, s),
                   "cudaMemcpy host to device failed");
        hip::check(hipStreamSynchronize(s), "cudaMemcpy host to device failed");
    } else {
        hip::check(hipMemcpy(data_, src, bytes, hipMemcpyHostToDevice),
                   "cudaMemcpy host to device failed");
    }
}

void TensorImpl::copy_to_host(void* dst, std::size_t bytes) const {
    if (bytes > nbytes()) throw std::runtime_error("copy_to_host exceeds tensor size");
    if (bytes == 0) return;
    if (!device_.is_cuda()) throw std::runtime_error("copy_to_host currently supports CUDA tensors only");
    hip::check(hipSetDevice(device_.index), "cudaSetDevice failed");
    // Ordered after the work queued on the current stream, then waited for.
    const hipStream_t s = static_cast<hipStream_t>(current_stream());
    if (s) {
        hip::check(hipMemcpyAsync(dst, data_, bytes, hipMemcpyDeviceToHost, s),
                   "cudaMemcpy device to host failed");
        hip::check(hipStreamSynchronize(s), "cudaMemcpy device to host failed");
    } else {
        hip::check(hipMemcpy(dst, data_, bytes, hipMemcpyDeviceToHost),
                   "cudaMemcpy device to host failed");
    }
}

void TensorImpl::copy_from(const TensorImpl& src) {
    if (src.nbytes() != nbytes()) throw std::runtime_error("tensor copy size mismatch");
    if (nbytes() == 0) return;
    if (!(src.device().is_cuda() && device_.is_cuda())) {
        throw std::runtime_error("copy_from currently supports CUDA to CUDA only");
    }
    hip::check(hipSetDevice(device_.index), "cudaSetDevice failed");
    const hipStream_t s = static_cast<hipStream_t>(current_stream());
    if (s) {
        hip::check(hipMemcpyAsync(data_, src.data(), nbytes(), hipMemcpyDeviceToDevice, s),
                   "cudaMemcpy device to device failed");
    } else {
        hip::check(hipMemcpy(data_, src.data(), nbytes(), hipMemcpyDeviceToDevice),
                   "cudaMemcpy device to device failed");
    }
}

void TensorImpl::zero_() {
    if (nbytes() == 0) return;
    if (!device_.is_cuda()) throw std::runtime_error("zero_ currently supports CUDA tensors only");
    hip::check(hipSetDevice(device_.index), "cudaSetDevice failed");
    const hipStream_t s = static_cast<hipStream_t>(current_stream());
    if (s) {
        hip::check(hipMemsetAsync(data_, 0, nbytes(), s), "cudaMemset failed");
    } else {
        hip::check(hipMemset(data_, 0, nbytes()), "cudaMemset failed");
    }
}

// -------------------------------------------------------------------- Tensor

Tensor::Tensor(const Shape& shape, DType dtype, Device device)
    : impl_(std::make_shared<TensorImpl>(shape, dtype, device)) {}

Tensor Tensor::empty(const Shape& shape, DType dtype, Device device) {
    return Tensor(shape, dtype, device);
}

Tensor Tensor::zeros(const Shape& shape, DType dtype, Device device) {
    Tensor t(shape, dtype, device);
    t.zero_();
    return t;
}

namespace {

Tensor random_tensor(const Shape& shape, DType dtype, Device device, const char* what) {
    if (dtype != DType::Float32) {
        throw std::runtime_error(std::string("Tensor::") + what + " currently supports Float32 only");
    }
    if (!device.is_cuda()) {
        throw std::runtime_error(std::string("Tensor::") + what + " currently supports CUDA only");
    }
    Tensor out(shape, dtype, device);
    hip::check(hipSetDevice(device.index), "cudaSetDevice failed");
    return out;
}

}  // namespace

Tensor Tensor::randn(Shape shape, DType dtype, Device device, float mean, float stddev, uint64_t seed) {
    Tensor out = random_tensor(shape, dtype, device, "randn");
    kernels::normal_float32(static_cast<float*>(out.data()), out.numel(), mean, stddev, seed);
    return out;
}

Tensor Tensor::uniform(Shape shape, DType dtype, Device device, float low, float high, uint64_t seed) {
    Tensor out = random_tensor(shape, dtype, device, "uniform");
    kernels::uniform_float32(static_cast<float*>(out.data()), out.numel(), low, high, seed);
    return out;
}

Tensor Tensor::xavier_uniform(Shape shape, DType dtype, Device device, uint64_t seed) {
    if (shape.rank() < 2) throw std::runtime_error("Tensor::xavier_uniform requires rank >= 2");
    const float fan_in = static_cast<float>(shape[static_cast<int>(shape.rank() - 2)]);
    const float fan_out = static_cast<float>(shape[static_cast<int>(shape.rank() - 1)]);
    const float limit = std::sqrt(6.0f / (fan_in + fan_out));
    return uniform(shape, dtype, device, -limit, limit, seed);
}

Tensor Tensor::kaiming_uniform(Shape shape, DType dtype, Device device, uint64_t seed) {
    if (shape.rank() < 2) throw std::runtime_error("Tensor::kaiming_uniform requires rank >= 2");
    const float fan_in = static_cast<float>(shape[static_cast<int>(shape.rank() - 2)]);
    const float limit = std::sqrt(6.0f / fan_in);
    return uniform(shape, dtype, device, -limit, limit, seed);
}

Tensor Tensor::empty_like(const Tensor& other) {
    if (!other.defined()) throw std::runtime_error("empty_like requires a defined tensor");
    return Tensor(other.shape(), other.dtype(), other.device());
}

Tensor Tensor::zeros_like(const Tensor& other) {
    Tensor t = empty_like(other);
    t.zero_();
    return t;
}

void* Tensor::data() { return impl_ ? impl_->data() : nullptr; }
const void* Tensor::data() const { return impl_ ? impl_->data() : nullptr; }
const Shape& Tensor::shape() const { return impl_ ? impl_->shape() : no_shape(); }
DType Tensor::dtype() const { return impl_ ? impl_->dtype() : DType::Float32; }
Device Tensor::device() const { return impl_ ? impl_->device() : Device(); }
int64_t Tensor::numel() const { return impl_ ? impl_->numel() : 0; }
std::size_t Tensor::nbytes() const { return impl_ ? impl_->nbytes() : 0; }
bool Tensor::defined() const { return impl_ && impl_->data() != nullptr; }

void Tensor::copy_from_host(const void* src, std::size_t bytes) {
    if (!impl_) throw std::runtime_error("copy_from_host requires a defined tensor");
    impl_->copy_from_host(src, bytes);
}

void Tensor::copy_to_host(void* dst, std::size_t bytes) const {
    if (!impl_) throw std::runtime_error("copy_to_host requires a defined tensor");
    impl_->copy_to_host(dst, bytes);
}

void Tensor::copy_from(const Tensor& src) {
    if (!impl_ || !src.impl_) throw std::runtime_error("copy_from requires defined tensors");
    impl_->copy_from(*src.impl_);
}

void Tensor::copy_to(Tensor& dst) const { dst.copy_from(*this); }

void Tensor::zero_() {
    if (!impl_) throw std::runtime_error("zero_ requires a defined tensor");
    impl_->zero_();
}

}  // namespace dl
