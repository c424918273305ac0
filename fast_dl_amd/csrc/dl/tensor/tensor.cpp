// Tensor / TensorImpl on the HIP runtime (reference src/tensor/Tensor.cpp and
// TensorImpl.cpp for the API behaviour and error strings).
//
// Device memory comes from the stream-ordered block cache of
// block_cache.hpp: a tensor's block belongs to the stream that was current
// when it was allocated and goes back to that stream's free list when the
// tensor dies; streams other than that one which the tensor's memory was
// used on (every data() call records the calling thread's current stream)
// hold the block back until they pass an event recorded at the release.  The
// cache is process-lifetime (never torn down at exit, when the HIP runtime
// may already be gone).
#include "block_cache.hpp"

#include <dl/core/HipUtils.hpp>
#include <dl/core/Stream.hpp>
#include <dl/kernels/random.hpp>
#include <dl/tensor/Tensor.hpp>
#include <dl/tensor/TensorImpl.hpp>
#include <fastdl_gemm.h>

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <mutex>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace dl {

namespace detail {

namespace {

std::atomic<int> g_inject_failures{0};

// The cache's view of the HIP runtime.  A failed call that the cache
// recovers from (an allocation it retries, an event not yet reached) must
// not leave HIP's per-thread error state set: every launcher in this library
// reports hipGetLastError() after its launch, so a stale failure would be
// reported by the next, unrelated op.  The state is cleared only when it was
// clear before the call, so an earlier failure is still reported.
class HipBackend final : public CacheBackend {
public:
    bool alloc(int device, std::size_t bytes, void** p) override {
        hip::check(hipSetDevice(device), "cudaSetDevice failed");
        const hipError_t before = hipPeekAtLastError();
        std::size_t ask = bytes;
        int left = g_inject_failures.load();
        while (left > 0 && !g_inject_failures.compare_exchange_weak(left, left - 1)) {
        }
        if (left > 0) ask = std::size_t(1) << 62;  // more than any device holds
        *p = nullptr;
        hipError_t err = hipMalloc(p, ask);
        if (err == hipSuccess && ask != bytes) {
            (void)hipFree(*p);
            *p = nullptr;
            err = hipErrorOutOfMemory;
        }
        if (err == hipSuccess) return true;
        {
            std::lock_guard<std::mutex> lock(mu_);
            last_ = hipGetErrorString(err);
        }
        *p = nullptr;
        if (before == hipSuccess) (void)hipGetLastError();
        return false;
    }

    void free(int device, void* p) override {
        (void)hipSetDevice(device);
        (void)hipFree(p);
    }

    // Runs in tensor destructors, so it does not throw: if no event can be
    // recorded it waits for the stream instead and returns no marker (done).
    void* mark(int device, void* stream) override {
        hipEvent_t ev = nullptr;
        {
            std::lock_guard<std::mutex> lock(mu_);
            if (!pool_.empty()) {
                ev = pool_.back();
                pool_.pop_back();
            }
        }
        const hipError_t before = hipPeekAtLastError();
        hipError_t err = hipSetDevice(device);
        if (err == hipSuccess && !ev) err = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (err == hipSuccess) err = hipEventRecord(ev, static_cast<hipStream_t>(stream));
        if (err == hipSuccess) return ev;
        if (ev) drop(ev);
        (void)hipStreamSynchronize(static_cast<hipStream_t>(stream));
        if (before == hipSuccess) (void)hipGetLastError();
        return nullptr;
    }

    bool done(void* marker) override {
        if (!marker) return true;
        const hipError_t before = hipPeekAtLastError();
        const hipError_t q = hipEventQuery(static_cast<hipEvent_t>(marker));
        if (q == hipSuccess) return true;
        if (before == hipSuccess) (void)hipGetLastError();
        if (q == hipErrorNotReady) return false;
        hip::check(q, "event query failed");
        return false;
    }

    void wait(void* marker) override {
        if (!marker) return;
        hip::check(hipEventSynchronize(static_cast<hipEvent_t>(marker)),
                   "event synchronize failed");
    }

    void drop(void* marker) override {
        if (!marker) return;
        std::lock_guard<std::mutex> lock(mu_);
        pool_.push_back(static_cast<hipEvent_t>(marker));
    }

    void sync(void* stream) override {
        hip::check(hipStreamSynchronize(static_cast<hipStream_t>(stream)),
                   "stream synchronize failed");
    }

    std::string last_error() override {
        std::lock_guard<std::mutex> lock(mu_);
        return last_;
    }

private:
    std::mutex mu_;
    std::string last_;
    std::vector<hipEvent_t> pool_;
};

}  // namespace

BlockCache& device_block_cache() {
    static HipBackend* backend = new HipBackend();
    static BlockCache* cache = new BlockCache(*backend);
    return *cache;
}

void inject_alloc_failures(int n) { g_inject_failures.store(std::max(0, n)); }

}  // namespace detail

namespace {

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
    : data_(o.data_), stream_(o.stream_), uses_(std::move(o.uses_)),
      shape_(std::move(o.shape_)), dtype_(o.dtype_), device_(o.device_),
      requires_grad_(o.requires_grad_), grad_(std::move(o.grad_)),
      grad_fn_(std::move(o.grad_fn_)) {
    o.data_ = nullptr;
}

TensorImpl& TensorImpl::operator=(TensorImpl&& o) noexcept {
    if (this != &o) {
        release();
        data_ = o.data_;
        stream_ = o.stream_;
        uses_ = std::move(o.uses_);
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

void* TensorImpl::data() {
    note_use();
    return data_;
}

const void* TensorImpl::data() const {
    note_use();
    return data_;
}

void TensorImpl::note_use() const {
    if (data_) record_stream(current_stream());
}

void TensorImpl::record_stream(void* stream) const {
    // stream_ is fixed from allocation on; only uses on other streams are listed
    if (stream != stream_) uses_.record(stream);
}
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
    stream_ = current_stream();
    data_ = detail::device_block_cache().acquire(device_.index, bytes, stream_);
}

void TensorImpl::release() {
    if (!data_) return;
    if (device_.is_cuda()) {
        detail::device_block_cache().release(device_.index, nbytes(), data_, stream_,
                                             uses_.take());
    }
    data_ = nullptr;
    uses_.take();
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
    note_use();
    src.note_use();
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
    note_use();
    // A kernel on the current stream, not hipMemsetAsync: zeros() and
    // Linear's bias stay capturable into a graph (a captured memset node
    // gave wrong results on replays).
    hip::check_fdl(fdl_zero_fill(data_, static_cast<int64_t>(nbytes()), current_stream()),
                   "cudaMemset failed");
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

void Tensor::record_stream(void* stream) const {
    if (impl_ && impl_->data_ptr_raw()) impl_->record_stream(stream);
}

void Tensor::zero_() {
    if (!impl_) throw std::runtime_error("zero_ requires a defined tensor");
    impl_->zero_();
}

}  // namespace dl
