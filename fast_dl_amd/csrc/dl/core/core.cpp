// dl:: value types (Device, DType, Shape), streams and HIP error checks.
// Behaviour follows src/core/{Device,DType,Shape,CudaUtils}.cpp of the reference.
#include <dl/core/DType.hpp>
#include <dl/core/Device.hpp>
#include <dl/core/HipUtils.hpp>
#include <dl/core/Shape.hpp>
#include <dl/core/Stream.hpp>

#include <fastdl_gemm.h>

#include "../tensor/block_cache.hpp"

#include <hip/hip_runtime_api.h>

#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>

namespace dl {

Device::Device(DeviceType t, int i) : type(t), index(i) {}

bool Device::is_cuda() const { return type == DeviceType::CUDA; }

bool Device::is_cpu() const { return type == DeviceType::CPU; }

std::string Device::str() const { return is_cuda() ? "cuda:" + std::to_string(index) : "cpu"; }

std::size_t dtype_size(DType dtype) {
    switch (dtype) {
        case DType::Float32: return 4;
        case DType::Float16: return 2;
        case DType::Int32: return 4;
        case DType::Int64: return 8;
        case DType::Bool: return 1;
    }
    throw std::invalid_argument("unknown dtype");
}

std::string dtype_name(DType dtype) {
    switch (dtype) {
        case DType::Float32: return "float32";
        case DType::Float16: return "float16";
        case DType::Int32: return "int32";
        case DType::Int64: return "int64";
        case DType::Bool: return "bool";
    }
    throw std::invalid_argument("unknown dtype");
}

Shape::Shape(std::initializer_list<int64_t> d) : dims(d) {}

Shape::Shape(std::vector<int64_t> d) : dims(std::move(d)) {}

int64_t Shape::rank() const { return static_cast<int64_t>(dims.size()); }

int64_t Shape::numel() const {
    if (dims.empty()) return 0;
    int64_t n = 1;
    for (int64_t d : dims) n *= d;
    return n;
}

int64_t Shape::operator[](int index) const { return dims[index]; }

std::string Shape::str() const {
    std::ostringstream os;
    os << "(";
    for (std::size_t i = 0; i < dims.size(); ++i) os << (i ? ", " : "") << dims[i];
    os << ")";
    return os.str();
}

// ------------------------------------------------------------------ streams

namespace {

thread_local void* t_current_stream = nullptr;

}  // namespace

Stream::Stream(const Device& device) {
    if (!device.is_cuda()) throw std::runtime_error("Stream: device must be a GPU");
    hip::check(hipSetDevice(device.index), "cudaSetDevice failed");
    hipStream_t s = nullptr;
    hip::check(hipStreamCreate(&s), "stream create failed");
    stream_ = s;
    detail::device_block_cache().stream_created(stream_);
}

namespace {

// Hands the stream's cached blocks to the shared pool (after its work has
// finished), then destroys it.
void destroy_stream(void* stream) noexcept {
    if (!stream) return;
    try {
        detail::device_block_cache().retire_stream(stream);
    } catch (...) {
        // The stream could not be synchronized; its blocks stay filed under
        // its handle and are freed on the next out-of-memory retry.
    }
    (void)hipStreamDestroy(static_cast<hipStream_t>(stream));
}

}  // namespace

Stream::~Stream() { destroy_stream(stream_); }

Stream::Stream(Stream&& other) noexcept : stream_(std::exchange(other.stream_, nullptr)) {}

Stream& Stream::operator=(Stream&& other) noexcept {
    if (this != &other) {
        destroy_stream(stream_);
        stream_ = std::exchange(other.stream_, nullptr);
    }
    return *this;
}

void retire_stream(void* stream) { detail::device_block_cache().retire_stream(stream); }

void Stream::synchronize() const {
    hip::check(hipStreamSynchronize(static_cast<hipStream_t>(stream_)), "stream synchronize failed");
}

void* current_stream() { return t_current_stream; }

void set_current_stream(void* stream) { t_current_stream = stream; }

StreamGuard::StreamGuard(void* stream) : previous_(t_current_stream) { t_current_stream = stream; }

StreamGuard::~StreamGuard() { t_current_stream = previous_; }

void synchronize() {
    hip::check(hipStreamSynchronize(static_cast<hipStream_t>(t_current_stream)),
               "stream synchronize failed");
}

namespace hip {

void check(hipError_t status, const char* action) {
    if (status != hipSuccess) {
        throw std::runtime_error(std::string(action) + ": " + hipGetErrorString(status));
    }
}

void check_fdl(int status, const char* action) {
    if (status != FDL_SUCCESS) {
        throw std::runtime_error(std::string(action) + ": " + fdl_last_error());
    }
}

}  // namespace hip

}  // namespace dl
