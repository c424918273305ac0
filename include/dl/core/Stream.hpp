#pragma once
// Streams for the dl:: API.  The reference enqueues all of its work on the
// legacy default stream (src/ops/Matmul.cpp:33-42 launch with no stream);
// this build keeps that as the default and lets a thread choose another
// stream for the dl:: work it issues.  A stream is a hipStream_t carried as
// void*, so using this header needs no HIP headers.

#include <dl/core/Device.hpp>

namespace dl {

// A HIP stream owned by this object, created on `device` with the default
// flags (it orders with the null stream) and the default priority.
class Stream {
public:
    explicit Stream(const Device& device = Device(DeviceType::CUDA, 0));
    ~Stream();
    Stream(const Stream&) = delete;
    Stream& operator=(const Stream&) = delete;
    Stream(Stream&& other) noexcept;
    Stream& operator=(Stream&& other) noexcept;

    void* handle() const { return stream_; }  // the hipStream_t
    void synchronize() const;                  // waits for all work on this stream

private:
    void* stream_ = nullptr;
};

// The stream every dl:: op, kernel launcher, tensor transfer and trainer step
// issued from the calling thread is enqueued on; nullptr (the default) is the
// null stream.  Tensor transfers to and from the host stay synchronous.
//
// Tensor memory is cached per stream: a tensor's block returns to the stream
// that was current when it was allocated.  A dl::Stream hands its cached
// blocks back when it is destroyed.  A raw hipStream_t made current with
// set_current_stream must be passed to retire_stream before the caller
// destroys it (that waits for its work and releases its cached blocks to
// every stream).
void* current_stream();
void set_current_stream(void* stream);
void retire_stream(void* stream);

// Makes `stream` the calling thread's current stream for the guard's lifetime
// and restores the previous one on destruction.
class StreamGuard {
public:
    explicit StreamGuard(void* stream);
    explicit StreamGuard(const Stream& stream) : StreamGuard(stream.handle()) {}
    ~StreamGuard();
    StreamGuard(const StreamGuard&) = delete;
    StreamGuard& operator=(const StreamGuard&) = delete;

private:
    void* previous_;
};

// Waits for all work on the calling thread's current stream.
void synchronize();

}  // namespace dl
