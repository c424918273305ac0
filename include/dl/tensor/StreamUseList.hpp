#pragma once
// The streams, other than the one it was allocated on, that a tensor's memory
// is used on (TensorImpl::record_stream).  Any thread may record a use: a
// shared const tensor, such as a model weight, is read by several threads,
// each with its own current stream, so the list takes a lock.

#include <algorithm>
#include <cstddef>
#include <mutex>
#include <utility>
#include <vector>

namespace dl::detail {

class StreamUseList {
public:
    StreamUseList() = default;
    StreamUseList(const StreamUseList&) = delete;
    StreamUseList& operator=(const StreamUseList&) = delete;
    StreamUseList(StreamUseList&& other) noexcept : uses_(other.take()) {}
    StreamUseList& operator=(StreamUseList&& other) noexcept {
        if (this != &other) {
            std::vector<void*> taken = other.take();
            std::lock_guard<std::mutex> lock(mu_);
            uses_ = std::move(taken);
        }
        return *this;
    }

    // Adds `stream` unless it is listed already.
    void record(void* stream) {
        std::lock_guard<std::mutex> lock(mu_);
        if (std::find(uses_.begin(), uses_.end(), stream) == uses_.end()) uses_.push_back(stream);
    }

    // The recorded streams, in first-use order; the list is left empty.
    std::vector<void*> take() {
        std::lock_guard<std::mutex> lock(mu_);
        std::vector<void*> out;
        out.swap(uses_);
        return out;
    }

    std::size_t size() const {
        std::lock_guard<std::mutex> lock(mu_);
        return uses_.size();
    }

private:
    mutable std::mutex mu_;
    std::vector<void*> uses_;
};

}  // namespace dl::detail
