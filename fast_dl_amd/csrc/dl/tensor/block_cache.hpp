#pragma once
// Stream-ordered cache of device blocks behind TensorImpl (the reference
// allocates and frees every tensor with cudaMalloc/cudaFree,
// src/tensor/TensorImpl.cpp:69-89; this cache keeps freed blocks for reuse).
//
// Rules that make reuse safe without waiting for the device:
//  * A block belongs to the stream it was allocated on (its "home").  When
//    it is freed it goes back to its home's free list, whichever stream is
//    current at that moment, and only allocations made on the home stream get
//    it again: work queued on the home stream that used the old tensor runs
//    before any work that uses the new one, by stream order.
//  * A block also used on other streams (recorded with record_use) is not
//    reusable until those streams have passed the point where it was freed:
//    at release a marker (a HIP event) is recorded on each of them, and the
//    block waits in a pending list until every marker has completed.
//  * A stream about to be destroyed is retired: it is synchronized, and its
//    idle blocks move to a shared pool that any stream may take from.  A block
//    released later under a retired home also goes to that pool.
//
// The device runtime is reached only through CacheBackend, so the
// bookkeeping builds and is tested on the host with a fake backend.  Blocks
// are handed out by size class (see round()); the cache is not tied to HIP.
#include <cstddef>
#include <cstdint>
#include <functional>
#include <map>
#include <mutex>
#include <set>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace dl {
namespace detail {

class CacheBackend {
public:
    virtual ~CacheBackend() = default;
    // Allocates `bytes` on `device`.  On failure returns false, leaving no
    // error state behind that a later, unrelated call would report.
    virtual bool alloc(int device, std::size_t bytes, void** p) = 0;
    virtual void free(int device, void* p) = 0;
    // Marker after the work queued on `stream` so far; done() says whether
    // that work has completed.  Markers are handed back with drop().
    virtual void* mark(int device, void* stream) = 0;
    virtual bool done(void* marker) = 0;
    virtual void wait(void* marker) = 0;
    virtual void drop(void* marker) = 0;
    // Waits for all work queued on `stream`.
    virtual void sync(void* stream) = 0;
    // Text of the last allocation failure, for the exception message.
    virtual std::string last_error() = 0;
};

class BlockCache {
public:
    explicit BlockCache(CacheBackend& backend) : be_(backend) {}
    BlockCache(const BlockCache&) = delete;
    BlockCache& operator=(const BlockCache&) = delete;

    // Size class: 512-byte granules below 2 MiB, 2 MiB granules above.
    static std::size_t round(std::size_t bytes) {
        constexpr std::size_t kSmall = 512;
        constexpr std::size_t kLarge = std::size_t(2) << 20;
        const std::size_t g = bytes < kLarge ? kSmall : kLarge;
        return (bytes + g - 1) / g * g;
    }

    // A block of at least `bytes` for use on `stream`.  Throws
    // std::runtime_error("cudaMalloc failed: ...") when the device has no
    // memory left even after every cached block was returned to it.
    void* acquire(int device, std::size_t bytes, void* stream) {
        const std::size_t sz = round(bytes);
        {
            std::lock_guard<std::mutex> lock(mu_);
            reap_locked();
            if (void* p = take_locked(Key{device, sz, stream})) return p;
            if (void* p = take_locked(Key{device, sz, shared()})) return p;
        }
        void* p = nullptr;
        if (be_.alloc(device, sz, &p)) return p;
        // Return every cached block of this device to the runtime and retry once.
        release_all(device);
        if (be_.alloc(device, sz, &p)) return p;
        throw std::runtime_error("cudaMalloc failed: " + be_.last_error());
    }

    // Gives back a block allocated on `home`.  `uses` are the other streams
    // that used it (the home stream and retired streams are skipped).
    void release(int device, std::size_t bytes, void* p, void* home,
                 const std::vector<void*>& uses) {
        if (!p) return;
        const std::size_t sz = round(bytes);
        std::lock_guard<std::mutex> lock(mu_);
        void* const owner = retired_.count(home) ? shared() : home;
        Pending pend{Key{device, sz, owner}, p, {}};
        for (void* s : uses) {
            // A retired stream's work has finished (and the stream may no
            // longer exist): nothing to wait for.
            if (s == home || retired_.count(s)) continue;
            pend.markers.push_back(be_.mark(device, s));
        }
        if (pend.markers.empty()) {
            free_[pend.key].push_back(p);
        } else {
            pending_.push_back(std::move(pend));
        }
    }

    // Frees every cached and pending block of `device` (waiting for the work
    // that may still use the pending ones first).
    void release_all(int device) {
        std::lock_guard<std::mutex> lock(mu_);
        for (auto it = pending_.begin(); it != pending_.end();) {
            if (it->key.device != device) {
                ++it;
                continue;
            }
            for (void* m : it->markers) {
                be_.wait(m);
                be_.drop(m);
            }
            be_.free(device, it->p);
            it = pending_.erase(it);
        }
        for (auto& kv : free_) {
            if (kv.first.device != device) continue;
            for (void* p : kv.second) be_.free(device, p);
            kv.second.clear();
        }
    }

    // `stream` is about to be destroyed: waits for its work, then moves its
    // idle blocks to the shared pool and files later releases of blocks
    // homed on it there too.
    void retire_stream(void* stream) {
        if (!stream) return;  // the null stream is never destroyed
        be_.sync(stream);
        std::lock_guard<std::mutex> lock(mu_);
        retired_.insert(stream);
        reap_locked();
        for (auto it = free_.begin(); it != free_.end(); ++it) {
            if (it->first.stream != stream || it->second.empty()) continue;
            auto& dst = free_[Key{it->first.device, it->first.bytes, shared()}];
            dst.insert(dst.end(), it->second.begin(), it->second.end());
            it->second.clear();
        }
        for (Pending& pd : pending_) {
            if (pd.key.stream == stream) pd.key.stream = shared();
        }
    }

    // A stream handle (re)created: a handle value reused by the runtime no
    // longer counts as retired.  Blocks still homed on the old stream of the
    // same value are idle (it was synchronized when retired), so they may go
    // to the new one.
    void stream_created(void* stream) {
        std::lock_guard<std::mutex> lock(mu_);
        retired_.erase(stream);
    }

    // Bookkeeping queries (tests).
    std::size_t free_blocks(int device, std::size_t bytes, void* stream) {
        std::lock_guard<std::mutex> lock(mu_);
        reap_locked();
        auto it = free_.find(Key{device, round(bytes), stream});
        return it == free_.end() ? 0 : it->second.size();
    }
    std::size_t shared_blocks(int device, std::size_t bytes) {
        return free_blocks(device, bytes, shared());
    }
    std::size_t pending_blocks() {
        std::lock_guard<std::mutex> lock(mu_);
        reap_locked();
        return pending_.size();
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
    struct Pending {
        Key key;
        void* p;
        std::vector<void*> markers;
    };

    // Key of the shared pool: not a valid stream handle (an odd address).
    static void* shared() { return reinterpret_cast<void*>(std::uintptr_t(1)); }

    void* take_locked(const Key& k) {
        auto it = free_.find(k);
        if (it == free_.end() || it->second.empty()) return nullptr;
        void* p = it->second.back();
        it->second.pop_back();
        return p;
    }

    // Moves pending blocks whose markers have all completed to their free list.
    void reap_locked() {
        for (auto it = pending_.begin(); it != pending_.end();) {
            bool all = true;
            for (void* m : it->markers) {
                if (!be_.done(m)) {
                    all = false;
                    break;
                }
            }
            if (!all) {
                ++it;
                continue;
            }
            for (void* m : it->markers) be_.drop(m);
            free_[it->key].push_back(it->p);
            it = pending_.erase(it);
        }
    }

    CacheBackend& be_;
    std::mutex mu_;
    std::map<Key, std::vector<void*>> free_;
    std::vector<Pending> pending_;
    std::set<void*> retired_;
};

// The dl:: library's process-wide cache (tensor.cpp), on the HIP runtime.
BlockCache& device_block_cache();

// Test hook: each of the next `n` device allocations first asks the runtime
// for an impossible size, so it fails for real (and leaves the runtime's
// error state set, as an out-of-memory failure does) before the cache frees
// its blocks and retries with the real size.
void inject_alloc_failures(int n);

}  // namespace detail
}  // namespace dl
