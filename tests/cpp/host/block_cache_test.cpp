// Host-only checks of the block cache's bookkeeping
// (fast_dl_amd/csrc/dl/tensor/block_cache.hpp) with a fake device backend:
// which stream gets a freed block back, when a block used on other streams
// becomes reusable, what retiring a stream does, and the out-of-memory retry.
// Each check prints "<name> : passed|not passed"; the exit status counts
// failures.
#include "block_cache.hpp"

#include <cstdint>
#include <cstdio>
#include <functional>
#include <iostream>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

using dl::detail::BlockCache;
using dl::detail::CacheBackend;

// Fake device: addresses count up from 0x1000; markers complete when the
// test says so; allocations fail while `fail` is positive.
class FakeBackend final : public CacheBackend {
public:
    int fail = 0;
    int allocs = 0;
    std::vector<void*> freed;
    std::set<std::uintptr_t> done_markers;
    std::vector<void*> synced;
    std::uintptr_t next_addr = 0x1000;
    std::uintptr_t next_marker = 1;
    std::vector<std::pair<void*, void*>> marks;  // (marker, stream)
    std::vector<void*> waited;

    bool alloc(int, std::size_t bytes, void** p) override {
        ++allocs;
        if (fail > 0) {
            --fail;
            return false;
        }
        *p = reinterpret_cast<void*>(next_addr);
        next_addr += bytes + 0x1000;
        return true;
    }
    void free(int, void* p) override { freed.push_back(p); }
    void* mark(int, void* stream) override {
        void* m = reinterpret_cast<void*>(next_marker++);
        marks.emplace_back(m, stream);
        return m;
    }
    bool done(void* m) override { return done_markers.count(reinterpret_cast<std::uintptr_t>(m)) > 0; }
    void wait(void* m) override {
        waited.push_back(m);
        done_markers.insert(reinterpret_cast<std::uintptr_t>(m));
    }
    void drop(void*) override {}
    void sync(void* stream) override {
        synced.push_back(stream);
        for (auto& ms : marks)
            if (ms.second == stream) done_markers.insert(reinterpret_cast<std::uintptr_t>(ms.first));
    }
    std::string last_error() override { return "out of memory"; }
};

void* S(int i) { return reinterpret_cast<void*>(std::uintptr_t(0x100 * i)); }

int g_failures = 0;

void check(const std::string& name, const std::function<bool()>& fn) {
    bool ok = false;
    try {
        ok = fn();
    } catch (const std::exception& e) {
        std::cout << name << " threw: " << e.what() << "\n";
    }
    std::cout << name << " : " << (ok ? "passed" : "not passed") << std::endl;
    if (!ok) ++g_failures;
}

}  // namespace

int main() {
    check("size_classes", [] {
        return BlockCache::round(1) == 512 && BlockCache::round(512) == 512 &&
               BlockCache::round(513) == 1024 && BlockCache::round((2 << 20) - 1) == (2u << 20) &&
               BlockCache::round(2 << 20) == (2u << 20) &&
               BlockCache::round((2 << 20) + 1) == (4u << 20);
    });

    check("same_stream_reuse", [] {
        FakeBackend be;
        BlockCache c(be);
        void* a = c.acquire(0, 4096, S(1));
        c.release(0, 4096, a, S(1), {S(1)});
        void* b = c.acquire(0, 4000, S(1));  // same size class
        return a == b && be.allocs == 1;
    });

    // A tensor allocated on T, freed while S is current: the block goes back
    // to T, so an allocation on S cannot overwrite it under T's queued work.
    check("freed_under_other_stream_returns_home", [] {
        FakeBackend be;
        BlockCache c(be);
        void* x = c.acquire(0, 1 << 20, S(2));     // home T = S(2)
        c.release(0, 1 << 20, x, S(2), {S(2)});    // freed (S current: irrelevant)
        void* y = c.acquire(0, 1 << 20, S(3));     // allocation on S
        void* z = c.acquire(0, 1 << 20, S(2));     // allocation on T
        return y != x && z == x && c.free_blocks(0, 1 << 20, S(3)) == 0;
    });

    // Home S, also used on T: pending until T's marker completes, then S's again.
    check("recorded_use_waits_for_marker", [] {
        FakeBackend be;
        BlockCache c(be);
        void* x = c.acquire(0, 8192, S(1));
        c.release(0, 8192, x, S(1), {S(1), S(2)});
        if (be.marks.size() != 1 || be.marks[0].second != S(2)) return false;
        if (c.pending_blocks() != 1) return false;
        void* y = c.acquire(0, 8192, S(1));  // T not yet past the release
        if (y == x) return false;
        be.done_markers.insert(reinterpret_cast<std::uintptr_t>(be.marks[0].first));
        void* z = c.acquire(0, 8192, S(1));
        return z == x && c.pending_blocks() == 0;
    });

    check("retire_moves_idle_blocks_to_shared_pool", [] {
        FakeBackend be;
        BlockCache c(be);
        void* a = c.acquire(0, 512, S(4));
        void* live = c.acquire(0, 512, S(4));
        c.release(0, 512, a, S(4), {});
        c.retire_stream(S(4));
        if (be.synced.size() != 1 || be.synced[0] != S(4)) return false;
        if (c.free_blocks(0, 512, S(4)) != 0 || c.shared_blocks(0, 512) != 1) return false;
        void* b = c.acquire(0, 512, S(5));  // any stream takes from the shared pool
        if (b != a) return false;
        c.release(0, 512, live, S(4), {});  // released after its home was retired
        if (c.shared_blocks(0, 512) != 1) return false;
        c.stream_created(S(4));  // the handle value reused by a new stream
        void* d = c.acquire(0, 512, S(6));
        c.release(0, 512, d, S(4), {});
        return d == live && c.free_blocks(0, 512, S(4)) == 1;
    });

    check("retire_reassigns_pending_blocks", [] {
        FakeBackend be;
        BlockCache c(be);
        void* a = c.acquire(0, 1024, S(7));
        c.release(0, 1024, a, S(7), {S(8)});
        c.retire_stream(S(7));                 // S(8)'s marker still open
        if (c.pending_blocks() != 1) return false;
        be.done_markers.insert(reinterpret_cast<std::uintptr_t>(be.marks[0].first));
        return c.pending_blocks() == 0 && c.shared_blocks(0, 1024) == 1;
    });

    // A tensor that outlives a stream it was used on (its home is another
    // stream): no marker may be recorded on the destroyed stream.
    check("use_on_retired_stream_needs_no_marker", [] {
        FakeBackend be;
        BlockCache c(be);
        void* x = c.acquire(0, 2048, nullptr);
        c.retire_stream(S(9));
        c.release(0, 2048, x, nullptr, {S(9)});
        return be.marks.empty() && c.free_blocks(0, 2048, nullptr) == 1;
    });

    check("null_stream_never_retired", [] {
        FakeBackend be;
        BlockCache c(be);
        void* a = c.acquire(0, 512, nullptr);
        c.release(0, 512, a, nullptr, {});
        c.retire_stream(nullptr);
        return be.synced.empty() && c.free_blocks(0, 512, nullptr) == 1;
    });

    // Out of memory: every cached block (pending ones after their markers)
    // goes back to the device, then one retry.
    check("oom_frees_cache_and_retries", [] {
        FakeBackend be;
        BlockCache c(be);
        void* a = c.acquire(0, 4096, S(1));
        void* b = c.acquire(0, 8192, S(2));
        void* other_dev = c.acquire(1, 4096, S(1));
        c.release(0, 4096, a, S(1), {});
        c.release(0, 8192, b, S(2), {S(3)});
        c.release(1, 4096, other_dev, S(1), {});
        be.fail = 1;
        void* d = c.acquire(0, 1 << 21, S(1));
        const bool freed_dev0 = be.freed.size() == 2 &&
                                ((be.freed[0] == a && be.freed[1] == b) ||
                                 (be.freed[0] == b && be.freed[1] == a));
        return d != nullptr && freed_dev0 && be.waited.size() == 1 &&
               c.free_blocks(1, 4096, S(1)) == 1 && c.pending_blocks() == 0;
    });

    check("oom_after_retry_throws", [] {
        FakeBackend be;
        BlockCache c(be);
        be.fail = 2;
        try {
            c.acquire(0, 512, nullptr);
        } catch (const std::runtime_error& e) {
            return std::string(e.what()) == "cudaMalloc failed: out of memory" && be.allocs == 2;
        }
        return false;
    });

    std::cout << (g_failures ? "block_cache_test : not passed" : "block_cache_test : passed")
              << std::endl;
    return g_failures;
}
