// Host-only check of dl::detail::StreamUseList (include/dl/tensor/StreamUseList.hpp),
// the streams TensorImpl::record_stream lists for a tensor: several threads
// record uses of one shared tensor at once, each on its own current stream
// (as when threads read a shared weight), while another thread takes the
// list.  Built with the thread sanitizer (host code only); prints
// "<name> : passed|not passed" and exits with the number of failures.
#include <dl/tensor/StreamUseList.hpp>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <set>
#include <thread>
#include <vector>

namespace {

int failures = 0;

void report(const char* name, bool ok) {
    std::printf("%s : %s\n", name, ok ? "passed" : "not passed");
    if (!ok) ++failures;
}

void* fake_stream(std::uintptr_t i) { return reinterpret_cast<void*>(0x1000 + 16 * i); }

}  // namespace

int main() {
    {
        // Eight threads, each recording its own stream and two shared ones
        // many times: every stream is listed once.
        dl::detail::StreamUseList uses;
        std::vector<std::thread> threads;
        for (std::uintptr_t t = 0; t < 8; ++t) {
            threads.emplace_back([&uses, t] {
                for (int i = 0; i < 20000; ++i) {
                    uses.record(fake_stream(100 + t));
                    uses.record(fake_stream(i & 1));
                }
            });
        }
        for (auto& th : threads) th.join();
        const std::vector<void*> got = uses.take();
        std::set<void*> distinct(got.begin(), got.end());
        bool ok = got.size() == 10 && distinct.size() == 10 && uses.size() == 0;
        for (std::uintptr_t t = 0; t < 8; ++t) ok = ok && distinct.count(fake_stream(100 + t));
        report("stream_use_list_concurrent_record", ok);
    }
    {
        // Records racing with takes: every recorded stream comes out of
        // exactly one take or is left at the end, and never twice in one.
        dl::detail::StreamUseList uses;
        std::atomic<bool> stop{false};
        std::vector<std::vector<void*>> taken;
        std::thread taker([&] {
            while (!stop.load()) taken.push_back(uses.take());
        });
        std::vector<std::thread> writers;
        for (std::uintptr_t t = 0; t < 4; ++t) {
            writers.emplace_back([&uses, t] {
                for (int i = 0; i < 20000; ++i) uses.record(fake_stream(t));
            });
        }
        for (auto& th : writers) th.join();
        stop = true;
        taker.join();
        taken.push_back(uses.take());
        bool ok = true;
        std::set<void*> seen;
        for (const auto& v : taken) {
            std::set<void*> once(v.begin(), v.end());
            ok = ok && once.size() == v.size();
            seen.insert(v.begin(), v.end());
        }
        ok = ok && seen.size() == 4;
        report("stream_use_list_record_while_taking", ok);
    }
    {
        // Moves carry the list and leave the source empty.
        dl::detail::StreamUseList a;
        a.record(fake_stream(1));
        a.record(fake_stream(2));
        a.record(fake_stream(1));
        dl::detail::StreamUseList b(std::move(a));
        dl::detail::StreamUseList c;
        c.record(fake_stream(9));
        c = std::move(b);
        const std::vector<void*> got = c.take();
        report("stream_use_list_move",
               a.size() == 0 && b.size() == 0 && got.size() == 2 && got[0] == fake_stream(1) &&
                   got[1] == fake_stream(2));
    }
    std::printf("stream_use_list_test : %s\n", failures ? "not passed" : "passed");
    return failures;
}
