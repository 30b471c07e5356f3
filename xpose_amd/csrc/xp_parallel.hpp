// Host thread pool helpers shared by the packers (int4 requantiser, native
// repack): a thread count and a work-stealing parallel for.
#pragma once

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <exception>
#include <thread>
#include <vector>

namespace xp {

// `t` threads, or every hardware thread when t == 0.
inline uint32_t n_threads(uint32_t t) {
    if (t) return t;
    const uint32_t h = std::thread::hardware_concurrency();
    return h ? h : 1;
}

// Runs fn(i) for i in [0, n) on up to `threads` threads (work stealing).
template <class F>
void parallel_for(uint32_t n, uint32_t threads, F&& fn) {
    const uint32_t nt = std::max(1u, std::min(threads, n));
    if (nt == 1) {
        for (uint32_t i = 0; i < n; ++i) fn(i);
        return;
    }
    std::atomic<uint32_t> next{0};
    std::exception_ptr err;
    std::atomic<bool> failed{false};
    std::vector<std::thread> pool;
    pool.reserve(nt);
    for (uint32_t w = 0; w < nt; ++w)
        pool.emplace_back([&] {
            for (;;) {
                const uint32_t i = next.fetch_add(1, std::memory_order_relaxed);
                if (i >= n || failed.load(std::memory_order_relaxed)) return;
                try {
                    fn(i);
                } catch (...) {
                    if (!failed.exchange(true)) err = std::current_exception();
                    return;
                }
            }
        });
    for (auto& t : pool) t.join();
    if (err) std::rethrow_exception(err);
}

}  // namespace xp
