// Exercises the engine's host thread pool (engine/src/parallel.cpp) under a sanitizer:
// disjoint writes from every chunk, sizes around the chunking thresholds, nested calls
// (which run inline), an exception thrown from a chunk, thread-count changes between
// calls and calls from several host threads at once (serialised by the pool).
#include <atomic>
#include <cstdio>
#include <stdexcept>
#include <thread>
#include <vector>

#include "engine/parallel.hpp"

namespace par = engine::parallel;

static int fail(const char* what) {
    std::fprintf(stderr, "pool_driver: %s\n", what);
    return 1;
}

static bool fill_and_check(size_t n, size_t min_per_thread) {
    std::vector<int> hits(n, 0);
    par::parallel_for(n, min_per_thread, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) hits[i] += 1;
    });
    for (int h : hits)
        if (h != 1) return false;
    return true;
}

int main() {
    for (size_t threads : {1u, 3u, 8u, 16u}) {
        par::set_num_threads(threads);
        for (size_t n : {size_t(0), size_t(1), size_t(7), size_t(1000), (size_t(1) << 17) + 3,
                         size_t(1) << 20})
            for (size_t min : {size_t(1), size_t(64), par::kElementsPerThread})
                if (!fill_and_check(n, min)) return fail("an element was not visited once");
    }
    par::set_num_threads(8);
    // Nested: the inner call runs inline on the calling worker.
    std::atomic<size_t> inner{0};
    std::atomic<bool> nested_inline{true};
    par::parallel_for(64, 1, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) {
            if (!par::inside_parallel_region()) nested_inline = false;
            par::parallel_for(100, 1, [&](size_t ib, size_t ie) { inner += ie - ib; });
        }
    });
    if (inner != 6400 || !nested_inline) return fail("nested calls");
    // An exception in one chunk reaches the caller; the pool stays usable.
    bool caught = false;
    try {
        par::parallel_for(1 << 16, 1, [&](size_t b, size_t) {
            if (b == 0) throw std::runtime_error("chunk failure");
        });
    } catch (const std::runtime_error&) {
        caught = true;
    }
    if (!caught) return fail("exception not propagated");
    if (!fill_and_check(1 << 18, 1)) return fail("pool unusable after an exception");
    // Several host threads calling at once.
    std::vector<std::thread> callers;
    std::atomic<int> bad{0};
    for (int t = 0; t < 4; ++t)
        callers.emplace_back([&] {
            for (int rep = 0; rep < 20; ++rep)
                if (!fill_and_check(1 << 15, 1)) ++bad;
        });
    for (auto& c : callers) c.join();
    if (bad) return fail("concurrent callers");
    std::printf("pool_driver: ok\n");
    return 0;
}
