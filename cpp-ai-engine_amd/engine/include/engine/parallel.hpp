// parallel.hpp -- the reference's host thread-pool API
// (include/engine/parallel.hpp): callers' own host loops split over threads.
// This engine computes on the GPU and never calls it; it is here so that
// programs and tests written against the reference's API build and behave
// the same (contiguous chunks, each run by one thread, so a loop whose chunks
// are independent gives the same bits with any thread count).
#ifndef ENGINE_PARALLEL_HPP
#define ENGINE_PARALLEL_HPP

#include <cstddef>
#include <functional>

namespace engine {
namespace parallel {

// The reference's split threshold for element-wise host loops.
constexpr size_t kElementsPerThread = 1u << 17;

// Threads in use: the ENGINE_NUM_THREADS environment variable, else the
// machine's hardware threads; at least 1.
size_t num_threads();

// Sets the thread count (0 counts as 1); with 1 everything runs on the caller.
void set_num_threads(size_t threads);

// body(begin, end) over [0, count) cut into at most num_threads() contiguous
// chunks of at least min_per_thread elements; runs inline when one chunk is
// enough or when called from inside another parallel_for. The first exception
// a chunk throws is rethrown on the caller after every chunk has finished.
void parallel_for(size_t count, size_t min_per_thread,
                  const std::function<void(size_t begin, size_t end)>& body);

// True on a thread that is running a parallel_for chunk.
bool inside_parallel_region();

}  // namespace parallel
}  // namespace engine

#endif  // ENGINE_PARALLEL_HPP
