// common.hpp -- internal helpers shared by the backend's translation units:
// status reporting, the launch guard, stream casts and the scratch buffer.
#ifndef EHIP_COMMON_HPP
#define EHIP_COMMON_HPP

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "ehip.h"

namespace ehip {

// Records a printf-style message for ehip_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Initialises on first use and checks the runtime switch. Every kernel entry
// point starts with it.
int ready();

// Launch bookkeeping. before_launch() implements the fault-injection hook
// (ENGINE_HIP_FAIL_LAUNCH=n refuses the n-th launch, counted from 1, without
// touching the GPU); after_launch() reads the launch status, counts the
// launch, and with ENGINE_HIP_SYNC=1 waits for the stream so that a fault is
// reported by the launch that caused it.
int before_launch(const char* name);
int after_launch(const char* name, hipStream_t stream);

// The stream of this thread's graph capture (ehip_graph_begin), or null. While
// it is set, every call made with a null stream is recorded into the graph
// instead of being queued on the null stream.
extern thread_local hipStream_t t_capture;

inline hipStream_t as_stream(void* s) {
    return s != nullptr ? reinterpret_cast<hipStream_t>(s) : t_capture;
}
inline bool capturing() { return t_capture != nullptr; }

// Grow-only device scratch owned by the library (never shrinks; replaced by a
// larger block when asked for more). Work is ordered on one stream, so a
// buffer released while queued kernels still use it is reused only by later
// work on that stream. Slots are independent buffers: an entry point uses
// slot 0, and helpers it calls (column_sums) use slot 1, so the two never
// overlap. Returns nullptr (with the error recorded) on failure.
constexpr int kScratchSlots = 2;
void* scratch(size_t bytes, int slot = 0);

// Kernels reported by ehip_kernel_occupancy: each source file registers its
// representative instantiations (name, kernel, the block size it launches
// with) through a file-scope OccupancyEntries object at load time.
struct OccupancyKernel {
    const char* name;
    const void* func;
    int block_threads;
};
void register_occupancy(const OccupancyKernel* kernels, int count);
struct OccupancyEntries {
    template <int N>
    explicit OccupancyEntries(const OccupancyKernel (&k)[N]) { register_occupancy(k, N); }
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Column sums of `slabs` row-major (rows, cols) matrices with row pitch `ld`,
// slab pitch x_slab, into out[slab][cols]. Deterministic: the summation order
// depends only on the shape (reduce.hip).
int column_sums(const float* x, int64_t slabs, int64_t rows, int64_t cols, int64_t ld,
                int64_t x_slab, float* out, hipStream_t s);
// column_sums of x into out0 and of x + x_second into out1 (one slab each,
// the same sums bit for bit) in the launches of one call.
int column_sums_pair(const float* x, int64_t rows, int64_t cols, int64_t ld, int64_t x_second,
                     float* out0, float* out1, hipStream_t s);

// Ordered sum of partial[chunk][o] over `chunks` chunks of O outputs, as one
// 256-thread block's share (block bx of ceil(O / (256 / rl))): rl lanes per
// output take chunks l, l + rl, ... (eight loads in flight), then the lane sums
// are added in lane order through `lanes` (256 floats of LDS). Returns true in
// the thread that holds output o's sum. The order depends only on the shape.
__device__ __forceinline__ bool partial_sums(const float* __restrict__ partial, int O, int chunks,
                                             int rl, int bx, float* lanes, float& sum, int& o) {
    const int cw = 256 / rl;
    const int lane = threadIdx.x / cw, cl = threadIdx.x % cw;
    o = bx * cw + cl;
    float acc = 0.0f;
    if (o < O && lane < chunks) {
        const float* p = partial + o + int64_t(lane) * O;
        const int64_t stride = int64_t(rl) * O;
        const int count = (chunks - lane + rl - 1) / rl;
        acc = p[0];
        int s = 1;
        for (; s + 8 <= count; s += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = p[int64_t(s + u) * stride];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += v[u];
        }
        for (; s < count; ++s) acc += p[int64_t(s) * stride];
    }
    lanes[threadIdx.x] = acc;
    __syncthreads();
    if (lane != 0 || o >= O) return false;
    sum = lanes[cl];
    for (int l = 1; l < rl && l < chunks; ++l) sum += lanes[l * cw + cl];
    return true;
}

// Block order of a partial_sums reduction of `nblocks` blocks: groups of 16
// are permuted so that the blocks computing outputs 2j and 2j + 1 (with 16
// outputs a block, the two 64-byte halves of the same 128-byte lines of every
// chunk) run on one XCD -- the dispatcher hands consecutive blocks to the
// eight XCDs in turn, so local blocks p and p + 8 share one -- and each line
// comes into one L2 once instead of into two. A last, incomplete group keeps
// its order. The sums do not depend on which block computes them.
__device__ __forceinline__ int xcd_paired_block(int p, int nblocks) {
    if ((p | 15) >= nblocks) return p;
    return (p & ~15) | ((p & 7) << 1) | ((p >> 3) & 1);
}

// Lanes per output of partial_sums: about one per eight chunks, at most 16, so
// that a block still reads 16 consecutive outputs (64 bytes) of each chunk
// (32 lanes measured no faster and fetched twice the bytes).
inline int reduce_lanes(int64_t chunks) {
    int rl = 1;
    while (rl < 16 && rl * 8 < chunks) rl *= 2;
    return rl;
}

// Validates a window: positive extents, non-negative padding, and out_h/out_w
// equal to the geometry's (layout.hip). Refusals carry `name`.
int check_window(const char* name, const ehip_window_t* w);

// First and last window index along one axis whose window covers position p.
__host__ __device__ __forceinline__ void covering(int64_t p, int64_t pad, int64_t k, int64_t s,
                                         int64_t out, int64_t& lo, int64_t& hi) {
    const int64_t t = p + pad - (k - 1);
    lo = t <= 0 ? 0 : (t + s - 1) / s;
    hi = (p + pad) / s;
    if (hi > out - 1) hi = out - 1;
}

__host__ __device__ inline bool aligned16(const void* p) {
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

}  // namespace ehip

// Launches `kernel` through the guard; returns from the calling entry point on
// any failure.
#define EHIP_LAUNCH(name, kernel, grid, block, shmem, stream, ...)                  \
    do {                                                                            \
        if (int rc_ = ::ehip::before_launch(name)) return rc_;                      \
        hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);        \
        if (int rc_ = ::ehip::after_launch(name, stream)) return rc_;               \
    } while (0)

#define EHIP_READY()                                   \
    do {                                               \
        if (int rc_ = ::ehip::ready()) return rc_;     \
    } while (0)

#endif  // EHIP_COMMON_HPP
