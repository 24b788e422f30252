// reduce.hip -- sum over one axis (bias gradients, fold_leading) and the
// whole-buffer double-precision sums behind Tensor::sum()/mean().
//
// No atomics: every sum has a fixed order that depends only on the shape, so
// two runs on the same data agree bit for bit.

#include "common.hpp"

namespace ehip {
namespace {

constexpr int kThreads = 256;

// Adds p[0], p[step], ..., p[(n-1) step] to acc in that order. Loads are
// issued sixteen at a time ahead of the additions, which stay in index order:
// a lane's chain of dependent HBM round trips is n / 16 long.
__device__ __forceinline__ float ordered_sum(float acc, const float* __restrict__ p, int64_t n,
                                             int64_t step) {
    constexpr int U = 16;
    int64_t i = 0;
    for (; i + U <= n; i += U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = p[(i + u) * step];
#pragma unroll
        for (int u = 0; u < U; ++u) acc += v[u];
    }
    for (; i + 4 <= n; i += 4) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = p[(i + u) * step];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc += v[u];
    }
    for (; i < n; ++i) acc += p[i * step];
    return acc;
}

// One thread per output element, axis ascending from zero: exactly the order
// of src/tensor.cpp:347-356, so the result is bit-identical to the CPU.
__global__ __launch_bounds__(kThreads) void sum_axis_serial(const float* __restrict__ x,
                                                            float* __restrict__ out,
                                                            int64_t axis_len, int64_t inner,
                                                            int64_t n_out) {
    const int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= n_out) return;
    const int64_t o = e / inner, i = e % inner;
    out[e] = ordered_sum(0.0f, x + o * axis_len * inner + i, axis_len, inner);
}

// Column sums over a block of rows, for the long-axis / few-outputs case
// (bias gradients: thousands of rows, 8 to 4096 columns). The 256 threads
// form RL row lanes x CW columns (CW = min(64, cols rounded up to a power of
// two)); block (b, t, o) covers rows [b*rpb, (b+1)*rpb) and columns
// [t*CW, (t+1)*CW) of slab o. Lane l adds rows r0+l, r0+l+RL, ... in order;
// then one thread per column adds the RL lane sums in lane order. The order
// depends only on the shape. Returns the sum in the lane-0 threads.
__device__ __forceinline__ float block_rows_sum(const float* __restrict__ xs, int64_t r0,
                                                int64_t r1, int64_t c, int64_t cols, int64_t ld,
                                                int cw, float* lanes) {
    const int rl = kThreads / cw;
    const int lane = threadIdx.x / cw, cl = threadIdx.x % cw;
    float acc = 0.0f;
    if (c < cols && r0 + lane < r1)
        acc = ordered_sum(0.0f, xs + (r0 + lane) * ld + c, (r1 - r0 - lane + rl - 1) / rl,
                          int64_t(rl) * ld);
    lanes[threadIdx.x] = acc;
    __syncthreads();
    float s = 0.0f;
    if (lane == 0)
        for (int l = 0; l < rl; ++l) s += lanes[l * cw + cl];
    __syncthreads();  // lanes may be reused
    return s;
}

// Slab z's output: out + z * out_slab, or out_second for slab 1 when given
// (two separate arrays).
__device__ __forceinline__ float* slab_out(float* out, float* out_second, int64_t out_slab) {
    return blockIdx.z == 1 && out_second != nullptr ? out_second
                                                   : out + int64_t(blockIdx.z) * out_slab;
}

__global__ __launch_bounds__(kThreads) void sum_cols(const float* __restrict__ x,
                                                     float* out, float* out_second, int64_t rows,
                                                     int64_t cols, int64_t ld, int64_t rpb,
                                                     int64_t x_slab, int64_t out_slab, int cw) {
    __shared__ float lanes[kThreads];
    const int64_t c = int64_t(blockIdx.y) * cw + threadIdx.x % cw;
    const int64_t r0 = int64_t(blockIdx.x) * rpb;
    const int64_t r1 = r0 + rpb < rows ? r0 + rpb : rows;
    const float s = block_rows_sum(x + int64_t(blockIdx.z) * x_slab, r0, r1, c, cols, ld, cw, lanes);
    if (threadIdx.x < cw && c < cols)
        slab_out(out, out_second, out_slab)[int64_t(blockIdx.x) * cols + c] = s;
}

// sum_cols for CW = 64 with four adjacent columns per thread (float4 loads,
// 1 KiB per wave and row instead of 256 bytes): the same row lanes, rows per
// lane and order per column as sum_cols, so the sums are bit-identical.
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ __forceinline__ float4 ordered_sum4(const float* __restrict__ p, int64_t n,
                                               int64_t step) {
    constexpr int U = 16;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    int64_t i = 0;
    for (; i + U <= n; i += U) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = *reinterpret_cast<const float4*>(p + (i + u) * step);
#pragma unroll
        for (int u = 0; u < U; ++u) acc = add4(acc, v[u]);
    }
    for (; i < n; ++i) acc = add4(acc, *reinterpret_cast<const float4*>(p + i * step));
    return acc;
}

__device__ __forceinline__ float4 block_rows_sum4(const float* __restrict__ xs, int64_t r0,
                                                  int64_t r1, int64_t c, int64_t cols, int64_t ld,
                                                  float4* lanes) {
    constexpr int kCw = 64, kRl = kThreads / kCw;
    const int lane = threadIdx.x / kCw, cl = threadIdx.x % kCw;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (c < cols && r0 + lane < r1)
        acc = ordered_sum4(xs + (r0 + lane) * ld + c, (r1 - r0 - lane + kRl - 1) / kRl,
                           int64_t(kRl) * ld);
    lanes[threadIdx.x] = acc;
    __syncthreads();
    float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (lane == 0)
        for (int l = 0; l < kRl; ++l) sum = add4(sum, lanes[l * kCw + cl]);
    __syncthreads();
    return sum;
}

__device__ __forceinline__ void store4(float* o, float4 v) {
    o[0] = v.x;
    o[1] = v.y;
    o[2] = v.z;
    o[3] = v.w;
}

__global__ __launch_bounds__(kThreads) void sum_cols4(const float* __restrict__ x,
                                                      float* out, float* out_second, int64_t rows,
                                                      int64_t cols, int64_t ld, int64_t rpb,
                                                      int64_t x_slab, int64_t out_slab) {
    __shared__ float4 lanes[kThreads];
    const int64_t c = (int64_t(blockIdx.y) * 64 + threadIdx.x % 64) * 4;
    const int64_t r0 = int64_t(blockIdx.x) * rpb;
    const int64_t r1 = r0 + rpb < rows ? r0 + rpb : rows;
    const float4 s = block_rows_sum4(x + int64_t(blockIdx.z) * x_slab, r0, r1, c, cols, ld, lanes);
    if (threadIdx.x < 64 && c < cols)
        store4(slab_out(out, out_second, out_slab) + int64_t(blockIdx.x) * cols + c, s);
}

// Whole-buffer sum in double: a fixed grid of blocks, each thread striding by
// the grid, then a fixed-shape tree per block.
constexpr int kReduceBlocks = 512;

template <bool SQUARES>
__global__ __launch_bounds__(kThreads) void reduce_stage1(const float* __restrict__ x, int64_t n,
                                                          double* __restrict__ partial) {
    __shared__ double sh[kThreads];
    double acc = 0.0;
    const int64_t step = int64_t(kReduceBlocks) * kThreads;
    for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < n; i += step) {
        const double v = x[i];
        acc += SQUARES ? v * v : v;
    }
    sh[threadIdx.x] = acc;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (int(threadIdx.x) < s) sh[threadIdx.x] += sh[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = sh[0];
}

__global__ __launch_bounds__(kThreads) void reduce_stage2(const double* __restrict__ partial,
                                                          double* out_d, float* out_f) {
    __shared__ double sh[kThreads];
    double acc = 0.0;
    for (int i = threadIdx.x; i < kReduceBlocks; i += kThreads) acc += partial[i];
    sh[threadIdx.x] = acc;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (int(threadIdx.x) < s) sh[threadIdx.x] += sh[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        if (out_d) *out_d = sh[0];
        if (out_f) *out_f = static_cast<float>(sh[0]);
    }
}

const OccupancyKernel kReduceKernels[] = {
    {"sum_cols4 (bias-gradient column sums)", reinterpret_cast<const void*>(&sum_cols4), kThreads},
    {"reduce_stage1 (double sum)", reinterpret_cast<const void*>(&reduce_stage1<false>), kThreads},
};
const OccupancyEntries kReduceKernelsReg(kReduceKernels);

}  // namespace

// Two passes of sum_cols: row blocks into partials, then the partials of each
// slab. The row blocks are sized so that the first pass has about a thousand
// workgroups and the second adds at most 64 partials per lane. (One launch
// with a last-block-adds pattern measured 25 us instead of 2 x 3: making the
// partials visible across the XCDs' L2 caches costs an L2 write-back.)
// Slab o's sums go to out + o * out_slab; plan_slabs is the slab count the
// row blocks are sized for (the order of every sum depends on it).
int column_sums_plan(const float* x, int64_t slabs, int64_t rows, int64_t cols, int64_t ld,
                     int64_t x_slab, float* out, int64_t out_slab, int64_t plan_slabs,
                     hipStream_t s, float* out_second = nullptr) {
    if (slabs == 0 || cols == 0) return EHIP_OK;
    int cw = 1;
    while (cw < cols && cw < 64) cw *= 2;
    const int64_t tiles = ceil_div(cols, cw);
    if (tiles > 65535 || slabs > 65535) return fail(EHIP_EINVAL, "column_sums: too many columns");
    const int rl = kThreads / cw;
    int64_t blocks = ceil_div(1024, tiles * plan_slabs);
    const int64_t max_blocks = ceil_div(rows, 2 * rl);  // at least two rows per lane
    if (blocks > max_blocks) blocks = max_blocks;
    if (blocks > 64 * rl) blocks = 64 * rl;
    if (blocks < 1) blocks = 1;
    const int64_t rpb = ceil_div(rows, blocks);
    blocks = ceil_div(rows, rpb);
    // Wide rows of aligned float4s take sum_cols4 (same order, a quarter of
    // the column tiles).
    const bool vec = cols >= 256 && cols % 4 == 0 && ld % 4 == 0 && x_slab % 4 == 0 &&
                     aligned16(x);
    const unsigned tiles4 = unsigned(ceil_div(cols, 4 * 64));
    if (blocks == 1) {
        if (vec) {
            EHIP_LAUNCH("column_sums", sum_cols4, dim3(1, tiles4, unsigned(slabs)), dim3(kThreads),
                        0, s, x, out, out_second, rows, cols, ld, rows, x_slab, out_slab);
        } else {
            EHIP_LAUNCH("column_sums", sum_cols, dim3(1, unsigned(tiles), unsigned(slabs)),
                        dim3(kThreads), 0, s, x, out, out_second, rows, cols, ld, rows, x_slab,
                        out_slab, cw);
        }
        return EHIP_OK;
    }
    float* partial =
        static_cast<float*>(scratch(size_t(slabs * blocks * cols) * sizeof(float), 1));
    if (partial == nullptr) return EHIP_ENOMEM;
    if (vec) {
        EHIP_LAUNCH("column_sums_blocks", sum_cols4, dim3(unsigned(blocks), tiles4, unsigned(slabs)),
                    dim3(kThreads), 0, s, x, partial, nullptr, rows, cols, ld, rpb, x_slab,
                    blocks * cols);
        EHIP_LAUNCH("column_sums_final", sum_cols4, dim3(1, tiles4, unsigned(slabs)),
                    dim3(kThreads), 0, s, partial, out, out_second, blocks, cols, cols, blocks,
                    blocks * cols, out_slab);
        return EHIP_OK;
    }
    EHIP_LAUNCH("column_sums_blocks", sum_cols, dim3(unsigned(blocks), unsigned(tiles), unsigned(slabs)),
                dim3(kThreads), 0, s, x, partial, nullptr, rows, cols, ld, rpb, x_slab, blocks * cols,
                cw);
    EHIP_LAUNCH("column_sums_final", sum_cols, dim3(1, unsigned(tiles), unsigned(slabs)),
                dim3(kThreads), 0, s, partial, out, out_second, blocks, cols, cols, blocks,
                blocks * cols, out_slab, cw);
    return EHIP_OK;
}

int column_sums(const float* x, int64_t slabs, int64_t rows, int64_t cols, int64_t ld,
                int64_t x_slab, float* out, hipStream_t s) {
    return column_sums_plan(x, slabs, rows, cols, ld, x_slab, out, cols, slabs, s);
}

// Two single-slab column sums in the launches of one: slab 1 writes to out1
// (a separate array, passed to the kernels as such), and the row blocks are
// sized for one slab, so each sum has the order a column_sums call of its own
// gives.
int column_sums_pair(const float* x, int64_t rows, int64_t cols, int64_t ld, int64_t x_second,
                     float* out0, float* out1, hipStream_t s) {
    return column_sums_plan(x, 2, rows, cols, ld, x_second, out0, 0, 1, s, out1);
}

}  // namespace ehip

using namespace ehip;

extern "C" {

int ehip_sum_axis_f32(const float* x, float* out, int64_t outer, int64_t axis_len, int64_t inner,
                      void* stream) {
    EHIP_READY();
    if (outer < 0 || axis_len < 0 || inner < 0) return fail(EHIP_EINVAL, "sum_axis: bad shape");
    if (!x || !out) return fail(EHIP_EINVAL, "sum_axis: null pointer");
    const int64_t n_out = outer * inner;
    if (n_out == 0) return EHIP_OK;
    hipStream_t s = as_stream(stream);
    if (axis_len <= 64 || n_out >= 16384) {
        EHIP_LAUNCH("sum_axis", sum_axis_serial, dim3(unsigned(ceil_div(n_out, kThreads))),
                    dim3(kThreads), 0, s, x, out, axis_len, inner, n_out);
        return EHIP_OK;
    }
    // Here outer * inner < 16384, so the slabs fit the grid's z extent.
    return column_sums(x, outer, axis_len, inner, inner, axis_len * inner, out, s);
}

int ehip_reduce_sum_f32(const float* x, int64_t n, int squares, double* out_d, float* out_f,
                        void* stream) {
    EHIP_READY();
    if (n < 0) return fail(EHIP_EINVAL, "reduce_sum: negative size");
    if (!x && n > 0) return fail(EHIP_EINVAL, "reduce_sum: null input");
    hipStream_t s = as_stream(stream);
    double* partial = static_cast<double*>(scratch(kReduceBlocks * sizeof(double)));
    if (partial == nullptr) return EHIP_ENOMEM;
    if (squares) {
        EHIP_LAUNCH("reduce_sum_squares", reduce_stage1<true>, dim3(kReduceBlocks), dim3(kThreads),
                    0, s, x, n, partial);
    } else {
        EHIP_LAUNCH("reduce_sum", reduce_stage1<false>, dim3(kReduceBlocks), dim3(kThreads), 0, s,
                    x, n, partial);
    }
    EHIP_LAUNCH("reduce_sum_final", reduce_stage2, dim3(1), dim3(kThreads), 0, s, partial, out_d,
                out_f);
    return EHIP_OK;
}

}  // extern "C"
