// reduce.hip -- sum over one axis (bias gradients, fold_leading) and the
// whole-buffer double-precision sums behind Tensor::sum()/mean().
//
// No atomics: every sum has a fixed order that depends only on the shape, so
// two runs on the same data agree bit for bit.

#include "common.hpp"

namespace ehip {
namespace {

constexpr int kThreads = 256;

// One thread per output element, axis ascending from zero: exactly the order
// of src/tensor.cpp:347-356, so the result is bit-identical to the CPU.
__global__ __launch_bounds__(kThreads) void sum_axis_serial(const float* __restrict__ x,
                                                            float* __restrict__ out,
                                                            int64_t axis_len, int64_t inner,
                                                            int64_t n_out) {
    const int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= n_out) return;
    const int64_t o = e / inner, i = e % inner;
    const float* p = x + o * axis_len * inner + i;
    float acc = 0.0f;
    for (int64_t a = 0; a < axis_len; ++a) acc += p[a * inner];
    out[e] = acc;
}

// Stage 1 of the chunked sum: partial[o][c][i] = serial sum of the c-th chunk
// of the axis.
__global__ __launch_bounds__(kThreads) void sum_axis_chunks(const float* __restrict__ x,
                                                            float* __restrict__ partial,
                                                            int64_t axis_len, int64_t inner,
                                                            int64_t chunks, int64_t chunk_len,
                                                            int64_t n_part) {
    const int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= n_part) return;
    const int64_t i = e % inner;
    const int64_t t = e / inner;
    const int64_t c = t % chunks, o = t / chunks;
    const int64_t a0 = c * chunk_len;
    int64_t a1 = a0 + chunk_len;
    if (a1 > axis_len) a1 = axis_len;
    const float* p = x + o * axis_len * inner + i;
    float acc = 0.0f;
    for (int64_t a = a0; a < a1; ++a) acc += p[a * inner];
    partial[e] = acc;
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

}  // namespace
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
    // Enough chunks to give ~64k threads, each chunk at least 32 long.
    int64_t chunks = ceil_div(65536, n_out);
    if (chunks > axis_len / 32) chunks = axis_len / 32;
    if (chunks > 1024) chunks = 1024;
    if (chunks < 2) chunks = 2;
    const int64_t chunk_len = ceil_div(axis_len, chunks);
    chunks = ceil_div(axis_len, chunk_len);
    const int64_t n_part = n_out * chunks;
    float* partial = static_cast<float*>(scratch(size_t(n_part) * sizeof(float)));
    if (partial == nullptr) return EHIP_ENOMEM;
    EHIP_LAUNCH("sum_axis_chunks", sum_axis_chunks, dim3(unsigned(ceil_div(n_part, kThreads))),
                dim3(kThreads), 0, s, x, partial, axis_len, inner, chunks, chunk_len, n_part);
    EHIP_LAUNCH("sum_axis", sum_axis_serial, dim3(unsigned(ceil_div(n_out, kThreads))),
                dim3(kThreads), 0, s, partial, out, chunks, inner, n_out);
    return EHIP_OK;
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
