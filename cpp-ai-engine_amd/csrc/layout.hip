// layout.hip -- index maps that move or gather floats: permute, the tiled
// last-two-axes transpose, im2col/col2im, max pooling and its scatter, and the
// row gather of Embedding with its ordered scatter-add.
//
// All of them are bit-exact with the reference CPU path: the moves copy bits,
// and every sum (col2im, the pooling backward, the row scatter) runs per
// output element in the order the reference's loops visit the contributions,
// starting from zero.

#include "common.hpp"

#include <cmath>

namespace ehip {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxDims = 8;

struct PermutePlan {
    int ndim;
    int64_t shape[kMaxDims];   // output shape
    int64_t stride[kMaxDims];  // source stride of each output axis
};

// One element per thread (src/tensor_ops.cpp:437-458).
__global__ __launch_bounds__(kThreads) void permute_scalar(const float* __restrict__ x,
                                                           float* __restrict__ out,
                                                           PermutePlan p, int64_t n) {
    const int64_t step = int64_t(gridDim.x) * kThreads;
    for (int64_t flat = int64_t(blockIdx.x) * kThreads + threadIdx.x; flat < n; flat += step) {
        int64_t rem = flat, off = 0;
        for (int d = p.ndim - 1; d >= 0; --d) {
            const int64_t c = rem % p.shape[d];
            rem /= p.shape[d];
            off += c * p.stride[d];
        }
        out[flat] = x[off];
    }
}

// The last axis stays contiguous (stride 1, length divisible by 4): one float4
// per thread. This is the attention head split/merge (0,2,1,3).
__global__ __launch_bounds__(kThreads) void permute_vec4(const float* __restrict__ x,
                                                         float* __restrict__ out, PermutePlan p,
                                                         int64_t nv) {
    const int64_t step = int64_t(gridDim.x) * kThreads;
    const int64_t last4 = p.shape[p.ndim - 1] >> 2;
    for (int64_t v = int64_t(blockIdx.x) * kThreads + threadIdx.x; v < nv; v += step) {
        int64_t rem = v / last4;
        int64_t off = (v % last4) << 2;
        for (int d = p.ndim - 2; d >= 0; --d) {
            const int64_t c = rem % p.shape[d];
            rem /= p.shape[d];
            off += c * p.stride[d];
        }
        reinterpret_cast<float4*>(out)[v] = *reinterpret_cast<const float4*>(x + off);
    }
}

// 64 x 64 tiles through LDS with a padded row, block 64 x 4 (src/tensor_ops.cpp:335-370).
constexpr int kT = 64;
__global__ __launch_bounds__(256) void transpose_tiled(const float* __restrict__ x,
                                                       float* __restrict__ out, int64_t rows,
                                                       int64_t cols, int64_t tiles_r,
                                                       int64_t tiles_c) {
    __shared__ float tile[kT][kT + 1];
    const int64_t t = blockIdx.x;
    const int64_t b = blockIdx.y;
    const int64_t tr = t / tiles_c, tc = t % tiles_c;
    const float* src = x + b * rows * cols;
    float* dst = out + b * rows * cols;
    const int tx = threadIdx.x, ty = threadIdx.y;
    const int64_t c = tc * kT + tx;
    for (int i = ty; i < kT; i += 4) {
        const int64_t r = tr * kT + i;
        if (r < rows && c < cols) tile[i][tx] = src[r * cols + c];
    }
    __syncthreads();
    const int64_t oc = tr * kT + tx;  // column of the output = row of the input
    for (int i = ty; i < kT; i += 4) {
        const int64_t orow = tc * kT + i;
        if (orow < cols && oc < rows) dst[orow * rows + oc] = tile[tx][i];
    }
}

// One thread per column element, output-contiguous (src/conv.cpp:61-150).
__global__ __launch_bounds__(kThreads) void im2col_kernel(const float* __restrict__ x,
                                                          float* __restrict__ cols,
                                                          ehip_window_t w, int64_t n) {
    const int64_t K = w.channels * w.kernel_h * w.kernel_w;
    const int64_t step = int64_t(gridDim.x) * kThreads;
    for (int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x; e < n; e += step) {
        const int64_t row = e / K, col = e % K;
        const int64_t ow = row % w.out_w;
        const int64_t t = row / w.out_w;
        const int64_t oh = t % w.out_h, nn = t / w.out_h;
        const int64_t j = col % w.kernel_w;
        const int64_t t2 = col / w.kernel_w;
        const int64_t i = t2 % w.kernel_h, c = t2 / w.kernel_h;
        const int64_t h = oh * w.stride + i - w.padding;
        const int64_t v = ow * w.stride + j - w.padding;
        float val = 0.0f;
        if (h >= 0 && h < w.height && v >= 0 && v < w.width)
            val = x[((nn * w.channels + c) * w.height + h) * w.width + v];
        cols[e] = val;
    }
}

// One thread per input pixel, summing its windows with oh then ow ascending
// from zero: the per-pixel order of src/conv.cpp:183-214.
__global__ __launch_bounds__(kThreads) void col2im_kernel(const float* __restrict__ cols,
                                                          float* __restrict__ x, ehip_window_t w,
                                                          int64_t n) {
    const int64_t K = w.channels * w.kernel_h * w.kernel_w;
    const int64_t step = int64_t(gridDim.x) * kThreads;
    for (int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x; e < n; e += step) {
        const int64_t v = e % w.width;
        int64_t t = e / w.width;
        const int64_t h = t % w.height;
        t /= w.height;
        const int64_t c = t % w.channels, nn = t / w.channels;
        int64_t oh_lo, oh_hi, ow_lo, ow_hi;
        covering(h, w.padding, w.kernel_h, w.stride, w.out_h, oh_lo, oh_hi);
        covering(v, w.padding, w.kernel_w, w.stride, w.out_w, ow_lo, ow_hi);
        float acc = 0.0f;
        for (int64_t oh = oh_lo; oh <= oh_hi; ++oh) {
            const int64_t i = h + w.padding - oh * w.stride;
            for (int64_t ow = ow_lo; ow <= ow_hi; ++ow) {
                const int64_t j = v + w.padding - ow * w.stride;
                const int64_t row = (nn * w.out_h + oh) * w.out_w + ow;
                acc += cols[row * K + (c * w.kernel_h + i) * w.kernel_w + j];
            }
        }
        x[e] = acc;
    }
}

// One thread per output; the first strict maximum in window order wins
// (src/conv.cpp:410-442). Idx is int32_t, or float for the reference's float
// argmax storage (exact for flat indices below 2^24).
template <typename Idx>
__global__ __launch_bounds__(kThreads) void maxpool_kernel(const float* __restrict__ x,
                                                           float* __restrict__ y,
                                                           Idx* __restrict__ argmax,
                                                           ehip_window_t w, int64_t n) {
    const int64_t step = int64_t(gridDim.x) * kThreads;
    for (int64_t o = int64_t(blockIdx.x) * kThreads + threadIdx.x; o < n; o += step) {
        const int64_t ow = o % w.out_w;
        int64_t t = o / w.out_w;
        const int64_t oh = t % w.out_h;
        const int64_t plane = t / w.out_h;  // n * C + c
        float best = -INFINITY;
        int64_t best_idx = 0;
        bool found = false;
        for (int64_t i = 0; i < w.kernel_h; ++i) {
            const int64_t h = oh * w.stride + i - w.padding;
            if (h < 0 || h >= w.height) continue;
            for (int64_t j = 0; j < w.kernel_w; ++j) {
                const int64_t v = ow * w.stride + j - w.padding;
                if (v < 0 || v >= w.width) continue;
                const int64_t idx = (plane * w.height + h) * w.width + v;
                const float xv = x[idx];
                if (!found || xv > best) {
                    best = xv;
                    best_idx = idx;
                    found = true;
                }
            }
        }
        y[o] = best;
        argmax[o] = static_cast<Idx>(best_idx);
    }
}

// One thread per input pixel: the gradients of the windows that chose it, in
// output order from zero (src/conv.cpp:461-469 visits outputs ascending).
template <typename Idx>
__global__ __launch_bounds__(kThreads) void maxpool_backward_kernel(
    const Idx* __restrict__ argmax, const float* __restrict__ g, float* __restrict__ dx,
    ehip_window_t w, int64_t n) {
    const int64_t step = int64_t(gridDim.x) * kThreads;
    for (int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x; e < n; e += step) {
        const int64_t v = e % w.width;
        int64_t t = e / w.width;
        const int64_t h = t % w.height;
        const int64_t plane = t / w.height;
        int64_t oh_lo, oh_hi, ow_lo, ow_hi;
        covering(h, w.padding, w.kernel_h, w.stride, w.out_h, oh_lo, oh_hi);
        covering(v, w.padding, w.kernel_w, w.stride, w.out_w, ow_lo, ow_hi);
        float acc = 0.0f;
        for (int64_t oh = oh_lo; oh <= oh_hi; ++oh)
            for (int64_t ow = ow_lo; ow <= ow_hi; ++ow) {
                const int64_t o = (plane * w.out_h + oh) * w.out_w + ow;
                if (argmax[o] == static_cast<Idx>(e)) acc += g[o];
            }
        dx[e] = acc;
    }
}

// Non-overlapping windows (kernel == stride, no padding), the usual pooling
// layer: 32-bit index math (every entry point caps the input below 2^31
// elements) and, in the backward pass, one thread per output that writes its
// whole window -- each input is covered by at most one window, so the
// gradient is 0 + g at the window's argmax and 0 elsewhere, which is what the
// covering-window sum of maxpool_backward_kernel gives. Inputs past the last
// whole window (H or W not a multiple of k) are written by the last row or
// column of windows. The forward keeps the first strict maximum in window
// order.
template <typename Idx>
__global__ __launch_bounds__(kThreads) void maxpool_tiles_kernel(const float* __restrict__ x,
                                                                 float* __restrict__ y,
                                                                 Idx* __restrict__ argmax,
                                                                 uint32_t width, uint32_t height,
                                                                 uint32_t out_w, uint32_t out_h,
                                                                 uint32_t k, uint32_t n) {
    const uint32_t step = gridDim.x * kThreads;
    for (uint32_t o = blockIdx.x * kThreads + threadIdx.x; o < n; o += step) {
        const uint32_t ow = o % out_w, t = o / out_w;
        const uint32_t oh = t % out_h, plane = t / out_h;
        const uint32_t base = (plane * height + oh * k) * width + ow * k;
        float best = x[base];
        uint32_t best_idx = base;
        for (uint32_t i = 0; i < k; ++i)
            for (uint32_t j = 0; j < k; ++j) {
                const uint32_t idx = base + i * width + j;
                const float xv = x[idx];
                if (xv > best) {
                    best = xv;
                    best_idx = idx;
                }
            }
        y[o] = best;
        argmax[o] = static_cast<Idx>(best_idx);
    }
}

template <typename Idx>
__global__ __launch_bounds__(kThreads) void maxpool_tiles_backward_kernel(
    const Idx* __restrict__ argmax, const float* __restrict__ g, float* __restrict__ dx,
    uint32_t width, uint32_t height, uint32_t out_w, uint32_t out_h, uint32_t k, uint32_t n) {
    const uint32_t step = gridDim.x * kThreads;
    for (uint32_t o = blockIdx.x * kThreads + threadIdx.x; o < n; o += step) {
        const uint32_t ow = o % out_w, t = o / out_w;
        const uint32_t oh = t % out_h, plane = t / out_h;
        const Idx am = argmax[o];
        const float gv = 0.0f + g[o];
        const uint32_t h0 = oh * k, v0 = ow * k;
        const uint32_t h1 = oh + 1 == out_h ? height : h0 + k;
        const uint32_t v1 = ow + 1 == out_w ? width : v0 + k;
        for (uint32_t h = h0; h < h1; ++h)
            for (uint32_t v = v0; v < v1; ++v) {
                const uint32_t idx = (plane * height + h) * width + v;
                const bool in = h < h0 + k && v < v0 + k;
                dx[idx] = (in && static_cast<Idx>(idx) == am) ? gv : 0.0f;
            }
    }
}

// 2 x 2 windows on even-sized planes: each window row is one aligned float2.
template <typename Idx>
__global__ __launch_bounds__(kThreads) void maxpool_2x2_kernel(const float* __restrict__ x,
                                                               float* __restrict__ y,
                                                               Idx* __restrict__ argmax,
                                                               uint32_t width, uint32_t out_w,
                                                               uint32_t n) {
    const uint32_t step = gridDim.x * kThreads;
    for (uint32_t o = blockIdx.x * kThreads + threadIdx.x; o < n; o += step) {
        const uint32_t ow = o % out_w, row = o / out_w;  // row = plane * out_h + oh
        const uint32_t base = 2 * row * width + 2 * ow;
        const float2 a = *reinterpret_cast<const float2*>(x + base);
        const float2 b = *reinterpret_cast<const float2*>(x + base + width);
        float best = a.x;
        uint32_t idx = base;
        if (a.y > best) { best = a.y; idx = base + 1; }
        if (b.x > best) { best = b.x; idx = base + width; }
        if (b.y > best) { best = b.y; idx = base + width + 1; }
        y[o] = best;
        argmax[o] = static_cast<Idx>(idx);
    }
}

template <typename Idx>
__global__ __launch_bounds__(kThreads) void maxpool_2x2_backward_kernel(
    const Idx* __restrict__ argmax, const float* __restrict__ g, float* __restrict__ dx,
    uint32_t width, uint32_t out_w, uint32_t n) {
    const uint32_t step = gridDim.x * kThreads;
    for (uint32_t o = blockIdx.x * kThreads + threadIdx.x; o < n; o += step) {
        const uint32_t ow = o % out_w, row = o / out_w;
        const uint32_t base = 2 * row * width + 2 * ow;
        const Idx am = argmax[o];
        const float gv = 0.0f + g[o];
        float2 a, b;
        a.x = static_cast<Idx>(base) == am ? gv : 0.0f;
        a.y = static_cast<Idx>(base + 1) == am ? gv : 0.0f;
        b.x = static_cast<Idx>(base + width) == am ? gv : 0.0f;
        b.y = static_cast<Idx>(base + width + 1) == am ? gv : 0.0f;
        *reinterpret_cast<float2*>(dx + base) = a;
        *reinterpret_cast<float2*>(dx + base + width) = b;
    }
}

bool even_2x2(const ehip_window_t* w, const void* p, const void* q) {
    return w->kernel_h == 2 && w->height % 2 == 0 && w->width % 2 == 0 &&
           reinterpret_cast<uintptr_t>(p) % 8 == 0 && reinterpret_cast<uintptr_t>(q) % 8 == 0;
}

bool tiled_window(const ehip_window_t* w) {
    return w->kernel_h == w->kernel_w && w->stride == w->kernel_h && w->padding == 0 &&
           w->out_h > 0 && w->out_w > 0;
}

// Row gather; an out-of-range index yields NaN rather than a wild read.
__global__ __launch_bounds__(kThreads) void select_rows_kernel(const float* __restrict__ x,
                                                               const int32_t* __restrict__ idx,
                                                               float* __restrict__ out,
                                                               int64_t row_size, int64_t n_rows,
                                                               int64_t n) {
    const int64_t step = int64_t(gridDim.x) * kThreads;
    for (int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x; e < n; e += step) {
        const int64_t i = e / row_size, j = e % row_size;
        const int64_t r = idx[i];
        out[e] = (r >= 0 && r < n_rows) ? x[r * row_size + j] : NAN;
    }
}

// CSR scatter-add: every destination element sums its sources in list order.
// kScatterBatch positions are read at a time, then their source rows, then added
// in order: two load round trips per batch instead of two per source row.
constexpr int kScatterBatch = 8;

__global__ __launch_bounds__(kThreads) void scatter_add_rows_kernel(
    const float* __restrict__ g, const int32_t* __restrict__ row_ptr,
    const int32_t* __restrict__ pos, float* __restrict__ dx, int64_t row_size, int64_t n_src,
    int64_t n, int accumulate) {
    const int64_t step = int64_t(gridDim.x) * kThreads;
    for (int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x; e < n; e += step) {
        const int64_t r = e / row_size, j = e % row_size;
        const int32_t p0 = row_ptr[r], p1 = row_ptr[r + 1];
        float acc = 0.0f;
        for (int32_t p = p0; p < p1; p += kScatterBatch) {
            int64_t src[kScatterBatch];
#pragma unroll
            for (int u = 0; u < kScatterBatch; ++u) src[u] = p + u < p1 ? pos[p + u] : 0;
            float v[kScatterBatch];
#pragma unroll
            for (int u = 0; u < kScatterBatch; ++u)
                v[u] = p + u >= p1 ? 0.0f
                       : (src[u] >= 0 && src[u] < n_src) ? g[src[u] * row_size + j]
                                                         : NAN;
#pragma unroll
            for (int u = 0; u < kScatterBatch; ++u)
                if (p + u < p1) acc += v[u];
        }
        dx[e] = accumulate ? dx[e] + acc : acc;
    }
}

unsigned grid_for(int64_t n) {
    int64_t g = ceil_div(n, kThreads);
    if (g > 131072) g = 131072;
    if (g < 1) g = 1;
    return unsigned(g);
}

template <typename Idx>
int maxpool_forward(const char* name, const float* x, float* y, Idx* argmax,
                    const ehip_window_t* w, int64_t max_in, void* stream) {
    EHIP_READY();
    if (int rc = check_window(name, w)) return rc;
    if (!x || !y || !argmax) return fail(EHIP_EINVAL, "%s: null pointer", name);
    const int64_t n_in = w->batch * w->channels * w->height * w->width;
    if (n_in > max_in)
        return fail(EHIP_EINVAL, "%s: %lld input elements beyond exact indices (%lld)", name,
                    (long long)n_in, (long long)max_in);
    const int64_t n = w->batch * w->channels * w->out_h * w->out_w;
    if (n == 0) return EHIP_OK;
    if (tiled_window(w) && even_2x2(w, x, x)) {
        EHIP_LAUNCH(name, maxpool_2x2_kernel<Idx>, dim3(grid_for(n)), dim3(kThreads), 0,
                    as_stream(stream), x, y, argmax, uint32_t(w->width), uint32_t(w->out_w),
                    uint32_t(n));
        return EHIP_OK;
    }
    if (tiled_window(w)) {
        EHIP_LAUNCH(name, maxpool_tiles_kernel<Idx>, dim3(grid_for(n)), dim3(kThreads), 0,
                    as_stream(stream), x, y, argmax, uint32_t(w->width), uint32_t(w->height),
                    uint32_t(w->out_w), uint32_t(w->out_h), uint32_t(w->kernel_h), uint32_t(n));
        return EHIP_OK;
    }
    EHIP_LAUNCH(name, maxpool_kernel<Idx>, dim3(grid_for(n)), dim3(kThreads), 0,
                as_stream(stream), x, y, argmax, *w, n);
    return EHIP_OK;
}

template <typename Idx>
int maxpool_backward(const char* name, const Idx* argmax, const float* g, float* dx,
                     const ehip_window_t* w, int64_t max_in, void* stream) {
    EHIP_READY();
    if (int rc = check_window(name, w)) return rc;
    if (!argmax || !g || !dx) return fail(EHIP_EINVAL, "%s: null pointer", name);
    const int64_t n = w->batch * w->channels * w->height * w->width;
    if (n > max_in)
        return fail(EHIP_EINVAL, "%s: %lld input elements beyond exact indices (%lld)", name,
                    (long long)n, (long long)max_in);
    if (n == 0) return EHIP_OK;
    if (tiled_window(w) && even_2x2(w, dx, dx)) {
        const int64_t n_out = w->batch * w->channels * w->out_h * w->out_w;
        EHIP_LAUNCH(name, maxpool_2x2_backward_kernel<Idx>, dim3(grid_for(n_out)), dim3(kThreads),
                    0, as_stream(stream), argmax, g, dx, uint32_t(w->width), uint32_t(w->out_w),
                    uint32_t(n_out));
        return EHIP_OK;
    }
    if (tiled_window(w)) {
        const int64_t n_out = w->batch * w->channels * w->out_h * w->out_w;
        EHIP_LAUNCH(name, maxpool_tiles_backward_kernel<Idx>, dim3(grid_for(n_out)),
                    dim3(kThreads), 0, as_stream(stream), argmax, g, dx, uint32_t(w->width),
                    uint32_t(w->height), uint32_t(w->out_w), uint32_t(w->out_h),
                    uint32_t(w->kernel_h), uint32_t(n_out));
        return EHIP_OK;
    }
    EHIP_LAUNCH(name, maxpool_backward_kernel<Idx>, dim3(grid_for(n)), dim3(kThreads), 0,
                as_stream(stream), argmax, g, dx, *w, n);
    return EHIP_OK;
}

const OccupancyKernel kLayoutKernels[] = {
    {"transpose_tiled", reinterpret_cast<const void*>(&transpose_tiled), kT * 4},
    {"maxpool_2x2_kernel", reinterpret_cast<const void*>(&maxpool_2x2_kernel<int32_t>), kThreads},
    {"im2col_kernel", reinterpret_cast<const void*>(&im2col_kernel), kThreads},
};
const OccupancyEntries kLayoutKernelsReg(kLayoutKernels);

}  // namespace

int check_window(const char* name, const ehip_window_t* w) {
    if (w == nullptr) return fail(EHIP_EINVAL, "%s: null window", name);
    if (w->batch < 0 || w->channels <= 0 || w->height <= 0 || w->width <= 0 ||
        w->kernel_h <= 0 || w->kernel_w <= 0 || w->stride <= 0 || w->padding < 0)
        return fail(EHIP_EINVAL, "%s: bad window geometry", name);
    const int64_t oh = (w->height + 2 * w->padding - w->kernel_h) / w->stride + 1;
    const int64_t ow = (w->width + 2 * w->padding - w->kernel_w) / w->stride + 1;
    if (w->height + 2 * w->padding < w->kernel_h || w->width + 2 * w->padding < w->kernel_w ||
        oh != w->out_h || ow != w->out_w)
        return fail(EHIP_EINVAL, "%s: out_h/out_w do not match the window", name);
    return EHIP_OK;
}

}  // namespace ehip

using namespace ehip;

extern "C" {

int ehip_permute_f32(const float* x, float* out, int ndim, const int64_t* out_shape,
                     const int64_t* src_strides, void* stream) {
    EHIP_READY();
    if (ndim < 1 || ndim > kMaxDims) return fail(EHIP_EINVAL, "permute: ndim %d out of 1..8", ndim);
    if (!x || !out || !out_shape || !src_strides) return fail(EHIP_EINVAL, "permute: null pointer");
    PermutePlan p{};
    p.ndim = ndim;
    int64_t n = 1;
    for (int d = 0; d < ndim; ++d) {
        if (out_shape[d] < 0 || src_strides[d] < 0)
            return fail(EHIP_EINVAL, "permute: negative extent or stride");
        p.shape[d] = out_shape[d];
        p.stride[d] = src_strides[d];
        n *= out_shape[d];
    }
    if (n == 0) return EHIP_OK;
    hipStream_t s = as_stream(stream);
    const bool vec = src_strides[ndim - 1] == 1 && out_shape[ndim - 1] % 4 == 0 && aligned16(x) &&
                     aligned16(out) && [&] {
                         for (int d = 0; d < ndim - 1; ++d)
                             if (src_strides[d] % 4 != 0) return false;
                         return true;
                     }();
    if (vec) {
        EHIP_LAUNCH("permute", permute_vec4, dim3(grid_for(n / 4)), dim3(kThreads), 0, s, x, out,
                    p, n / 4);
    } else {
        EHIP_LAUNCH("permute", permute_scalar, dim3(grid_for(n)), dim3(kThreads), 0, s, x, out, p,
                    n);
    }
    return EHIP_OK;
}

int ehip_transpose_f32(const float* x, float* out, int64_t batch, int64_t rows, int64_t cols,
                       void* stream) {
    EHIP_READY();
    if (batch < 0 || rows < 0 || cols < 0) return fail(EHIP_EINVAL, "transpose: bad shape");
    if (!x || !out) return fail(EHIP_EINVAL, "transpose: null pointer");
    if (batch == 0 || rows == 0 || cols == 0) return EHIP_OK;
    const int64_t tr = ceil_div(rows, kT), tc = ceil_div(cols, kT);
    if (tr * tc > 0x7fffffff) return fail(EHIP_EINVAL, "transpose: too many tiles");
    // The batch is the grid's y extent (at most 65535): longer batches run as
    // several launches over consecutive matrices.
    const int64_t mat = rows * cols;
    for (int64_t z0 = 0; z0 < batch; z0 += 65535) {
        const int64_t nz = batch - z0 < 65535 ? batch - z0 : 65535;
        EHIP_LAUNCH("transpose", transpose_tiled, dim3(unsigned(tr * tc), unsigned(nz)),
                    dim3(kT, 4), 0, as_stream(stream), x + z0 * mat, out + z0 * mat, rows, cols,
                    tr, tc);
    }
    return EHIP_OK;
}

int ehip_im2col_f32(const float* x, float* cols, const ehip_window_t* w, void* stream) {
    EHIP_READY();
    if (int rc = check_window("im2col", w)) return rc;
    if (!x || !cols) return fail(EHIP_EINVAL, "im2col: null pointer");
    const int64_t n = w->batch * w->out_h * w->out_w * w->channels * w->kernel_h * w->kernel_w;
    if (n == 0) return EHIP_OK;
    EHIP_LAUNCH("im2col", im2col_kernel, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream),
                x, cols, *w, n);
    return EHIP_OK;
}

int ehip_col2im_f32(const float* cols, float* x, const ehip_window_t* w, void* stream) {
    EHIP_READY();
    if (int rc = check_window("col2im", w)) return rc;
    if (!x || !cols) return fail(EHIP_EINVAL, "col2im: null pointer");
    const int64_t n = w->batch * w->channels * w->height * w->width;
    if (n == 0) return EHIP_OK;
    EHIP_LAUNCH("col2im", col2im_kernel, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream),
                cols, x, *w, n);
    return EHIP_OK;
}

int ehip_maxpool_f32(const float* x, float* y, int32_t* argmax, const ehip_window_t* w,
                     void* stream) {
    return maxpool_forward("maxpool", x, y, argmax, w, 0x7fffffff, stream);
}

int ehip_maxpool_backward_f32(const int32_t* argmax, const float* g, float* dx,
                              const ehip_window_t* w, void* stream) {
    return maxpool_backward("maxpool_backward", argmax, g, dx, w, 0x7fffffff, stream);
}

int ehip_maxpool_fidx_f32(const float* x, float* y, float* argmax, const ehip_window_t* w,
                          void* stream) {
    return maxpool_forward("maxpool_fidx", x, y, argmax, w, int64_t(1) << 24, stream);
}

int ehip_maxpool_backward_fidx_f32(const float* argmax, const float* g, float* dx,
                                   const ehip_window_t* w, void* stream) {
    return maxpool_backward("maxpool_backward_fidx", argmax, g, dx, w, int64_t(1) << 24, stream);
}

int ehip_select_rows_f32(const float* x, const int32_t* idx, float* out, int64_t n_idx,
                         int64_t row_size, int64_t n_rows, void* stream) {
    EHIP_READY();
    if (n_idx < 0 || row_size < 0 || n_rows < 0) return fail(EHIP_EINVAL, "select_rows: bad shape");
    if (!x || !idx || !out) return fail(EHIP_EINVAL, "select_rows: null pointer");
    const int64_t n = n_idx * row_size;
    if (n == 0) return EHIP_OK;
    EHIP_LAUNCH("select_rows", select_rows_kernel, dim3(grid_for(n)), dim3(kThreads), 0,
                as_stream(stream), x, idx, out, row_size, n_rows, n);
    return EHIP_OK;
}

int ehip_scatter_add_rows_f32(const float* g, const int32_t* row_ptr, const int32_t* pos,
                              float* dx, int64_t n_rows, int64_t row_size, int64_t n_src,
                              int accumulate, void* stream) {
    EHIP_READY();
    if (n_rows < 0 || row_size < 0) return fail(EHIP_EINVAL, "scatter_add_rows: bad shape");
    if (!g || !row_ptr || !pos || !dx) return fail(EHIP_EINVAL, "scatter_add_rows: null pointer");
    const int64_t n = n_rows * row_size;
    if (n == 0) return EHIP_OK;
    EHIP_LAUNCH("scatter_add_rows", scatter_add_rows_kernel, dim3(grid_for(n)), dim3(kThreads), 0,
                as_stream(stream), g, row_ptr, pos, dx, row_size, n_src, n, accumulate);
    return EHIP_OK;
}

}  // extern "C"
