// conv.hip -- direct 2-D convolution for narrow layers: forward, input
// gradient, and the fused weight + bias gradient, with no im2col columns in
// HBM and the output written straight in (N, C, H, W).
//
// The reference composes Conv2d::forward from im2col, a product with the
// transposed weight, a broadcast bias add and a permute (src/conv.cpp:280-338);
// autograd derives the backward from those four nodes. Here each direction is
// one kernel (the weight gradient two: per-chunk partials and their ordered
// reduction), so a conv layer costs three to four launches per step instead of
// ten, and the columns (kH * kW times the input) never touch HBM.
//
// Exactness. The forward sums the K = C_in kH kW products of each output in
// k-ascending order from zero, skipping zero inputs, then adds the bias: the
// reference's i-k-j loop with its zero skip (src/tensor_ops.cpp:553-560) and
// its separately rounded bias add, so the result is bit-identical. The input
// gradient computes, for every window that covers a pixel (oh then ow
// ascending), the C_out-term dot product of that column entry (co ascending,
// zero gradients skipped) and adds those in order from zero: the reference's
// product dcols = g W followed by col2im (src/conv.cpp:183-214), bit for bit.
// The weight and bias gradients are sums over all N oH oW pixels; they are
// split into chunks and reduced in a fixed order (deterministic, within the
// K-term tolerance of the reference's serial sums).
//
// Narrow means out_channels * C_in * kH * kW <= 8192 (the weights fit in
// 32 KiB of LDS): the cfg2 layers (8 x 9 and 16 x 72). Wider layers go through
// im2col and the MFMA GEMM, where the product dominates.

#include "common.hpp"

#include <algorithm>

namespace ehip {
namespace {

constexpr int kThreads = 256;
constexpr int kCoGroup = 4;              // output channels per thread in the forward
constexpr int64_t kMaxWeights = 8192;    // out_channels * K
constexpr size_t kMaxLds = 64 * 1024;    // bytes of LDS per weight-gradient block

struct Geo {
    int n, cin, h, w, kh, kw, stride, pad, oh, ow, cout, k;
};

Geo geo_of(const ehip_window_t& win, int64_t cout) {
    Geo g;
    g.n = int(win.batch);
    g.cin = int(win.channels);
    g.h = int(win.height);
    g.w = int(win.width);
    g.kh = int(win.kernel_h);
    g.kw = int(win.kernel_w);
    g.stride = int(win.stride);
    g.pad = int(win.padding);
    g.oh = int(win.out_h);
    g.ow = int(win.out_w);
    g.cout = int(cout);
    g.k = g.cin * g.kh * g.kw;
    return g;
}

// One thread per output pixel and group of kCoGroup output channels; the group
// is blockIdx.y, so every weight read is uniform across the block (scalar
// loads). x is read through the caches, kH kW times per pixel at most.
__global__ __launch_bounds__(kThreads) void conv_forward_direct(const float* __restrict__ x,
                                                                const float* __restrict__ wt,
                                                                const float* __restrict__ bias,
                                                                float* __restrict__ out, Geo g) {
    const int64_t pixels = int64_t(g.n) * g.oh * g.ow;
    const int64_t m = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    const int co0 = int(blockIdx.y) * kCoGroup;
    if (m >= pixels) return;
    const int ow = int(m % g.ow);
    const int64_t t = m / g.ow;
    const int oh = int(t % g.oh);
    const int n = int(t / g.oh);
    float c[kCoGroup];
#pragma unroll
    for (int q = 0; q < kCoGroup; ++q) c[q] = 0.0f;
    const float* xn = x + int64_t(n) * g.cin * g.h * g.w;
    int k = 0;
    for (int ci = 0; ci < g.cin; ++ci) {
        const float* xc = xn + int64_t(ci) * g.h * g.w;
        for (int i = 0; i < g.kh; ++i) {
            const int h = oh * g.stride + i - g.pad;
            for (int j = 0; j < g.kw; ++j, ++k) {
                const int v = ow * g.stride + j - g.pad;
                const float a = (h >= 0 && h < g.h && v >= 0 && v < g.w) ? xc[h * g.w + v] : 0.0f;
#pragma unroll
                for (int q = 0; q < kCoGroup; ++q) {
                    if (co0 + q < g.cout) {
                        const float b = wt[int64_t(co0 + q) * g.k + k];
                        c[q] = (a != 0.0f) ? c[q] + a * b : c[q];
                    }
                }
            }
        }
    }
    const int64_t plane = int64_t(g.oh) * g.ow;
    float* on = out + int64_t(n) * g.cout * plane + int64_t(oh) * g.ow + ow;
#pragma unroll
    for (int q = 0; q < kCoGroup; ++q) {
        const int co = co0 + q;
        if (co < g.cout) on[int64_t(co) * plane] = bias ? c[q] + bias[co] : c[q];
    }
}

// One thread per input element (n, ci, h, w); the weights sit in LDS.
__global__ __launch_bounds__(kThreads) void conv_backward_input_direct(
    const float* __restrict__ gout, const float* __restrict__ wt, float* __restrict__ dx, Geo g) {
    extern __shared__ float ws[];
    const int nw = g.cout * g.k;
    for (int e = threadIdx.x; e < nw; e += kThreads) ws[e] = wt[e];
    __syncthreads();
    const int64_t n_in = int64_t(g.n) * g.cin * g.h * g.w;
    const int64_t plane = int64_t(g.oh) * g.ow;
    const int64_t step = int64_t(gridDim.x) * kThreads;
    for (int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x; e < n_in; e += step) {
        const int v = int(e % g.w);
        int64_t t = e / g.w;
        const int h = int(t % g.h);
        t /= g.h;
        const int ci = int(t % g.cin);
        const int n = int(t / g.cin);
        int64_t oh_lo, oh_hi, ow_lo, ow_hi;
        covering(h, g.pad, g.kh, g.stride, g.oh, oh_lo, oh_hi);
        covering(v, g.pad, g.kw, g.stride, g.ow, ow_lo, ow_hi);
        const float* gn = gout + int64_t(n) * g.cout * plane;
        const float* wc = ws + ci * g.kh * g.kw;
        float acc = 0.0f;
        for (int64_t oh = oh_lo; oh <= oh_hi; ++oh) {
            const int i = int(h + g.pad - oh * g.stride);
            for (int64_t ow = ow_lo; ow <= ow_hi; ++ow) {
                const int j = int(v + g.pad - ow * g.stride);
                const float* gp = gn + oh * g.ow + ow;
                const float* wp = wc + i * g.kw + j;
                float d = 0.0f;
                for (int co = 0; co < g.cout; ++co) {
                    const float gv = gp[int64_t(co) * plane];
                    d = (gv != 0.0f) ? d + gv * wp[co * g.k] : d;
                }
                acc += d;
            }
        }
        dx[e] = acc;
    }
}

// Staging helper: copies n elements into LDS, U independent global loads in
// flight per thread before any LDS store. at(e, slot) returns element e (doing
// its own bounds checks) and sets its LDS slot in `base`.
template <int U, class At>
__device__ __forceinline__ void stage(int n, float* base, At at) {
    for (int first = 0; first < n; first += U * kThreads) {
        float v[U];
        int slot[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = first + u * kThreads + int(threadIdx.x);
            slot[u] = -1;
            v[u] = e < n ? at(e, slot[u]) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (slot[u] >= 0) base[slot[u]] = v[u];
    }
}

// LDS pitches: odd, so rows, planes and channels that are a power-of-two
// multiple apart do not fall in the same bank.
__device__ __forceinline__ int odd(int v) { return v | 1; }

// Forward over a tile of `rows` output rows of one image and CG output
// channels (blockIdx.y). The input rows the tile reads, zero-padded on every
// side, and the weights of the CG channels (laid out [k][CG], one 128-bit
// broadcast read per k) sit in LDS; each thread then computes whole pixels
// (all CG channels) from LDS in the same k order and with the same zero skip
// as conv_forward_direct. The skip is a select after an unconditional
// multiply-add, so no LDS read waits behind a branch. KH = KW = 0 reads the
// kernel size at run time; 3 x 3 is compiled unrolled. blockIdx.x = n * tiles
// + tile.
template <int CG, int KH, int KW>
__global__ __launch_bounds__(kThreads) void conv_forward_tiled(const float* __restrict__ x,
                                                               const float* __restrict__ wt,
                                                               const float* __restrict__ bias,
                                                               float* __restrict__ out, Geo g,
                                                               int rows, int tiles) {
    extern __shared__ __align__(16) float sm[];
    const int kh = KH ? KH : g.kh, kw = KW ? KW : g.kw;
    const int n = int(blockIdx.x) / tiles, tile = int(blockIdx.x) % tiles;
    const int co0 = int(blockIdx.y) * CG;
    const int oh0 = tile * rows;
    const int oh1 = min(oh0 + rows, g.oh);
    const int r0 = oh0 * g.stride - g.pad;               // first input row read
    const int rows_in = (oh1 - oh0 - 1) * g.stride + kh;
    const int wp = g.w + 2 * g.pad;                      // padded row width
    const int wps = odd(wp), plane_s = odd(rows_in * wps); // LDS pitches
    float* w_s = sm;                                     // [K][CG]
    float* x_s = sm + CG * g.k;                          // [cin][rows_in][wps]
    const float* xn = x + int64_t(n) * g.cin * g.h * g.w;
    const int plane_in = rows_in * wp;
    stage<4>(CG * g.k, w_s, [&](int e, int& slot) {
        const int co = co0 + e % CG;
        slot = e;
        return co < g.cout ? wt[co * g.k + e / CG] : 0.0f;
    });
    stage<8>(g.cin * plane_in, x_s, [&](int e, int& slot) {
        const unsigned ci = unsigned(e) / unsigned(plane_in);
        const unsigned rem = unsigned(e) - ci * unsigned(plane_in);
        const unsigned rr = rem / unsigned(wp), cc = rem - rr * unsigned(wp);
        slot = int(ci) * plane_s + int(rr) * wps + int(cc);
        const int h = r0 + int(rr), v = int(cc) - g.pad;
        return (h >= 0 && h < g.h && v >= 0 && v < g.w) ? xn[(int(ci) * g.h + h) * g.w + v] : 0.0f;
    });
    __syncthreads();
    const int npix = (oh1 - oh0) * g.ow;
    const int64_t plane = int64_t(g.oh) * g.ow;
    for (int p = threadIdx.x; p < npix; p += kThreads) {
        const int ohl = p / g.ow, ow = p - ohl * g.ow;
        float c[CG];
#pragma unroll
        for (int q = 0; q < CG; ++q) c[q] = 0.0f;
        const float* wk = w_s;
        for (int ci = 0; ci < g.cin; ++ci) {
            const float* xr = x_s + ci * plane_s + ohl * g.stride * wps + ow * g.stride;
#pragma unroll
            for (int i = 0; i < (KH ? KH : 1); ++i) {
                for (int ii = 0; ii < (KH ? 1 : kh); ++ii) {
                    const float* xi = xr + (KH ? i : ii) * wps;
#pragma unroll
                    for (int j = 0; j < (KW ? KW : 1); ++j) {
                        for (int jj = 0; jj < (KW ? 1 : kw); ++jj, wk += CG) {
                            const float a = xi[KW ? j : jj];
                            float wv[CG];
#pragma unroll
                            for (int q = 0; q < CG; ++q) wv[q] = wk[q];
#pragma unroll
                            for (int q = 0; q < CG; ++q) {
                                const float t = c[q] + a * wv[q];
                                c[q] = (a != 0.0f) ? t : c[q];
                            }
                        }
                    }
                }
            }
        }
        float* on = out + int64_t(n) * g.cout * plane + int64_t(oh0 + ohl) * g.ow + ow;
#pragma unroll
        for (int q = 0; q < CG; ++q) {
            const int co = co0 + q;
            if (co < g.cout) on[int64_t(co) * plane] = bias ? c[q] + bias[co] : c[q];
        }
    }
}

// Conv2d -> ReLU -> MaxPool2d (disjoint pk x pk windows) over a tile of
// `prows` pooled rows of one image and CG output channels. The convolution
// values of the tile's windows are computed exactly as conv_forward_tiled does
// and kept in LDS; each window is then ReLU'd and reduced to its first strict
// maximum in window order (src/conv.cpp:410-442), written with its flat index
// into the (N, C, oH, oW) convolution output. Only the pooled tensor reaches
// HBM. blockIdx.x = n * tiles + tile.
template <int CG, int KH, int KW>
__global__ __launch_bounds__(kThreads) void conv_relu_pool_tiled(
    const float* __restrict__ x, const float* __restrict__ wt, const float* __restrict__ bias,
    float* __restrict__ pooled, int32_t* __restrict__ argmax, Geo g, int pk, int ph, int pw,
    int prows, int tiles) {
    extern __shared__ __align__(16) float sm[];
    const int kh = KH ? KH : g.kh, kw = KW ? KW : g.kw;
    const int n = int(blockIdx.x) / tiles, tile = int(blockIdx.x) % tiles;
    const int co0 = int(blockIdx.y) * CG;
    const int pr0 = tile * prows;
    const int pr1 = min(pr0 + prows, ph);
    const int oh0 = pr0 * pk, crows = (pr1 - pr0) * pk, ccols = pw * pk;
    const int r0 = oh0 * g.stride - g.pad;
    const int rows_in = (crows - 1) * g.stride + kh;
    const int wp = g.w + 2 * g.pad;
    const int wps = odd(wp), plane_s = odd(rows_in * wps);
    float* w_s = sm;                                     // [K][CG]
    float* x_s = w_s + CG * g.k;                         // [cin][rows_in][wps]
    float* y_s = x_s + g.cin * plane_s;                  // [CG][crows][ccols]
    const float* xn = x + int64_t(n) * g.cin * g.h * g.w;
    const int plane_in = rows_in * wp;
    stage<4>(CG * g.k, w_s, [&](int e, int& slot) {
        const int co = co0 + e % CG;
        slot = e;
        return co < g.cout ? wt[co * g.k + e / CG] : 0.0f;
    });
    stage<8>(g.cin * plane_in, x_s, [&](int e, int& slot) {
        const unsigned ci = unsigned(e) / unsigned(plane_in);
        const unsigned rem = unsigned(e) - ci * unsigned(plane_in);
        const unsigned rr = rem / unsigned(wp), cc = rem - rr * unsigned(wp);
        slot = int(ci) * plane_s + int(rr) * wps + int(cc);
        const int h = r0 + int(rr), v = int(cc) - g.pad;
        return (h >= 0 && h < g.h && v >= 0 && v < g.w) ? xn[(int(ci) * g.h + h) * g.w + v] : 0.0f;
    });
    __syncthreads();
    const int npix = crows * ccols;
    for (int p = threadIdx.x; p < npix; p += kThreads) {
        const int ohl = p / ccols, ow = p - ohl * ccols;
        float c[CG];
#pragma unroll
        for (int q = 0; q < CG; ++q) c[q] = 0.0f;
        const float* wk = w_s;
        for (int ci = 0; ci < g.cin; ++ci) {
            const float* xr = x_s + ci * plane_s + ohl * g.stride * wps + ow * g.stride;
#pragma unroll
            for (int i = 0; i < (KH ? KH : 1); ++i) {
                for (int ii = 0; ii < (KH ? 1 : kh); ++ii) {
                    const float* xi = xr + (KH ? i : ii) * wps;
#pragma unroll
                    for (int j = 0; j < (KW ? KW : 1); ++j) {
                        for (int jj = 0; jj < (KW ? 1 : kw); ++jj, wk += CG) {
                            const float a = xi[KW ? j : jj];
                            float wv[CG];
#pragma unroll
                            for (int q = 0; q < CG; ++q) wv[q] = wk[q];
#pragma unroll
                            for (int q = 0; q < CG; ++q) {
                                const float t = c[q] + a * wv[q];
                                c[q] = (a != 0.0f) ? t : c[q];
                            }
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int q = 0; q < CG; ++q) {
            const int co = co0 + q;
            const float v = (bias && co < g.cout) ? c[q] + bias[co] : c[q];
            y_s[(q * crows + ohl) * ccols + ow] = (0.0f < v) ? v : 0.0f;  // ReLU
        }
    }
    __syncthreads();
    const int nwin = CG * (pr1 - pr0) * pw;
    for (int e = threadIdx.x; e < nwin; e += kThreads) {
        const int q = e / ((pr1 - pr0) * pw), r = e - q * ((pr1 - pr0) * pw);
        const int co = co0 + q;
        if (co >= g.cout) continue;
        const int prl = r / pw, pc = r - prl * pw;
        float best = 0.0f;
        int bi = 0, bj = 0;
        bool found = false;
        for (int i = 0; i < pk; ++i)
            for (int j = 0; j < pk; ++j) {
                const float v = y_s[(q * crows + prl * pk + i) * ccols + pc * pk + j];
                if (!found || v > best) {
                    best = v;
                    bi = i;
                    bj = j;
                    found = true;
                }
            }
        const int64_t plane_c = int64_t(n) * g.cout + co;
        const int64_t o = (plane_c * ph + pr0 + prl) * pw + pc;
        pooled[o] = best;
        argmax[o] = int32_t((plane_c * g.oh + oh0 + prl * pk + bi) * g.ow + pc * pk + bj);
    }
}

// n / d for 0 <= n < 2^31 with a multiply-high, an add and a shift instead of
// a division sequence (Granlund and Montgomery, "Division by invariant
// integers using multiplication", PLDI 1994): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, n / d = (mulhi(n, m) + n) >> l. The sum
// stays below 2^32 because mulhi(n, m) < n < 2^31. The tile kernels decode
// their staging and item indices with it.
struct FastDiv {
    uint32_t d, m, l;
};

FastDiv fast_div(uint32_t d) {
    uint32_t l = 0;
    while ((uint64_t(1) << l) < d) ++l;
    const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1;
    return FastDiv{d, uint32_t(m), l};
}

__device__ __forceinline__ int fdiv(int n, const FastDiv& f) {
    return int((__umulhi(uint32_t(n), f.m) + uint32_t(n)) >> f.l);
}

// The (image, tile) of a tile kernel's block. Workgroups go to the 8 XCDs in
// turn (block b to XCD b % 8), each with its own L2; when the batch is a
// multiple of 8, the tiles of one image are given blocks on the same XCD, so
// the rows and pooled cells that neighbouring tiles both stage (halo rows,
// cache lines shared by short rows) are fetched from HBM once per image.
__device__ __forceinline__ void image_tile(int b, int tiles, int images, int& n, int& tile) {
    if (images % 8 == 0) {
        const int slot = b / 8;
        n = 8 * (slot / tiles) + b % 8;
        tile = slot % tiles;
    } else {
        n = b / tiles;
        tile = b % tiles;
    }
}

// Conv2d (3 x 3, stride 1, padding 1) -> ReLU -> MaxPool2d (disjoint pk x pk
// windows) over a tile of `rows` convolution rows (a multiple of pk) of one
// image and every output channel. The input rows r0 - 1 .. r0 + rows
// (zero-padded) and the weights as [k][cout] sit in LDS once for all output
// channels; one thread per (pixel, group of CG output channels) sums the K
// products of each channel in k order from zero, skipping zero inputs, then
// adds the bias (conv_forward_direct's order, bit-identical), and ReLU'd
// values go to LDS for the pool. When every weight is finite a skipped product
// a * w, a = +-0, is +-0 and leaves the sum as it is (a sum that starts at +0
// never becomes -0), so the skip is dropped with the same bits. Each window is
// then reduced to its first strict maximum in window order
// (src/conv.cpp:410-442) and written with its flat index into the (N, C, oH,
// oW) convolution output.
struct PoolFwdTile {
    int rows, tiles;     // convolution rows per tile (a multiple of pk), tiles per image
    int wp, plane;       // LDS row and plane pitch of the input rows (odd)
    int coutp;           // output channels padded to CG
    int ws_off, ys_off;  // LDS offsets (floats) of the weights and the ReLU'd outputs
    // divisors: W + 2, rows + 2, coutp, rows * W, W, pw, rows / pk
    FastDiv wcols, srows, fcoutp, npx, w, pw, prows;
};

template <int CG, bool FAST>
__device__ __forceinline__ void pool_fwd_items(const float* xs, const float* ws,
                                               const float* __restrict__ bias, float* ys,
                                               const Geo& g, const PoolFwdTile& ft, int rows,
                                               int first, int step) {
    const int npx = ft.rows * g.w;
    const int items = npx * (ft.coutp / CG);
    for (int it = first; it < items; it += step) {
        const int cgi = fdiv(it, ft.npx), p = it - cgi * npx;
        const int hl = fdiv(p, ft.w), v = p - hl * g.w;
        if (hl >= rows) continue;
        float c[CG];
#pragma unroll
        for (int q = 0; q < CG; ++q) c[q] = 0.0f;
        const float* wk = ws + cgi * CG;
        for (int ci = 0; ci < g.cin; ++ci) {
            const float* xr = xs + ci * ft.plane + hl * ft.wp + v;
#pragma unroll
            for (int i = 0; i < 3; ++i)
#pragma unroll
                for (int j = 0; j < 3; ++j, wk += ft.coutp) {
                    const float a = xr[i * ft.wp + j];
                    float wv[CG];
                    if constexpr (CG == 4) {
                        const float4 t = *reinterpret_cast<const float4*>(wk);
                        wv[0] = t.x; wv[1] = t.y; wv[2] = t.z; wv[3] = t.w;
                    } else if constexpr (CG == 2) {
                        const float2 t = *reinterpret_cast<const float2*>(wk);
                        wv[0] = t.x; wv[1] = t.y;
                    } else {
                        wv[0] = wk[0];
                    }
#pragma unroll
                    for (int q = 0; q < CG; ++q) {
                        const float t = c[q] + a * wv[q];
                        c[q] = (FAST || a != 0.0f) ? t : c[q];
                    }
                }
        }
#pragma unroll
        for (int q = 0; q < CG; ++q) {
            const int co = cgi * CG + q;
            if (co >= g.cout) continue;
            const float y = bias ? c[q] + bias[co] : c[q];
            ys[(co * ft.rows + hl) * g.w + v] = (0.0f < y) ? y : 0.0f;   // ReLU
        }
    }
}

template <int CG, int NT>
__global__ __launch_bounds__(NT) void conv3_relu_pool(const float* __restrict__ x,
                                                      const float* __restrict__ wt,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ pooled,
                                                      int32_t* __restrict__ argmax, Geo g, int pk,
                                                      int ph, int pw, PoolFwdTile ft) {
    extern __shared__ __align__(16) float sm[];
    const int tid = int(threadIdx.x);
    int n, tile;
    image_tile(int(blockIdx.x), ft.tiles, g.n, n, tile);
    const int r0 = tile * ft.rows;
    const int rows = min(ft.rows, g.h - r0);
    const int srows = ft.rows + 2, wcols = g.w + 2;
    float* xs = sm;                  // [cin][plane]: input rows r0 - 1 .. r0 + rows
    float* ws = sm + ft.ws_off;      // [K][coutp]
    float* ys = sm + ft.ys_off;      // [cout][rows][W]
    const int xn = g.cin * srows * wcols;
    const int wn = g.k * ft.coutp;
    bool nonfinite = false;
    for (int rd = 0; rd * 4 * NT < xn || rd * 4 * NT < wn; ++rd) {
        float xv[4], wv[4];
        int xslot[4], wslot[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = rd * 4 * NT + u * NT + tid;
            xslot[u] = -1;
            xv[u] = 0.0f;
            if (e < xn) {
                const int q = fdiv(e, ft.wcols), cc = e - q * wcols;
                const int ci = fdiv(q, ft.srows), rr = q - ci * srows;
                const int r = r0 - 1 + rr, c = cc - 1;
                xslot[u] = ci * ft.plane + rr * ft.wp + cc;
                if (r >= 0 && r < g.h && c >= 0 && c < g.w)
                    xv[u] = x[((int64_t(n) * g.cin + ci) * g.h + r) * g.w + c];
            }
            wslot[u] = -1;
            wv[u] = 0.0f;
            if (e < wn) {
                const int k = fdiv(e, ft.fcoutp), co = e - k * ft.coutp;
                wslot[u] = e;
                if (co < g.cout) wv[u] = wt[co * g.k + k];
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (xslot[u] >= 0) xs[xslot[u]] = xv[u];
            if (wslot[u] >= 0) {
                ws[wslot[u]] = wv[u];
                nonfinite |= !isfinite(wv[u]);
            }
        }
    }
    const bool fast = !__syncthreads_or(nonfinite);
    if (fast)
        pool_fwd_items<CG, true>(xs, ws, bias, ys, g, ft, rows, tid, NT);
    else
        pool_fwd_items<CG, false>(xs, ws, bias, ys, g, ft, rows, tid, NT);
    __syncthreads();
    const int pr0 = r0 / pk;
    const int prows = ft.rows / pk;
    const int prn = max(min(pr0 + prows, ph) - pr0, 0);
    const int nwin = g.cout * prows * pw;
    for (int e = tid; e < nwin; e += NT) {
        const int q = fdiv(e, ft.pw), pc = e - q * pw;
        const int co = fdiv(q, ft.prows), prl = q - co * prows;
        if (prl >= prn) continue;
        float best = 0.0f;
        int bi = 0, bj = 0;
        bool found = false;
        for (int i = 0; i < pk; ++i)
            for (int j = 0; j < pk; ++j) {
                const float v = ys[(co * ft.rows + prl * pk + i) * g.w + pc * pk + j];
                if (!found || v > best) {
                    best = v;
                    bi = i;
                    bj = j;
                    found = true;
                }
            }
        const int64_t plane_c = int64_t(n) * g.cout + co;
        const int64_t o = (plane_c * ph + pr0 + prl) * pw + pc;
        pooled[o] = best;
        argmax[o] = int32_t((plane_c * g.oh + r0 + prl * pk + bi) * g.ow + pc * pk + bj);
    }
}

// A ReLU and a max pool with disjoint pk x pk windows after the convolution
// (Conv2d -> ReLU -> MaxPool2d fused): the pooled output, its gradient and the
// argmax (flat index into the convolution's output) replace the convolution's
// own output gradient, which is gathered on the fly.
struct PoolGather {
    const float* gp;        // gradient of the pooled output (N, C, ph, pw)
    const float* pooled;    // the pooled output
    const int32_t* argmax;  // flat index of each window's maximum in (N, C, oH, oW)
    int pk, ph, pw;
};

// The convolution's output gradient at (n, co, oh, ow): the reference's
// maxpool backward (src/conv.cpp:461-469, one window per position here) then
// its ReLU backward (src/tensor_ops.cpp:603-615). The pooled value is the
// chosen position's ReLU output, so "pooled > 0" is "conv output > 0" there,
// and every other position's gradient is zero either way: bit-exact.
template <bool POOL>
__device__ __forceinline__ float out_grad(const float* gout, const PoolGather& pg, const Geo& g,
                                          int n, int co, int oh, int ow) {
    const int64_t flat = ((int64_t(n) * g.cout + co) * g.oh + oh) * g.ow + ow;
    if (!POOL) return gout[flat];
    const int pr = oh / pg.pk, pc = ow / pg.pk;
    if (pr >= pg.ph || pc >= pg.pw) return 0.0f;
    const int64_t o = ((int64_t(n) * g.cout + co) * pg.ph + pr) * pg.pw + pc;
    return (pg.argmax[o] == flat && pg.pooled[o] > 0.0f) ? pg.gp[o] : 0.0f;
}

// First and last window index along one axis whose window covers position p,
// in 32-bit arithmetic (stride 1 needs no division).
__device__ __forceinline__ void cover32(int p, int pad, int k, int s, int out, int& lo, int& hi) {
    const int t = p + pad - (k - 1);
    if (s == 1) {
        lo = t <= 0 ? 0 : t;
        hi = p + pad;
    } else {
        lo = t <= 0 ? 0 : (t + s - 1) / s;
        hi = (p + pad) / s;
    }
    if (hi > out - 1) hi = out - 1;
}

// Input gradient over a tile of `rows` input rows of one image and CG input
// channels (blockIdx.y). The output-gradient rows whose windows cover the tile
// (all out_channels) and the weights of the CG channels (laid out
// [tap][cout][CG]) sit in LDS; each thread computes one input pixel for all
// CG channels, every channel in the order of conv_backward_input_direct (zero
// gradients skipped by a select after an unconditional multiply-add).
// blockIdx.x = n * tiles + tile.
template <int CG, bool POOL>
__device__ __forceinline__ void backward_input_block(const float* __restrict__ gout,
                                                     const PoolGather& pgat,
                                                     const float* __restrict__ wt,
                                                     float* __restrict__ dx, const Geo& g,
                                                     int rows, int tiles, int bx, int by,
                                                     float* sm) {
    const int n = bx / tiles, tile = bx % tiles;
    const int ci0 = by * CG;
    const int h0 = tile * rows;
    const int h1 = min(h0 + rows, g.h);
    int lo, hi, lo2, hi2;
    cover32(h0, g.pad, g.kh, g.stride, g.oh, lo, hi);
    cover32(h1 - 1, g.pad, g.kh, g.stride, g.oh, lo2, hi2);
    const int oh_first = lo;
    const int oh_rows = max(0, hi2 - oh_first + 1);
    const int khw = g.kh * g.kw;
    const int gplane = oh_rows * g.ow;
    const int gplane_s = odd(gplane), tap_s = odd(g.cout * CG);   // LDS pitches
    float* g_s = sm;                                   // [cout][oh_rows][ow]
    float* w_s = sm + g.cout * gplane_s;               // [tap][cout][CG]
    const int64_t plane = int64_t(g.oh) * g.ow;
    const float* gn = POOL ? nullptr : gout + int64_t(n) * g.cout * plane + int64_t(oh_first) * g.ow;
    stage<8>(g.cout * gplane, g_s, [&](int e, int& slot) {
        const unsigned co = unsigned(e) / unsigned(gplane);
        const unsigned r = unsigned(e) - co * unsigned(gplane);
        slot = int(co) * gplane_s + int(r);
        if (POOL) {
            const unsigned rr = r / unsigned(g.ow);
            return out_grad<true>(gout, pgat, g, n, int(co), oh_first + int(rr),
                                  int(r - rr * unsigned(g.ow)));
        }
        return gn[int64_t(co) * plane + r];
    });
    stage<4>(khw * g.cout * CG, w_s, [&](int e, int& slot) {
        const int cl = e % CG, r = e / CG;             // r = tap * cout + co
        const int co = r % g.cout, tap = r / g.cout;
        const int ci = ci0 + cl;
        slot = tap * tap_s + co * CG + cl;
        return ci < g.cin ? wt[(co * g.cin + ci) * khw + tap] : 0.0f;
    });
    __syncthreads();
    const int band = (h1 - h0) * g.w;
    for (int e = threadIdx.x; e < band; e += kThreads) {
        const int hl = e / g.w;
        const int h = h0 + hl, v = e - hl * g.w;
        int oh_lo, oh_hi, ow_lo, ow_hi;
        cover32(h, g.pad, g.kh, g.stride, g.oh, oh_lo, oh_hi);
        cover32(v, g.pad, g.kw, g.stride, g.ow, ow_lo, ow_hi);
        float acc[CG];
#pragma unroll
        for (int cl = 0; cl < CG; ++cl) acc[cl] = 0.0f;
        for (int oh = oh_lo; oh <= oh_hi; ++oh) {
            const int i = h + g.pad - oh * g.stride;
            for (int ow = ow_lo; ow <= ow_hi; ++ow) {
                const int j = v + g.pad - ow * g.stride;
                const float* gp = g_s + (oh - oh_first) * g.ow + ow;
                const float* wp = w_s + (i * g.kw + j) * tap_s;
                float d[CG];
#pragma unroll
                for (int cl = 0; cl < CG; ++cl) d[cl] = 0.0f;
                int co = 0;
                for (; co + 8 <= g.cout; co += 8) {
                    float gv[8], wv[8][CG];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        gv[u] = gp[(co + u) * gplane_s];
#pragma unroll
                        for (int cl = 0; cl < CG; ++cl) wv[u][cl] = wp[(co + u) * CG + cl];
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u)
#pragma unroll
                        for (int cl = 0; cl < CG; ++cl) {
                            const float t = d[cl] + gv[u] * wv[u][cl];
                            d[cl] = (gv[u] != 0.0f) ? t : d[cl];
                        }
                }
                for (; co < g.cout; ++co) {
                    const float gv = gp[co * gplane_s];
#pragma unroll
                    for (int cl = 0; cl < CG; ++cl) {
                        const float t = d[cl] + gv * wp[co * CG + cl];
                        d[cl] = (gv != 0.0f) ? t : d[cl];
                    }
                }
#pragma unroll
                for (int cl = 0; cl < CG; ++cl) acc[cl] += d[cl];
            }
        }
#pragma unroll
        for (int cl = 0; cl < CG; ++cl)
            if (ci0 + cl < g.cin)
                dx[((int64_t(n) * g.cin + ci0 + cl) * g.h + h) * g.w + v] = acc[cl];
    }
}

template <int CG, bool POOL>
__global__ __launch_bounds__(kThreads) void conv_backward_input_tiled(
    const float* __restrict__ gout, PoolGather pgat, const float* __restrict__ wt,
    float* __restrict__ dx, Geo g, int rows, int tiles) {
    extern __shared__ __align__(16) float sm[];
    backward_input_block<CG, POOL>(gout, pgat, wt, dx, g, rows, tiles, int(blockIdx.x),
                                   int(blockIdx.y), sm);
}

// Weight and bias gradient partials over a band of `rows` output rows of one
// image: the input rows the band reads (zero-padded) and its output gradient
// rows are staged in LDS; a thread owns a CT x KT tile of (output channel,
// column k) sums -- column K is the bias, whose "input" is 1 -- over one of PG
// pixel groups, and the groups are combined in group order. partial[block][o],
// o = co (K + 1) + k, is then reduced over blocks by conv_weight_reduce. The
// order of every sum depends only on the shape.
template <int CT, int KT, bool POOL>
__device__ __forceinline__ void weight_band_block(const float* __restrict__ x,
                                                  const float* __restrict__ gout,
                                                  const PoolGather& pgat,
                                                  float* __restrict__ partial, const Geo& g,
                                                  int rows, int bands, int bx, float* sm) {
    const int n = bx / bands, band = bx % bands;
    const int oh0 = band * rows;
    const int oh1 = min(oh0 + rows, g.oh);
    const int np = (oh1 - oh0) * g.ow;
    const int rows_in = (oh1 - oh0 - 1) * g.stride + g.kh;
    const int wp = g.w + 2 * g.pad;
    const int K1 = g.k + 1;
    const int tiles_k = (K1 + KT - 1) / KT, tiles = ((g.cout + CT - 1) / CT) * tiles_k;
    const int PG = tiles >= kThreads ? 1 : kThreads / tiles;
    const int wps = odd(wp), plane_s = odd(rows_in * wps), nps = odd(np);   // LDS pitches
    float* x_s = sm;                                   // [cin][rows_in][wps]
    float* dy_s = x_s + g.cin * plane_s;               // [cout][nps]
    float* red = dy_s + g.cout * nps;                  // [PG][tiles][CT * KT]
    const int r0 = oh0 * g.stride - g.pad;
    const float* xn = x + int64_t(n) * g.cin * g.h * g.w;
    const int plane_in = rows_in * wp;
    stage<8>(g.cin * plane_in, x_s, [&](int e, int& slot) {
        const unsigned ci = unsigned(e) / unsigned(plane_in);
        const unsigned rem = unsigned(e) - ci * unsigned(plane_in);
        const unsigned rr = rem / unsigned(wp), cc = rem - rr * unsigned(wp);
        slot = int(ci) * plane_s + int(rr) * wps + int(cc);
        const int h = r0 + int(rr), v = int(cc) - g.pad;
        return (h >= 0 && h < g.h && v >= 0 && v < g.w) ? xn[(int(ci) * g.h + h) * g.w + v] : 0.0f;
    });
    const int64_t plane = int64_t(g.oh) * g.ow;
    const float* gn = POOL ? nullptr : gout + int64_t(n) * g.cout * plane + int64_t(oh0) * g.ow;
    stage<8>(g.cout * np, dy_s, [&](int e, int& slot) {
        const unsigned co = unsigned(e) / unsigned(np);
        const unsigned r = unsigned(e) - co * unsigned(np);
        slot = int(co) * nps + int(r);
        if (POOL) {
            const unsigned rr = r / unsigned(g.ow);
            return out_grad<true>(gout, pgat, g, n, int(co), oh0 + int(rr),
                                  int(r - rr * unsigned(g.ow)));
        }
        return gn[int64_t(co) * plane + r];
    });
    __syncthreads();
    const int khw = g.kh * g.kw;
    for (int tbase = 0; tbase < tiles; tbase += kThreads) {
        const int t = tbase + int(threadIdx.x) % (tiles >= kThreads ? kThreads : tiles);
        const int pg = tiles >= kThreads ? 0 : int(threadIdx.x) / tiles;
        const bool active = t < tiles && pg < PG;
        float acc[CT][KT];
#pragma unroll
        for (int q = 0; q < CT; ++q)
#pragma unroll
            for (int kk = 0; kk < KT; ++kk) acc[q][kk] = 0.0f;
        const int co_base = (t / tiles_k) * CT, k_base = (t % tiles_k) * KT;
        int xoff[KT];   // offset of column k within the band for pixel (0, 0); -1 bias; -2 none
#pragma unroll
        for (int kk = 0; kk < KT; ++kk) {
            const int k = k_base + kk;
            if (k < g.k) {
                const int ci = k / khw, ij = k - ci * khw;
                const int i = ij / g.kw, j = ij - i * g.kw;
                xoff[kk] = ci * plane_s + i * wps + j;
            } else {
                xoff[kk] = k == g.k ? -1 : -2;
            }
        }
        if (active) {
            int ohl = pg / g.ow, ow = pg - (pg / g.ow) * g.ow;
            for (int p = pg; p < np; p += PG) {
                const int pix = ohl * g.stride * wps + ow * g.stride;
                float xv[KT], dv[CT];
#pragma unroll
                for (int kk = 0; kk < KT; ++kk)
                    xv[kk] = xoff[kk] >= 0 ? x_s[xoff[kk] + pix] : (xoff[kk] == -1 ? 1.0f : 0.0f);
#pragma unroll
                for (int q = 0; q < CT; ++q)
                    dv[q] = co_base + q < g.cout ? dy_s[(co_base + q) * nps + p] : 0.0f;
#pragma unroll
                for (int q = 0; q < CT; ++q)
#pragma unroll
                    for (int kk = 0; kk < KT; ++kk) acc[q][kk] = fmaf(dv[q], xv[kk], acc[q][kk]);
                ow += PG;
                while (ow >= g.ow) {
                    ow -= g.ow;
                    ++ohl;
                }
            }
        }
        if (PG > 1) {
            // All PG groups park their tiles in LDS; every thread then adds the
            // groups of a few outputs in group order.
            if (active) {
                float* r = red + (pg * tiles + t) * (CT * KT);
#pragma unroll
                for (int q = 0; q < CT; ++q)
#pragma unroll
                    for (int kk = 0; kk < KT; ++kk) r[q * KT + kk] = acc[q][kk];
            }
            __syncthreads();
            float* pc = partial + int64_t(bx) * g.cout * K1;
            const int span = tiles * CT * KT;
            for (int o = threadIdx.x; o < span; o += kThreads) {
                float sum = red[o];
                for (int g2 = 1; g2 < PG; ++g2) sum += red[g2 * span + o];
                const int tt = o / (CT * KT), e = o % (CT * KT);
                const int co = (tt / tiles_k) * CT + e / KT, k = (tt % tiles_k) * KT + e % KT;
                if (co < g.cout && k < K1) pc[co * K1 + k] = sum;
            }
        } else if (active) {
            float* pc = partial + int64_t(bx) * g.cout * K1;
#pragma unroll
            for (int q = 0; q < CT; ++q)
#pragma unroll
                for (int kk = 0; kk < KT; ++kk) {
                    const int co = co_base + q, k = k_base + kk;
                    if (co < g.cout && k < K1) pc[co * K1 + k] = acc[q][kk];
                }
        }
    }
}

template <int CT, int KT, bool POOL>
__global__ __launch_bounds__(kThreads) void conv_weight_band(const float* __restrict__ x,
                                                             const float* __restrict__ gout,
                                                             PoolGather pgat,
                                                             float* __restrict__ partial, Geo g,
                                                             int rows, int bands) {
    extern __shared__ __align__(16) float sm[];
    weight_band_block<CT, KT, POOL>(x, gout, pgat, partial, g, rows, bands, int(blockIdx.x), sm);
}

// The input-gradient tiles and the weight-gradient bands of one layer in a
// single launch: blocks [0, in_blocks) run backward_input_block (x-major over
// in_x), the rest weight_band_block. The two read the same operands and write
// disjoint outputs; at these sizes each alone leaves most CUs idle, so
// together they take about as long as the longer one.
struct PairGeo {
    int in_rows, in_tiles, in_x, in_blocks;
    int band_rows, bands;
};

template <int CG, int T, bool POOL>
__global__ __launch_bounds__(kThreads) void conv_backward_pair(
    const float* __restrict__ x, const float* __restrict__ gout, PoolGather pgat,
    const float* __restrict__ wt, float* __restrict__ dx, float* __restrict__ partial, Geo g,
    PairGeo pg) {
    extern __shared__ __align__(16) float sm[];
    const int b = int(blockIdx.x);
    if (b < pg.in_blocks)
        backward_input_block<CG, POOL>(gout, pgat, wt, dx, g, pg.in_rows, pg.in_tiles,
                                       b % pg.in_x, b / pg.in_x, sm);
    else
        weight_band_block<T, T, POOL>(x, gout, pgat, partial, g, pg.band_rows, pg.bands,
                                      b - pg.in_blocks, sm);
}

// Backward of a 3 x 3, stride 1, padding 1 convolution followed by ReLU and a
// max pool with disjoint pk x pk windows, over a tile of `rows` convolution
// rows (a multiple of pk, so every pooled cell belongs to one tile) of one
// image: the input gradient of those rows and the weight and bias gradient
// partials of those positions, in one block.
//
// The convolution's output gradient around the tile (rows r0 - 1 .. r0 +
// rows, columns -1 .. W, zero wherever there is no output) is built in LDS
// by scattering each pooled cell's gradient to its argmax position when the
// pooled value is positive: out_grad() for every position, with a quarter of
// the loads. The input rows r0 - 1 .. r0 + rows (zero-padded) and, for the
// input gradient, the weights as [tap][cout][ci] sit beside it.
//
// Threads [0, dx_threads) compute the input gradient, one per (pixel, group
// of CG input channels): for the nine windows in (oh, ow) order, the
// cout-term dot product in co order with zero gradients skipped, added to the
// pixel's sum: conv_backward_input_direct's order, so the result is
// bit-identical. Windows outside the output read the zero border; their dot
// products are +0 and leave the sum unchanged (a sum that starts at +0 never
// becomes -0 in round-to-nearest). When every weight is finite a skipped
// product g * w, g = +-0, is itself +-0, so the skip is dropped with the same
// bits; a non-finite weight keeps it.
//
// The other threads compute the weight and bias partials as
// weight_band_block does -- CT x CT tiles of (co, k), column K the bias,
// over pg pixel groups combined in group order -- into partial[n * tiles + tile].
struct PoolTile {
    int rows, tiles;         // convolution rows per tile (a multiple of pk), tiles per image
    int dx_threads;          // threads computing dx (a multiple of 64; 0 = no dx)
    int pg;                  // pixel groups of the weight partials (0 = no weight gradient)
    int wp, plane;           // LDS row and plane pitch (odd)
    int cinp;                // input channels padded to CG
    int xs_off, ws_off, red_off;   // LDS offsets (floats) of the input rows, weights, group sums
    int prows;               // pooled rows a tile's halo can reach: rows / pk + 2
    int own, cells, cell_off;  // the tile's own pooled rows (rows / pk), cout * own * pw
                               // cells, LDS offset of their positions and gradients
    // divisors: pw, prows, W + 2, rows + 2, C_in, rows * W, W
    FastDiv pw, fprows, wcols, srows, cin, npx, w;
};

// Weights of one (co, input-channel group) in the tile kernel's LDS: nine taps
// of CG channels, padded to whole 16-byte reads.
template <int CG>
constexpr int tap_pitch() { return (9 * CG + 3) / 4 * 4; }

// One thread per (pixel, group of CG channels). The nine windows' dot
// products run side by side with co as the outer loop (each still sums its
// co terms in co order), so every round of LDS reads feeds 9 CG products.
template <int CG, bool FAST>
__device__ __forceinline__ void pool_tile_dx(const float* gs, const float* ws, float* dx,
                                             const Geo& g, const PoolTile& pt, int n, int r0,
                                             int rows, int first, int step) {
    constexpr int WS = tap_pitch<CG>();
    const int npx = pt.rows * g.w;
    const int groups = pt.cinp / CG;
    const int items = npx * groups;
    for (int it = first; it < items; it += step) {
        const int cgi = fdiv(it, pt.npx), p = it - cgi * npx;
        const int hl = fdiv(p, pt.w), v = p - hl * g.w;
        if (hl >= rows) continue;
        float d[9][CG];
#pragma unroll
        for (int t = 0; t < 9; ++t)
#pragma unroll
            for (int cl = 0; cl < CG; ++cl) d[t][cl] = 0.0f;
        const float* gb = gs + hl * pt.wp + v;
        const float* wb = ws + cgi * WS;
#pragma unroll 2
        for (int co = 0; co < g.cout; ++co) {
            float gv[9];
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
                for (int b = 0; b < 3; ++b) gv[a * 3 + b] = gb[co * pt.plane + a * pt.wp + b];
            float wv[WS];
            const float4* wq = reinterpret_cast<const float4*>(wb + co * groups * WS);
#pragma unroll
            for (int q = 0; q < WS / 4; ++q) {
                const float4 t = wq[q];
                wv[4 * q] = t.x;
                wv[4 * q + 1] = t.y;
                wv[4 * q + 2] = t.z;
                wv[4 * q + 3] = t.w;
            }
            // window (a, b) is (oh, ow) = (h - 1 + a, v - 1 + b), tap (2 - a, 2 - b)
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
                for (int b = 0; b < 3; ++b) {
                    const int tap = (2 - a) * 3 + (2 - b);
                    const float gq = gv[a * 3 + b];
#pragma unroll
                    for (int cl = 0; cl < CG; ++cl) {
                        const float t = d[a * 3 + b][cl] + gq * wv[tap * CG + cl];
                        d[a * 3 + b][cl] = (FAST || gq != 0.0f) ? t : d[a * 3 + b][cl];
                    }
                }
        }
        const int h = r0 + hl;
#pragma unroll
        for (int cl = 0; cl < CG; ++cl) {
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < 9; ++t) acc += d[t][cl];
            const int ci = cgi * CG + cl;
            if (ci < g.cin) dx[((int64_t(n) * g.cin + ci) * g.h + h) * g.w + v] = acc;
        }
    }
}

template <int CG, int CT, int NT>
__global__ __launch_bounds__(NT) void conv3_pool_backward(const float* __restrict__ x,
                                                          const float* __restrict__ wt,
                                                          PoolGather pgat, float* __restrict__ dx,
                                                          float* __restrict__ partial, Geo g,
                                                          PoolTile pt) {
    extern __shared__ __align__(16) float sm[];
    const int tid = int(threadIdx.x);
    int n, tile;
    image_tile(int(blockIdx.x), pt.tiles, g.n, n, tile);
    const int r0 = tile * pt.rows;
    const int rows = min(pt.rows, g.h - r0);
    const int srows = pt.rows + 2;
    const bool want_dx = pt.dx_threads > 0, want_dw = pt.pg > 0;
    // gs: [cout rounded up to CT][plane], output gradient rows r0 - 1 .. r0 + rows
    // (planes beyond cout stay zero); xs: [cin + 2][plane], input rows r0 - 1 ..
    // r0 + rows, then a plane of ones (the bias column) and one of zeros.
    float* gs = sm;
    float* xs = sm + pt.xs_off;
    float* ws = sm + pt.ws_off;       // [cout][cinp / CG][tap_pitch]: tap-major CG channels
    float* red = sm + pt.red_off;     // [pg][tiles][CT * CT]
    // The tile's own pooled cells ([cout][own][pw]): the position of the argmax
    // in the tile (row * wp + column) and its gradient when it carries one, else
    // position 0 and gradient 0 (which adds nothing, see the sums below).
    int* cpos = reinterpret_cast<int*>(sm + pt.cell_off);
    float* cgrad = sm + pt.cell_off + pt.cells;
    __shared__ __align__(16) int flags;   // bit 0: a non-finite weight; bit 1: a non-finite input

    // The zero border and every position no pooled cell selects.
    const int zero_n = pt.xs_off;
    for (int e = tid; e < zero_n; e += NT) gs[e] = 0.0f;
    if (want_dw)
        for (int e = tid; e < pt.cells; e += NT) {
            cpos[e] = 0;
            cgrad[e] = 0.0f;
        }
    if (tid == 0) flags = 0;
    if (want_dw)
        for (int e = tid; e < 2 * pt.plane; e += NT)
            xs[g.cin * pt.plane + e] = e < pt.plane ? 1.0f : 0.0f;
    if (want_dx && pt.cinp != g.cin)
        for (int e = tid; e < g.cout * (pt.cinp / CG) * tap_pitch<CG>(); e += NT) ws[e] = 0.0f;
    __syncthreads();

    // Pooled rows whose windows reach rows r0 - 1 .. r0 + rows.
    const int pk = pgat.pk, pw = pgat.pw;
    const int pr_lo = max(r0 / pk - 1, 0), pr_hi = min((r0 + pt.rows) / pk, pgat.ph - 1);
    const int prn = max(pr_hi - pr_lo + 1, 0);
    const int cells = g.cout * pt.prows * pw;   // rows prl >= prn are skipped
    const int wcols = g.w + 2;
    const int xn = want_dw ? g.cin * srows * wcols : 0;
    const int wn = want_dx ? g.cout * g.cin * 9 : 0;
    const int64_t oplane = int64_t(g.h) * g.w;
    bool nonfinite = false, nonfinite_x = false;
    // One round issues up to 2 cells (3 loads each), 2 input and 5 weight
    // loads per thread before any LDS store.
    for (int rd = 0; rd * 2 * NT < cells || rd * 2 * NT < xn || rd * 5 * NT < wn; ++rd) {
        int cslot[2], ccell[2], cpix[2];
        float cval[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int e = rd * 2 * NT + u * NT + tid;
            cslot[u] = -1;
            ccell[u] = -1;
            cpix[u] = 0;
            cval[u] = 0.0f;
            const int q = fdiv(e, pt.pw), pc = e - q * pw;
            const int co = fdiv(q, pt.fprows), prl = q - co * pt.prows;
            if (e < cells && prl < prn) {
                const int pr = pr_lo + prl;
                const int64_t nc = int64_t(n) * g.cout + co;
                const int64_t o = (nc * pgat.ph + pr) * pw + pc;
                const int32_t am = pgat.argmax[o];
                const float pv = pgat.pooled[o];
                const float gv = pgat.gp[o];
                const int64_t off = int64_t(am) - (nc * oplane + int64_t(pr) * pk * g.w + pc * pk);
                if (pv > 0.0f && off >= 0 && off < int64_t(pk) * g.w) {
                    const int offi = int(off);
                    const int dr = offi / g.w, dc = offi - dr * g.w;
                    const int r = pr * pk + dr;
                    if (dr < pk && dc < pk && r >= r0 - 1 && r <= r0 + pt.rows) {
                        cslot[u] = co * pt.plane + (r - r0 + 1) * pt.wp + pc * pk + dc + 1;
                        cval[u] = gv;
                        const int own = pr - r0 / pk;
                        if (want_dw && own >= 0 && own < pt.own) {
                            ccell[u] = (co * pt.own + own) * pw + pc;
                            cpix[u] = (r - r0) * pt.wp + pc * pk + dc;
                        }
                    }
                }
            }
        }
        int xslot[2];
        float xval[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int e = rd * 2 * NT + u * NT + tid;
            xslot[u] = -1;
            xval[u] = 0.0f;
            if (e < xn) {
                const int q = fdiv(e, pt.wcols), cc = e - q * wcols;
                const int ci = fdiv(q, pt.srows), rr = q - ci * srows;
                const int r = r0 - 1 + rr, c = cc - 1;
                xslot[u] = ci * pt.plane + rr * pt.wp + cc;
                if (r >= 0 && r < g.h && c >= 0 && c < g.w)
                    xval[u] = x[((int64_t(n) * g.cin + ci) * g.h + r) * g.w + c];
            }
        }
        int wslot[5];
        float wval[5];
#pragma unroll
        for (int u = 0; u < 5; ++u) {
            const int e = rd * 5 * NT + u * NT + tid;
            wslot[u] = -1;
            wval[u] = 0.0f;
            if (e < wn) {
                const int q = e / 9, tap = e - q * 9;   // e = (co cin + ci) 9 + tap
                const int co = fdiv(q, pt.cin), ci = q - co * g.cin;
                wval[u] = wt[e];
                wslot[u] = (co * (pt.cinp / CG) + ci / CG) * tap_pitch<CG>() + tap * CG + ci % CG;
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (cslot[u] >= 0) gs[cslot[u]] = cval[u];
            if (ccell[u] >= 0) {
                cpos[ccell[u]] = cpix[u];
                cgrad[ccell[u]] = cval[u];
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u)
            if (xslot[u] >= 0) {
                xs[xslot[u]] = xval[u];
                nonfinite_x |= !isfinite(xval[u]);
            }
#pragma unroll
        for (int u = 0; u < 5; ++u)
            if (wslot[u] >= 0) {
                ws[wslot[u]] = wval[u];
                nonfinite |= !isfinite(wval[u]);
            }
    }
    if (nonfinite || nonfinite_x) atomicOr(&flags, (nonfinite ? 1 : 0) | (nonfinite_x ? 2 : 0));
    __syncthreads();
    const int fl = flags;
    const bool fast = (fl & 1) == 0;

    if (tid < pt.dx_threads) {
        if (fast)
            pool_tile_dx<CG, true>(gs, ws, dx, g, pt, n, r0, rows, tid, pt.dx_threads);
        else
            pool_tile_dx<CG, false>(gs, ws, dx, g, pt, n, r0, rows, tid, pt.dx_threads);
    }
    if (!want_dw) return;   // uniform across the block
    const int K1 = g.k + 1;

    // With every input finite, only the positions that carry a gradient (one per
    // pooled cell at most) add to the weight and bias sums: a thread owns four
    // columns k of one output channel and adds the channel's cells in cell order,
    // four cells per round of LDS reads. A cell without a gradient adds 0 * x =
    // +-0 (x finite), which leaves a sum that starts at +0 as it is. (A
    // non-finite input times a zero gradient is NaN in the full sum, so such
    // tiles take the full sum below.)
    if ((fl & 2) == 0) {
        const int wtid = tid - pt.dx_threads, wthreads = NT - pt.dx_threads;
        const int kt = (K1 + 3) / 4, ncell = pt.own * pgat.pw, stiles = g.cout * kt;
        // sg cell groups per tile when there are fewer tiles than threads; group
        // r adds cells r, r + sg, ... and the groups are added in group order.
        const int sg = max(1, wthreads / stiles);
        float* pc = partial + (int64_t(n) * pt.tiles + tile) * g.cout * K1;
        for (int t0 = 0; t0 < stiles; t0 += wthreads) {
            const int t = sg == 1 ? wtid + t0 : wtid % stiles, grp = sg == 1 ? 0 : wtid / stiles;
            const bool active = wtid >= 0 && t < stiles && grp < sg;
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            const int co = active ? t / kt : 0, k0 = active ? (t - co * kt) * 4 : 0;
            if (active) {
                int xoff[4];
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    const int k = k0 + kk;
                    if (k < g.k) {
                        const int ci = k / 9, ij = k - ci * 9;
                        const int i = ij / 3, j = ij - i * 3;
                        xoff[kk] = ci * pt.plane + i * pt.wp + j;
                    } else {
                        xoff[kk] = (k == g.k ? g.cin : g.cin + 1) * pt.plane;
                    }
                }
                const int* cp = cpos + co * ncell;
                const float* cv = cgrad + co * ncell;
                for (int c0 = grp; c0 < ncell; c0 += 4 * sg) {
                    int pos[4];
                    float gv[4], xv[4][4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int c = c0 + u * sg;
                        pos[u] = c < ncell ? cp[c] : 0;
                        gv[u] = c < ncell ? cv[c] : 0.0f;
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u)
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) xv[u][kk] = xs[xoff[kk] + pos[u]];
#pragma unroll
                    for (int u = 0; u < 4; ++u)
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk)
                            acc[kk] = fmaf(gv[u], xv[u][kk], acc[kk]);
                }
            }
            if (sg == 1) {
                if (active)
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk)
                        if (k0 + kk < K1) pc[co * K1 + k0 + kk] = acc[kk];
            } else {
                if (active)
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) red[(grp * stiles + t) * 4 + kk] = acc[kk];
                __syncthreads();
                for (int o = tid; o < stiles * 4; o += NT) {
                    float sum = red[o];
                    for (int r = 1; r < sg; ++r) sum += red[r * stiles * 4 + o];
                    const int tt = o / 4, kk = o - tt * 4;
                    const int cco = tt / kt, k = (tt - cco * kt) * 4 + kk;
                    if (k < K1) pc[cco * K1 + k] = sum;
                }
            }
        }
        return;
    }

    const int tiles_k = (K1 + CT - 1) / CT, tiles = ((g.cout + CT - 1) / CT) * tiles_k;
    const int wtid = tid - pt.dx_threads;
    if (wtid >= 0 && wtid < tiles * pt.pg) {
        const int t = wtid % tiles, pgi = wtid / tiles;
        const int co_base = (t / tiles_k) * CT, k_base = (t % tiles_k) * CT;
        int xoff[CT];   // plane offset of column k: an input plane, the ones or the zero plane
#pragma unroll
        for (int kk = 0; kk < CT; ++kk) {
            const int k = k_base + kk;
            if (k < g.k) {
                const int ci = k / 9, ij = k - ci * 9;
                const int i = ij / 3, j = ij - i * 3;
                xoff[kk] = ci * pt.plane + i * pt.wp + j;
            } else {
                xoff[kk] = (k == g.k ? g.cin : g.cin + 1) * pt.plane;
            }
        }
        const float* gq = gs + co_base * pt.plane + pt.wp + 1;
        float acc[CT][CT];
#pragma unroll
        for (int q = 0; q < CT; ++q)
#pragma unroll
            for (int kk = 0; kk < CT; ++kk) acc[q][kk] = 0.0f;
        // Position p of the tile (row p / W, column p % W) sits at p + (p / W)(wp - W)
        // in a plane; the row is (p + 1/2) * RN(1 / W) rounded down, exact for
        // p < 2^22 / rows.
        const int np = rows * g.w, skip = pt.wp - g.w;
        const float inv_w = 1.0f / float(g.w);
        const auto at = [&](int q) { return q + int((float(q) + 0.5f) * inv_w) * skip; };
        // Positions pgi, pgi + pg, ... in that order, two per round of LDS reads.
        int p = pgi;
        for (; p + pt.pg < np; p += 2 * pt.pg) {
            const int pix0 = at(p), pix1 = at(p + pt.pg);
            float xv[2][CT], dv[2][CT];
#pragma unroll
            for (int kk = 0; kk < CT; ++kk) {
                xv[0][kk] = xs[xoff[kk] + pix0];
                xv[1][kk] = xs[xoff[kk] + pix1];
            }
#pragma unroll
            for (int q = 0; q < CT; ++q) {
                dv[0][q] = gq[q * pt.plane + pix0];
                dv[1][q] = gq[q * pt.plane + pix1];
            }
#pragma unroll
            for (int q = 0; q < CT; ++q)
#pragma unroll
                for (int kk = 0; kk < CT; ++kk) acc[q][kk] = fmaf(dv[0][q], xv[0][kk], acc[q][kk]);
#pragma unroll
            for (int q = 0; q < CT; ++q)
#pragma unroll
                for (int kk = 0; kk < CT; ++kk) acc[q][kk] = fmaf(dv[1][q], xv[1][kk], acc[q][kk]);
        }
        if (p < np) {
            const int pix = at(p);
            float xv[CT], dv[CT];
#pragma unroll
            for (int kk = 0; kk < CT; ++kk) xv[kk] = xs[xoff[kk] + pix];
#pragma unroll
            for (int q = 0; q < CT; ++q) dv[q] = gq[q * pt.plane + pix];
#pragma unroll
            for (int q = 0; q < CT; ++q)
#pragma unroll
                for (int kk = 0; kk < CT; ++kk) acc[q][kk] = fmaf(dv[q], xv[kk], acc[q][kk]);
        }
        float* r = red + (pgi * tiles + t) * (CT * CT);
#pragma unroll
        for (int q = 0; q < CT; ++q)
#pragma unroll
            for (int kk = 0; kk < CT; ++kk) r[q * CT + kk] = acc[q][kk];
    }
    __syncthreads();
    float* pc = partial + (int64_t(n) * pt.tiles + tile) * g.cout * K1;
    const int span = tiles * CT * CT;
    for (int o = tid; o < span; o += NT) {
        float sum = red[o];
        for (int g2 = 1; g2 < pt.pg; ++g2) sum += red[g2 * span + o];
        const int tt = o / (CT * CT), e = o % (CT * CT);
        const int co = (tt / tiles_k) * CT + e / CT, k = (tt % tiles_k) * CT + e % CT;
        if (co < g.cout && k < K1) pc[co * K1 + k] = sum;
    }
}

// Partial weight and bias gradients of one chunk of P output pixels. The
// chunk's gradients (cout x P) and columns ((K + 1) x P, the last column all
// ones so that its row is the bias gradient) are staged in LDS with a padded
// pitch; output o = co (K + 1) + k sums its P products. With fewer outputs
// than threads, G thread groups split the pixels and are combined in group
// order. partial[chunk][o]; the order of every sum depends only on the shape.
__global__ __launch_bounds__(kThreads) void conv_weight_partial(const float* __restrict__ x,
                                                                const float* __restrict__ gout,
                                                                float* __restrict__ partial,
                                                                Geo g, int P) {
    extern __shared__ __align__(16) float sm[];
    const int ld = P + 1;
    const int K1 = g.k + 1;
    float* dy_s = sm;
    float* col_s = sm + g.cout * ld;
    float* red = col_s + K1 * ld;
    const int64_t pixels = int64_t(g.n) * g.oh * g.ow;
    const int64_t plane = int64_t(g.oh) * g.ow;
    const int64_t m0 = int64_t(blockIdx.x) * P;
    stage<8>(g.cout * P, dy_s, [&](int e, int& slot) {
        const int co = e / P, p = e - co * P;
        slot = co * ld + p;
        const int64_t m = m0 + p;
        if (m >= pixels) return 0.0f;
        const unsigned mu = unsigned(m), pl = unsigned(plane);
        const unsigned n = mu / pl, r = mu - n * pl;
        return gout[(int64_t(n) * g.cout + co) * plane + r];
    });
    stage<8>(K1 * P, col_s, [&](int e, int& slot) {
        const int k = e / P, p = e - k * P;
        slot = k * ld + p;
        const int64_t m = m0 + p;
        if (m >= pixels) return 0.0f;
        if (k == g.k) return 1.0f;
        const unsigned mu = unsigned(m);
        const unsigned t = mu / unsigned(g.ow), ow = mu - t * unsigned(g.ow);
        const unsigned n = t / unsigned(g.oh), oh = t - n * unsigned(g.oh);
        const int ij = k % (g.kh * g.kw), ci = k / (g.kh * g.kw);
        const int i = ij / g.kw, j = ij - i * g.kw;
        const int h = int(oh) * g.stride + i - g.pad, v = int(ow) * g.stride + j - g.pad;
        return (h >= 0 && h < g.h && v >= 0 && v < g.w)
                   ? x[((int64_t(n) * g.cin + ci) * g.h + h) * g.w + v]
                   : 0.0f;
    });
    __syncthreads();
    const int O = g.cout * K1;
    float* pc = partial + int64_t(blockIdx.x) * O;
    if (O >= kThreads) {
        for (int o = threadIdx.x; o < O; o += kThreads) {
            const float* a = dy_s + (o / K1) * ld;
            const float* b = col_s + (o % K1) * ld;
            float acc = 0.0f;
            for (int p = 0; p < P; ++p) acc += a[p] * b[p];
            pc[o] = acc;
        }
    } else {
        const int G = kThreads / O;
        const int o = threadIdx.x % O, grp = threadIdx.x / O;
        float acc = 0.0f;
        if (grp < G) {
            const float* a = dy_s + (o / K1) * ld;
            const float* b = col_s + (o % K1) * ld;
            for (int p = grp; p < P; p += G) acc += a[p] * b[p];
        }
        red[threadIdx.x] = acc;
        __syncthreads();
        if (threadIdx.x < O) {
            float s = red[threadIdx.x];
            for (int q = 1; q < G; ++q) s += red[q * O + threadIdx.x];
            pc[threadIdx.x] = s;
        }
    }
}

// dw / db from the partials (partial_sums in common.hpp gives the order).
__device__ __forceinline__ void weight_reduce_block(const float* __restrict__ partial,
                                                    float* __restrict__ dw,
                                                    float* __restrict__ db, int cout, int k,
                                                    int chunks, int rl, int bx, float* lanes) {
    float sum;
    int o;
    const int nb = (cout * (k + 1) + 256 / rl - 1) / (256 / rl);
    if (partial_sums(partial, cout * (k + 1), chunks, rl, xcd_paired_block(bx, nb), lanes, sum,
                     o)) {
        const int co = o / (k + 1), kk = o % (k + 1);
        if (kk < k)
            dw[int64_t(co) * k + kk] = sum;
        else if (db != nullptr)
            db[co] = sum;
    }
}

__global__ __launch_bounds__(256) void conv_weight_reduce(const float* __restrict__ partial,
                                                          float* __restrict__ dw,
                                                          float* __restrict__ db, int cout,
                                                          int k, int chunks, int rl) {
    __shared__ float lanes[256];
    weight_reduce_block(partial, dw, db, cout, k, chunks, rl, int(blockIdx.x), lanes);
}

// Several layers' reductions in one launch: job j owns blocks [first, next
// job's first), each with the rl of its own chunk count -- the same sums as
// one conv_weight_reduce per job.
constexpr int kMaxReduceJobs = 32;

struct ReduceJob {
    const float* partial;
    float* dw;
    float* db;
    int cout, k, chunks, rl, first;
};

struct ReduceBatch {
    ReduceJob job[kMaxReduceJobs];
    int count;
};

__global__ __launch_bounds__(256) void conv_weight_reduce_batch(ReduceBatch b) {
    __shared__ float lanes[256];
    int j = 0;
    while (j + 1 < b.count && int(blockIdx.x) >= b.job[j + 1].first) ++j;
    const ReduceJob& r = b.job[j];
    weight_reduce_block(r.partial, r.dw, r.db, r.cout, r.k, r.chunks, r.rl,
                        int(blockIdx.x) - r.first, lanes);
}

constexpr size_t kTileLds = 48 * 1024;   // bytes of LDS per tiled block

// Rows per tile so that n * groups * tiles reaches about 512 blocks: two per
// CU, whose waves hide each other's LDS and load latency (measured best for
// the cfg2 layers over 128..3584 blocks).
int rows_for_fill(int64_t n_groups, int extent, int64_t target = 512) {
    int64_t tiles = ceil_div(target, n_groups < 1 ? 1 : n_groups);
    if (tiles > extent) tiles = extent;
    if (tiles < 1) tiles = 1;
    return int(ceil_div(extent, tiles));
}

size_t odd_h(size_t v) { return v | 1; }

size_t forward_lds(const Geo& g, int cg, int rows) {
    const size_t rows_in = size_t(rows - 1) * g.stride + g.kh;
    return (size_t(g.cin) * odd_h(rows_in * odd_h(g.w + 2 * g.pad)) + size_t(cg) * g.k) *
           sizeof(float);
}

// Largest number of output-gradient rows any tile of `rows` input rows needs.
int grad_rows_for(const Geo& g, int rows) {
    int most = 0;
    for (int h0 = 0; h0 < g.h; h0 += rows) {
        const int h1 = h0 + rows < g.h ? h0 + rows : g.h;
        int64_t lo, hi, lo2, hi2;
        covering(h0, g.pad, g.kh, g.stride, g.oh, lo, hi);
        covering(h1 - 1, g.pad, g.kh, g.stride, g.oh, lo2, hi2);
        const int r = int(hi2 - lo + 1);
        if (r > most) most = r;
    }
    return most;
}

// Tile edge (CT = KT = t) of the weight-gradient band kernel: the largest of
// 4, 2, 1 that still gives at least 64 tiles, so at most four pixel groups
// share a tile.
int weight_tile(const Geo& g) {
    for (int t : {4, 2}) {
        if (ceil_div(g.cout, t) * ceil_div(g.k + 1, t) >= 64) return t;
    }
    return 1;
}

size_t weight_band_lds(const Geo& g, int rows) {
    const size_t rows_in = size_t(rows - 1) * g.stride + g.kh;
    const size_t np = size_t(rows) * g.ow;
    const int t = weight_tile(g);
    const size_t tiles = size_t(ceil_div(g.cout, t)) * size_t(ceil_div(g.k + 1, t));
    const size_t red = tiles >= kThreads ? 0 : (kThreads / tiles) * tiles * size_t(t * t);
    return (size_t(g.cin) * odd_h(rows_in * odd_h(g.w + 2 * g.pad)) + size_t(g.cout) * odd_h(np) +
            red) *
           sizeof(float);
}

size_t backward_input_lds(const Geo& g, int cg, int rows) {
    return (size_t(g.cout) * odd_h(size_t(grad_rows_for(g, rows)) * g.ow) +
            size_t(g.kh) * g.kw * odd_h(size_t(g.cout) * cg)) *
           sizeof(float);
}

template <int CG>
int forward_tiled(const float* x, const float* wt, const float* bias, float* out, const Geo& g,
                  hipStream_t s) {
    const int groups = int(ceil_div(g.cout, CG));
    int rows = rows_for_fill(int64_t(g.n) * groups, g.oh);
    while (rows > 1 && forward_lds(g, CG, rows) > kTileLds) rows = (rows + 1) / 2;
    const int tiles = int(ceil_div(g.oh, rows));
    const dim3 grid{unsigned(int64_t(g.n) * tiles), unsigned(groups)};
    const size_t lds = forward_lds(g, CG, rows);
    if (g.kh == 3 && g.kw == 3)
        EHIP_LAUNCH("conv2d_forward", (conv_forward_tiled<CG, 3, 3>), grid, dim3(kThreads), lds, s,
                    x, wt, bias, out, g, rows, tiles);
    else
        EHIP_LAUNCH("conv2d_forward", (conv_forward_tiled<CG, 0, 0>), grid, dim3(kThreads), lds, s,
                    x, wt, bias, out, g, rows, tiles);
    return EHIP_OK;
}

template <int CG, bool POOL>
int backward_input_tiled(const float* gout, const PoolGather& pg, const float* wt, float* dx,
                         const Geo& g, hipStream_t s) {
    const int groups = int(ceil_div(g.cin, CG));
    int rows = rows_for_fill(int64_t(g.n) * groups, g.h);
    while (rows > 1 && backward_input_lds(g, CG, rows) > kTileLds) rows = (rows + 1) / 2;
    const int tiles = int(ceil_div(g.h, rows));
    const dim3 grid{unsigned(int64_t(g.n) * tiles), unsigned(groups)};
    EHIP_LAUNCH("conv2d_backward_input", (conv_backward_input_tiled<CG, POOL>), grid,
                dim3(kThreads), backward_input_lds(g, CG, rows), s, gout, pg, wt, dx, g, rows,
                tiles);
    return EHIP_OK;
}

bool input_tiles_fit(const Geo& g) {
    const int cg = g.cin >= 2 ? 2 : 1;
    return backward_input_lds(g, cg, 1) <= kTileLds && int64_t(g.n) * g.h <= 0x7fffffff;
}

// The input gradient; POOL gathers the output gradient through a fused pool.
template <bool POOL>
int backward_input(const float* gout, const PoolGather& pg, const float* wt, float* dx,
                   const Geo& g, hipStream_t s) {
    const int64_t n_in = int64_t(g.n) * g.cin * g.h * g.w;
    if (n_in == 0) return EHIP_OK;
    if (input_tiles_fit(g)) {
        if (g.cin >= 2) return backward_input_tiled<2, POOL>(gout, pg, wt, dx, g, s);
        return backward_input_tiled<1, POOL>(gout, pg, wt, dx, g, s);
    }
    if (POOL) return fail(EHIP_EINVAL, "conv2d: the fused pool needs LDS tiles");
    int64_t grid = ceil_div(n_in, kThreads);
    if (grid > 65536) grid = 65536;
    const size_t lds = size_t(g.cout) * g.k * sizeof(float);
    EHIP_LAUNCH("conv2d_backward_input", conv_backward_input_direct, dim3(unsigned(grid)),
                dim3(kThreads), lds, s, gout, wt, dx, g);
    return EHIP_OK;
}

int band_rows(const Geo& g, int64_t target = 512) {
    int rows = rows_for_fill(g.n, g.oh, target);
    while (rows > 1 && weight_band_lds(g, rows) > kTileLds) rows = (rows + 1) / 2;
    return rows;
}

bool weight_bands_fit(const Geo& g) {
    return weight_band_lds(g, band_rows(g)) <= kTileLds && int64_t(g.n) * g.oh <= 0x7fffffff;
}

template <int T, bool POOL>
int launch_band(const float* x, const float* gout, const PoolGather& pg, float* partial,
                const Geo& g, int rows, int bands, hipStream_t s) {
    EHIP_LAUNCH("conv2d_weight_band", (conv_weight_band<T, T, POOL>),
                dim3(unsigned(int64_t(g.n) * bands)), dim3(kThreads), weight_band_lds(g, rows), s,
                x, gout, pg, partial, g, rows, bands);
    return EHIP_OK;
}

// dweight / dbias from the per-band (or per-chunk) partials, in chunk order.

int weight_reduce(const float* partial, float* dweight, float* dbias, const Geo& g,
                  int64_t chunks, hipStream_t s) {
    const int O = g.cout * (g.k + 1);
    const int rl = reduce_lanes(chunks);
    const int per_block = 256 / rl;
    EHIP_LAUNCH("conv2d_weight_reduce", conv_weight_reduce, dim3(unsigned(ceil_div(O, per_block))),
                dim3(256), 0, s, partial, dweight, dbias, g.cout, g.k, int(chunks), rl);
    return EHIP_OK;
}

// Weight and bias gradients: per-band (or per-chunk) partials, then their
// ordered reduction. POOL gathers the output gradient through a fused pool.
template <bool POOL>
int backward_weight(const float* x, const float* gout, const PoolGather& pg, float* dweight,
                    float* dbias, const Geo& g, hipStream_t s) {
    const int64_t pixels = int64_t(g.n) * g.oh * g.ow;
    const int O = g.cout * (g.k + 1);
    if (pixels == 0) {
        if (int rc = ehip_fill_f32(dweight, int64_t(g.cout) * g.k, 0.0f, s)) return rc;
        return dbias ? ehip_fill_f32(dbias, g.cout, 0.0f, s) : EHIP_OK;
    }
    int64_t chunks = 0;
    float* partial = nullptr;
    // Bands of output rows (one image each, about 512 blocks) when a band's
    // input rows and gradient rows fit in LDS; otherwise chunks of P pixels
    // with their im2col columns staged.
    if (weight_bands_fit(g)) {
        const int rows = band_rows(g);
        const int bands = int(ceil_div(g.oh, rows));
        chunks = int64_t(g.n) * bands;
        partial = static_cast<float*>(scratch(size_t(chunks) * O * sizeof(float)));
        if (partial == nullptr) return EHIP_ENOMEM;
        const int t = weight_tile(g);
        const int rc = t == 4   ? launch_band<4, POOL>(x, gout, pg, partial, g, rows, bands, s)
                       : t == 2 ? launch_band<2, POOL>(x, gout, pg, partial, g, rows, bands, s)
                                : launch_band<1, POOL>(x, gout, pg, partial, g, rows, bands, s);
        if (rc != EHIP_OK) return rc;
    } else {
        if (POOL) return fail(EHIP_EINVAL, "conv2d: the fused pool needs LDS bands");
        // Chunk size: about 256 chunks to fill the CUs, 16..256 pixels each, and
        // the staged chunk within the LDS budget.
        int P = 16;
        while (P < 256 && ceil_div(pixels, P) > 256) P *= 2;
        const auto lds_for = [&](int p) {
            return (size_t(g.cout) + size_t(g.k) + 1) * size_t(p + 1) * sizeof(float) +
                   kThreads * sizeof(float);
        };
        while (P > 1 && lds_for(P) > kMaxLds) P /= 2;
        chunks = ceil_div(pixels, P);
        if (chunks > 0x7fffffff)
            return fail(EHIP_EINVAL, "conv2d_backward_weight: too many pixels");
        partial = static_cast<float*>(scratch(size_t(chunks) * O * sizeof(float)));
        if (partial == nullptr) return EHIP_ENOMEM;
        EHIP_LAUNCH("conv2d_weight_partial", conv_weight_partial, dim3(unsigned(chunks)),
                    dim3(kThreads), lds_for(P), s, x, gout, partial, g, P);
    }
    return weight_reduce(partial, dweight, dbias, g, chunks, s);
}

// The input and weight gradients of a fused conv block in one launch
// (conv_backward_pair), then the weight partials' reduction. Needs both
// tiled paths to fit.
template <int CG, int T>
int launch_pair(const float* x, const PoolGather& pg, const float* wt, float* dx, float* partial,
                const Geo& g, const PairGeo& pr, size_t lds, hipStream_t s) {
    EHIP_LAUNCH("conv2d_backward_pair", (conv_backward_pair<CG, T, true>),
                dim3(unsigned(pr.in_blocks + int64_t(g.n) * pr.bands)), dim3(kThreads), lds, s, x,
                static_cast<const float*>(nullptr), pg, wt, dx, partial, g, pr);
    return EHIP_OK;
}

int backward_pair(const float* x, const PoolGather& pg, const float* wt, float* dx,
                  float* dweight, float* dbias, const Geo& g, hipStream_t s) {
    const int cg = g.cin >= 2 ? 2 : 1;
    const int groups = int(ceil_div(g.cin, cg));
    int in_rows = rows_for_fill(int64_t(g.n) * groups, g.h);
    while (in_rows > 1 && backward_input_lds(g, cg, in_rows) > kTileLds) in_rows = (in_rows + 1) / 2;
    PairGeo pr{};
    pr.in_rows = in_rows;
    pr.in_tiles = int(ceil_div(g.h, in_rows));
    pr.in_x = g.n * pr.in_tiles;
    pr.in_blocks = pr.in_x * groups;
    // The usual band count: a quarter (fewer partials) measured 23 us per launch
    // pair and twice as many 25 us, against 20 us here.
    pr.band_rows = band_rows(g);
    pr.bands = int(ceil_div(g.oh, pr.band_rows));
    const int64_t chunks = int64_t(g.n) * pr.bands;
    if (int64_t(pr.in_blocks) + chunks > 0x7fffffff)
        return fail(EHIP_EINVAL, "conv2d_relu_maxpool_backward: too many blocks");
    const int O = g.cout * (g.k + 1);
    float* partial = static_cast<float*>(scratch(size_t(chunks) * O * sizeof(float)));
    if (partial == nullptr) return EHIP_ENOMEM;
    const size_t lds = std::max(backward_input_lds(g, cg, in_rows), weight_band_lds(g, pr.band_rows));
    const int t = weight_tile(g);
    int rc;
    if (cg == 2)
        rc = t == 4   ? launch_pair<2, 4>(x, pg, wt, dx, partial, g, pr, lds, s)
             : t == 2 ? launch_pair<2, 2>(x, pg, wt, dx, partial, g, pr, lds, s)
                      : launch_pair<2, 1>(x, pg, wt, dx, partial, g, pr, lds, s);
    else
        rc = t == 4   ? launch_pair<1, 4>(x, pg, wt, dx, partial, g, pr, lds, s)
             : t == 2 ? launch_pair<1, 2>(x, pg, wt, dx, partial, g, pr, lds, s)
                      : launch_pair<1, 1>(x, pg, wt, dx, partial, g, pr, lds, s);
    if (rc != EHIP_OK) return rc;
    return weight_reduce(partial, dweight, dbias, g, chunks, s);
}

// The fused 3 x 3 tile path: a stride-1, padding-1, 3 x 3 convolution (its
// output as large as its input) and a tile configuration.
bool conv3_same(const Geo& g) {
    return g.kh == 3 && g.kw == 3 && g.stride == 1 && g.pad == 1 && g.oh == g.h && g.ow == g.w;
}

struct PoolTileCfg {
    int rows;         // convolution rows per tile (a multiple of pk)
    int cg, ct, nt;   // input channels per dx thread, weight tile edge, threads per block
    int dx_threads;   // threads computing dx when dx is wanted
};

int weight_tiles(const Geo& g, int ct) {
    return int(ceil_div(g.cout, ct) * ceil_div(g.k + 1, ct));
}

// Fills `pt` and the LDS bytes for `c`; false when the configuration does not
// fit (too little LDS, too few weight threads, misaligned rows).
bool pool_tile_plan(const Geo& g, int pk, const PoolTileCfg& c, bool want_dx, bool want_dw,
                    PoolTile& pt, size_t& lds) {
    if (c.rows < pk || c.rows % pk != 0 || c.rows > g.h + pk) return false;
    pt = PoolTile{};
    pt.rows = c.rows;
    pt.tiles = int(ceil_div(g.h, c.rows));
    pt.dx_threads = want_dx ? c.dx_threads : 0;
    if (want_dx && (c.dx_threads < 64 || c.dx_threads % 64 != 0 || c.dx_threads > c.nt))
        return false;
    const int tiles = weight_tiles(g, c.ct);
    const int wthreads = c.nt - pt.dx_threads;
    if (want_dw) {
        if (tiles > wthreads) return false;
        pt.pg = wthreads / tiles;
    }
    pt.wp = int(odd_h(size_t(g.w) + 2));
    pt.plane = int(odd_h(size_t(c.rows + 2) * pt.wp));
    pt.cinp = int(ceil_div(g.cin, c.cg) * c.cg);
    pt.prows = c.rows / pk + 2;
    pt.pw = fast_div(uint32_t(std::max(g.w / pk, 1)));
    pt.fprows = fast_div(uint32_t(pt.prows));
    pt.wcols = fast_div(uint32_t(g.w + 2));
    pt.srows = fast_div(uint32_t(c.rows + 2));
    pt.cin = fast_div(uint32_t(g.cin));
    pt.npx = fast_div(uint32_t(c.rows * g.w));
    pt.w = fast_div(uint32_t(g.w));
    int64_t off = (want_dw ? ceil_div(g.cout, c.ct) * c.ct : int64_t(g.cout)) * pt.plane;
    pt.xs_off = int(off);
    if (want_dw) off += int64_t(g.cin + 2) * pt.plane;
    off = ceil_div(off, 4) * 4;
    pt.ws_off = int(off);
    if (want_dx) off += int64_t(g.cout) * (pt.cinp / c.cg) * ((9 * c.cg + 3) / 4 * 4);
    pt.red_off = int(off);
    if (want_dw)
        off += std::max<int64_t>(int64_t(pt.pg) * tiles * c.ct * c.ct, 4 * int64_t(wthreads));
    pt.own = c.rows / pk;
    pt.cells = want_dw ? g.cout * pt.own * (g.w / pk) : 0;
    pt.cell_off = int(off);
    off += 2 * int64_t(pt.cells);
    lds = size_t(off) * sizeof(float);
    return lds <= kTileLds && int64_t(g.n) * pt.tiles <= 0x7fffffff;
}

template <int CG, int CT, int NT>
int launch_pool_tile(const float* x, const float* wt, const PoolGather& pg, float* dx,
                     float* partial, const Geo& g, const PoolTile& pt, size_t lds, hipStream_t s) {
    EHIP_LAUNCH("conv2d_relu_maxpool_backward", (conv3_pool_backward<CG, CT, NT>),
                dim3(unsigned(int64_t(g.n) * pt.tiles)), dim3(NT), lds, s, x, wt, pg, dx, partial,
                g, pt);
    return EHIP_OK;
}

template <int CG, int CT>
int launch_pool_tile_nt(const float* x, const float* wt, const PoolGather& pg, float* dx,
                        float* partial, const Geo& g, const PoolTile& pt, size_t lds, int nt,
                        hipStream_t s) {
    if (nt == 512) return launch_pool_tile<CG, CT, 512>(x, wt, pg, dx, partial, g, pt, lds, s);
    return launch_pool_tile<CG, CT, 256>(x, wt, pg, dx, partial, g, pt, lds, s);
}

template <int CG>
int launch_pool_tile_ct(const float* x, const float* wt, const PoolGather& pg, float* dx,
                        float* partial, const Geo& g, const PoolTile& pt, size_t lds,
                        const PoolTileCfg& c, hipStream_t s) {
    if (c.ct == 4) return launch_pool_tile_nt<CG, 4>(x, wt, pg, dx, partial, g, pt, lds, c.nt, s);
    if (c.ct == 2) return launch_pool_tile_nt<CG, 2>(x, wt, pg, dx, partial, g, pt, lds, c.nt, s);
    return launch_pool_tile_nt<CG, 1>(x, wt, pg, dx, partial, g, pt, lds, c.nt, s);
}

int pool_tile_launch(const float* x, const PoolGather& pg, const float* wt, float* dx,
                     float* partial, const Geo& g, const PoolTileCfg& c, const PoolTile& pt,
                     size_t lds, hipStream_t s) {
    return c.cg == 4   ? launch_pool_tile_ct<4>(x, wt, pg, dx, partial, g, pt, lds, c, s)
           : c.cg == 2 ? launch_pool_tile_ct<2>(x, wt, pg, dx, partial, g, pt, lds, c, s)
                       : launch_pool_tile_ct<1>(x, wt, pg, dx, partial, g, pt, lds, c, s);
}

// Input gradient (dx may be null) and weight + bias gradients (dweight may be
// null) of a fused 3 x 3 block with configuration `c`: one tile launch, then
// the partials' ordered reduction.
int pool_tile_backward(const float* x, const PoolGather& pg, const float* wt, float* dx,
                       float* dweight, float* dbias, const Geo& g, const PoolTileCfg& c,
                       const PoolTile& pt, size_t lds, hipStream_t s) {
    const int64_t chunks = int64_t(g.n) * pt.tiles;
    float* partial = nullptr;
    if (dweight != nullptr) {
        partial = static_cast<float*>(scratch(size_t(chunks) * g.cout * (g.k + 1) * sizeof(float)));
        if (partial == nullptr) return EHIP_ENOMEM;
    }
    const int rc = pool_tile_launch(x, pg, wt, dx, partial, g, c, pt, lds, s);
    if (rc != EHIP_OK || dweight == nullptr) return rc;
    return weight_reduce(partial, dweight, dbias, g, chunks, s);
}

// The tile configuration for a layer: about one 512-thread block per CU
// (fewer rows per tile only when the LDS needs it), two input channels per dx
// thread, the largest weight tile that still gives 16 tiles, and enough dx
// threads for one item each (measured best for the cfg2 layers over rows
// 2..8, 1..4 channels per thread, tiles 1..4, 256 or 512 threads and every dx
// thread count). Returns false when no configuration fits.
bool pool_tile_choice(const Geo& g, int pk, bool want_dx, bool want_dw, PoolTileCfg& c,
                      PoolTile& pt, size_t& lds) {
    c = PoolTileCfg{};
    c.nt = 512;
    c.cg = g.cin >= 2 ? 2 : 1;
    c.ct = 1;
    for (int t : {4, 2})
        if (weight_tiles(g, t) >= 16) {
            c.ct = t;
            break;
        }
    const int64_t per_image = std::min<int64_t>(ceil_div(256, std::max(g.n, 1)), std::max(g.h, 1));
    int rows = int(ceil_div(ceil_div(g.h, per_image), pk) * pk);
    for (;;) {
        c.rows = rows;
        const int64_t items = int64_t(rows) * g.w * ceil_div(g.cin, c.cg);
        const int64_t reserve = want_dw ? ceil_div(weight_tiles(g, c.ct), 64) * 64 : 0;
        const int64_t room = c.nt - reserve;
        c.dx_threads = !want_dx ? 0 : int(std::max<int64_t>(64, std::min(ceil_div(items, 64) * 64, room)));
        if (pool_tile_plan(g, pk, c, want_dx, want_dw, pt, lds)) return true;
        if (rows <= pk) return false;
        rows = std::max(pk, rows / 2 / pk * pk);
    }
}

// The 3 x 3 forward tile: `rows` convolution rows per block, CG output
// channels per thread. False when it does not fit the LDS budget.
bool pool_fwd_plan(const Geo& g, int pk, int rows, int cg, PoolFwdTile& ft, size_t& lds) {
    if (rows < pk || rows % pk != 0 || rows > g.h + pk) return false;
    ft = PoolFwdTile{};
    ft.rows = rows;
    ft.tiles = int(ceil_div(g.h, rows));
    ft.wp = int(odd_h(size_t(g.w) + 2));
    ft.plane = int(odd_h(size_t(rows + 2) * ft.wp));
    ft.coutp = int(ceil_div(g.cout, cg) * cg);
    int64_t off = ceil_div(int64_t(g.cin) * ft.plane, 4) * 4;
    ft.ws_off = int(off);
    off += int64_t(g.k) * ft.coutp;
    ft.ys_off = int(off);
    off += int64_t(g.cout) * rows * g.w;
    lds = size_t(off) * sizeof(float);
    ft.wcols = fast_div(uint32_t(g.w + 2));
    ft.srows = fast_div(uint32_t(rows + 2));
    ft.fcoutp = fast_div(uint32_t(ft.coutp));
    ft.npx = fast_div(uint32_t(rows * g.w));
    ft.w = fast_div(uint32_t(g.w));
    ft.pw = fast_div(uint32_t(std::max(g.w / pk, 1)));
    ft.prows = fast_div(uint32_t(rows / pk));
    return lds <= kTileLds && int64_t(g.n) * ft.tiles <= 0x7fffffff;
}

template <int CG, int NT>
int launch_pool_fwd(const float* x, const float* wt, const float* bias, float* pooled,
                    int32_t* argmax, const Geo& g, int pk, int ph, int pw, const PoolFwdTile& ft,
                    size_t lds, hipStream_t s) {
    EHIP_LAUNCH("conv2d_relu_maxpool", (conv3_relu_pool<CG, NT>),
                dim3(unsigned(int64_t(g.n) * ft.tiles)), dim3(NT), lds, s, x, wt, bias, pooled,
                argmax, g, pk, ph, pw, ft);
    return EHIP_OK;
}

int pool_fwd_launch(const float* x, const float* wt, const float* bias, float* pooled,
                    int32_t* argmax, const Geo& g, int pk, int ph, int pw, const PoolFwdTile& ft,
                    size_t lds, int cg, int nt, hipStream_t s) {
    if (nt == 256) {
        if (cg == 4) return launch_pool_fwd<4, 256>(x, wt, bias, pooled, argmax, g, pk, ph, pw, ft, lds, s);
        if (cg == 2) return launch_pool_fwd<2, 256>(x, wt, bias, pooled, argmax, g, pk, ph, pw, ft, lds, s);
        return launch_pool_fwd<1, 256>(x, wt, bias, pooled, argmax, g, pk, ph, pw, ft, lds, s);
    }
    if (cg == 4) return launch_pool_fwd<4, 512>(x, wt, bias, pooled, argmax, g, pk, ph, pw, ft, lds, s);
    if (cg == 2) return launch_pool_fwd<2, 512>(x, wt, bias, pooled, argmax, g, pk, ph, pw, ft, lds, s);
    return launch_pool_fwd<1, 512>(x, wt, bias, pooled, argmax, g, pk, ph, pw, ft, lds, s);
}

// Rows per tile for about one 512-thread block per CU (fewer when the LDS
// needs it) and the fewest output channels per thread that keep a tile's
// items within the block (measured best for the cfg2 layers over rows 2..8,
// 1..4 channels per thread and 256 or 512 threads). Returns the rows, or 0
// when no tile fits.
int pool_fwd_choice(const Geo& g, int pk, int& cg, PoolFwdTile& ft, size_t& lds) {
    const int64_t per_image = std::min<int64_t>(ceil_div(256, std::max(g.n, 1)), std::max(g.h, 1));
    int rows = int(ceil_div(ceil_div(g.h, per_image), pk) * pk);
    for (;;) {
        cg = 4;
        for (int c : {1, 2})
            if (int64_t(rows) * g.w * ceil_div(g.cout, c) <= 512) {
                cg = c;
                break;
            }
        if (pool_fwd_plan(g, pk, rows, cg, ft, lds)) return rows;
        if (rows <= pk) return 0;
        rows = std::max(pk, rows / 2 / pk * pk);
    }
}

size_t pool_forward_lds(const Geo& g, int cg, int pk, int pw, int prows) {
    const size_t crows = size_t(prows) * pk;
    const size_t rows_in = (crows - 1) * g.stride + g.kh;
    return (size_t(cg) * g.k + size_t(g.cin) * odd_h(rows_in * odd_h(g.w + 2 * g.pad)) +
            size_t(cg) * crows * size_t(pw) * pk) *
           sizeof(float);
}

// Validates the pool window of a fused Conv2d -> ReLU -> MaxPool2d: disjoint
// square windows (kernel == stride, no padding) over the convolution output.
int check_pool(const char* name, const ehip_window_t* c, int64_t cout, const ehip_window_t* p) {
    if (int rc = check_window(name, p)) return rc;
    if (p->kernel_h != p->kernel_w || p->kernel_h != p->stride || p->padding != 0)
        return fail(EHIP_EINVAL, "%s: the pool must have kernel == stride and no padding", name);
    if (p->batch != c->batch || p->channels != cout || p->height != c->out_h ||
        p->width != c->out_w)
        return fail(EHIP_EINVAL, "%s: the pool window does not match the convolution output",
                    name);
    return EHIP_OK;
}

bool fused_fits(const Geo& g, const ehip_window_t& p) {
    const int cg = g.cout >= 3 ? 4 : g.cout;
    return pool_forward_lds(g, cg, int(p.kernel_h), int(p.out_w), 1) <= kTileLds &&
           input_tiles_fit(g) && weight_bands_fit(g) && int64_t(g.n) * g.oh <= 0x7fffffff;
}

template <int CG>
int pool_forward_tiled(const float* x, const float* wt, const float* bias, float* pooled,
                       int32_t* argmax, const Geo& g, int pk, int ph, int pw, hipStream_t s) {
    const int groups = int(ceil_div(g.cout, CG));
    int prows = rows_for_fill(int64_t(g.n) * groups, ph);
    while (prows > 1 && pool_forward_lds(g, CG, pk, pw, prows) > kTileLds) prows = (prows + 1) / 2;
    const int tiles = int(ceil_div(ph, prows));
    const dim3 grid{unsigned(int64_t(g.n) * tiles), unsigned(groups)};
    const size_t lds = pool_forward_lds(g, CG, pk, pw, prows);
    if (g.kh == 3 && g.kw == 3)
        EHIP_LAUNCH("conv2d_relu_maxpool", (conv_relu_pool_tiled<CG, 3, 3>), grid, dim3(kThreads),
                    lds, s, x, wt, bias, pooled, argmax, g, pk, ph, pw, prows, tiles);
    else
        EHIP_LAUNCH("conv2d_relu_maxpool", (conv_relu_pool_tiled<CG, 0, 0>), grid, dim3(kThreads),
                    lds, s, x, wt, bias, pooled, argmax, g, pk, ph, pw, prows, tiles);
    return EHIP_OK;
}

int check_conv(const char* name, const ehip_window_t* w, int64_t cout) {
    if (int rc = check_window(name, w)) return rc;
    if (cout <= 0) return fail(EHIP_EINVAL, "%s: out_channels must be positive", name);
    const int64_t k = w->channels * w->kernel_h * w->kernel_w;
    if (cout * k > kMaxWeights)
        return fail(EHIP_EINVAL,
                    "%s: out_channels * C_in * kH * kW = %lld exceeds the direct path's %lld",
                    name, (long long)(cout * k), (long long)kMaxWeights);
    const int64_t n_in = w->batch * w->channels * w->height * w->width;
    const int64_t n_out = w->batch * cout * w->out_h * w->out_w;
    if (n_in > 0x7fffffff || n_out > 0x7fffffff)
        return fail(EHIP_EINVAL, "%s: tensors beyond 2^31 elements", name);
    return EHIP_OK;
}

const OccupancyKernel kConvKernels[] = {
    {"conv_weight_reduce", reinterpret_cast<const void*>(&conv_weight_reduce), 256},
    {"conv_weight_reduce_batch", reinterpret_cast<const void*>(&conv_weight_reduce_batch), 256},
};
const OccupancyEntries kConvKernelsReg(kConvKernels);

}  // namespace
}  // namespace ehip

using namespace ehip;

extern "C" {

int ehip_conv2d_direct_supported(const ehip_window_t* w, int64_t out_channels) {
    if (w == nullptr || out_channels <= 0) return 0;
    return out_channels * w->channels * w->kernel_h * w->kernel_w <= kMaxWeights ? 1 : 0;
}

int ehip_conv2d_forward_f32(const float* x, const float* weight, const float* bias, float* out,
                            const ehip_window_t* w, int64_t out_channels, void* stream) {
    EHIP_READY();
    if (int rc = check_conv("conv2d_forward", w, out_channels)) return rc;
    if (!x || !weight || !out) return fail(EHIP_EINVAL, "conv2d_forward: null pointer");
    const Geo g = geo_of(*w, out_channels);
    const int64_t pixels = int64_t(g.n) * g.oh * g.ow;
    if (pixels == 0) return EHIP_OK;
    hipStream_t s = as_stream(stream);
    // LDS tiles when one input row band fits; the per-pixel kernel otherwise.
    const int cg = g.cout >= 3 ? 4 : g.cout;
    if (forward_lds(g, cg, 1) <= kTileLds && int64_t(g.n) * g.oh <= 0x7fffffff) {
        if (cg == 4) return forward_tiled<4>(x, weight, bias, out, g, s);
        if (cg == 2) return forward_tiled<2>(x, weight, bias, out, g, s);
        return forward_tiled<1>(x, weight, bias, out, g, s);
    }
    const dim3 grid{unsigned(ceil_div(pixels, kThreads)), unsigned(ceil_div(g.cout, kCoGroup))};
    EHIP_LAUNCH("conv2d_forward", conv_forward_direct, grid, dim3(kThreads), 0, s, x, weight, bias,
                out, g);
    return EHIP_OK;
}

int ehip_conv2d_backward_input_f32(const float* grad_out, const float* weight, float* dx,
                                   const ehip_window_t* w, int64_t out_channels, void* stream) {
    EHIP_READY();
    if (int rc = check_conv("conv2d_backward_input", w, out_channels)) return rc;
    if (!grad_out || !weight || !dx) return fail(EHIP_EINVAL, "conv2d_backward_input: null pointer");
    return backward_input<false>(grad_out, PoolGather{}, weight, dx, geo_of(*w, out_channels),
                                 as_stream(stream));
}

int ehip_conv2d_backward_weight_f32(const float* x, const float* grad_out, float* dweight,
                                    float* dbias, const ehip_window_t* w, int64_t out_channels,
                                    void* stream) {
    EHIP_READY();
    if (int rc = check_conv("conv2d_backward_weight", w, out_channels)) return rc;
    if (!x || !grad_out || !dweight)
        return fail(EHIP_EINVAL, "conv2d_backward_weight: null pointer");
    return backward_weight<false>(x, grad_out, PoolGather{}, dweight, dbias,
                                  geo_of(*w, out_channels), as_stream(stream));
}

int ehip_conv2d_relu_maxpool_supported(const ehip_window_t* conv, int64_t out_channels,
                                       const ehip_window_t* pool) {
    if (conv == nullptr || pool == nullptr || out_channels <= 0) return 0;
    if (!ehip_conv2d_direct_supported(conv, out_channels)) return 0;
    if (pool->kernel_h != pool->kernel_w || pool->kernel_h != pool->stride || pool->padding != 0 ||
        pool->kernel_h <= 0)
        return 0;
    if (pool->batch != conv->batch || pool->channels != out_channels ||
        pool->height != conv->out_h || pool->width != conv->out_w)
        return 0;
    const int64_t n_out = conv->batch * out_channels * conv->out_h * conv->out_w;
    if (n_out > 0x7fffffff) return 0;
    return fused_fits(geo_of(*conv, out_channels), *pool) ? 1 : 0;
}

int ehip_conv2d_relu_maxpool_f32(const float* x, const float* weight, const float* bias,
                                 float* out, int32_t* argmax, const ehip_window_t* conv,
                                 int64_t out_channels, const ehip_window_t* pool, void* stream) {
    EHIP_READY();
    if (int rc = check_conv("conv2d_relu_maxpool", conv, out_channels)) return rc;
    if (int rc = check_pool("conv2d_relu_maxpool", conv, out_channels, pool)) return rc;
    if (!x || !weight || !out || !argmax)
        return fail(EHIP_EINVAL, "conv2d_relu_maxpool: null pointer");
    const Geo g = geo_of(*conv, out_channels);
    if (!fused_fits(g, *pool))
        return fail(EHIP_EINVAL, "conv2d_relu_maxpool: the layer does not fit the LDS tiles");
    const int pk = int(pool->kernel_h), ph = int(pool->out_h), pw = int(pool->out_w);
    if (int64_t(g.n) * g.cout * ph * pw == 0) return EHIP_OK;
    hipStream_t s = as_stream(stream);
    // 3 x 3 "same" convolutions: every output channel of a tile in one block.
    if (conv3_same(g)) {
        PoolFwdTile ft;
        size_t lds = 0;
        int cgf = 0;
        const int rows = pool_fwd_choice(g, pk, cgf, ft, lds);
        if (rows > 0)
            return pool_fwd_launch(x, weight, bias, out, argmax, g, pk, ph, pw, ft, lds, cgf, 512, s);
    }
    const int cg = g.cout >= 3 ? 4 : g.cout;
    if (cg == 4) return pool_forward_tiled<4>(x, weight, bias, out, argmax, g, pk, ph, pw, s);
    if (cg == 2) return pool_forward_tiled<2>(x, weight, bias, out, argmax, g, pk, ph, pw, s);
    return pool_forward_tiled<1>(x, weight, bias, out, argmax, g, pk, ph, pw, s);
}

int ehip_conv2d_relu_maxpool_backward_f32(const float* x, const float* weight,
                                          const float* grad_out, const float* out,
                                          const int32_t* argmax, float* dx, float* dweight,
                                          float* dbias, const ehip_window_t* conv,
                                          int64_t out_channels, const ehip_window_t* pool,
                                          void* stream) {
    EHIP_READY();
    if (int rc = check_conv("conv2d_relu_maxpool_backward", conv, out_channels)) return rc;
    if (int rc = check_pool("conv2d_relu_maxpool_backward", conv, out_channels, pool)) return rc;
    if (!grad_out || !out || !argmax || (dx && !weight) || ((dweight || dbias) && !x))
        return fail(EHIP_EINVAL, "conv2d_relu_maxpool_backward: null pointer");
    if (dbias && !dweight)
        return fail(EHIP_EINVAL, "conv2d_relu_maxpool_backward: dbias needs dweight");
    const Geo g = geo_of(*conv, out_channels);
    if (!fused_fits(g, *pool))
        return fail(EHIP_EINVAL, "conv2d_relu_maxpool_backward: the layer does not fit the LDS tiles");
    const PoolGather pg{grad_out, out, argmax, int(pool->kernel_h), int(pool->out_h),
                        int(pool->out_w)};
    hipStream_t s = as_stream(stream);
    if (!dx && !dweight) return EHIP_OK;
    if (int64_t(g.n) * g.h * g.w == 0) {
        if (dweight) {
            if (int rc = ehip_fill_f32(dweight, int64_t(g.cout) * g.k, 0.0f, s)) return rc;
            if (dbias) return ehip_fill_f32(dbias, g.cout, 0.0f, s);
        }
        return EHIP_OK;
    }
    // 3 x 3 "same" convolutions: one tile launch for dx and the weight partials.
    if (conv3_same(g)) {
        PoolTileCfg c;
        PoolTile pt;
        size_t lds = 0;
        if (pool_tile_choice(g, pg.pk, dx != nullptr, dweight != nullptr, c, pt, lds))
            return pool_tile_backward(x, pg, weight, dx, dweight, dbias, g, c, pt, lds, s);
    }
    if (dx && dweight && input_tiles_fit(g) && weight_bands_fit(g))
        return backward_pair(x, pg, weight, dx, dweight, dbias, g, s);
    if (dx)
        if (int rc = backward_input<true>(nullptr, pg, weight, dx, g, s)) return rc;
    if (dweight) return backward_weight<true>(x, nullptr, pg, dweight, dbias, g, s);
    return EHIP_OK;
}

int64_t ehip_conv2d_relu_maxpool_partials(const ehip_window_t* conv, int64_t out_channels,
                                          const ehip_window_t* pool, int want_dx,
                                          int64_t* chunks) {
    if (chunks != nullptr) *chunks = 0;
    if (!ehip_conv2d_relu_maxpool_supported(conv, out_channels, pool)) return 0;
    if (check_window("conv2d_relu_maxpool_partials", conv) != EHIP_OK ||
        check_window("conv2d_relu_maxpool_partials", pool) != EHIP_OK)
        return 0;
    const Geo g = geo_of(*conv, out_channels);
    if (!conv3_same(g) || int64_t(g.n) * g.h * g.w == 0) return 0;
    PoolTileCfg c;
    PoolTile pt;
    size_t lds = 0;
    if (!pool_tile_choice(g, int(pool->kernel_h), want_dx != 0, true, c, pt, lds)) return 0;
    const int64_t ch = int64_t(g.n) * pt.tiles;
    if (chunks != nullptr) *chunks = ch;
    return ch * g.cout * (g.k + 1);
}

int ehip_conv2d_relu_maxpool_backward_partials_f32(
    const float* x, const float* weight, const float* grad_out, const float* out,
    const int32_t* argmax, float* dx, float* partials, int64_t chunks, const ehip_window_t* conv,
    int64_t out_channels, const ehip_window_t* pool, void* stream) {
    EHIP_READY();
    const char* name = "conv2d_relu_maxpool_backward_partials";
    if (int rc = check_conv(name, conv, out_channels)) return rc;
    if (int rc = check_pool(name, conv, out_channels, pool)) return rc;
    if (!x || !weight || !grad_out || !out || !argmax || !partials)
        return fail(EHIP_EINVAL, "%s: null pointer", name);
    const Geo g = geo_of(*conv, out_channels);
    PoolTileCfg c;
    PoolTile pt;
    size_t lds = 0;
    if (!fused_fits(g, *pool) || !conv3_same(g) || int64_t(g.n) * g.h * g.w == 0 ||
        !pool_tile_choice(g, int(pool->kernel_h), dx != nullptr, true, c, pt, lds))
        return fail(EHIP_EINVAL, "%s: the layer has no tile partials "
                    "(ehip_conv2d_relu_maxpool_partials returned 0)", name);
    if (chunks != int64_t(g.n) * pt.tiles)
        return fail(EHIP_EINVAL, "%s: %lld chunks given, the tile plan has %lld", name,
                    (long long)chunks, (long long)(int64_t(g.n) * pt.tiles));
    const PoolGather pg{grad_out, out, argmax, int(pool->kernel_h), int(pool->out_h),
                        int(pool->out_w)};
    return pool_tile_launch(x, pg, weight, dx, partials, g, c, pt, lds, as_stream(stream));
}

int ehip_conv_weight_reduce_f32(const ehip_conv_reduce_t* jobs, int count, void* stream) {
    EHIP_READY();
    if (count < 0 || (count > 0 && jobs == nullptr))
        return fail(EHIP_EINVAL, "conv_weight_reduce: bad job list");
    hipStream_t s = as_stream(stream);
    for (int first = 0; first < count; first += kMaxReduceJobs) {
        ReduceBatch b{};
        int64_t blocks = 0;
        for (int j = first; j < count && b.count < kMaxReduceJobs; ++j) {
            const ehip_conv_reduce_t& q = jobs[j];
            if (!q.partials || !q.dweight || q.chunks <= 0 || q.out_channels <= 0 || q.k <= 0 ||
                q.chunks > 0x7fffffff || q.out_channels * (q.k + 1) > 0x7fffffff)
                return fail(EHIP_EINVAL, "conv_weight_reduce: bad job %d", j);
            ReduceJob& r = b.job[b.count++];
            r.partial = q.partials;
            r.dw = q.dweight;
            r.db = q.dbias;
            r.cout = int(q.out_channels);
            r.k = int(q.k);
            r.chunks = int(q.chunks);
            r.rl = reduce_lanes(q.chunks);
            r.first = int(blocks);
            blocks += ceil_div(q.out_channels * (q.k + 1), 256 / r.rl);
        }
        if (blocks > 0x7fffffff) return fail(EHIP_EINVAL, "conv_weight_reduce: too many outputs");
        EHIP_LAUNCH("conv_weight_reduce", conv_weight_reduce_batch, dim3(unsigned(blocks)),
                    dim3(256), 0, s, b);
    }
    return EHIP_OK;
}

}  // extern "C"
