// rows.hip -- kernels that work row by row over the last axis: softmax and its
// derivative, LayerNorm forward and backward, and the fused softmax
// cross-entropy (forward, backward from saved probabilities, and the one-pass
// backward straight from the logits).
//
// A row is handled by a "group" of T threads that keeps the whole row in
// registers, V values per thread: T = 64 (one wavefront, four rows per
// 256-thread block) for rows up to 2048 values, T = 256 or 1024 (one block
// per row, 128-bit loads) above that. The row is read from HBM once and
// written once. Reductions go through wavefront shuffles and, across the
// wavefronts of a block, LDS in wavefront order: a fixed order per shape, so
// results are deterministic. Rows longer than the register path holds use a
// looped fallback that streams the row three times.

#include "common.hpp"

#include <algorithm>
#include <cmath>

namespace ehip {
namespace {

// ------------------------------------------------------------ reductions

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Reduction over the T threads of a group. T == 64 stays in the wavefront;
// larger T combines the wavefront results through `sh` in wavefront order.
// Every thread of the block must call it (it may hold barriers).
template <int T, bool MAX>
__device__ __forceinline__ float group_reduce(float v, float* sh) {
    v = MAX ? wave_max(v) : wave_sum(v);
    if (T == 64) return v;
    constexpr int W = T / 64;
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    __syncthreads();  // sh may still be read by the previous reduction
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float r = sh[0];
#pragma unroll
    for (int w = 1; w < W; ++w) r = MAX ? fmaxf(r, sh[w]) : r + sh[w];
    return r;
}

// ------------------------------------------------------------ row fragments

// Rows of at least this many elements in total are streamed with non-temporal
// loads and stores (no reuse; 64 MiB per operand is past every cache level).
constexpr int64_t kNontemporalMin = int64_t(1) << 24;

typedef float nf4 __attribute__((ext_vector_type(4)));

// V values of one row held by thread `tid` of a T-thread group. VEC4 loads
// 128 bits at a time: value t sits at column 4 * (tid + T * (t / 4)) + t % 4;
// otherwise at column tid + T * t. Column arithmetic is 32-bit (register rows
// are at most 32768 wide), which keeps the register count low enough for two
// 1024-thread groups per CU.
template <int T, int V, bool VEC4, bool NT = false>
struct Frag {
    float v[V];
    __device__ static int col(int tid, int t) {
        return VEC4 ? 4 * (tid + T * (t / 4)) + (t % 4) : tid + T * t;
    }
    // Slot of column c in the fragment of the thread that owns it, or -1 when
    // this thread does not own c.
    __device__ static int slot(int tid, int64_t c) {
        if (c < 0) return -1;
        const int ci = int(c);
        if (VEC4) {
            const int c4 = ci >> 2;
            return (c4 % T == tid) ? 4 * (c4 / T) + (ci & 3) : -1;
        }
        return (ci % T == tid) ? ci / T : -1;
    }
    __device__ void load(const float* row, int cols, int tid, float fill) {
        if (VEC4) {
            const nf4* r4 = reinterpret_cast<const nf4*>(row);
#pragma unroll
            for (int q = 0; q < V / 4; ++q) {
                const int c4 = tid + T * q;
                nf4 x = {fill, fill, fill, fill};
                if (4 * c4 < cols) {
                    x = NT ? __builtin_nontemporal_load(r4 + c4) : r4[c4];
                    // A limit inside the vector (the causal diagonal): the
                    // lanes past it are read with the vector but count as
                    // `fill`, so their memory never reaches the result.
                    if (4 * c4 + 4 > cols) {
                        if (4 * c4 + 1 >= cols) x.y = fill;
                        if (4 * c4 + 2 >= cols) x.z = fill;
                        if (4 * c4 + 3 >= cols) x.w = fill;
                    }
                }
                v[4 * q] = x.x;
                v[4 * q + 1] = x.y;
                v[4 * q + 2] = x.z;
                v[4 * q + 3] = x.w;
            }
        } else {
#pragma unroll
            for (int t = 0; t < V; ++t) {
                const int c = col(tid, t);
                v[t] = c < cols ? row[c] : fill;
            }
        }
    }
    __device__ void store(float* row, int cols, int tid) const {
        if (VEC4) {
            nf4* r4 = reinterpret_cast<nf4*>(row);
#pragma unroll
            for (int q = 0; q < V / 4; ++q) {
                const int c4 = tid + T * q;
                if (4 * c4 < cols) {
                    const nf4 x = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                    if (NT)
                        __builtin_nontemporal_store(x, r4 + c4);
                    else
                        r4[c4] = x;
                }
            }
        } else {
#pragma unroll
            for (int t = 0; t < V; ++t) {
                const int c = col(tid, t);
                if (c < cols) row[c] = v[t];
            }
        }
    }
};

// Group geometry inside a block of max(T, 256) threads. kMinWaves asks the
// compiler for two 1024-thread groups per CU (8 waves per SIMD) in kernels
// that hold one fragment.
template <int T>
struct Group {
    static constexpr int kBlock = T < 256 ? 256 : T;
    static constexpr int kPerBlock = kBlock / T;
    static constexpr int kMinWaves = T == 1024 ? 8 : 1;
    __device__ static int tid() { return threadIdx.x % T; }
    __device__ static int64_t first_row() { return int64_t(blockIdx.x) * kPerBlock + threadIdx.x / T; }
    __device__ static int64_t row_step() { return int64_t(gridDim.x) * kPerBlock; }
};

// Softmax of the fragment in place; returns the row max and the sum of
// exponentials through m and s. Columns past the end hold -inf and give 0.
// The exponentials are scaled by one correctly rounded reciprocal of the sum
// (within an ulp of dividing each, and a division per element costs more than
// the row's HBM traffic).
template <int T, int V, bool VEC4, bool NT>
__device__ __forceinline__ void frag_softmax(Frag<T, V, VEC4, NT>& f, float* sh, float& m,
                                             float& s) {
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < V; ++t) mx = fmaxf(mx, f.v[t]);
    mx = group_reduce<T, true>(mx, sh);
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < V; ++t) {
        f.v[t] = expf(f.v[t] - mx);
        sum += f.v[t];
    }
    sum = group_reduce<T, false>(sum, sh);
    const float rs = 1.0f / sum;
#pragma unroll
    for (int t = 0; t < V; ++t) f.v[t] = f.v[t] * rs;
    m = mx;
    s = sum;
}

// ------------------------------------------------------------ softmax

// Columns of row r that are read: all, or with `causal` (rows stacked in
// cols x cols matrices whose entries right of the diagonal are masked) the
// first (r mod cols) + 1. A masked entry that is not read counts as -inf in
// the forward (exp gives 0, as for a masked score far below the row's
// maximum) and as 0 in the backward (where y is 0), so the sums and the other
// outputs keep their bits; the masked outputs are stored as 0.
__device__ __forceinline__ int read_cols(int64_t r, int64_t cols, int causal) {
    return causal ? int(r % cols) + 1 : int(cols);
}

template <int T, int V, bool VEC4, bool NT>
__global__ __launch_bounds__(Group<T>::kBlock, Group<T>::kMinWaves) void softmax_rows(
    const float* __restrict__ x, float* __restrict__ y, int64_t rows, int64_t cols, int causal) {
    __shared__ float sh[Group<T>::kBlock / 64];
    for (int64_t r = Group<T>::first_row(); r < rows; r += Group<T>::row_step()) {
        Frag<T, V, VEC4, NT> f;
        f.load(x + r * cols, read_cols(r, cols, causal), Group<T>::tid(), -INFINITY);
        float m, s;
        frag_softmax(f, sh, m, s);
        f.store(y + r * cols, int(cols), Group<T>::tid());
    }
}

// dx may alias g: every element of a row is loaded before any is stored.
template <int T, int V, bool VEC4, bool NT>
__global__ __launch_bounds__(Group<T>::kBlock) void softmax_rows_backward(
    const float* __restrict__ y, const float* g, float* dx, int64_t rows, int64_t cols,
    float scale, int causal) {
    __shared__ float sh[Group<T>::kBlock / 64];
    for (int64_t r = Group<T>::first_row(); r < rows; r += Group<T>::row_step()) {
        Frag<T, V, VEC4, NT> fy, fg;
        const int rc = read_cols(r, cols, causal);
        fy.load(y + r * cols, rc, Group<T>::tid(), 0.0f);
        fg.load(g + r * cols, rc, Group<T>::tid(), 0.0f);
        float dot = 0.0f;
#pragma unroll
        for (int t = 0; t < V; ++t) dot += fg.v[t] * fy.v[t];
        dot = group_reduce<T, false>(dot, sh);
#pragma unroll
        for (int t = 0; t < V; ++t) fg.v[t] = (fy.v[t] * (fg.v[t] - dot)) * scale;
        fg.store(dx + r * cols, int(cols), Group<T>::tid());
    }
}

// Looped fallback for rows beyond the register path: one block per row,
// three passes over global memory.
constexpr int kLoopThreads = 1024;

__device__ float block_reduce_loop(float v, float* sh, bool is_max) {
    v = is_max ? wave_max(v) : wave_sum(v);
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float r = sh[0];
    for (int w = 1; w < kLoopThreads / 64; ++w) r = is_max ? fmaxf(r, sh[w]) : r + sh[w];
    return r;
}

// Both honour `causal` as the register path does: columns at or past
// read_cols() are not read, count as -inf (forward) or 0 (backward), and
// their outputs come from the same expressions on those values.
__global__ __launch_bounds__(kLoopThreads) void softmax_rows_loop(const float* __restrict__ x,
                                                                  float* __restrict__ y,
                                                                  int64_t rows, int64_t cols,
                                                                  int causal) {
    __shared__ float sh[kLoopThreads / 64];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + r * cols;
        float* yr = y + r * cols;
        const int64_t rc = read_cols(r, cols, causal);
        float mx = -INFINITY;
        for (int64_t c = threadIdx.x; c < rc; c += kLoopThreads) mx = fmaxf(mx, xr[c]);
        mx = block_reduce_loop(mx, sh, true);
        float sum = 0.0f;
        for (int64_t c = threadIdx.x; c < rc; c += kLoopThreads) sum += expf(xr[c] - mx);
        sum = block_reduce_loop(sum, sh, false);
        const float rs = 1.0f / sum;
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads)
            yr[c] = expf((c < rc ? xr[c] : -INFINITY) - mx) * rs;
    }
}

__global__ __launch_bounds__(kLoopThreads) void softmax_rows_backward_loop(
    const float* __restrict__ y, const float* g, float* dx, int64_t rows, int64_t cols,
    float scale, int causal) {
    __shared__ float sh[kLoopThreads / 64];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* yr = y + r * cols;
        const float* gr = g + r * cols;
        const int64_t rc = read_cols(r, cols, causal);
        float dot = 0.0f;
        for (int64_t c = threadIdx.x; c < rc; c += kLoopThreads) dot += gr[c] * yr[c];
        dot = block_reduce_loop(dot, sh, false);
        // dx may alias g: each element is read by the thread that stores it.
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) {
            const float yv = c < rc ? yr[c] : 0.0f, gv = c < rc ? gr[c] : 0.0f;
            dx[r * cols + c] = (yv * (gv - dot)) * scale;
        }
    }
}

// LayerNorm rows wider than the register path (more than 8192 columns): one
// block per row, passes over global memory (the row stays in the caches
// between them), the expressions of layernorm_rows and
// layernorm_rows_backward. The backward's dgamma / dbeta partials accumulate
// per group in partial[group][2][cols]; column c always belongs to thread
// c mod kLoopThreads of its group's block, so each partial has one writer.
__global__ __launch_bounds__(kLoopThreads) void layernorm_rows_loop(
    const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    float* __restrict__ out, float* __restrict__ xhat, float* __restrict__ inv_std, int64_t rows,
    int64_t cols, float eps) {
    __shared__ float sh[kLoopThreads / 64];
    const float inv_d = 1.0f / static_cast<float>(cols);
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + r * cols;
        float sum = 0.0f;
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) sum += xr[c];
        const float mean = block_reduce_loop(sum, sh, false) * inv_d;
        float q = 0.0f;
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) {
            const float d = xr[c] - mean;
            q += d * d;
        }
        const float var = block_reduce_loop(q, sh, false) * inv_d;
        const float inv = 1.0f / sqrtf(var + eps);
        if (threadIdx.x == 0) inv_std[r] = inv;
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) {
            const float h = (xr[c] - mean) * inv;
            xhat[r * cols + c] = h;
            out[r * cols + c] = gamma[c] * h + beta[c];
        }
    }
}

__global__ __launch_bounds__(kLoopThreads) void layernorm_rows_backward_loop(
    const float* __restrict__ dy, const float* __restrict__ xhat, const float* __restrict__ gamma,
    const float* __restrict__ inv_std, float* __restrict__ dx, float* __restrict__ partial,
    int64_t rows, int64_t cols) {
    __shared__ float sh[kLoopThreads / 64];
    const float inv_d = 1.0f / static_cast<float>(cols);
    float* pg = partial + int64_t(blockIdx.x) * 2 * cols;
    for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) {
        pg[c] = 0.0f;
        pg[cols + c] = 0.0f;
    }
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* dr = dy + r * cols;
        const float* hr = xhat + r * cols;
        float s1 = 0.0f, s2 = 0.0f;
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) {
            const float dxh = dr[c] * gamma[c];
            s1 += dxh;
            s2 += dxh * hr[c];
        }
        s1 = block_reduce_loop(s1, sh, false);
        s2 = block_reduce_loop(s2, sh, false);
        const float inv = inv_std[r];
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) {
            const float d = dr[c], h = hr[c];
            const float dxh = d * gamma[c];
            dx[r * cols + c] = inv * (dxh - inv_d * s1 - h * inv_d * s2);
            pg[c] = pg[c] + d * h;
            pg[cols + c] = pg[cols + c] + d;
        }
    }
}

// ------------------------------------------------------------ cross-entropy

// probs = softmax(logits); row_loss[r] = -((x[t] - max) - log(sum)), the
// expression of src/nn.cpp:371-373. An out-of-range target gives NaN.
template <int T, int V, bool VEC4, bool NT>
__global__ __launch_bounds__(Group<T>::kBlock, Group<T>::kMinWaves) void xent_rows(
    const float* __restrict__ logits, const int32_t* __restrict__ targets,
    float* __restrict__ probs, float* __restrict__ row_loss, int64_t rows, int64_t cols) {
    __shared__ float sh[Group<T>::kBlock / 64];
    for (int64_t r = Group<T>::first_row(); r < rows; r += Group<T>::row_step()) {
        Frag<T, V, VEC4, NT> f;
        f.load(logits + r * cols, int(cols), Group<T>::tid(), -INFINITY);
        float m, s;
        frag_softmax(f, sh, m, s);
        f.store(probs + r * cols, int(cols), Group<T>::tid());
        if (Group<T>::tid() == 0) {
            const int64_t t = targets[r];
            row_loss[r] = (t >= 0 && t < cols) ? -((logits[r * cols + t] - m) - logf(s)) : NAN;
        }
    }
}

// A classifier head's batch (at most 1024 rows of at most 128 classes) in one
// block: xent_rows' arithmetic per row (16 wavefronts; each loads four of its
// rows, and their targets, before computing any, and takes the target's logit
// from the lane that holds it), the row losses kept in LDS, then mean_rows'
// tree over them -- the two launches' results bit for bit, in one. The tree
// starts at half the smallest power of two >= rows: the levels above it only
// add the zero entries beyond the rows, which leaves every sum as it is. With
// dlogits, each row's gradient for an upstream gradient of 1 is written too,
// as xent_backward_from_probs computes it from the stored probabilities.
constexpr int kXentMeanRows = 1024;

template <int V>
__global__ __launch_bounds__(1024) void xent_rows_mean(const float* __restrict__ logits,
                                                       const int32_t* __restrict__ targets,
                                                       float* __restrict__ probs,
                                                       float* __restrict__ loss,
                                                       float* __restrict__ dlogits, int rows,
                                                       int cols) {
    constexpr int kAhead = 4;
    __shared__ float row_loss[kXentMeanRows];
    __shared__ double sh[1024];
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    for (int r0 = wave; r0 < rows; r0 += 16 * kAhead) {
        Frag<64, V, false, false> f[kAhead];
        int32_t tg[kAhead];
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {
            const int r = r0 + 16 * u;
            tg[u] = -1;
            if (r < rows) {
                f[u].load(logits + int64_t(r) * cols, cols, lane, -INFINITY);
                tg[u] = targets[r];
            }
        }
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {
            const int r = r0 + 16 * u;
            if (r >= rows) break;
            const int32_t t = tg[u];
            const bool valid = t >= 0 && t < cols;
            // column t sits in slot t / 64 of lane t % 64 (the slot is uniform)
            const int ts = valid ? t : 0;
            float own = f[u].v[0];
#pragma unroll
            for (int q = 1; q < V; ++q)
                if (ts / 64 == q) own = f[u].v[q];
            const float xt = __shfl(own, ts % 64);
            float m, sum;
            frag_softmax(f[u], nullptr, m, sum);  // one wavefront: no LDS in the reduction
            f[u].store(probs + int64_t(r) * cols, cols, lane);
            if (lane == 0) row_loss[r] = valid ? -((xt - m) - logf(sum)) : NAN;
            if (dlogits != nullptr) {
                const float scale = 1.0f / static_cast<float>(rows);
                const int ts = Frag<64, V, false, false>::slot(lane, t);
#pragma unroll
                for (int q = 0; q < V; ++q) {
                    float p = f[u].v[q];
                    if (q == ts) p -= 1.0f;
                    f[u].v[q] = p * scale;
                }
                f[u].store(dlogits + int64_t(r) * cols, cols, lane);
            }
        }
    }
    __syncthreads();
    double acc = 0.0;
    if (int(threadIdx.x) < rows) acc += row_loss[threadIdx.x];
    sh[threadIdx.x] = acc;
    __syncthreads();
    int h = 1;
    while (h < rows) h <<= 1;
    for (h >>= 1; h > 0; h >>= 1) {
        if (int(threadIdx.x) < h) sh[threadIdx.x] += sh[threadIdx.x + h];
        __syncthreads();
    }
    if (threadIdx.x == 0) loss[0] = static_cast<float>(sh[0]) / static_cast<float>(rows);
}

// dx = (softmax - onehot) * (grad / rows), from the logits in one pass. The
// softmax is the same code as xent_rows, so the result equals the two-kernel
// path bit for bit.
template <int T, int V, bool VEC4, bool NT>
__global__ __launch_bounds__(Group<T>::kBlock, Group<T>::kMinWaves) void xent_rows_backward_fused(
    const float* __restrict__ logits, const int32_t* __restrict__ targets, float* __restrict__ dx,
    int64_t rows, int64_t cols, const float* __restrict__ grad) {
    __shared__ float sh[Group<T>::kBlock / 64];
    const float scale = grad[0] / static_cast<float>(rows);
    const int tid = Group<T>::tid();
    for (int64_t r = Group<T>::first_row(); r < rows; r += Group<T>::row_step()) {
        Frag<T, V, VEC4, NT> f;
        f.load(logits + r * cols, int(cols), tid, -INFINITY);
        float m, s;
        frag_softmax(f, sh, m, s);
        const int64_t t = targets[r];
        // Only the thread holding the target column subtracts the one-hot.
        const int ts = t < cols ? Frag<T, V, VEC4, NT>::slot(tid, t) : -1;
#pragma unroll
        for (int q = 0; q < V; ++q) {
            float p = f.v[q];
            if (q == ts) p -= 1.0f;
            f.v[q] = p * scale;
        }
        f.store(dx + r * cols, int(cols), tid);
    }
}

__global__ __launch_bounds__(kLoopThreads) void xent_rows_loop(const float* __restrict__ logits,
                                                               const int32_t* __restrict__ targets,
                                                               float* __restrict__ probs,
                                                               float* __restrict__ row_loss,
                                                               int64_t rows, int64_t cols) {
    __shared__ float sh[kLoopThreads / 64];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = logits + r * cols;
        float mx = -INFINITY;
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) mx = fmaxf(mx, xr[c]);
        mx = block_reduce_loop(mx, sh, true);
        float sum = 0.0f;
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) sum += expf(xr[c] - mx);
        sum = block_reduce_loop(sum, sh, false);
        const float rs = 1.0f / sum;
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads)
            probs[r * cols + c] = expf(xr[c] - mx) * rs;
        if (threadIdx.x == 0) {
            const int64_t t = targets[r];
            row_loss[r] = (t >= 0 && t < cols) ? -((xr[t] - mx) - logf(sum)) : NAN;
        }
    }
}

__global__ __launch_bounds__(kLoopThreads) void xent_rows_backward_loop(
    const float* __restrict__ logits, const int32_t* __restrict__ targets, float* __restrict__ dx,
    int64_t rows, int64_t cols, const float* __restrict__ grad) {
    __shared__ float sh[kLoopThreads / 64];
    const float scale = grad[0] / static_cast<float>(rows);
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = logits + r * cols;
        float mx = -INFINITY;
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) mx = fmaxf(mx, xr[c]);
        mx = block_reduce_loop(mx, sh, true);
        float sum = 0.0f;
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) sum += expf(xr[c] - mx);
        sum = block_reduce_loop(sum, sh, false);
        const int64_t t = targets[r];
        const float rs = 1.0f / sum;
        for (int64_t c = threadIdx.x; c < cols; c += kLoopThreads) {
            float p = expf(xr[c] - mx) * rs;
            if (c == t) p -= 1.0f;
            dx[r * cols + c] = p * scale;
        }
    }
}

// src/nn.cpp:386-405: (p - onehot) * (grad / N), element by element.
__global__ __launch_bounds__(256) void xent_backward_from_probs(
    const float* __restrict__ probs, const int32_t* __restrict__ targets, float* __restrict__ dx,
    int64_t rows, int64_t cols, const float* __restrict__ grad) {
    const float scale = grad[0] / static_cast<float>(rows);
    const int64_t n = rows * cols;
    const int64_t step = int64_t(gridDim.x) * 256;
    for (int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x; e < n; e += step) {
        const int64_t r = e / cols, c = e % cols;
        float p = probs[e];
        if (c == targets[r]) p -= 1.0f;
        dx[e] = p * scale;
    }
}

// mean over rows of row_loss, summed in double over a fixed tree.
__global__ __launch_bounds__(1024) void mean_rows(const float* __restrict__ row_loss, int64_t rows,
                                                  float* __restrict__ loss) {
    __shared__ double sh[1024];
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < rows; i += 1024) acc += row_loss[i];
    sh[threadIdx.x] = acc;
    __syncthreads();
    for (int s = 512; s > 0; s >>= 1) {
        if (int(threadIdx.x) < s) sh[threadIdx.x] += sh[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) loss[0] = static_cast<float>(sh[0]) / static_cast<float>(rows);
}

// ------------------------------------------------------------ LayerNorm

// src/transformer.cpp:53-73: mean = (sum x) * (1/D); var = (sum (x-mean)^2) * (1/D);
// inv = 1 / sqrt(var + eps); xhat = (x - mean) * inv; out = gamma * xhat + beta.
template <int T, int V, bool VEC4, bool NT = false>
__global__ __launch_bounds__(Group<T>::kBlock) void layernorm_rows(
    const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    float* __restrict__ out, float* __restrict__ xhat, float* __restrict__ inv_std, int64_t rows,
    int64_t cols, float eps) {
    using F = Frag<T, V, VEC4, NT>;
    __shared__ float sh[Group<T>::kBlock / 64];
    const float inv_d = 1.0f / static_cast<float>(cols);
    const int tid = Group<T>::tid();
    float gm[V], bt[V];
#pragma unroll
    for (int t = 0; t < V; ++t) {
        const int64_t c = F::col(tid, t);
        gm[t] = c < cols ? gamma[c] : 0.0f;
        bt[t] = c < cols ? beta[c] : 0.0f;
    }
    // The next row is loaded before the current one is reduced, so a group
    // keeps loads in flight while it computes and stores.
    const int64_t step = Group<T>::row_step();
    int64_t r = Group<T>::first_row();
    F nf;
    if (r < rows) nf.load(x + r * cols, int(cols), tid, 0.0f);
    for (; r < rows; r += step) {
        const F f = nf;
        if (r + step < rows) nf.load(x + (r + step) * cols, int(cols), tid, 0.0f);
        float s = 0.0f;
#pragma unroll
        for (int t = 0; t < V; ++t) s += f.v[t];
        const float mean = group_reduce<T, false>(s, sh) * inv_d;
        float q = 0.0f;
#pragma unroll
        for (int t = 0; t < V; ++t) {
            const float d = F::col(tid, t) < cols ? f.v[t] - mean : 0.0f;
            q += d * d;
        }
        const float var = group_reduce<T, false>(q, sh) * inv_d;
        const float inv = 1.0f / sqrtf(var + eps);
        if (tid == 0) inv_std[r] = inv;
        F fh, fo;
#pragma unroll
        for (int t = 0; t < V; ++t) {
            fh.v[t] = (f.v[t] - mean) * inv;
            fo.v[t] = gm[t] * fh.v[t] + bt[t];
        }
        fh.store(xhat + r * cols, int(cols), tid);
        fo.store(out + r * cols, int(cols), tid);
    }
}

// dx per row (src/transformer.cpp:147-171); dgamma/dbeta partial sums per
// group over the rows it visits, ascending, into partial[group][2][cols].
// One group per block of T threads (group = blockIdx.x, rows group, group +
// groups, ...), so that few groups still spread over every CU; the next two
// rows' dy and xhat are loaded before the current row is reduced, keeping
// loads in flight behind the arithmetic of a group's serial row chain.
template <int T, int V, bool VEC4>
__global__ __launch_bounds__(T) void layernorm_rows_backward(
    const float* __restrict__ dy, const float* __restrict__ xhat, const float* __restrict__ gamma,
    const float* __restrict__ inv_std, float* __restrict__ dx, float* __restrict__ partial,
    int64_t rows, int64_t cols) {
    using F = Frag<T, V, VEC4>;
    constexpr int kAhead = 3;  // rows in registers: the current one and two ahead
    __shared__ float sh[T / 64];
    const float inv_d = 1.0f / static_cast<float>(cols);
    const int tid = threadIdx.x;
    const int64_t group = blockIdx.x, step = gridDim.x;
    float dg[V], db[V], gm[V];
#pragma unroll
    for (int t = 0; t < V; ++t) {
        dg[t] = 0.0f;
        db[t] = 0.0f;
        const int64_t c = F::col(tid, t);
        gm[t] = c < cols ? gamma[c] : 0.0f;
    }
    F fd[kAhead], fh[kAhead];
    float iv[kAhead];
#pragma unroll
    for (int a = 0; a < kAhead - 1; ++a) {
        const int64_t ra = group + a * step;
        iv[a] = 0.0f;
        if (ra < rows) {
            fd[a].load(dy + ra * cols, int(cols), tid, 0.0f);
            fh[a].load(xhat + ra * cols, int(cols), tid, 0.0f);
            iv[a] = inv_std[ra];
        }
    }
    int64_t r = group;
    for (; r < rows; r += step) {
        // Rotate by value so the register arrays keep static indices.
        const int64_t rn = r + (kAhead - 1) * step;
        iv[kAhead - 1] = 0.0f;
        if (rn < rows) {
            fd[kAhead - 1].load(dy + rn * cols, int(cols), tid, 0.0f);
            fh[kAhead - 1].load(xhat + rn * cols, int(cols), tid, 0.0f);
            iv[kAhead - 1] = inv_std[rn];
        }
        float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
        for (int t = 0; t < V; ++t) {
            const float dxh = fd[0].v[t] * gm[t];
            s1 += dxh;
            s2 += dxh * fh[0].v[t];
        }
        s1 = group_reduce<T, false>(s1, sh);
        s2 = group_reduce<T, false>(s2, sh);
        const float inv = iv[0];
        F fo;
#pragma unroll
        for (int t = 0; t < V; ++t) {
            const float dxh = fd[0].v[t] * gm[t];
            fo.v[t] = inv * (dxh - inv_d * s1 - fh[0].v[t] * inv_d * s2);
            dg[t] = dg[t] + fd[0].v[t] * fh[0].v[t];
            db[t] = db[t] + fd[0].v[t];
        }
        fo.store(dx + r * cols, int(cols), tid);
#pragma unroll
        for (int a = 0; a + 1 < kAhead; ++a) {
            fd[a] = fd[a + 1];
            fh[a] = fh[a + 1];
            iv[a] = iv[a + 1];
        }
    }
    float* pg = partial + group * 2 * cols;
#pragma unroll
    for (int t = 0; t < V; ++t) {
        const int64_t c = F::col(tid, t);
        if (c < cols) {
            pg[c] = dg[t];
            pg[cols + c] = db[t];
        }
    }
}

// The same as layernorm_rows_backward<64, V, VEC4> for groups of at most
// kSplitRows rows, with the group's rows shared by W waves instead of walked
// by one: wave w takes the group's rows i = w, w + W, ... (row group + i
// groups), computes dx as above, and parks the row's dy and xhat in LDS; after
// a barrier one thread per column runs the serial kernel's dgamma / dbeta
// recurrences over them in row order, with the same expressions, so the sums
// match it bit for bit.
constexpr int kSplitRows = 16;

template <int V, bool VEC4, int W>
__global__ __launch_bounds__(64 * W) void layernorm_rows_backward_split(
    const float* __restrict__ dy, const float* __restrict__ xhat, const float* __restrict__ gamma,
    const float* __restrict__ inv_std, float* __restrict__ dx, float* __restrict__ partial,
    int64_t rows, int64_t cols) {
    using F = Frag<64, V, VEC4>;
    constexpr int kC = 64 * V;   // columns the fragment holds
    __shared__ float rows_dh[kSplitRows][2][kC];
    const float inv_d = 1.0f / static_cast<float>(cols);
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int64_t group = blockIdx.x, step = gridDim.x;
    const int nrows = int(group < rows ? (rows - 1 - group) / step + 1 : 0);
    float gm[V];
#pragma unroll
    for (int t = 0; t < V; ++t) {
        const int64_t c = F::col(lane, t);
        gm[t] = c < cols ? gamma[c] : 0.0f;
    }
    for (int i = wave; i < nrows; i += W) {
        const int64_t r = group + int64_t(i) * step;
        F fd, fh;
        fd.load(dy + r * cols, int(cols), lane, 0.0f);
        fh.load(xhat + r * cols, int(cols), lane, 0.0f);
        const float inv = inv_std[r];
        float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
        for (int t = 0; t < V; ++t) {
            const float dxh = fd.v[t] * gm[t];
            s1 += dxh;
            s2 += dxh * fh.v[t];
        }
        s1 = group_reduce<64, false>(s1, nullptr);
        s2 = group_reduce<64, false>(s2, nullptr);
        F fo;
#pragma unroll
        for (int t = 0; t < V; ++t) {
            const float dxh = fd.v[t] * gm[t];
            fo.v[t] = inv * (dxh - inv_d * s1 - fh.v[t] * inv_d * s2);
            const int c = F::col(lane, t);
            rows_dh[i][0][c] = fd.v[t];
            rows_dh[i][1][c] = fh.v[t];
        }
        fo.store(dx + r * cols, int(cols), lane);
    }
    __syncthreads();
    float* pg = partial + group * 2 * cols;
    for (int c = threadIdx.x; c < cols; c += 64 * W) {
        float dg = 0.0f, db = 0.0f;
        for (int i = 0; i < nrows; ++i) {
            const float d = rows_dh[i][0][c], h = rows_dh[i][1][c];
            dg = dg + d * h;
            db = db + d;
        }
        pg[c] = dg;
        pg[cols + c] = db;
    }
}

constexpr int kLnWaves = 8;

// acc of wave 0 += acc of waves 1..kLnWaves-1 by a fixed halving tree
// (wave w adds wave w + half for half = kLnWaves / 2, ..., 1).
template <int V>
__device__ __forceinline__ void combine_waves(float (&acc)[V], float (*tree)[V][64], int wave,
                                              int lane) {
#pragma unroll
    for (int half = kLnWaves / 2; half >= 1; half /= 2) {
        if (wave >= half && wave < 2 * half) {
#pragma unroll
            for (int t = 0; t < V; ++t) tree[wave - half][t][lane] = acc[t];
        }
        __syncthreads();
        if (wave < half) {
#pragma unroll
            for (int t = 0; t < V; ++t) acc[t] = acc[t] + tree[wave][t][lane];
        }
        __syncthreads();
    }
}

// The large-problem form: a group is a block of kLnWaves waves; wave w of
// group g takes rows g + groups (w + kLnWaves i), ascending i, AHEAD of them at
// a time with every load issued before the first of them is reduced, so that
// every CU holds many independent rows while the partials stay few (one
// dgamma / dbeta row per group). The waves' partial sums are combined by a
// fixed tree through LDS (w += w + half, halving), then written interleaved,
// partial[group][c][2] = (dgamma, dbeta): the layout of a convolution
// weight-gradient job with one weight per output channel, so that the ordered
// sum over groups is conv_weight_reduce's (here, in ehip_conv_weight_reduce_f32,
// or inside the Adam launch of ehip_adam_multi_reduce_f32). Measured at
// 8192 x 1024 (cfg5): four rows ahead with nontemporal accesses 16.6 us against
// 19.0 us for the previous one-row prefetch; at 2^28 elements one row at a time
// is faster (545 against 564 us).
//
// ACC: dx += the rows' gradient (the held gradient read with the row), a
// template parameter so that the plain form holds no registers for it.
template <int V, bool VEC4, int AHEAD, bool ACC>
__global__ __launch_bounds__(64 * kLnWaves) void layernorm_rows_backward_wide(
    const float* __restrict__ dy, const float* __restrict__ xhat, const float* __restrict__ gamma,
    const float* __restrict__ inv_std, float* __restrict__ dx, float* __restrict__ partial,
    int64_t rows, int64_t cols) {
    using F = Frag<64, V, VEC4, true>;
    __shared__ float tree[kLnWaves / 2][V][64];
    const float inv_d = 1.0f / static_cast<float>(cols);
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int64_t group = blockIdx.x, groups = gridDim.x;
    float dg[V], db[V];
    F gmf;  // gamma, zero past the row
    gmf.load(gamma, int(cols), lane, 0.0f);
    const float* gm = gmf.v;
#pragma unroll
    for (int t = 0; t < V; ++t) {
        dg[t] = 0.0f;
        db[t] = 0.0f;
    }
    const int64_t step = groups * kLnWaves;
    for (int64_t r0 = group + groups * wave; r0 < rows; r0 += step * AHEAD) {
        F fd[AHEAD], fh[AHEAD], fx[ACC ? AHEAD : 1];
        float iv[AHEAD];
#pragma unroll
        for (int a = 0; a < AHEAD; ++a) {
            const int64_t r = r0 + a * step;
            iv[a] = 0.0f;
            if (r < rows) {
                fd[a].load(dy + r * cols, int(cols), lane, 0.0f);
                fh[a].load(xhat + r * cols, int(cols), lane, 0.0f);
                if constexpr (ACC) fx[a].load(dx + r * cols, int(cols), lane, 0.0f);
                iv[a] = inv_std[r];
            }
        }
#pragma unroll
        for (int a = 0; a < AHEAD; ++a) {
            const int64_t r = r0 + a * step;
            if (r >= rows) break;
            float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
            for (int t = 0; t < V; ++t) {
                const float dxh = fd[a].v[t] * gm[t];
                s1 += dxh;
                s2 += dxh * fh[a].v[t];
            }
            s1 = wave_sum(s1);
            s2 = wave_sum(s2);
            // dx overwrites dy's registers once dgamma and dbeta have read them.
            F& fo = fd[a];
#pragma unroll
            for (int t = 0; t < V; ++t) {
                const float g = fd[a].v[t];
                dg[t] = dg[t] + g * fh[a].v[t];
                db[t] = db[t] + g;
                fo.v[t] = iv[a] * (g * gm[t] - inv_d * s1 - fh[a].v[t] * inv_d * s2);
            }
            // Accumulating: the gradient already held plus this one, one add
            // (the bits of a separate accumulate pass).
            if constexpr (ACC) {
#pragma unroll
                for (int t = 0; t < V; ++t) fo.v[t] = fx[a].v[t] + fo.v[t];
            }
            fo.store(dx + r * cols, int(cols), lane);
        }
    }
    combine_waves<V>(dg, tree, wave, lane);
    combine_waves<V>(db, tree, wave, lane);
    if (wave == 0) {
        float* pg = partial + group * 2 * cols;
        if (VEC4) {
            // Columns t and t + 1 of a float4 slot are adjacent: one 16-byte store
            // (cols is a multiple of 4 here, so a slot is inside or outside whole).
#pragma unroll
            for (int t = 0; t < V; t += 2) {
                const int64_t c = F::col(lane, t);
                if (c < cols)
                    *reinterpret_cast<float4*>(pg + 2 * c) =
                        make_float4(dg[t], db[t], dg[t + 1], db[t + 1]);
            }
        } else {
#pragma unroll
            for (int t = 0; t < V; ++t) {
                const int64_t c = F::col(lane, t);
                if (c < cols) *reinterpret_cast<float2*>(pg + 2 * c) = make_float2(dg[t], db[t]);
            }
        }
    }
}

// ------------------------------------------------------------ dispatch

unsigned row_grid(int64_t rows, int per_block) {
    int64_t g = ceil_div(rows, per_block);
    if (g > (int64_t(1) << 20)) g = int64_t(1) << 20;
    return unsigned(g < 1 ? 1 : g);
}

// Calls f.template operator()<T, V, VEC4>() for the register path that holds
// `cols`, or returns false when the row needs the looped fallback.
// Calls f.template run<T, V, VEC4, NT>() for the register path that holds
// `cols`, or returns false when the row needs the looped fallback. Rows whose
// width is a multiple of 4 (and 16-byte aligned) load 128 bits at a time;
// large totals stream non-temporally.
template <int T, int V, class F>
bool run_vec(bool nt, F& f) {
    return nt ? f.template run<T, V, true, true>() : f.template run<T, V, true, false>();
}

template <class F>
bool dispatch_row(int64_t rows, int64_t cols, bool vec_ok, F&& f) {
    const bool nt = rows * cols >= kNontemporalMin;
    if (cols <= 64) return f.template run<64, 1, false, false>();
    if (cols <= 128) return f.template run<64, 2, false, false>();
    if (!vec_ok) {
        if (cols <= 256) return f.template run<64, 4, false, false>();
        if (cols <= 512) return f.template run<64, 8, false, false>();
        if (cols <= 1024) return f.template run<64, 16, false, false>();
        if (cols <= 2048) return f.template run<64, 32, false, false>();
        return false;
    }
    if (cols <= 256) return run_vec<64, 4>(nt, f);
    if (cols <= 512) return run_vec<64, 8>(nt, f);
    if (cols <= 1024) return run_vec<64, 16>(nt, f);
    if (cols <= 2048) return run_vec<64, 32>(nt, f);
    if (cols <= 4096) return run_vec<256, 16>(nt, f);
    if (cols <= 8192) return run_vec<256, 32>(nt, f);
    if (cols <= 16384) return run_vec<1024, 16>(nt, f);
    if (cols <= 32768) return run_vec<1024, 32>(nt, f);
    return false;
}

struct SoftmaxLaunch {
    const float* x;
    float* y;
    int64_t rows, cols;
    hipStream_t s;
    int* rc;
    int causal;
    template <int T, int V, bool VEC4, bool NT>
    bool run() {
        constexpr int B = Group<T>::kBlock, G = Group<T>::kPerBlock;
        *rc = [&] {
            EHIP_LAUNCH("softmax", (softmax_rows<T, V, VEC4, NT>), dim3(row_grid(rows, G)), dim3(B), 0,
                        s, x, y, rows, cols, causal);
            return int(EHIP_OK);
        }();
        return true;
    }
};

struct SoftmaxBackwardLaunch {
    const float* y;
    const float* g;
    float* dx;
    int64_t rows, cols;
    float scale;
    hipStream_t s;
    int* rc;
    int causal;
    template <int T, int V, bool VEC4, bool NT>
    bool run() {
        constexpr int B = Group<T>::kBlock, G = Group<T>::kPerBlock;
        *rc = [&] {
            EHIP_LAUNCH("softmax_backward", (softmax_rows_backward<T, V, VEC4, NT>),
                        dim3(row_grid(rows, G)), dim3(B), 0, s, y, g, dx, rows, cols, scale,
                        causal);
            return int(EHIP_OK);
        }();
        return true;
    }
};

struct XentLaunch {
    const float* logits;
    const int32_t* targets;
    float* probs;
    float* row_loss;
    int64_t rows, cols;
    hipStream_t s;
    int* rc;
    template <int T, int V, bool VEC4, bool NT>
    bool run() {
        constexpr int B = Group<T>::kBlock, G = Group<T>::kPerBlock;
        *rc = [&] {
            EHIP_LAUNCH("cross_entropy", (xent_rows<T, V, VEC4, NT>), dim3(row_grid(rows, G)), dim3(B),
                        0, s, logits, targets, probs, row_loss, rows, cols);
            return int(EHIP_OK);
        }();
        return true;
    }
};

struct XentBackwardLaunch {
    const float* logits;
    const int32_t* targets;
    float* dx;
    int64_t rows, cols;
    const float* grad;
    hipStream_t s;
    int* rc;
    template <int T, int V, bool VEC4, bool NT>
    bool run() {
        constexpr int B = Group<T>::kBlock, G = Group<T>::kPerBlock;
        *rc = [&] {
            EHIP_LAUNCH("softmax_xent_backward", (xent_rows_backward_fused<T, V, VEC4, NT>),
                        dim3(row_grid(rows, G)), dim3(B), 0, s, logits, targets, dx, rows, cols,
                        grad);
            return int(EHIP_OK);
        }();
        return true;
    }
};

bool rows_vec_ok(int64_t cols, std::initializer_list<const void*> ptrs) {
    if (cols % 4 != 0) return false;
    for (const void* p : ptrs)
        if (!aligned16(p)) return false;
    return true;
}

// Groups of the large-problem form for rows x cols, or 0 when the shape takes
// the small-problem kernels (fewer than 2^17 elements, or rows beyond 2048
// columns). About 32 rows per group, at most 256 (one per CU); the group count
// fixes the order of the dgamma / dbeta sums. From 2^17 elements up (the char
// Transformer's 2048 x 96) the engine queues those sums into the step's Adam
// launch, two launches fewer per LayerNorm than the small form's separate sums.
// Widest LayerNorm row held in registers; wider rows take the looped kernels.
constexpr int64_t kLnRegisterCols = 8192;

int64_t ln_wide_groups(int64_t rows, int64_t cols) {
    if (rows <= 0 || rows * cols < (int64_t(1) << 17) || cols > 2048) return 0;
    return std::min<int64_t>(ceil_div(rows, 32), 256);
}

// One width class of the large-problem row kernel: four rows in flight per
// wave below 2^25 elements for rows of up to 1024 columns (512 without
// 16-byte rows), one otherwise. Wider rows take one row at a time always
// (four would need more registers than a lane has: the compiler spills), so
// those instantiations are never compiled.
template <int V, bool VEC>
int launch_ln_wide_v(bool ahead, const float* dy, const float* xhat, const float* gamma,
                     const float* inv_std, float* dx, float* partial, int64_t groups,
                     int64_t rows, int64_t cols, int accumulate, hipStream_t s) {
#define EHIP_LN_WIDE(AHEAD, ACC)                                                                   \
    EHIP_LAUNCH("layernorm_backward", (layernorm_rows_backward_wide<V, VEC, AHEAD, ACC>),          \
                dim3(unsigned(groups)), dim3(64 * kLnWaves), 0, s, dy, xhat, gamma, inv_std, dx,   \
                partial, rows, cols)
    if constexpr (V <= (VEC ? 16 : 8)) {
        if (ahead) {
            // Accumulating holds a third row per row in flight: two ahead at
            // 1024 columns, where four would spill.
            if (!accumulate)
                EHIP_LN_WIDE(4, false);
            else if constexpr (V >= 16)
                EHIP_LN_WIDE(2, true);
            else
                EHIP_LN_WIDE(4, true);
            return EHIP_OK;
        }
    }
    // Accumulating rows of 2048 columns would spill even one row at a time:
    // the entry point refuses them, so that form is never compiled.
    if constexpr (V < 32) {
        if (accumulate) {
            EHIP_LN_WIDE(1, true);
            return EHIP_OK;
        }
    }
    EHIP_LN_WIDE(1, false);
#undef EHIP_LN_WIDE
    return EHIP_OK;
}

// Launches the large-problem row kernel for `groups` groups (dx = or, with
// accumulate, dx += the rows' input gradient).
int launch_ln_wide(const float* dy, const float* xhat, const float* gamma, const float* inv_std,
                   float* dx, float* partial, int64_t groups, int64_t rows, int64_t cols,
                   hipStream_t s, int accumulate = 0) {
    const bool vec = cols >= 256 && rows_vec_ok(cols, {dy, xhat, gamma, dx});
    // Four rows ahead below the last-level cache size, one beyond it (2^25 elements).
    const bool ahead = rows * cols < (int64_t(1) << 25);
#define EHIP_LNW(V, VEC) \
    return launch_ln_wide_v<V, VEC>(ahead, dy, xhat, gamma, inv_std, dx, partial, groups, rows, \
                                    cols, accumulate, s)
    if (vec) {
        if (cols <= 256) EHIP_LNW(4, true);
        if (cols <= 512) EHIP_LNW(8, true);
        if (cols <= 1024) EHIP_LNW(16, true);
        EHIP_LNW(32, true);
    }
    if (cols <= 64) EHIP_LNW(1, false);
    if (cols <= 128) EHIP_LNW(2, false);
    if (cols <= 256) EHIP_LNW(4, false);
    if (cols <= 512) EHIP_LNW(8, false);
    if (cols <= 1024) EHIP_LNW(16, false);
    EHIP_LNW(32, false);
#undef EHIP_LNW
}

unsigned loop_grid(int64_t rows) { return unsigned(rows < 65536 ? rows : 65536); }

const OccupancyKernel kRowKernels[] = {
    {"softmax_rows, 64-lane rows of 512", reinterpret_cast<const void*>(&softmax_rows<64, 8, true, false>), 256},
    {"softmax_rows, 1024-thread rows of 32768",
     reinterpret_cast<const void*>(&softmax_rows<1024, 32, true, true>), 1024},
    {"xent_rows_backward_fused, rows of 32000",
     reinterpret_cast<const void*>(&xent_rows_backward_fused<1024, 32, true, true>), 1024},
    {"layernorm_rows, rows of 1024", reinterpret_cast<const void*>(&layernorm_rows<64, 16, true, false>), 256},
    {"layernorm_rows_backward_wide, rows of 1024, 4 ahead",
     reinterpret_cast<const void*>(&layernorm_rows_backward_wide<16, true, 4, false>), 64 * kLnWaves},
    {"softmax_rows_loop", reinterpret_cast<const void*>(&softmax_rows_loop), kLoopThreads},
};
const OccupancyEntries kRowKernelsReg(kRowKernels);

}  // namespace
}  // namespace ehip

using namespace ehip;

extern "C" {

}  // extern "C"

namespace {

int softmax_run(const float* x, float* y, int64_t rows, int64_t cols, int causal, void* stream) {
    EHIP_READY();
    if (rows < 0 || cols <= 0) return fail(EHIP_EINVAL, "softmax: bad shape");
    if (!x || !y) return fail(EHIP_EINVAL, "softmax: null pointer");
    if (causal && rows % cols != 0)
        return fail(EHIP_EINVAL, "softmax (causal): %lld rows are not whole %lld x %lld matrices",
                    (long long)rows, (long long)cols, (long long)cols);
    if (rows == 0) return EHIP_OK;
    hipStream_t s = as_stream(stream);
    int rc = EHIP_OK;
    if (dispatch_row(rows, cols, rows_vec_ok(cols, {x, y}),
                     SoftmaxLaunch{x, y, rows, cols, s, &rc, causal}))
        return rc;
    EHIP_LAUNCH("softmax", softmax_rows_loop, dim3(loop_grid(rows)), dim3(kLoopThreads), 0, s, x, y,
                rows, cols, causal);
    return EHIP_OK;
}

int softmax_backward_run(const float* y, const float* g, float* dx, int64_t rows, int64_t cols,
                         float scale, int causal, void* stream) {
    EHIP_READY();
    if (rows < 0 || cols <= 0) return fail(EHIP_EINVAL, "softmax_backward: bad shape");
    if (!y || !g || !dx) return fail(EHIP_EINVAL, "softmax_backward: null pointer");
    if (causal && rows % cols != 0)
        return fail(EHIP_EINVAL,
                    "softmax_backward (causal): %lld rows are not whole %lld x %lld matrices",
                    (long long)rows, (long long)cols, (long long)cols);
    if (rows == 0) return EHIP_OK;
    hipStream_t s = as_stream(stream);
    int rc = EHIP_OK;
    if (dispatch_row(rows, cols, rows_vec_ok(cols, {y, g, dx}),
                     SoftmaxBackwardLaunch{y, g, dx, rows, cols, scale, s, &rc, causal}))
        return rc;
    EHIP_LAUNCH("softmax_backward", softmax_rows_backward_loop, dim3(loop_grid(rows)),
                dim3(kLoopThreads), 0, s, y, g, dx, rows, cols, scale, causal);
    return EHIP_OK;
}

}  // namespace

extern "C" {

int ehip_softmax_f32(const float* x, float* y, int64_t rows, int64_t cols, void* stream) {
    return softmax_run(x, y, rows, cols, 0, stream);
}

int ehip_softmax_causal_f32(const float* x, float* y, int64_t rows, int64_t cols, void* stream) {
    return softmax_run(x, y, rows, cols, 1, stream);
}

int ehip_softmax_backward_f32(const float* y, const float* g, float* dx, int64_t rows,
                              int64_t cols, void* stream) {
    return ehip_softmax_backward_scaled_f32(y, g, dx, rows, cols, 1.0f, stream);
}

int ehip_softmax_backward_scaled_f32(const float* y, const float* g, float* dx, int64_t rows,
                                     int64_t cols, float scale, void* stream) {
    return softmax_backward_run(y, g, dx, rows, cols, scale, 0, stream);
}

int ehip_softmax_backward_scaled_causal_f32(const float* y, const float* g, float* dx,
                                            int64_t rows, int64_t cols, float scale,
                                            void* stream) {
    return softmax_backward_run(y, g, dx, rows, cols, scale, 1, stream);
}

int ehip_cross_entropy_f32(const float* logits, const int32_t* targets, float* probs, float* loss,
                           int64_t rows, int64_t cols, void* stream) {
    EHIP_READY();
    if (rows <= 0 || cols <= 0) return fail(EHIP_EINVAL, "cross_entropy: bad shape");
    if (!logits || !targets || !probs || !loss)
        return fail(EHIP_EINVAL, "cross_entropy: null pointer");
    hipStream_t s = as_stream(stream);
    if (rows <= kXentMeanRows && cols <= 128) {
        if (cols <= 64)
            EHIP_LAUNCH("cross_entropy", xent_rows_mean<1>, dim3(1), dim3(1024), 0, s, logits,
                        targets, probs, loss, static_cast<float*>(nullptr), int(rows), int(cols));
        else
            EHIP_LAUNCH("cross_entropy", xent_rows_mean<2>, dim3(1), dim3(1024), 0, s, logits,
                        targets, probs, loss, static_cast<float*>(nullptr), int(rows), int(cols));
        return EHIP_OK;
    }
    float* row_loss = static_cast<float*>(scratch(size_t(rows) * sizeof(float)));
    if (row_loss == nullptr) return EHIP_ENOMEM;
    int rc = EHIP_OK;
    if (!dispatch_row(rows, cols, rows_vec_ok(cols, {logits, probs}),
                      XentLaunch{logits, targets, probs, row_loss, rows, cols, s, &rc})) {
        EHIP_LAUNCH("cross_entropy", xent_rows_loop, dim3(loop_grid(rows)), dim3(kLoopThreads), 0,
                    s, logits, targets, probs, row_loss, rows, cols);
    }
    if (rc != EHIP_OK) return rc;
    EHIP_LAUNCH("cross_entropy_mean", mean_rows, dim3(1), dim3(1024), 0, s, row_loss, rows, loss);
    return EHIP_OK;
}

int ehip_cross_entropy_fused_supported(int64_t rows, int64_t cols) {
    return rows > 0 && cols > 0 && rows <= kXentMeanRows && cols <= 128 ? 1 : 0;
}

int ehip_cross_entropy_fused_f32(const float* logits, const int32_t* targets, float* probs,
                                 float* loss, float* dlogits, int64_t rows, int64_t cols,
                                 void* stream) {
    EHIP_READY();
    if (!ehip_cross_entropy_fused_supported(rows, cols))
        return fail(EHIP_EINVAL, "cross_entropy_fused: shape %lld x %lld beyond one block",
                    (long long)rows, (long long)cols);
    if (!logits || !targets || !probs || !loss || !dlogits)
        return fail(EHIP_EINVAL, "cross_entropy_fused: null pointer");
    hipStream_t s = as_stream(stream);
    if (cols <= 64)
        EHIP_LAUNCH("cross_entropy_fused", xent_rows_mean<1>, dim3(1), dim3(1024), 0, s, logits,
                    targets, probs, loss, dlogits, int(rows), int(cols));
    else
        EHIP_LAUNCH("cross_entropy_fused", xent_rows_mean<2>, dim3(1), dim3(1024), 0, s, logits,
                    targets, probs, loss, dlogits, int(rows), int(cols));
    return EHIP_OK;
}

int ehip_cross_entropy_backward_f32(const float* probs, const int32_t* targets, float* dx,
                                    int64_t rows, int64_t cols, const float* grad, void* stream) {
    EHIP_READY();
    if (rows <= 0 || cols <= 0) return fail(EHIP_EINVAL, "cross_entropy_backward: bad shape");
    if (!probs || !targets || !dx || !grad)
        return fail(EHIP_EINVAL, "cross_entropy_backward: null pointer");
    int64_t grid = ceil_div(rows * cols, 256);
    if (grid > 131072) grid = 131072;
    EHIP_LAUNCH("cross_entropy_backward", xent_backward_from_probs, dim3(unsigned(grid)), dim3(256),
                0, as_stream(stream), probs, targets, dx, rows, cols, grad);
    return EHIP_OK;
}

int ehip_softmax_xent_backward_f32(const float* logits, const int32_t* targets, float* dx,
                                   int64_t rows, int64_t cols, const float* grad, void* stream) {
    EHIP_READY();
    if (rows <= 0 || cols <= 0) return fail(EHIP_EINVAL, "softmax_xent_backward: bad shape");
    if (!logits || !targets || !dx || !grad)
        return fail(EHIP_EINVAL, "softmax_xent_backward: null pointer");
    hipStream_t s = as_stream(stream);
    int rc = EHIP_OK;
    if (dispatch_row(rows, cols, rows_vec_ok(cols, {logits, dx}),
                     XentBackwardLaunch{logits, targets, dx, rows, cols, grad, s, &rc}))
        return rc;
    EHIP_LAUNCH("softmax_xent_backward", xent_rows_backward_loop, dim3(loop_grid(rows)),
                dim3(kLoopThreads), 0, s, logits, targets, dx, rows, cols, grad);
    return EHIP_OK;
}

int ehip_layernorm_f32(const float* x, const float* gamma, const float* beta, float* out,
                       float* xhat, float* inv_std, int64_t rows, int64_t cols, float eps,
                       void* stream) {
    EHIP_READY();
    if (rows < 0 || cols <= 0) return fail(EHIP_EINVAL, "layernorm: bad shape");
    if (!x || !gamma || !beta || !out || !xhat || !inv_std)
        return fail(EHIP_EINVAL, "layernorm: null pointer");
    if (rows == 0) return EHIP_OK;
    hipStream_t s = as_stream(stream);
    if (cols > kLnRegisterCols) {
        EHIP_LAUNCH("layernorm", layernorm_rows_loop, dim3(loop_grid(rows)), dim3(kLoopThreads), 0,
                    s, x, gamma, beta, out, xhat, inv_std, rows, cols, eps);
        return EHIP_OK;
    }
    const bool vec = cols >= 256 && rows_vec_ok(cols, {x, gamma, beta, out, xhat});
    // At most 512 blocks (two per CU): large inputs give each group several rows,
    // so that its loads of the next row overlap the stores of the current one.
    // Inputs beyond the last-level cache (2^25 elements and up) stream with
    // nontemporal loads and stores from up to 16384 blocks (measured 75 % of
    // HBM peak at 2^28 elements against 67 % for the cached form; at 2^23 the
    // cached form with 512 blocks is faster).
    const bool stream_nt = rows * cols >= (int64_t(1) << 25);
#define EHIP_LN(T, V, VEC)                                                                    \
    do {                                                                                      \
        if (stream_nt)                                                                        \
            EHIP_LAUNCH("layernorm", (layernorm_rows<T, V, VEC, true>),                       \
                        dim3(std::min(row_grid(rows, Group<T>::kPerBlock), 16384u)),          \
                        dim3(Group<T>::kBlock), 0, s, x, gamma, beta, out, xhat, inv_std, rows, \
                        cols, eps);                                                           \
        else                                                                                  \
            EHIP_LAUNCH("layernorm", (layernorm_rows<T, V, VEC>),                             \
                        dim3(std::min(row_grid(rows, Group<T>::kPerBlock), 512u)),            \
                        dim3(Group<T>::kBlock), 0, s, x, gamma, beta, out, xhat, inv_std, rows, \
                        cols, eps);                                                           \
    } while (0)
    if (vec) {
        if (cols <= 256) EHIP_LN(64, 4, true);
        else if (cols <= 512) EHIP_LN(64, 8, true);
        else if (cols <= 1024) EHIP_LN(64, 16, true);
        else if (cols <= 2048) EHIP_LN(64, 32, true);
        else if (cols <= 4096) EHIP_LN(256, 16, true);
        else EHIP_LN(256, 32, true);
    } else if (cols <= 64) EHIP_LN(64, 1, false);
    else if (cols <= 128) EHIP_LN(64, 2, false);
    else if (cols <= 256) EHIP_LN(64, 4, false);
    else if (cols <= 512) EHIP_LN(64, 8, false);
    else if (cols <= 1024) EHIP_LN(64, 16, false);
    else if (cols <= 2048) EHIP_LN(64, 32, false);
    else if (cols <= 4096) EHIP_LN(256, 16, false);
    else EHIP_LN(256, 32, false);
#undef EHIP_LN
    return EHIP_OK;
}

int ehip_layernorm_backward_f32(const float* dy, const float* xhat, const float* gamma,
                                const float* inv_std, float* dx, float* dgamma, float* dbeta,
                                int64_t rows, int64_t cols, void* stream) {
    EHIP_READY();
    if (rows < 0 || cols <= 0) return fail(EHIP_EINVAL, "layernorm_backward: bad shape");
    if (!dy || !xhat || !gamma || !inv_std || !dx || !dgamma || !dbeta)
        return fail(EHIP_EINVAL, "layernorm_backward: null pointer");
    hipStream_t s = as_stream(stream);
    if (cols > kLnRegisterCols) {
        // Row groups as for the small problems, fewer for very wide rows so
        // that the partials stay within 2^24 floats.
        int64_t groups = std::min<int64_t>(ceil_div(rows, 16), 256);
        groups = std::min<int64_t>(groups, std::max<int64_t>(1, (int64_t(1) << 23) / cols));
        if (groups < 1) groups = 1;
        float* partial =
            static_cast<float*>(scratch(size_t(groups) * 2 * size_t(cols) * sizeof(float)));
        if (partial == nullptr) return EHIP_ENOMEM;
        EHIP_LAUNCH("layernorm_backward", layernorm_rows_backward_loop, dim3(unsigned(groups)),
                    dim3(kLoopThreads), 0, s, dy, xhat, gamma, inv_std, dx, partial, rows, cols);
        return column_sums_pair(partial, groups, cols, 2 * cols, cols, dgamma, dbeta, s);
    }
    // A fixed number of row groups per shape, which fixes the order of the
    // dgamma / dbeta sums.
    const bool vec = cols >= 256 && rows_vec_ok(cols, {dy, xhat, gamma, dx});
    if (const int64_t groups = ln_wide_groups(rows, cols)) {
        // Large problems: the row kernel with per-group partials, then their
        // ordered sums (the same as the deferred form of
        // ehip_layernorm_backward_partials_f32 followed by the job's reduction).
        float* partial =
            static_cast<float*>(scratch(size_t(groups) * 2 * size_t(cols) * sizeof(float)));
        if (partial == nullptr) return EHIP_ENOMEM;
        if (int rc = launch_ln_wide(dy, xhat, gamma, inv_std, dx, partial, groups, rows, cols, s))
            return rc;
        const ehip_conv_reduce_t job{partial, groups, cols, 1, dgamma, dbeta};
        return ehip_conv_weight_reduce_f32(&job, 1, stream);
    }
    // Small problems: one wave per group of about 16 rows (at most 512 groups).
    int64_t groups = ceil_div(rows, 16);
    if (groups > 512) groups = 512;
    if (groups < 1) groups = 1;
    const unsigned grid = unsigned(groups);
    float* partial = static_cast<float*>(scratch(size_t(groups) * 2 * size_t(cols) * sizeof(float)));
    if (partial == nullptr) return EHIP_ENOMEM;
#define EHIP_LNB(T, V, VEC)                                                                     \
    EHIP_LAUNCH("layernorm_backward", (layernorm_rows_backward<T, V, VEC>), dim3(grid),         \
                dim3(T), 0, s, dy, xhat, gamma, inv_std, dx, partial, rows, cols)
#define EHIP_LNS(V, VEC)                                                                        \
    EHIP_LAUNCH("layernorm_backward", (layernorm_rows_backward_split<V, VEC, 4>), dim3(grid),   \
                dim3(256), 0, s, dy, xhat, gamma, inv_std, dx, partial, rows, cols)
    // Groups of at most kSplitRows rows of at most 256 columns: the group's rows
    // go to four waves side by side (the same bits, a quarter of the serial
    // row chain).
    if (ceil_div(rows, groups) <= kSplitRows && cols <= 256) {
        if (vec) EHIP_LNS(4, true);
        else if (cols <= 64) EHIP_LNS(1, false);
        else if (cols <= 128) EHIP_LNS(2, false);
        else EHIP_LNS(4, false);
    } else if (vec) {
        if (cols <= 256) EHIP_LNB(64, 4, true);
        else if (cols <= 512) EHIP_LNB(64, 8, true);
        else if (cols <= 1024) EHIP_LNB(64, 16, true);
        else if (cols <= 2048) EHIP_LNB(64, 32, true);
        else if (cols <= 4096) EHIP_LNB(256, 16, true);
        else EHIP_LNB(256, 32, true);
    } else if (cols <= 64) EHIP_LNB(64, 1, false);
    else if (cols <= 128) EHIP_LNB(64, 2, false);
    else if (cols <= 256) EHIP_LNB(64, 4, false);
    else if (cols <= 512) EHIP_LNB(64, 8, false);
    else if (cols <= 1024) EHIP_LNB(64, 16, false);
    else if (cols <= 2048) EHIP_LNB(64, 32, false);
    else if (cols <= 4096) EHIP_LNB(256, 16, false);
    else EHIP_LNB(256, 32, false);
#undef EHIP_LNB
#undef EHIP_LNS
    return column_sums_pair(partial, groups, cols, 2 * cols, cols, dgamma, dbeta, s);
}


int64_t ehip_layernorm_backward_partials(int64_t rows, int64_t cols, int64_t* groups) {
    const int64_t g = cols > 0 ? ln_wide_groups(rows, cols) : 0;
    if (groups) *groups = g;
    return g * 2 * (cols > 0 ? cols : 0);
}

int ehip_layernorm_backward_partials_f32(const float* dy, const float* xhat, const float* gamma,
                                         const float* inv_std, float* dx, float* partials,
                                         int64_t groups, int64_t rows, int64_t cols,
                                         int accumulate, void* stream) {
    EHIP_READY();
    if (rows < 0 || cols <= 0) return fail(EHIP_EINVAL, "layernorm_backward_partials: bad shape");
    if (!dy || !xhat || !gamma || !inv_std || !dx || !partials)
        return fail(EHIP_EINVAL, "layernorm_backward_partials: null pointer");
    if (accumulate && cols > 1024)
        return fail(EHIP_EINVAL,
                    "layernorm_backward_partials: accumulating rows of %lld columns (at most 1024)",
                    (long long)cols);
    const int64_t want = ln_wide_groups(rows, cols);
    if (want == 0 || groups != want)
        return fail(EHIP_EINVAL,
                    "layernorm_backward_partials: %lld groups for %lld x %lld (expected %lld)",
                    (long long)groups, (long long)rows, (long long)cols, (long long)want);
    return launch_ln_wide(dy, xhat, gamma, inv_std, dx, partials, groups, rows, cols,
                          as_stream(stream), accumulate ? 1 : 0);
}

}  // extern "C"
