// attention.hip -- scaled dot-product attention of short sequences (at most
// 64 positions, heads of at most 64 values) in one launch per direction: one
// workgroup per (batch, head) holds the head's Q, K, V (and in the backward
// dOut and the attention weights) in LDS and runs the whole composition of
// the reference's scaled_dot_product_attention (src/transformer.cpp:279-304:
// scores = Q K^T * scale [+ causal mask], softmax, weights V) and its autograd
// backward (src/tensor_ops.cpp:565-586 for each product's two materialised-
// transpose products, 663-670 for the softmax, 303-322 for the scale), each
// sum in the reference CPU loop's order: ascending index from 0, zero A
// operands skipped (src/tensor_ops.cpp:553-560), the softmax's denominator
// and the backward's row dot product serial in column order, the weights
// divided by the denominator. Masked entries (right of the diagonal under a
// causal mask) are skipped where the reference adds exact zeros there, so
// only the device exp (within an ulp of the host's) separates the results.
//
// Activations are (batch, seq, width) rows with head h at columns
// [h head_dim, (h + 1) head_dim), as the projections leave them; the weights
// are (batch, heads, seq, seq). The products and kernels of the general path
// (gemm.hip, rows.hip) take longer sequences.

#include "common.hpp"

namespace ehip {
namespace {

constexpr int kAttnMax = 64;       // positions and head values held in LDS
constexpr int kAttnPitch = 65;     // LDS row pitch (odd: column walks hit distinct banks)
constexpr int kFwdThreads = 256;
constexpr int kFwdRows = 16;       // query rows per forward workgroup
constexpr int kBwdThreads = 1024;
constexpr int kGroup = 4;          // score entries (consecutive keys) per thread and pass

struct AttnShape {
    int64_t batch, seq, width, heads, head_dim;
    float scale;
    int causal;
};

// Row i of head h of batch b in a (batch, seq, width) activation.
__device__ __forceinline__ int64_t head_row(const AttnShape& a, int64_t b, int64_t h, int64_t i) {
    return (b * a.seq + i) * a.width + h * a.head_dim;
}

// Rows [i0, i0 + rows) of one head into dst[0 .. rows).
template <int THREADS>
__device__ __forceinline__ void load_head(float (*dst)[kAttnPitch], const float* __restrict__ src,
                                          const AttnShape& a, int64_t b, int64_t h, int i0,
                                          int rows) {
    const int hd = int(a.head_dim), n = rows * hd;
    for (int e = threadIdx.x; e < n; e += THREADS) {
        const int i = e / hd, c = e - i * hd;
        dst[i][c] = src[head_row(a, b, h, i0 + i) + c];
    }
}

// acc[t] += x * y[t] in the reference's product order, the term skipped where the A
// operand x is zero (src/tensor_ops.cpp:553-560); a select keeps the lanes together.
__device__ __forceinline__ float mac(float acc, float x, float y) {
    return x != 0.0f ? acc + x * y : acc;
}

// dst[r][j] = sum_c a[r][c] b[j][c] (ascending c) for rows r < rows and keys j < S, kGroup
// consecutive keys per thread so that their chains interleave; entries right of the diagonal
// (causal, query row i0 + r) are left alone. The results pass through OUT(value) first.
template <int THREADS, typename Out>
__device__ __forceinline__ void row_products(float (*dst)[kAttnPitch], float (*a)[kAttnPitch],
                                             float (*b)[kAttnPitch], int rows, int S, int hd,
                                             int i0, bool causal, Out out) {
    const int ng = (S + kGroup - 1) / kGroup;
    for (int g = threadIdx.x; g < rows * ng; g += THREADS) {
        const int r = g / ng, j0 = (g - r * ng) * kGroup, i = i0 + r;
        if (causal && j0 > i) continue;
        float acc[kGroup] = {};
#pragma unroll 4
        for (int c = 0; c < hd; ++c) {
            const float x = a[r][c];
#pragma unroll
            for (int t = 0; t < kGroup; ++t) acc[t] = mac(acc[t], x, b[j0 + t][c]);
        }
#pragma unroll
        for (int t = 0; t < kGroup; ++t) {
            const int j = j0 + t;
            if (j < S && !(causal && j > i)) dst[r][j] = out(acc[t]);
        }
    }
}

// Forward of one block of kFwdRows query rows of one (batch, head).
__global__ __launch_bounds__(kFwdThreads) void attention_short_forward(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ weights, float* __restrict__ out, AttnShape a) {
    __shared__ float sq[kFwdRows][kAttnPitch], sk[kAttnMax][kAttnPitch];
    __shared__ float sv[kAttnMax][kAttnPitch], sp[kFwdRows][kAttnPitch];
    const int S = int(a.seq), hd = int(a.head_dim);
    const int blocks = (S + kFwdRows - 1) / kFwdRows;
    const int64_t bh = blockIdx.x / blocks, b = bh / a.heads, h = bh % a.heads;
    const int i0 = int(blockIdx.x % blocks) * kFwdRows, rows = min(kFwdRows, S - i0);
    const int keys = a.causal ? i0 + rows : S;  // keys any row of the block attends to
    load_head<kFwdThreads>(sq, q, a, b, h, i0, rows);
    load_head<kFwdThreads>(sk, k, a, b, h, 0, keys);
    load_head<kFwdThreads>(sv, v, a, b, h, 0, keys);
    __syncthreads();
    // scores[i][j] = (sum_c q[i][c] k[j][c]) * scale
    const float scale = a.scale;
    row_products<kFwdThreads>(sp, sq, sk, rows, keys, hd, i0, a.causal != 0,
                              [scale](float x) { return x * scale; });
    __syncthreads();
    // Row softmax, one thread per row (the reference's serial denominator).
    if (int(threadIdx.x) < rows) {
        const int r = threadIdx.x, n = a.causal ? i0 + r + 1 : S;
        float mx = sp[r][0];
        for (int j = 1; j < n; ++j) mx = fmaxf(mx, sp[r][j]);
        float denom = 0.0f;
#pragma unroll 8
        for (int j = 0; j < n; ++j) {
            const float ex = expf(sp[r][j] - mx);
            sp[r][j] = ex;
            denom += ex;
        }
        for (int j = 0; j < n; ++j) sp[r][j] = sp[r][j] / denom;
        for (int j = n; j < S; ++j) sp[r][j] = 0.0f;
    }
    __syncthreads();
    float* wbase = weights + (bh * S + i0) * S;
    for (int e = threadIdx.x; e < rows * S; e += kFwdThreads) {
        const int r = e / S, j = e - r * S;
        wbase[e] = sp[r][j];
    }
    // out[i][c] = sum_j weights[i][j] v[j][c]
    for (int e = threadIdx.x; e < rows * hd; e += kFwdThreads) {
        const int r = e / hd, c = e - r * hd;
        const int n = a.causal ? i0 + r + 1 : S;
        float acc = 0.0f;
#pragma unroll 8
        for (int j = 0; j < n; ++j) acc = mac(acc, sp[r][j], sv[j][c]);
        out[head_row(a, b, h, i0 + r) + c] = acc;
    }
}

// dv = weights^T g; dP = g v^T; dS = (weights (dP - rowdot(dP, weights))) * scale;
// dq = dS k; dk = dS^T q (each of dq, dk, dv may be null). One workgroup per (batch, head).
__global__ __launch_bounds__(kBwdThreads) void attention_short_backward(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ weights, const float* __restrict__ g, float* __restrict__ dq,
    float* __restrict__ dk, float* __restrict__ dv, AttnShape a) {
    __shared__ float sq[kAttnMax][kAttnPitch], sk[kAttnMax][kAttnPitch], sv[kAttnMax][kAttnPitch];
    __shared__ float sg[kAttnMax][kAttnPitch], sp[kAttnMax][kAttnPitch], sd[kAttnMax][kAttnPitch];
    __shared__ float sdot[kAttnMax];
    const int64_t bh = blockIdx.x, b = bh / a.heads, h = bh % a.heads;
    const int S = int(a.seq), hd = int(a.head_dim);
    const bool want_qk = dq != nullptr || dk != nullptr;
    if (dk != nullptr) load_head<kBwdThreads>(sq, q, a, b, h, 0, S);
    if (dq != nullptr) load_head<kBwdThreads>(sk, k, a, b, h, 0, S);
    if (want_qk) load_head<kBwdThreads>(sv, v, a, b, h, 0, S);
    load_head<kBwdThreads>(sg, g, a, b, h, 0, S);
    const float* wbase = weights + bh * S * S;
    for (int e = threadIdx.x; e < S * S; e += kBwdThreads) {
        const int i = e / S, j = e - i * S;
        sp[i][j] = wbase[e];
    }
    __syncthreads();
    if (dv != nullptr) {  // dv[j][c] = sum_i weights[i][j] g[i][c]
        for (int e = threadIdx.x; e < S * hd; e += kBwdThreads) {
            const int j = e / hd, c = e - j * hd;
            float acc = 0.0f;
#pragma unroll 8
            for (int i = a.causal ? j : 0; i < S; ++i) acc = mac(acc, sp[i][j], sg[i][c]);
            dv[head_row(a, b, h, j) + c] = acc;
        }
    }
    if (!want_qk) return;
    // dP[i][j] = sum_c g[i][c] v[j][c]
    row_products<kBwdThreads>(sd, sg, sv, S, S, hd, 0, a.causal != 0,
                              [](float x) { return x; });
    __syncthreads();
    if (int(threadIdx.x) < S) {  // the row dot products, serial in column order
        const int i = threadIdx.x, n = a.causal ? i + 1 : S;
        float dot = 0.0f;
#pragma unroll 8
        for (int j = 0; j < n; ++j) dot += sd[i][j] * sp[i][j];
        sdot[i] = dot;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < S * S; e += kBwdThreads) {
        const int i = e / S, j = e - i * S;
        sd[i][j] = a.causal && j > i ? 0.0f : (sp[i][j] * (sd[i][j] - sdot[i])) * a.scale;
    }
    __syncthreads();
    if (dq != nullptr) {  // dq[i][c] = sum_j dS[i][j] k[j][c]
        for (int e = threadIdx.x; e < S * hd; e += kBwdThreads) {
            const int i = e / hd, c = e - i * hd;
            const int n = a.causal ? i + 1 : S;
            float acc = 0.0f;
#pragma unroll 8
            for (int j = 0; j < n; ++j) acc = mac(acc, sd[i][j], sk[j][c]);
            dq[head_row(a, b, h, i) + c] = acc;
        }
    }
    if (dk != nullptr) {  // dk[j][c] = sum_i q[i][c] dS[i][j]
        for (int e = threadIdx.x; e < S * hd; e += kBwdThreads) {
            const int j = e / hd, c = e - j * hd;
            float acc = 0.0f;
#pragma unroll 8
            for (int i = a.causal ? j : 0; i < S; ++i) acc = mac(acc, sq[i][c], sd[i][j]);
            dk[head_row(a, b, h, j) + c] = acc;
        }
    }
}

const OccupancyKernel kAttentionKernels[] = {
    {"attention_short_forward", reinterpret_cast<const void*>(&attention_short_forward),
     kFwdThreads},
    {"attention_short_backward", reinterpret_cast<const void*>(&attention_short_backward),
     kBwdThreads},
};
const OccupancyEntries kAttentionKernelsReg(kAttentionKernels);

int check_shape(const char* name, int64_t batch, int64_t seq, int64_t width, int64_t heads,
                int64_t head_dim) {
    if (batch < 0 || seq < 1 || heads < 1 || head_dim < 1 || width < heads * head_dim)
        return fail(EHIP_EINVAL, "%s: bad shape", name);
    if (seq > kAttnMax || head_dim > kAttnMax)
        return fail(EHIP_EINVAL, "%s: %lld positions of %lld values exceed %d (use the products)",
                    name, (long long)seq, (long long)head_dim, kAttnMax);
    if (batch * heads * ((seq + kFwdRows - 1) / kFwdRows) > 0x7fffffffLL)
        return fail(EHIP_EINVAL, "%s: too many heads", name);
    return EHIP_OK;
}

}  // namespace
}  // namespace ehip

using namespace ehip;

extern "C" {

int ehip_attention_short_supported(int64_t seq, int64_t head_dim) {
    return seq >= 1 && head_dim >= 1 && seq <= kAttnMax && head_dim <= kAttnMax ? 1 : 0;
}

int ehip_attention_short_f32(const float* q, const float* k, const float* v, float* weights,
                             float* out, int64_t batch, int64_t seq, int64_t width, int64_t heads,
                             int64_t head_dim, float scale, int causal, void* stream) {
    EHIP_READY();
    if (int rc = check_shape("attention_short", batch, seq, width, heads, head_dim)) return rc;
    if (!q || !k || !v || !weights || !out) return fail(EHIP_EINVAL, "attention_short: null pointer");
    if (batch == 0) return EHIP_OK;
    const AttnShape a{batch, seq, width, heads, head_dim, scale, causal ? 1 : 0};
    const int64_t blocks = batch * heads * ((seq + kFwdRows - 1) / kFwdRows);
    EHIP_LAUNCH("attention_short", attention_short_forward, dim3(unsigned(blocks)),
                dim3(kFwdThreads), 0, as_stream(stream), q, k, v, weights, out, a);
    return EHIP_OK;
}

int ehip_attention_short_backward_f32(const float* q, const float* k, const float* v,
                                      const float* weights, const float* grad, float* dq,
                                      float* dk, float* dv, int64_t batch, int64_t seq,
                                      int64_t width, int64_t heads, int64_t head_dim, float scale,
                                      int causal, void* stream) {
    EHIP_READY();
    if (int rc = check_shape("attention_short_backward", batch, seq, width, heads, head_dim))
        return rc;
    if (!weights || !grad || (dk && !q) || (dq && !k) || ((dq || dk) && !v))
        return fail(EHIP_EINVAL, "attention_short_backward: null pointer");
    if (batch == 0 || (!dq && !dk && !dv)) return EHIP_OK;
    const AttnShape a{batch, seq, width, heads, head_dim, scale, causal ? 1 : 0};
    EHIP_LAUNCH("attention_short_backward", attention_short_backward,
                dim3(unsigned(batch * heads)), dim3(kBwdThreads), 0, as_stream(stream), q, k, v,
                weights, grad, dq, dk, dv, a);
    return EHIP_OK;
}

}  // extern "C"
