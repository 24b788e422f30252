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
// Query rows per forward workgroup: 8 (1024 workgroups at the char model's 128
// heads of 64) measured 10.4 us against 12.4 for 16 rows and 14.6 for 4 on
// MI355X, the same bits (each output's sum is one thread's whatever the
// split).
constexpr int kFwdRows = 8;
constexpr int kBwdThreads = 1024;
constexpr int kGroup = 4;          // score entries (consecutive keys) per thread and pass

struct AttnShape {
    int64_t batch, seq, width, heads, head_dim;
    float scale;
    int causal;
};

// e / d for 0 <= e < 16384 and 1 <= d <= 64 from the divisor's reciprocal:
// (e + 1/2) / d is at least 1/128 from an integer and the two roundings move it
// by under 2^-23 of at most 16384, so the truncation is exact.
__device__ __forceinline__ int quot(int e, float inv) { return int((float(e) + 0.5f) * inv); }

// Row i of head h of batch b in a (batch, seq, width) activation.
__device__ __forceinline__ int64_t head_row(const AttnShape& a, int64_t b, int64_t h, int64_t i) {
    return (b * a.seq + i) * a.width + h * a.head_dim;
}

// Rows [i0, i0 + rows) of one head, fetched into registers (every load of the
// thread issued before any is waited on; SLOTS float4s, or 4 SLOTS floats, cover
// the largest tile) and then placed in LDS rows dst[0 .. rows).
template <bool VEC, int THREADS, int SLOTS>
struct HeadTile {
    float4 v4[VEC ? SLOTS : 1];
    float v1[VEC ? 1 : 4 * SLOTS];
    int n = 0, i0 = 0;

    __device__ __forceinline__ void fetch(const float* __restrict__ src, const AttnShape& a,
                                          int64_t b, int64_t h, int first, int rows) {
        const int hd = int(a.head_dim);
        i0 = first;
        if (VEC) {
            const int q = hd / 4;
            const float inv = 1.0f / float(q);
            n = rows * q;
#pragma unroll
            for (int t = 0; t < SLOTS; ++t) {
                const int e = int(threadIdx.x) + t * THREADS;
                if (e < n) {
                    const int i = quot(e, inv), c4 = e - i * q;
                    v4[t] = *reinterpret_cast<const float4*>(src + head_row(a, b, h, i0 + i) +
                                                             4 * c4);
                }
            }
        } else {
            const float inv = 1.0f / float(hd);
            n = rows * hd;
#pragma unroll
            for (int t = 0; t < 4 * SLOTS; ++t) {
                const int e = int(threadIdx.x) + t * THREADS;
                if (e < n) {
                    const int i = quot(e, inv), c = e - i * hd;
                    v1[t] = src[head_row(a, b, h, i0 + i) + c];
                }
            }
        }
    }

    // Returns 1 when a placed value is not finite.
    __device__ __forceinline__ int place(float (*dst)[kAttnPitch], const AttnShape& a) const {
        const int hd = int(a.head_dim);
        int bad = 0;
        if (VEC) {
            const int q = hd / 4;
            const float inv = 1.0f / float(q);
#pragma unroll
            for (int t = 0; t < SLOTS; ++t) {
                const int e = int(threadIdx.x) + t * THREADS;
                if (e < n) {
                    const int i = quot(e, inv), c = 4 * (e - i * q);
                    dst[i][c] = v4[t].x;
                    dst[i][c + 1] = v4[t].y;
                    dst[i][c + 2] = v4[t].z;
                    dst[i][c + 3] = v4[t].w;
                    bad |= !(isfinite(v4[t].x) && isfinite(v4[t].y) && isfinite(v4[t].z) &&
                             isfinite(v4[t].w));
                }
            }
        } else {
            const float inv = 1.0f / float(hd);
#pragma unroll
            for (int t = 0; t < 4 * SLOTS; ++t) {
                const int e = int(threadIdx.x) + t * THREADS;
                if (e < n) {
                    const int i = quot(e, inv), c = e - i * hd;
                    dst[i][c] = v1[t];
                    bad |= !isfinite(v1[t]);
                }
            }
        }
        return bad;
    }
};

// acc + x * y in the reference's product order, the term skipped where the A
// operand x is zero (src/tensor_ops.cpp:553-560). A sum that starts at +0.0
// never becomes -0.0, so the skip changes a sum only when y is not finite:
// FAST (y known finite) computes the product and the add alone.
template <bool FAST>
__device__ __forceinline__ float mac(float acc, float x, float y) {
    if (FAST) return acc + x * y;
    return x != 0.0f ? acc + x * y : acc;
}

// dst[r][j] = OUT(sum_c a[r][c] b[j][c]) (ascending c) for rows r < rows and keys
// j < S, kGroup consecutive keys per thread so that their chains interleave;
// entries right of the diagonal (causal, query row i0 + r) are left alone.
template <bool FAST, int THREADS, typename Out>
__device__ __forceinline__ void row_products(float (*dst)[kAttnPitch], float (*a)[kAttnPitch],
                                             float (*b)[kAttnPitch], int rows, int S, int hd,
                                             int i0, bool causal, Out out) {
    const int ng = (S + kGroup - 1) / kGroup;
    const float inv = 1.0f / float(ng);
    for (int g = threadIdx.x; g < rows * ng; g += THREADS) {
        const int r = quot(g, inv), j0 = (g - r * ng) * kGroup, i = i0 + r;
        if (causal && j0 > i) continue;
        float acc[kGroup] = {};
#pragma unroll 4
        for (int c = 0; c < hd; ++c) {
            const float x = a[r][c];
#pragma unroll
            for (int t = 0; t < kGroup; ++t) acc[t] = mac<FAST>(acc[t], x, b[j0 + t][c]);
        }
#pragma unroll
        for (int t = 0; t < kGroup; ++t) {
            const int j = j0 + t;
            if (j < S && !(causal && j > i)) dst[r][j] = out(acc[t]);
        }
    }
}

// out[i][c] = sum_{j < n(i)} p[i][j] y[j][c] for rows i < rows (p: rows x S in
// LDS, y: S x hd), n(i) = i0 + i + 1 under the causal mask, else S; written
// through STORE(i, c, value).
template <bool FAST, int THREADS, typename Store>
__device__ __forceinline__ void row_times(float (*p)[kAttnPitch], float (*y)[kAttnPitch], int rows,
                                          int S, int hd, int i0, bool causal, Store store) {
    const float inv = 1.0f / float(hd);
    for (int e = threadIdx.x; e < rows * hd; e += THREADS) {
        const int i = quot(e, inv), c = e - i * hd;
        const int n = causal ? i0 + i + 1 : S;
        float acc = 0.0f;
#pragma unroll 8
        for (int j = 0; j < n; ++j) acc = mac<FAST>(acc, p[i][j], y[j][c]);
        store(i, c, acc);
    }
}

// out[j][c] = sum_{i >= i_min(j)} x[i][?] ... the column walks of the backward:
// out[j][c] = sum_i X(i, j, c) over i from (causal ? j : 0) to S - 1, with
// X given by TERM(acc, i, j, c); written through STORE(j, c, value).
template <int THREADS, typename Term, typename Store>
__device__ __forceinline__ void col_walk(int S, int hd, bool causal, Term term, Store store) {
    const float inv = 1.0f / float(hd);
    for (int e = threadIdx.x; e < S * hd; e += THREADS) {
        const int j = quot(e, inv), c = e - j * hd;
        float acc = 0.0f;
#pragma unroll 8
        for (int i = causal ? j : 0; i < S; ++i) acc = term(acc, i, j, c);
        store(j, c, acc);
    }
}

// Forward of one block of kFwdRows query rows of one (batch, head).
template <bool VEC>
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
    const bool causal = a.causal != 0;
    constexpr int kSlots = (kAttnMax * kAttnMax / 4 + kFwdThreads - 1) / kFwdThreads;
    constexpr int kQSlots = (kFwdRows * kAttnMax / 4 + kFwdThreads - 1) / kFwdThreads;
    HeadTile<VEC, kFwdThreads, kQSlots> tq;
    HeadTile<VEC, kFwdThreads, kSlots> tk, tv;
    tq.fetch(q, a, b, h, i0, rows);
    tk.fetch(k, a, b, h, 0, keys);
    tv.fetch(v, a, b, h, 0, keys);
    tq.place(sq, a);
    const int flags = tk.place(sk, a) | (tv.place(sv, a) << 1);
    const int bad_k = __syncthreads_or(flags & 1);
    const int bad_v = __syncthreads_or(flags & 2);
    // scores[i][j] = (sum_c q[i][c] k[j][c]) * scale
    const float scale = a.scale;
    const auto scaled = [scale](float x) { return x * scale; };
    if (bad_k)
        row_products<false, kFwdThreads>(sp, sq, sk, rows, keys, hd, i0, causal, scaled);
    else
        row_products<true, kFwdThreads>(sp, sq, sk, rows, keys, hd, i0, causal, scaled);
    __syncthreads();
    // Row softmax, a wave per row, lane j holding column j: the maximum over the
    // lanes (exact in any order), exp per lane, the denominator summed by lane 0
    // in column order (the reference's serial sum), the division per lane.
    const int wave = int(threadIdx.x) / 64, lane = int(threadIdx.x) % 64;
    for (int r = wave; r < rows; r += kFwdThreads / 64) {
        const int n = causal ? i0 + r + 1 : S;
        float x = lane < n ? sp[r][lane] : -INFINITY;
        float mx = x;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float ex = lane < n ? expf(x - mx) : 0.0f;
        if (lane < n) sp[r][lane] = ex;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float denom = 0.0f;
        if (lane == 0) {
#pragma unroll 16
            for (int j = 0; j < n; ++j) denom += sp[r][j];
        }
        denom = __shfl(denom, 0);
        if (lane < S) sp[r][lane] = lane < n ? ex / denom : 0.0f;
    }
    __syncthreads();
    float* wbase = weights + (bh * S + i0) * S;
    const float inv_s = 1.0f / float(S);
    for (int e = threadIdx.x; e < rows * S; e += kFwdThreads) {
        const int r = quot(e, inv_s), j = e - r * S;
        wbase[e] = sp[r][j];
    }
    // out[i][c] = sum_j weights[i][j] v[j][c]
    const auto store = [&](int i, int c, float val) { out[head_row(a, b, h, i0 + i) + c] = val; };
    if (bad_v)
        row_times<false, kFwdThreads>(sp, sv, rows, S, hd, i0, causal, store);
    else
        row_times<true, kFwdThreads>(sp, sv, rows, S, hd, i0, causal, store);
}

// dv = weights^T g; dP = g v^T; dS = (weights (dP - rowdot(dP, weights))) * scale;
// dq = dS k; dk = dS^T q (each of dq, dk, dv may be null). Two workgroups per
// (batch, head): blockIdx.x = 2 (batch * heads + head) + role; role 0 forms dv
// and dq, role 1 dk, and both form dP and dS (the same values), so the longest
// chain is three products instead of four over twice the workgroups.
template <bool VEC>
__global__ __launch_bounds__(kBwdThreads) void attention_short_backward(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ weights, const float* __restrict__ g, float* __restrict__ dq,
    float* __restrict__ dk, float* __restrict__ dv, AttnShape a) {
    __shared__ float sq[kAttnMax][kAttnPitch], sk[kAttnMax][kAttnPitch], sv[kAttnMax][kAttnPitch];
    __shared__ float sg[kAttnMax][kAttnPitch], sp[kAttnMax][kAttnPitch], sd[kAttnMax][kAttnPitch];
    __shared__ float sdot[kAttnMax];
    if (blockIdx.x & 1) {
        dq = nullptr;
        dv = nullptr;
    } else {
        dk = nullptr;
    }
    if (dq == nullptr && dk == nullptr && dv == nullptr) return;
    const int64_t bh = blockIdx.x / 2, b = bh / a.heads, h = bh % a.heads;
    const int S = int(a.seq), hd = int(a.head_dim);
    const bool causal = a.causal != 0;
    const bool want_qk = dq != nullptr || dk != nullptr;
    constexpr int kSlots = (kAttnMax * kAttnMax / 4 + kBwdThreads - 1) / kBwdThreads;
    HeadTile<VEC, kBwdThreads, kSlots> tq, tk, tv, tg;
    if (dk != nullptr) tq.fetch(q, a, b, h, 0, S);
    if (dq != nullptr) tk.fetch(k, a, b, h, 0, S);
    if (want_qk) tv.fetch(v, a, b, h, 0, S);
    tg.fetch(g, a, b, h, 0, S);
    const float* wbase = weights + bh * S * S;
    const float inv_s = 1.0f / float(S);
    float w[4 * kSlots];
#pragma unroll
    for (int t = 0; t < 4 * kSlots; ++t) {
        const int e = int(threadIdx.x) + t * kBwdThreads;
        if (e < S * S) w[t] = wbase[e];
    }
    if (dk != nullptr) tq.place(sq, a);
    const int bad_k = dq != nullptr ? tk.place(sk, a) : 0;
    const int bad_v = want_qk ? tv.place(sv, a) : 0;
    const int bad_g = tg.place(sg, a);
#pragma unroll
    for (int t = 0; t < 4 * kSlots; ++t) {
        const int e = int(threadIdx.x) + t * kBwdThreads;
        if (e < S * S) {
            const int i = quot(e, inv_s);
            sp[i][e - i * S] = w[t];
        }
    }
    const int flags = (bad_k ? 1 : 0) | (bad_v ? 2 : 0) | (bad_g ? 4 : 0);
    const int any_k = __syncthreads_or(flags & 1), any_v = __syncthreads_or(flags & 2),
              any_g = __syncthreads_or(flags & 4);
    if (dv != nullptr) {  // dv[j][c] = sum_i weights[i][j] g[i][c]
        const auto store = [&](int j, int c, float val) { dv[head_row(a, b, h, j) + c] = val; };
        if (any_g)
            col_walk<kBwdThreads>(S, hd, causal, [&](float acc, int i, int j, int c) {
                return mac<false>(acc, sp[i][j], sg[i][c]); }, store);
        else
            col_walk<kBwdThreads>(S, hd, causal, [&](float acc, int i, int j, int c) {
                return mac<true>(acc, sp[i][j], sg[i][c]); }, store);
    }
    if (!want_qk) return;
    // dP[i][j] = sum_c g[i][c] v[j][c]
    const auto same = [](float x) { return x; };
    if (any_v)
        row_products<false, kBwdThreads>(sd, sg, sv, S, S, hd, 0, causal, same);
    else
        row_products<true, kBwdThreads>(sd, sg, sv, S, S, hd, 0, causal, same);
    __syncthreads();
    if (int(threadIdx.x) < S) {  // the row dot products, serial in column order
        const int i = threadIdx.x, n = causal ? i + 1 : S;
        float dot = 0.0f;
#pragma unroll 8
        for (int j = 0; j < n; ++j) dot += sd[i][j] * sp[i][j];
        sdot[i] = dot;
    }
    __syncthreads();
    int bad_ds = 0;
    {
        for (int e = threadIdx.x; e < S * S; e += kBwdThreads) {
            const int i = quot(e, inv_s), j = e - i * S;
            const float ds = causal && j > i ? 0.0f : (sp[i][j] * (sd[i][j] - sdot[i])) * a.scale;
            sd[i][j] = ds;
            bad_ds |= !isfinite(ds);
        }
    }
    const int any_ds = __syncthreads_or(bad_ds);
    if (dq != nullptr) {  // dq[i][c] = sum_j dS[i][j] k[j][c]
        const auto store = [&](int i, int c, float val) { dq[head_row(a, b, h, i) + c] = val; };
        if (any_k)
            row_times<false, kBwdThreads>(sd, sk, S, S, hd, 0, causal, store);
        else
            row_times<true, kBwdThreads>(sd, sk, S, S, hd, 0, causal, store);
    }
    if (dk != nullptr) {  // dk[j][c] = sum_i q[i][c] dS[i][j]
        const auto store = [&](int j, int c, float val) { dk[head_row(a, b, h, j) + c] = val; };
        if (any_ds)
            col_walk<kBwdThreads>(S, hd, causal, [&](float acc, int i, int j, int c) {
                return mac<false>(acc, sq[i][c], sd[i][j]); }, store);
        else
            col_walk<kBwdThreads>(S, hd, causal, [&](float acc, int i, int j, int c) {
                return mac<true>(acc, sq[i][c], sd[i][j]); }, store);
    }
}

const OccupancyKernel kAttentionKernels[] = {
    {"attention_short_forward", reinterpret_cast<const void*>(&attention_short_forward<true>),
     kFwdThreads},
    {"attention_short_backward", reinterpret_cast<const void*>(&attention_short_backward<true>),
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
    const bool vec = head_dim % 4 == 0 && width % 4 == 0 && aligned16(q) && aligned16(k) &&
                     aligned16(v) && aligned16(out);
    const AttnShape a{batch, seq, width, heads, head_dim, scale, causal ? 1 : 0};
    const int64_t blocks = batch * heads * ((seq + kFwdRows - 1) / kFwdRows);
    if (vec)
        EHIP_LAUNCH("attention_short", attention_short_forward<true>, dim3(unsigned(blocks)),
                    dim3(kFwdThreads), 0, as_stream(stream), q, k, v, weights, out, a);
    else
        EHIP_LAUNCH("attention_short", attention_short_forward<false>, dim3(unsigned(blocks)),
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
    const bool vec = head_dim % 4 == 0 && width % 4 == 0 && (!q || aligned16(q)) &&
                     (!k || aligned16(k)) && (!v || aligned16(v)) && aligned16(grad);
    const AttnShape a{batch, seq, width, heads, head_dim, scale, causal ? 1 : 0};
    if (2 * batch * heads > 0x7fffffffLL)
        return fail(EHIP_EINVAL, "attention_short_backward: too many heads");
    const dim3 grid(unsigned(2 * batch * heads));
    if (vec)
        EHIP_LAUNCH("attention_short_backward", attention_short_backward<true>, grid,
                    dim3(kBwdThreads), 0, as_stream(stream), q, k, v, weights, grad, dq, dk, dv,
                    a);
    else
        EHIP_LAUNCH("attention_short_backward", attention_short_backward<false>, grid,
                    dim3(kBwdThreads), 0, as_stream(stream), q, k, v, weights, grad, dq, dk, dv,
                    a);
    return EHIP_OK;
}

}  // extern "C"
