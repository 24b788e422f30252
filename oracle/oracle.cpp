// oracle.cpp -- CPU restatement of cpp-ai-engine's fp32 training path.
//
// TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg, as the checker, never by the product.
//
// Built with -ffp-contract=off and no -march (oracle/Makefile): every multiply
// and add rounds on its own, as in the reference's Release build, so float
// results are bit-identical to the reference CPU path. Each loop keeps the
// reference's accumulation order; where a loop is reordered the comment says
// why the order does not reach the result.

#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <vector>

namespace {

inline void clear(float* p, int64_t n) {
    if (n > 0) std::memset(p, 0, static_cast<size_t>(n) * sizeof(float));
}

// True if a window coordinate lands inside the unpadded input.
inline int64_t in_range(int64_t v, int64_t hi) { return v >= 0 && v < hi; }

}  // namespace

extern "C" {

// src/tensor_ops.cpp:539-562. C starts at zero; each output row is owned by
// one loop iteration and summed over k ascending, skipping a_ik == 0.
void orc_matmul(const float* a, const float* b, float* c, int64_t batch, int64_t m, int64_t k,
                int64_t n, int a_batched, int b_batched) {
    const int64_t sa = a_batched ? m * k : 0;
    const int64_t sb = b_batched ? k * n : 0;
    clear(c, batch * m * n);
    for (int64_t bi = 0; bi < batch; ++bi) {
        const float* ab = a + bi * sa;
        const float* bb = b + bi * sb;
        float* cb = c + bi * m * n;
        for (int64_t i = 0; i < m; ++i) {
            float* crow = cb + i * n;
            for (int64_t kk = 0; kk < k; ++kk) {
                const float aik = ab[i * k + kk];
                if (aik == 0.0f) continue;
                const float* brow = bb + kk * n;
                for (int64_t j = 0; j < n; ++j) crow[j] += aik * brow[j];
            }
        }
    }
}

// src/tensor_detail.hpp:82-108 (blocked there for cache reasons; a pure move,
// so the traversal order does not reach the result).
void orc_transpose(const float* src, float* dst, int64_t batch, int64_t rows, int64_t cols) {
    for (int64_t b = 0; b < batch; ++b) {
        const float* s = src + b * rows * cols;
        float* d = dst + b * rows * cols;
        for (int64_t i = 0; i < rows; ++i)
            for (int64_t j = 0; j < cols; ++j) d[j * rows + i] = s[i * cols + j];
    }
}

// src/tensor_ops.cpp:387-394 (output shape and source strides) and 437-458
// (the gather). A pure move.
void orc_permute(const float* src, float* dst, int ndim, const int64_t* in_shape,
                 const int64_t* order) {
    std::vector<int64_t> in_stride(ndim), out_shape(ndim), src_stride(ndim), idx(ndim, 0);
    int64_t s = 1, total = 1;
    for (int d = ndim - 1; d >= 0; --d) {
        in_stride[d] = s;
        s *= in_shape[d];
    }
    for (int d = 0; d < ndim; ++d) {
        out_shape[d] = in_shape[order[d]];
        src_stride[d] = in_stride[order[d]];
        total *= out_shape[d];
    }
    for (int64_t flat = 0; flat < total; ++flat) {
        int64_t off = 0;
        for (int d = 0; d < ndim; ++d) off += idx[d] * src_stride[d];
        dst[flat] = src[off];
        for (int d = ndim - 1; d >= 0; --d) {
            if (++idx[d] < out_shape[d]) break;
            idx[d] = 0;
        }
    }
}

// src/tensor_ops.cpp:52-71 (add), 121-137 (sub), 176-192 (mul), 232-248 (div).
void orc_binary(int op, const float* a, const float* b, float* out, int64_t inner,
                int64_t repeat) {
    for (int64_t r = 0; r < repeat; ++r) {
        const float* l = a + r * inner;
        float* o = out + r * inner;
        for (int64_t j = 0; j < inner; ++j) {
            switch (op) {
                case 0: o[j] = l[j] + b[j]; break;
                case 1: o[j] = l[j] - b[j]; break;
                case 2: o[j] = l[j] * b[j]; break;
                default: o[j] = l[j] / b[j]; break;
            }
        }
    }
}

// src/tensor_ops.cpp:280-285 and 307-312.
void orc_scalar_add(const float* x, float* out, int64_t n, float k) {
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] + k;
}
void orc_scalar_mul(const float* x, float* out, int64_t n, float k) {
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] * k;
}

// src/tensor_ops.cpp:594-599: std::max(0.0f, x) yields +0 unless 0 < x.
void orc_relu(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = (0.0f < x[i]) ? x[i] : 0.0f;
}
// src/tensor_ops.cpp:607-613.
void orc_relu_backward(const float* x, const float* g, float* dx, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dx[i] = (x[i] > 0.0f) ? g[i] : 0.0f;
}

// src/tensor.cpp:193-202.
void orc_accumulate(float* grad, const float* g, int64_t n) {
    for (int64_t i = 0; i < n; ++i) grad[i] += g[i];
}

// src/tensor.cpp:347-356.
void orc_sum_axis(const float* x, float* out, int64_t outer, int64_t axis_len, int64_t inner) {
    clear(out, outer * inner);
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t a = 0; a < axis_len; ++a) {
            const float* src = x + (o * axis_len + a) * inner;
            float* dst = out + o * inner;
            for (int64_t i = 0; i < inner; ++i) dst[i] += src[i];
        }
}

// src/tensor_ops.cpp:688-693; src/optim.cpp:186-193.
double orc_sum(const float* x, int64_t n) {
    double t = 0.0;
    for (int64_t i = 0; i < n; ++i) t += x[i];
    return t;
}
double orc_sum_squares(const float* x, int64_t n) {
    double t = 0.0;
    for (int64_t i = 0; i < n; ++i) t += static_cast<double>(x[i]) * x[i];
    return t;
}

// src/conv.cpp:61-150: cols[(n,oh,ow)][(c,i,j)] = x[n,c,oh*s+i-p,ow*s+j-p], or
// zero in the padding. A pure move.
void orc_im2col(const float* x, float* cols, const orc_window* w) {
    const int64_t K = w->channels * w->kernel_h * w->kernel_w;
    int64_t row = 0;
    for (int64_t n = 0; n < w->batch; ++n)
        for (int64_t oh = 0; oh < w->out_h; ++oh)
            for (int64_t ow = 0; ow < w->out_w; ++ow, ++row) {
                float* d = cols + row * K;
                for (int64_t c = 0; c < w->channels; ++c)
                    for (int64_t i = 0; i < w->kernel_h; ++i)
                        for (int64_t j = 0; j < w->kernel_w; ++j) {
                            const int64_t h = oh * w->stride + i - w->padding;
                            const int64_t v = ow * w->stride + j - w->padding;
                            const int64_t col = (c * w->kernel_h + i) * w->kernel_w + j;
                            d[col] = (in_range(h, w->height) && in_range(v, w->width))
                                         ? x[((n * w->channels + c) * w->height + h) * w->width + v]
                                         : 0.0f;
                        }
            }
}

// src/conv.cpp:183-214.
void orc_col2im(const float* cols, float* x, const orc_window* w) {
    const int64_t K = w->channels * w->kernel_h * w->kernel_w;
    clear(x, w->batch * w->channels * w->height * w->width);
    for (int64_t n = 0; n < w->batch; ++n)
        for (int64_t oh = 0; oh < w->out_h; ++oh)
            for (int64_t ow = 0; ow < w->out_w; ++ow) {
                const int64_t row = (n * w->out_h + oh) * w->out_w + ow;
                for (int64_t c = 0; c < w->channels; ++c)
                    for (int64_t i = 0; i < w->kernel_h; ++i) {
                        const int64_t h = oh * w->stride + i - w->padding;
                        if (!in_range(h, w->height)) continue;
                        for (int64_t j = 0; j < w->kernel_w; ++j) {
                            const int64_t v = ow * w->stride + j - w->padding;
                            if (!in_range(v, w->width)) continue;
                            const int64_t col = (c * w->kernel_h + i) * w->kernel_w + j;
                            x[((n * w->channels + c) * w->height + h) * w->width + v] +=
                                cols[row * K + col];
                        }
                    }
            }
}

// src/conv.cpp:410-442: the first window position with a strictly larger
// value wins.
void orc_maxpool(const float* x, float* y, int32_t* argmax, const orc_window* w) {
    for (int64_t n = 0; n < w->batch; ++n)
        for (int64_t c = 0; c < w->channels; ++c)
            for (int64_t oh = 0; oh < w->out_h; ++oh)
                for (int64_t ow = 0; ow < w->out_w; ++ow) {
                    float best = -std::numeric_limits<float>::infinity();
                    int64_t best_idx = 0;
                    bool found = false;
                    for (int64_t i = 0; i < w->kernel_h; ++i) {
                        const int64_t h = oh * w->stride + i - w->padding;
                        if (!in_range(h, w->height)) continue;
                        for (int64_t j = 0; j < w->kernel_w; ++j) {
                            const int64_t v = ow * w->stride + j - w->padding;
                            if (!in_range(v, w->width)) continue;
                            const int64_t idx =
                                ((n * w->channels + c) * w->height + h) * w->width + v;
                            if (!found || x[idx] > best) {
                                best = x[idx];
                                best_idx = idx;
                                found = true;
                            }
                        }
                    }
                    const int64_t o = ((n * w->channels + c) * w->out_h + oh) * w->out_w + ow;
                    y[o] = best;
                    argmax[o] = static_cast<int32_t>(best_idx);
                }
}

// src/conv.cpp:461-469.
void orc_maxpool_backward(const int32_t* argmax, const float* g, float* dx, int64_t n_out,
                          int64_t n_in) {
    clear(dx, n_in);
    for (int64_t i = 0; i < n_out; ++i) dx[argmax[i]] += g[i];
}

// src/tensor_ops.cpp:633-645.
void orc_softmax(const float* x, float* y, int64_t rows, int64_t cols) {
    for (int64_t i = 0; i < rows; ++i) {
        const float* row = x + i * cols;
        float* out = y + i * cols;
        const float mx = *std::max_element(row, row + cols);
        float denom = 0.0f;
        for (int64_t j = 0; j < cols; ++j) {
            const float e = std::exp(row[j] - mx);
            out[j] = e;
            denom += e;
        }
        for (int64_t j = 0; j < cols; ++j) out[j] /= denom;
    }
}

// src/tensor_ops.cpp:663-670.
void orc_softmax_backward(const float* y, const float* g, float* dx, int64_t rows, int64_t cols) {
    for (int64_t i = 0; i < rows; ++i) {
        const float* yr = y + i * cols;
        const float* gr = g + i * cols;
        float dot = 0.0f;
        for (int64_t j = 0; j < cols; ++j) dot += gr[j] * yr[j];
        for (int64_t j = 0; j < cols; ++j) dx[i * cols + j] = yr[j] * (gr[j] - dot);
    }
}

// src/transformer.cpp:53-73; inv_d = 1/D in float (transformer.cpp:90).
void orc_layernorm(const float* x, const float* gamma, const float* beta, float* out,
                   float* xhat, float* inv_std, int64_t rows, int64_t d, float eps) {
    const float inv_d = 1.0f / static_cast<float>(d);
    for (int64_t i = 0; i < rows; ++i) {
        const float* row = x + i * d;
        float mean = 0.0f;
        for (int64_t j = 0; j < d; ++j) mean += row[j];
        mean *= inv_d;
        float var = 0.0f;
        for (int64_t j = 0; j < d; ++j) {
            const float t = row[j] - mean;
            var += t * t;
        }
        var *= inv_d;
        const float inv = 1.0f / std::sqrt(var + eps);
        inv_std[i] = inv;
        for (int64_t j = 0; j < d; ++j) {
            const float h = (row[j] - mean) * inv;
            xhat[i * d + j] = h;
            out[i * d + j] = gamma[j] * h + beta[j];
        }
    }
}

// src/transformer.cpp:147-171: dx row by row; dgamma/dbeta over rows ascending.
void orc_layernorm_backward(const float* dy, const float* xhat, const float* gamma,
                            const float* inv_std, float* dx, float* dgamma, float* dbeta,
                            int64_t rows, int64_t d) {
    const float inv_d = 1.0f / static_cast<float>(d);
    clear(dgamma, d);
    clear(dbeta, d);
    for (int64_t i = 0; i < rows; ++i) {
        float sum_dxhat = 0.0f;
        float sum_dxhat_h = 0.0f;
        for (int64_t j = 0; j < d; ++j) {
            const float dxhat = dy[i * d + j] * gamma[j];
            sum_dxhat += dxhat;
            sum_dxhat_h += dxhat * xhat[i * d + j];
        }
        for (int64_t j = 0; j < d; ++j) {
            const int64_t k = i * d + j;
            const float dxhat = dy[k] * gamma[j];
            dx[k] = inv_std[i] * (dxhat - inv_d * sum_dxhat - xhat[k] * inv_d * sum_dxhat_h);
            dgamma[j] += dy[k] * xhat[k];
            dbeta[j] += dy[k];
        }
    }
}

// src/nn.cpp:352-376.
float orc_cross_entropy(const float* logits, const int64_t* targets, float* probs, int64_t n,
                        int64_t c) {
    float total = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        if (targets[i] < 0 || targets[i] >= c) return std::numeric_limits<float>::quiet_NaN();
        const float* row = logits + i * c;
        float* p = probs + i * c;
        const float mx = *std::max_element(row, row + c);
        float sum_exp = 0.0f;
        for (int64_t j = 0; j < c; ++j) {
            const float e = std::exp(row[j] - mx);
            p[j] = e;
            sum_exp += e;
        }
        for (int64_t j = 0; j < c; ++j) p[j] /= sum_exp;
        const float log_prob = (row[targets[i]] - mx) - std::log(sum_exp);
        total += -log_prob;
    }
    return total / static_cast<float>(n);
}

// src/nn.cpp:387-404.
void orc_cross_entropy_backward(const float* probs, const int64_t* targets, float* dx, int64_t n,
                                int64_t c, float grad) {
    const float scale = grad / static_cast<float>(n);
    for (int64_t i = 0; i < n; ++i)
        for (int64_t j = 0; j < c; ++j) {
            float g = probs[i * c + j];
            if (j == targets[i]) g -= 1.0f;
            dx[i * c + j] = g * scale;
        }
}

// src/optim.cpp:119-120.
void orc_adam_bias(float beta1, float beta2, int64_t t, float* bias_c1, float* bias_c2) {
    *bias_c1 = 1.0f - std::pow(beta1, static_cast<float>(t));
    *bias_c2 = 1.0f - std::pow(beta2, static_cast<float>(t));
}

// src/optim.cpp:147-160.
void orc_adam(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1,
              float beta2, float eps, float weight_decay, float bias_c1, float bias_c2) {
    for (int64_t j = 0; j < n; ++j) {
        float grad = g[j];
        if (weight_decay != 0.0f) grad += weight_decay * p[j];
        m[j] = beta1 * m[j] + (1.0f - beta1) * grad;
        v[j] = beta2 * v[j] + (1.0f - beta2) * grad * grad;
        const float m_hat = m[j] / bias_c1;
        const float v_hat = v[j] / bias_c2;
        p[j] -= lr * m_hat / (std::sqrt(v_hat) + eps);
    }
}

// src/optim.cpp:71-84.
void orc_sgd(float* p, const float* g, float* velocity, int64_t n, float lr, float momentum,
             float weight_decay) {
    float* vel = (velocity != nullptr && momentum != 0.0f) ? velocity : nullptr;
    for (int64_t j = 0; j < n; ++j) {
        float grad = g[j];
        if (weight_decay != 0.0f) grad += weight_decay * p[j];
        if (vel != nullptr) {
            vel[j] = momentum * vel[j] + grad;
            grad = vel[j];
        }
        p[j] -= lr * grad;
    }
}

// src/tensor.cpp:583-585 and 593-600.
void orc_select_rows(const float* x, const int64_t* idx, float* out, int64_t n_idx,
                     int64_t row_size) {
    for (int64_t i = 0; i < n_idx; ++i)
        std::memcpy(out + i * row_size, x + idx[i] * row_size,
                    static_cast<size_t>(row_size) * sizeof(float));
}
void orc_scatter_add_rows(const float* g, const int64_t* idx, float* dx, int64_t n_idx,
                          int64_t row_size) {
    for (int64_t i = 0; i < n_idx; ++i)
        for (int64_t j = 0; j < row_size; ++j) dx[idx[i] * row_size + j] += g[i * row_size + j];
}

// src/transformer.cpp:255-265 (float std::pow, std::sin, std::cos).
void orc_positional_encoding(float* out, int64_t seq_len, int64_t d_model) {
    for (int64_t pos = 0; pos < seq_len; ++pos)
        for (int64_t i = 0; i < d_model; ++i) {
            const int64_t pair = i / 2;
            const float exponent = 2.0f * static_cast<float>(pair) / static_cast<float>(d_model);
            const float angle = static_cast<float>(pos) / std::pow(10000.0f, exponent);
            out[pos * d_model + i] = (i % 2 == 0) ? std::sin(angle) : std::cos(angle);
        }
}

// src/transformer.cpp:269-277.
void orc_causal_mask(float* out, int64_t seq_len, float masked_value) {
    for (int64_t i = 0; i < seq_len; ++i)
        for (int64_t j = 0; j < seq_len; ++j) out[i * seq_len + j] = j > i ? masked_value : 0.0f;
}

void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        if (r > 0) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = uint64_t(0xD2511F53u) * c0, p1 = uint64_t(0xCD9E8D57u) * c2;
        const uint32_t hi0 = uint32_t(p0 >> 32), lo0 = uint32_t(p0);
        const uint32_t hi1 = uint32_t(p1 >> 32), lo1 = uint32_t(p1);
        const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

void orc_dropout(const float* x, float* y, float* mask, int64_t n, float p, uint64_t seed,
                 uint64_t offset) {
    const float keep = 1.0f - p;
    const float scale = 1.0f / keep;
    const uint32_t key[2] = {uint32_t(seed), uint32_t(seed >> 32)};
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t c = offset + uint64_t(i), b = c / 4;
        const uint32_t ctr[4] = {uint32_t(b), uint32_t(b >> 32), 0u, 0u};
        uint32_t w[4];
        orc_philox4x32_10(ctr, key, w);
        const float u = float(w[c % 4] >> 8) * (1.0f / 16777216.0f);
        const float m = u < keep ? scale : 0.0f;
        mask[i] = m;
        y[i] = x[i] * m;
    }
}

}  // extern "C"
