/*
 * oracle.h -- CPU restatement of cpp-ai-engine's fp32 training path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP backend, the C++
 * engine, bench.py's GPU leg) links or calls this library. Only tests/,
 * __graft_entry__.smoke() and bench.py's `cpu_baseline` leg load it, and only
 * as the checker.
 *
 * Every function restates one loop nest of the reference CPU path in the same
 * accumulation order, so that for float work the oracle is bit-identical to
 * the reference (compiled without FMA contraction, as the reference is). The
 * reference file:line each function follows is given beside it; paths are
 * relative to the reference repository root.
 *
 * Pinning (what checks each function against something other than itself):
 *   - the 23 PyTorch-replay fixtures under tests/golden/fixtures/;
 *   - the compiled reference itself (oracle/_ref, built from the reference
 *     sources by oracle/Makefile), bit-exact on seeded inputs;
 *   - closed forms and brute force on tiny inputs (tests/test_oracle_*.py).
 * Functions with no such check would say "parity unpinned"; every function
 * below is pinned by at least one of the three. The whole-tensor sums are
 * pinned through the reference's Tensor::sum()/mean() (orc_sum) and the norm
 * clip_grad_norm returns (orc_sum_squares), bit for bit after the reference's
 * own cast to float, and by exact integer closed forms that only a double
 * accumulator meets; orc_scalar_add/orc_scalar_mul bit for bit against the
 * reference's t + k and t * k.
 */
#ifndef ORACLE_H
#define ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* C[b] = A[b] . B[b]; a_batched/b_batched = 0 means the operand is shared
 * across the batch (stride 0). C is overwritten. i -> k -> j with the a_ik == 0
 * skip, mul and add rounded separately (src/tensor_ops.cpp:539-562). */
void orc_matmul(const float* a, const float* b, float* c, int64_t batch, int64_t m, int64_t k,
                int64_t n, int a_batched, int b_batched);

/* dst[b][j][i] = src[b][i][j] (src/tensor_detail.hpp:82-108). */
void orc_transpose(const float* src, float* dst, int64_t batch, int64_t rows, int64_t cols);

/* General permutation: out axis i is input axis order[i]
 * (src/tensor_ops.cpp:375-471). */
void orc_permute(const float* src, float* dst, int ndim, const int64_t* in_shape,
                 const int64_t* order);

/* out = a op b with b repeated `repeat` times over blocks of `inner`
 * (src/tensor_ops.cpp:36-273). op: 0 add, 1 sub, 2 mul, 3 div. */
void orc_binary(int op, const float* a, const float* b, float* out, int64_t inner,
                int64_t repeat);

/* out = x + k (src/tensor_ops.cpp:276-299) and out = x * k (303-322). */
void orc_scalar_add(const float* x, float* out, int64_t n, float k);
void orc_scalar_mul(const float* x, float* out, int64_t n, float k);

/* ReLU and its derivative (src/tensor_ops.cpp:591-618). */
void orc_relu(const float* x, float* y, int64_t n);
void orc_relu_backward(const float* x, const float* g, float* dx, int64_t n);

/* grad += g (src/tensor.cpp:168-203, the accumulate branch; the first write
 * lands on a zero-filled buffer, so initialise == zero then accumulate). */
void orc_accumulate(float* grad, const float* g, int64_t n);

/* Sum over the middle axis of an (outer, axis_len, inner) view, a ascending,
 * from 0 (src/tensor.cpp:347-356; fold_leading is outer = 1,
 * src/tensor_detail.hpp:182-206). out is overwritten. */
void orc_sum_axis(const float* x, float* out, int64_t outer, int64_t axis_len, int64_t inner);

/* Whole-buffer sums in double, index order (src/tensor_ops.cpp:679-703). */
double orc_sum(const float* x, int64_t n);
double orc_sum_squares(const float* x, int64_t n);

/* Window geometry, the same fields as cuda::ops::WindowShape. */
typedef struct {
    int64_t batch, channels, height, width;
    int64_t kernel_h, kernel_w, stride, padding;
    int64_t out_h, out_w;
} orc_window;

/* im2col: (N,C,H,W) -> (N*oH*oW, C*kH*kW), padding left at zero
 * (src/conv.cpp:61-150). */
void orc_im2col(const float* x, float* cols, const orc_window* w);
/* col2im: the adjoint, summing per pixel in (n, oh, ow, c, i, j) order from 0
 * (src/conv.cpp:152-217). x is overwritten. */
void orc_col2im(const float* cols, float* x, const orc_window* w);

/* Max pooling with the flat input index of the first strict maximum
 * (src/conv.cpp:367-446); backward scatters in output order (449-470). */
void orc_maxpool(const float* x, float* y, int32_t* argmax, const orc_window* w);
void orc_maxpool_backward(const int32_t* argmax, const float* g, float* dx, int64_t n_out,
                          int64_t n_in);

/* Row softmax and its derivative (src/tensor_ops.cpp:621-676). */
void orc_softmax(const float* x, float* y, int64_t rows, int64_t cols);
void orc_softmax_backward(const float* y, const float* g, float* dx, int64_t rows, int64_t cols);

/* LayerNorm forward, two-pass (src/transformer.cpp:33-73), and backward with
 * dgamma/dbeta summed over rows in order (src/transformer.cpp:123-150).
 * dx, dgamma, dbeta are overwritten. */
void orc_layernorm(const float* x, const float* gamma, const float* beta, float* out,
                   float* xhat, float* inv_std, int64_t rows, int64_t d, float eps);
void orc_layernorm_backward(const float* dy, const float* xhat, const float* gamma,
                            const float* inv_std, float* dx, float* dgamma, float* dbeta,
                            int64_t rows, int64_t d);

/* Fused log-softmax + NLL, mean over rows accumulated serially in float
 * (src/nn.cpp:324-380). Returns the loss; probs receives the softmax.
 * Returns NaN and writes nothing further if a label is out of range. */
float orc_cross_entropy(const float* logits, const int64_t* targets, float* probs, int64_t n,
                        int64_t c);
/* dlogits = (probs - onehot) * (grad / N) (src/nn.cpp:386-405). */
void orc_cross_entropy_backward(const float* probs, const int64_t* targets, float* dx, int64_t n,
                                int64_t c, float grad);

/* Adam bias corrections, float std::pow (src/optim.cpp:119-120). */
void orc_adam_bias(float beta1, float beta2, int64_t t, float* bias_c1, float* bias_c2);
/* One Adam update in place (src/optim.cpp:147-160). */
void orc_adam(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1,
              float beta2, float eps, float weight_decay, float bias_c1, float bias_c2);
/* One SGD(+momentum, weight decay) update in place (src/optim.cpp:54-85). */
void orc_sgd(float* p, const float* g, float* velocity, int64_t n, float lr, float momentum,
             float weight_decay);

/* Row gather and its scatter-add adjoint, i ascending
 * (src/tensor.cpp:556-604). dx is accumulated into, not overwritten. */
void orc_select_rows(const float* x, const int64_t* idx, float* out, int64_t n_idx,
                     int64_t row_size);
void orc_scatter_add_rows(const float* g, const int64_t* idx, float* dx, int64_t n_idx,
                          int64_t row_size);

/* Constant tensors used by the Transformer path
 * (src/transformer.cpp:249-277). */
void orc_positional_encoding(float* out, int64_t seq_len, int64_t d_model);
void orc_causal_mask(float* out, int64_t seq_len, float masked_value);

/* Philox4x32-10 (Salmon et al., SC'11) on counter {c0..c3} and key {k0, k1}.
 * Pinned by the published Random123 known-answer vectors
 * (tests/test_oracle_fixtures.py). */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* Dropout as the device computes it: element i kept when the top 24 bits of
 * word (offset + i) % 4 of philox((offset + i) / 4; seed), over 2^24, are
 * below keep = 1 - p; mask[i] = keep ? 1 / keep : 0 and y = x * mask. The
 * reference (src/nn.cpp:206-244) draws from a sequential mt19937 instead, so
 * the masks are not the reference's: the checks are the generator's known
 * answers, the keep rate, and y and the backward given the mask. */
void orc_dropout(const float* x, float* y, float* mask, int64_t n, float p, uint64_t seed,
                 uint64_t offset);

#ifdef __cplusplus
}
#endif

#endif /* ORACLE_H */
