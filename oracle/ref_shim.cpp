// ref_shim.cpp -- a C ABI over the compiled reference engine.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file together with
// the reference's own CPU sources (read in place under the reference checkout,
// never copied) into oracle/_ref/libref_engine.so. Tests use it to pin the
// oracle restatement bit-exactly; bench.py's cpu_baseline leg times it
// ("kind": "reference").
//
// Every entry point builds reference Tensors from plain buffers, runs the
// reference's own public API (Tensor ops, nn layers, autograd, optim::Adam),
// and copies the results out. Errors become a nonzero return plus a message
// from ref_last_error().

#include "engine/autograd.hpp"
#include "engine/conv.hpp"
#include "engine/nn.hpp"
#include "engine/optim.hpp"
#include "engine/parallel.hpp"
#include "engine/serialize.hpp"
#include "engine/tensor.hpp"
#include "engine/transformer.hpp"

#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <string>
#include <vector>

using engine::Tensor;
namespace nn = engine::nn;
namespace optim = engine::optim;

namespace {

thread_local std::string g_error;

template <typename F>
int guarded(F&& body) {
    try {
        body();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 1;
    }
}

Tensor make(const std::vector<size_t>& shape, const float* data, bool req) {
    size_t n = 1;
    for (size_t d : shape) n *= d;
    return Tensor(shape, std::vector<float>(data, data + n), req);
}

void put(const Tensor& t, float* out) {
    if (out == nullptr) return;
    std::memcpy(out, t.data(), t.size() * sizeof(float));
}

void load_params(std::vector<Tensor> params, const float* flat) {
    size_t off = 0;
    for (Tensor& p : params) {
        std::memcpy(p.data(), flat + off, p.size() * sizeof(float));
        off += p.size();
    }
}

void store_params(const std::vector<Tensor>& params, float* flat) {
    size_t off = 0;
    for (const Tensor& p : params) {
        std::memcpy(flat + off, p.data(), p.size() * sizeof(float));
        off += p.size();
    }
}

std::vector<size_t> labels_of(const int64_t* t, int64_t n) {
    return std::vector<size_t>(t, t + n);
}

// The BASELINE cfg-2 network: conv 1->8 k3 p1, ReLU, pool 2, conv 8->16 k3 p1,
// ReLU, pool 2, flatten, linear 784->10.
std::unique_ptr<nn::Sequential> cnn_model(size_t in_c, size_t c1, size_t c2, size_t hw,
                                          size_t classes) {
    const size_t flat = c2 * (hw / 4) * (hw / 4);
    return std::make_unique<nn::Sequential>(
        nn::make<nn::Conv2d>(in_c, c1, nn::Window2d(3, 3, 1, 1)), nn::make<nn::ReLU>(),
        nn::make<nn::MaxPool2d>(2, 2), nn::make<nn::Conv2d>(c1, c2, nn::Window2d(3, 3, 1, 1)),
        nn::make<nn::ReLU>(), nn::make<nn::MaxPool2d>(2, 2), nn::make<nn::Flatten>(),
        nn::make<nn::Linear>(flat, classes));
}

// The character model of examples/charlm_demo.cpp:57-87: embedding plus the
// sinusoidal encoding, pre-LN blocks, a linear head.
struct CharModel {
    nn::Embedding embedding;
    std::vector<nn::TransformerBlock> blocks;
    nn::Linear head;
    Tensor positions;
    CharModel(size_t vocab, size_t seq, size_t d, size_t heads, size_t ff, size_t layers)
        : embedding(vocab, d), head(d, vocab), positions(nn::positional_encoding(seq, d)) {
        blocks.reserve(layers);
        for (size_t i = 0; i < layers; ++i) blocks.emplace_back(d, heads, ff);
    }
    Tensor forward(const Tensor& ids, const Tensor& mask) {
        Tensor h = embedding.forward(ids) + positions;
        for (nn::TransformerBlock& b : blocks) h = b.forward(h, &mask);
        return head.forward(h);
    }
    std::vector<Tensor> parameters() {
        std::vector<Tensor> out = embedding.parameters();
        for (nn::TransformerBlock& b : blocks)
            for (const Tensor& p : b.parameters()) out.push_back(p);
        for (const Tensor& p : head.parameters()) out.push_back(p);
        return out;
    }
};

}  // namespace

extern "C" {

const char* ref_last_error() { return g_error.c_str(); }

void ref_set_threads(int n) { engine::parallel::set_num_threads(static_cast<size_t>(n)); }
int ref_num_threads() { return static_cast<int>(engine::parallel::num_threads()); }

// Tensor::matmul forward only (src/tensor_ops.cpp:475-563). A 2-D operand is
// shared across the batch when its *_batched flag is 0.
int ref_matmul(const float* a, const float* b, float* c, int64_t batch, int64_t m, int64_t k,
               int64_t n, int a_batched, int b_batched) {
    return guarded([&] {
        std::vector<size_t> sa = {size_t(m), size_t(k)}, sb = {size_t(k), size_t(n)};
        if (a_batched) sa.insert(sa.begin(), size_t(batch));
        if (b_batched) sb.insert(sb.begin(), size_t(batch));
        put(make(sa, a, false).matmul(make(sb, b, false)), c);
    });
}

// 2-D matmul forward and backward through autograd.
int ref_matmul_fwd_bwd(const float* a, const float* b, const float* dc, int64_t m, int64_t k,
                       int64_t n, float* c, float* da, float* db) {
    return guarded([&] {
        Tensor A = make({size_t(m), size_t(k)}, a, true);
        Tensor B = make({size_t(k), size_t(n)}, b, true);
        Tensor C = A.matmul(B);
        C.backward(make({size_t(m), size_t(n)}, dc, false));
        put(C, c);
        put(A.grad(), da);
        put(B.grad(), db);
    });
}

// Any element-wise binary op with suffix broadcast, forward and backward.
// op: 0 add, 1 sub, 2 mul, 3 div.
int ref_binary_fwd_bwd(int op, const float* a, const int64_t* a_shape, int a_nd, const float* b,
                       const int64_t* b_shape, int b_nd, const float* dy, float* y, float* da,
                       float* db) {
    return guarded([&] {
        std::vector<size_t> sa(a_shape, a_shape + a_nd), sb(b_shape, b_shape + b_nd);
        Tensor A = make(sa, a, true), B = make(sb, b, true);
        Tensor Y = op == 0 ? A + B : op == 1 ? A - B : op == 2 ? A * B : A / B;
        Y.backward(make(sa, dy, false));
        put(Y, y);
        put(A.grad(), da);
        put(B.grad(), db);
    });
}

// Tensor::permute forward and backward.
int ref_permute_fwd_bwd(const float* x, const int64_t* shape, int nd, const int64_t* order,
                        const float* dy, float* y, float* dx) {
    return guarded([&] {
        std::vector<size_t> s(shape, shape + nd), o(order, order + nd), so(nd);
        for (int i = 0; i < nd; ++i) so[i] = s[o[i]];
        Tensor X = make(s, x, true);
        Tensor Y = X.permute(o);
        Y.backward(make(so, dy, false));
        put(Y, y);
        put(X.grad(), dx);
    });
}

// Tensor::sum(axis) forward and backward.
int ref_sum_axis_fwd_bwd(const float* x, const int64_t* shape, int nd, int axis, const float* dy,
                         float* y, float* dx) {
    return guarded([&] {
        std::vector<size_t> s(shape, shape + nd);
        Tensor X = make(s, x, true);
        Tensor Y = X.sum(size_t(axis));
        Y.backward(make(Y.shape(), dy, false));
        put(Y, y);
        put(X.grad(), dx);
    });
}

// ReLU / softmax forward and backward. which: 0 relu, 1 softmax (last axis).
int ref_unary_fwd_bwd(int which, const float* x, int64_t rows, int64_t cols, const float* dy,
                      float* y, float* dx) {
    return guarded([&] {
        Tensor X = make({size_t(rows), size_t(cols)}, x, true);
        Tensor Y = which == 0 ? X.relu() : X.softmax();
        Y.backward(make({size_t(rows), size_t(cols)}, dy, false));
        put(Y, y);
        put(X.grad(), dx);
    });
}

// Whole-tensor sum (double accumulation, src/tensor_ops.cpp:679-703).
int ref_sum(const float* x, int64_t n, float* out) {
    return guarded([&] { put(make({size_t(n)}, x, false).sum(), out); });
}

// Tensor::mean() (src/tensor_ops.cpp:706-712): the double sum cast to float,
// times 1/n in float.
int ref_mean(const float* x, int64_t n, float* out) {
    return guarded([&] { put(make({size_t(n)}, x, false).mean(), out); });
}

// Tensor::operator+(float) (src/tensor_ops.cpp:276-295) when mul is 0, and
// Tensor::operator*(float) (src/tensor_ops.cpp:303-322) otherwise.
int ref_scalar(const float* x, int64_t n, float k, int mul, float* out) {
    return guarded([&] {
        const Tensor X = make({size_t(n)}, x, false);
        put(mul ? X * k : X + k, out);
    });
}

// nn::im2col and nn::col2im on their own.
int ref_im2col(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, int64_t kh,
               int64_t kw, int64_t stride, int64_t pad, float* cols) {
    return guarded([&] {
        Tensor X = make({size_t(N), size_t(C), size_t(H), size_t(W)}, x, false);
        put(nn::im2col(X, nn::Window2d(kh, kw, stride, pad)), cols);
    });
}
int ref_col2im(const float* cols, int64_t N, int64_t C, int64_t H, int64_t W, int64_t kh,
               int64_t kw, int64_t stride, int64_t pad, float* x) {
    return guarded([&] {
        nn::Window2d win(kh, kw, stride, pad);
        const size_t rows = size_t(N) * win.out_h(H) * win.out_w(W);
        Tensor Cc = make({rows, size_t(C * kh * kw)}, cols, false);
        put(nn::col2im(Cc, {size_t(N), size_t(C), size_t(H), size_t(W)}, win), x);
    });
}

// nn::Conv2d forward and backward with given weights.
int ref_conv2d_fwd_bwd(const float* x, const float* w, const float* bias, int64_t N, int64_t C,
                       int64_t H, int64_t W, int64_t out_c, int64_t k, int64_t stride,
                       int64_t pad, const float* dy, float* y, float* dx, float* dw, float* db) {
    return guarded([&] {
        nn::Conv2d conv(static_cast<size_t>(C), static_cast<size_t>(out_c), nn::Window2d(k, k, stride, pad));
        load_params(conv.parameters(), w);
        std::memcpy(conv.bias().data(), bias, size_t(out_c) * sizeof(float));
        Tensor X = make({size_t(N), size_t(C), size_t(H), size_t(W)}, x, true);
        Tensor Y = conv(X);
        Y.backward(make(Y.shape(), dy, false));
        put(Y, y);
        put(X.grad(), dx);
        put(conv.weight().grad(), dw);
        put(conv.bias().grad(), db);
    });
}

// nn::MaxPool2d forward and backward.
int ref_maxpool_fwd_bwd(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, int64_t k,
                        int64_t stride, const float* dy, float* y, float* dx) {
    return guarded([&] {
        nn::MaxPool2d pool(static_cast<size_t>(k), static_cast<size_t>(stride));
        Tensor X = make({size_t(N), size_t(C), size_t(H), size_t(W)}, x, true);
        Tensor Y = pool(X);
        Y.backward(make(Y.shape(), dy, false));
        put(Y, y);
        put(X.grad(), dx);
    });
}

// nn::LayerNorm forward and backward.
int ref_layernorm_fwd_bwd(const float* x, const float* gamma, const float* beta, int64_t rows,
                          int64_t d, const float* dy, float* y, float* dx, float* dgamma,
                          float* dbeta) {
    return guarded([&] {
        nn::LayerNorm ln(static_cast<size_t>(d));
        std::memcpy(ln.gamma().data(), gamma, size_t(d) * sizeof(float));
        std::memcpy(ln.beta().data(), beta, size_t(d) * sizeof(float));
        Tensor X = make({size_t(rows), size_t(d)}, x, true);
        Tensor Y = ln(X);
        Y.backward(make(Y.shape(), dy, false));
        put(Y, y);
        put(X.grad(), dx);
        put(ln.gamma().grad(), dgamma);
        put(ln.beta().grad(), dbeta);
    });
}

// nn::cross_entropy_loss forward and backward (implicit dL/dL = 1).
int ref_cross_entropy(const float* logits, const int64_t* targets, int64_t n, int64_t c,
                      float* loss, float* dlogits) {
    return guarded([&] {
        Tensor L = make({size_t(n), size_t(c)}, logits, true);
        Tensor loss_t = nn::cross_entropy_loss(L, labels_of(targets, n));
        loss_t.backward();
        put(loss_t, loss);
        put(L.grad(), dlogits);
    });
}

// Embedding forward and backward: ids (B,S) as floats, table (V,D).
int ref_embedding_fwd_bwd(const float* table, int64_t vocab, int64_t d, const float* ids,
                          int64_t batch, int64_t seq, const float* dy, float* y, float* dtable) {
    return guarded([&] {
        nn::Embedding emb(static_cast<size_t>(vocab), static_cast<size_t>(d));
        std::memcpy(emb.weight().data(), table, size_t(vocab * d) * sizeof(float));
        Tensor Y = emb(make({size_t(batch), size_t(seq)}, ids, false));
        Y.backward(make(Y.shape(), dy, false));
        put(Y, y);
        put(emb.weight().grad(), dtable);
    });
}

// optim::Adam over one flat parameter for `steps` steps of a fixed gradient
// sequence: grads holds steps * n values.
int ref_adam_steps(float* p, const float* grads, int64_t n, int64_t steps, float lr, float b1,
                   float b2, float eps, float wd) {
    return guarded([&] {
        Tensor P = make({size_t(n)}, p, true);
        optim::Adam opt({P}, lr, b1, b2, eps, wd);
        for (int64_t s = 0; s < steps; ++s) {
            opt.zero_grad();
            P.add_grad(make({size_t(n)}, grads + s * n, false));
            opt.step();
        }
        put(P, p);
    });
}

// optim::clip_grad_norm over `count` parameters: parameter i has |sizes[i]|
// elements and, when sizes[i] > 0, the gradient taken from `grads`
// (concatenated); a negative size is a parameter without a gradient. Clipped
// gradients are written back over `grads`, the norm to *norm.
int ref_clip_grad_norm(float* grads, const int64_t* sizes, int count, float max_norm,
                       float* norm) {
    return guarded([&] {
        std::vector<Tensor> ps;
        size_t off = 0;
        for (int i = 0; i < count; ++i) {
            const size_t n = size_t(sizes[i] < 0 ? -sizes[i] : sizes[i]);
            Tensor P({n}, 0.0f, true);
            if (sizes[i] > 0) {
                P.add_grad(make({n}, grads + off, false));
                off += n;
            }
            ps.push_back(P);
        }
        *norm = optim::clip_grad_norm(ps, max_norm);
        off = 0;
        for (int i = 0; i < count; ++i) {
            if (sizes[i] <= 0) continue;
            put(ps[size_t(i)].grad(), grads + off);
            off += size_t(sizes[i]);
        }
    });
}

// Scaled dot-product attention with an optional mask (S,S), forward and
// backward: q,k,v (B,H,S,dk).
int ref_attention_fwd_bwd(const float* q, const float* k, const float* v, const float* mask,
                          int64_t b, int64_t h, int64_t s, int64_t dk, const float* dy, float* y,
                          float* weights, float* dq, float* dkk, float* dv) {
    return guarded([&] {
        std::vector<size_t> sh = {size_t(b), size_t(h), size_t(s), size_t(dk)};
        Tensor Q = make(sh, q, true), K = make(sh, k, true), V = make(sh, v, true);
        Tensor M;
        if (mask != nullptr) M = make({size_t(s), size_t(s)}, mask, false);
        Tensor W;
        Tensor Y = nn::scaled_dot_product_attention(Q, K, V, mask ? &M : nullptr, &W);
        Y.backward(make(sh, dy, false));
        put(Y, y);
        put(W, weights);
        put(Q.grad(), dq);
        put(K.grad(), dkk);
        put(V.grad(), dv);
    });
}

// A TransformerBlock forward and backward with given parameters (flat, in
// parameters() order) and an optional causal mask.
int ref_block_fwd_bwd(const float* x, int64_t b, int64_t s, int64_t d, int64_t heads, int64_t ff,
                      int causal, const float* params, const float* dy, float* y, float* dx,
                      float* dparams) {
    return guarded([&] {
        nn::TransformerBlock block(static_cast<size_t>(d), static_cast<size_t>(heads), static_cast<size_t>(ff));
        load_params(block.parameters(), params);
        Tensor X = make({size_t(b), size_t(s), size_t(d)}, x, true);
        Tensor M = nn::causal_mask(size_t(s));
        Tensor Y = block.forward(X, causal ? &M : nullptr);
        Y.backward(make(Y.shape(), dy, false));
        put(Y, y);
        put(X.grad(), dx);
        size_t off = 0;
        for (const Tensor& p : block.parameters()) {
            put(p.grad(), dparams + off);
            off += p.size();
        }
    });
}

int64_t ref_block_num_params(int64_t d, int64_t heads, int64_t ff) {
    nn::TransformerBlock block(static_cast<size_t>(d), static_cast<size_t>(heads), static_cast<size_t>(ff));
    return int64_t(block.num_parameters());
}

// cfg 2: the small CNN, `steps` Adam steps on one fixed batch. params is the
// flat parameters() concatenation; losses receives one value per step.
// The CNN of cnn_model with the flat parameters `params`, saved by the
// reference's save_parameters to `path`.
int ref_cnn_save(const float* params, int64_t in_c, int64_t c1, int64_t c2, int64_t hw,
                 int64_t classes, const char* path) {
    return guarded([&] {
        auto model = cnn_model(size_t(in_c), size_t(c1), size_t(c2), size_t(hw), size_t(classes));
        load_params(model->parameters(), params);
        engine::save_parameters(*model, path);
    });
}

// A CNN of cnn_model loaded by the reference's load_parameters (strict) from
// `path`; its flat parameters go to params_out.
int ref_cnn_load(const char* path, int64_t in_c, int64_t c1, int64_t c2, int64_t hw,
                 int64_t classes, float* params_out) {
    return guarded([&] {
        auto model = cnn_model(size_t(in_c), size_t(c1), size_t(c2), size_t(hw), size_t(classes));
        engine::load_parameters(*model, path, true);
        store_params(model->parameters(), params_out);
    });
}

// One forward and backward of the CNN: the loss and every parameter's gradient
// (flat, parameter order).
int ref_cnn_grads(const float* x, const int64_t* labels, int64_t batch, int64_t in_c, int64_t c1,
                  int64_t c2, int64_t hw, int64_t classes, const float* params, float* loss_out,
                  float* grads_out) {
    return guarded([&] {
        auto model = cnn_model(size_t(in_c), size_t(c1), size_t(c2), size_t(hw), size_t(classes));
        load_params(model->parameters(), params);
        Tensor X = make({size_t(batch), size_t(in_c), size_t(hw), size_t(hw)}, x, false);
        Tensor loss = nn::cross_entropy_loss((*model)(X), labels_of(labels, batch));
        loss.backward();
        put(loss, loss_out);
        size_t off = 0;
        for (const Tensor& p : model->parameters()) {
            put(p.grad(), grads_out + off);
            off += p.size();
        }
    });
}

int ref_cnn_train(const float* x, const int64_t* labels, int64_t batch, int64_t in_c, int64_t c1,
                  int64_t c2, int64_t hw, int64_t classes, const float* params, int64_t steps,
                  float lr, float* losses, float* params_out) {
    return guarded([&] {
        auto model = cnn_model(size_t(in_c), size_t(c1), size_t(c2), size_t(hw), size_t(classes));
        load_params(model->parameters(), params);
        optim::Adam opt(model->parameters(), lr);
        Tensor X = make({size_t(batch), size_t(in_c), size_t(hw), size_t(hw)}, x, false);
        const std::vector<size_t> y = labels_of(labels, batch);
        for (int64_t s = 0; s < steps; ++s) {
            opt.zero_grad();
            Tensor loss = nn::cross_entropy_loss((*model)(X), y);
            loss.backward();
            opt.step();
            if (losses) losses[s] = loss.data()[0];
        }
        if (params_out) store_params(model->parameters(), params_out);
    });
}

// cfg 3 / cfg 5: the character Transformer, `steps` Adam steps on one batch.
int ref_charlm_train(const float* ids, const int64_t* targets, int64_t batch, int64_t seq,
                     int64_t vocab, int64_t d, int64_t heads, int64_t ff, int64_t layers,
                     const float* params, int64_t steps, float lr, float* losses,
                     float* params_out) {
    return guarded([&] {
        CharModel model{size_t(vocab), size_t(seq), size_t(d), size_t(heads), size_t(ff),
                        size_t(layers)};
        load_params(model.parameters(), params);
        optim::Adam opt(model.parameters(), lr);
        const Tensor mask = nn::causal_mask(size_t(seq));
        Tensor X = make({size_t(batch), size_t(seq)}, ids, false);
        const std::vector<size_t> y = labels_of(targets, batch * seq);
        for (int64_t s = 0; s < steps; ++s) {
            opt.zero_grad();
            Tensor logits = model.forward(X, mask).reshape({size_t(batch * seq), size_t(vocab)});
            Tensor loss = nn::cross_entropy_loss(logits, y);
            loss.backward();
            opt.step();
            if (losses) losses[s] = loss.data()[0];
        }
        if (params_out) store_params(model.parameters(), params_out);
    });
}

// As ref_charlm_train, and the first step's gradients (after backward, before
// the update; parameter order) go to grads0 when it is not NULL.
int ref_charlm_train_grads(const float* ids, const int64_t* targets, int64_t batch, int64_t seq,
                           int64_t vocab, int64_t d, int64_t heads, int64_t ff, int64_t layers,
                           const float* params, int64_t steps, float lr, float* losses,
                           float* grads0, float* params_out) {
    return guarded([&] {
        CharModel model{size_t(vocab), size_t(seq), size_t(d), size_t(heads), size_t(ff),
                        size_t(layers)};
        load_params(model.parameters(), params);
        optim::Adam opt(model.parameters(), lr);
        const Tensor mask = nn::causal_mask(size_t(seq));
        Tensor X = make({size_t(batch), size_t(seq)}, ids, false);
        const std::vector<size_t> y = labels_of(targets, batch * seq);
        for (int64_t s = 0; s < steps; ++s) {
            opt.zero_grad();
            Tensor logits = model.forward(X, mask).reshape({size_t(batch * seq), size_t(vocab)});
            Tensor loss = nn::cross_entropy_loss(logits, y);
            loss.backward();
            if (s == 0 && grads0) {
                size_t off = 0;
                for (const Tensor& p : model.parameters()) {
                    put(p.grad(), grads0 + off);
                    off += p.size();
                }
            }
            opt.step();
            if (losses) losses[s] = loss.data()[0];
        }
        if (params_out) store_params(model.parameters(), params_out);
    });
}

int64_t ref_charlm_num_params(int64_t vocab, int64_t seq, int64_t d, int64_t heads, int64_t ff,
                              int64_t layers) {
    CharModel model{size_t(vocab), size_t(seq), size_t(d), size_t(heads), size_t(ff),
                    size_t(layers)};
    int64_t total = 0;
    for (const Tensor& p : model.parameters()) total += int64_t(p.size());
    return total;
}

}  // extern "C"
