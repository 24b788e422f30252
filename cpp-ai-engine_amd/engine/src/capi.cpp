// capi.cpp -- a C ABI over the engine for callers outside C++ (the tests and
// the benchmark). Every eng_* function below has the signature and meaning of
// the matching ref_* function that oracle/ref_shim.cpp builds over the
// reference engine, so the same inputs can be run through both and compared.
// Inputs and outputs are host buffers; the work runs on the GPU through the
// engine's Tensor API. Errors become a nonzero return plus eng_last_error().
//
// The trainer handles (eng_trainer_*) keep a model, its optimiser and one
// resident batch on the device, so that a training step can be timed without
// host transfers: eng_trainer_step() enqueues forward, backward and the Adam
// update and returns without waiting.

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "ehip.h"
#include "engine/autograd.hpp"
#include "engine/conv.hpp"
#include "engine/hip.hpp"
#include "engine/nn.hpp"
#include "engine/optim.hpp"
#include "engine/serialize.hpp"
#include "engine/tensor.hpp"
#include "engine/transformer.hpp"

namespace engine::data {
size_t idx_payload_bytes(const std::string& path, uint32_t magic, size_t max_items,
                         size_t* count);
}

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

void load_params(const std::vector<Tensor>& params, const float* flat) {
    size_t off = 0;
    for (Tensor p : params) {
        float* dst = p.data();
        std::memcpy(dst, flat + off, p.size() * sizeof(float));
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

std::unique_ptr<nn::Sequential> cnn_model(size_t in_c, size_t c1, size_t c2, size_t hw,
                                          size_t classes) {
    const size_t flat = c2 * (hw / 4) * (hw / 4);
    return std::make_unique<nn::Sequential>(
        nn::make<nn::Conv2d>(in_c, c1, nn::Window2d(3, 3, 1, 1)), nn::make<nn::ReLU>(),
        nn::make<nn::MaxPool2d>(2, 2), nn::make<nn::Conv2d>(c1, c2, nn::Window2d(3, 3, 1, 1)),
        nn::make<nn::ReLU>(), nn::make<nn::MaxPool2d>(2, 2), nn::make<nn::Flatten>(),
        nn::make<nn::Linear>(flat, classes));
}

// Token embedding plus the sinusoidal encoding, pre-LN blocks, a linear head
// (the character model of the reference's examples/charlm_demo.cpp:57-87).
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
    engine::NamedTensors named_parameters() {
        engine::NamedTensors out = embedding.named_parameters("embedding.");
        for (size_t i = 0; i < blocks.size(); ++i)
            for (auto& np : blocks[i].named_parameters("block" + std::to_string(i) + "."))
                out.push_back(np);
        for (auto& np : head.named_parameters("head.")) out.push_back(np);
        return out;
    }
    std::vector<Tensor> parameters() {
        std::vector<Tensor> out = embedding.parameters();
        for (nn::TransformerBlock& b : blocks)
            for (const Tensor& p : b.parameters()) out.push_back(p);
        for (const Tensor& p : head.parameters()) out.push_back(p);
        return out;
    }
};

// A model, its Adam state and one resident batch.
struct Trainer {
    std::unique_ptr<nn::Sequential> cnn;
    std::unique_ptr<CharModel> lm;
    std::unique_ptr<optim::Adam> opt;
    Tensor x;     // images (cnn) or ids (lm)
    Tensor mask;  // lm only
    std::vector<size_t> labels;
    nn::Labels device_labels;  // the batch's labels, resident like x
    size_t rows = 0, classes = 0;
    Tensor loss;

    // Graph mode: the second step is captured into a hip::Graph (the first
    // runs eagerly and creates the optimiser state), later steps refresh
    // Adam's device scalars and replay it with one launch.
    bool use_graph = false;
    size_t steps_run = 0;
    engine::hip::Graph graph;
    std::vector<Tensor> graph_params;

    std::vector<Tensor> parameters() { return cnn ? cnn->parameters() : lm->parameters(); }

    void eager_step() {
        opt->zero_grad();
        Tensor logits = cnn ? (*cnn)(x) : lm->forward(x, mask).reshape({rows, classes});
        loss = nn::cross_entropy_loss(logits, device_labels);
        loss.backward();
        opt->step();
    }

    void step() {
        if (!use_graph || steps_run == 0) {
            eager_step();
            ++steps_run;
            return;
        }
        if (!graph.ready()) {
            opt->set_device_scalars(true);
            try {
                graph.capture([&] { eager_step(); });
            } catch (...) {
                opt->set_device_scalars(false);
                use_graph = false;
                throw;
            }
            graph_params = parameters();
        }
        opt->prepare_replay();
        graph.launch();
        // The replay rewrote these on the device behind the host's back.
        for (Tensor& p : graph_params) {
            (void)p.storage().device_write();
            if (p.has_grad()) (void)p.get_impl()->grad->storage.device_write();
        }
        (void)loss.storage().device_write();
        ++steps_run;
    }

    void drop_graph() {
        graph.reset();
        graph_params.clear();
        opt->set_device_scalars(false);
    }

    void set_graph(bool on) {
        if (!on && graph.ready()) drop_graph();
        use_graph = on;
    }
};

}  // namespace

extern "C" {

const char* eng_last_error() { return g_error.c_str(); }

int eng_available() { return engine::hip::available() ? 1 : 0; }

// engine::hip's control API (the reference's cuda.hpp:28-29, 67-69, 100-125).
int eng_enabled() { return engine::hip::enabled() ? 1 : 0; }
void eng_set_enabled(int on) { engine::hip::set_enabled(on != 0); }
void eng_versions(int* compiled, int* runtime, int* driver) {
    *compiled = engine::hip::compiled_version();
    *runtime = engine::hip::runtime_version();
    *driver = engine::hip::driver_version();
}
// Writes up to `capacity` lines "name|threads|registers|lds|blocks|occupancy|limiter"
// into out (NUL-separated lines in one buffer of `bytes`); returns the kernel count.
int eng_kernel_occupancy(char* out, int64_t bytes) {
    const auto all = engine::hip::kernel_occupancy();
    std::string text;
    for (const auto& k : all)
        text += k.name + "|" + std::to_string(k.block_threads) + "|" +
                std::to_string(k.registers) + "|" + std::to_string(k.shared_bytes) + "|" +
                std::to_string(k.blocks_per_cu) + "|" + std::to_string(k.occupancy) + "|" +
                k.limiter + "\n";
    if (out != nullptr && bytes > 0) {
        const size_t n = std::min(text.size(), size_t(bytes - 1));
        std::memcpy(out, text.data(), n);
        out[n] = '\0';
    }
    return int(all.size());
}

// Host-only: reads an IDX file's header and payload (engine/src/data.cpp)
// and returns the items kept and the payload size, or the reader's error.
int eng_idx_probe(const char* path, uint32_t magic, int64_t max_items, int64_t* count,
                  int64_t* bytes) {
    return guarded([&] {
        size_t n = 0;
        *bytes = int64_t(engine::data::idx_payload_bytes(path, magic, size_t(max_items), &n));
        *count = int64_t(n);
    });
}

int eng_synchronize() {
    return guarded([&] { engine::hip::synchronize(); });
}

int eng_matmul(const float* a, const float* b, float* c, int64_t batch, int64_t m, int64_t k,
               int64_t n, int a_batched, int b_batched) {
    return guarded([&] {
        std::vector<size_t> sa = {size_t(m), size_t(k)}, sb = {size_t(k), size_t(n)};
        if (a_batched) sa.insert(sa.begin(), size_t(batch));
        if (b_batched) sb.insert(sb.begin(), size_t(batch));
        put(make(sa, a, false).matmul(make(sb, b, false)), c);
    });
}

int eng_matmul_fwd_bwd(const float* a, const float* b, const float* dc, int64_t m, int64_t k,
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

int eng_binary_fwd_bwd(int op, const float* a, const int64_t* a_shape, int a_nd, const float* b,
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

int eng_permute_fwd_bwd(const float* x, const int64_t* shape, int nd, const int64_t* order,
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

int eng_sum_axis_fwd_bwd(const float* x, const int64_t* shape, int nd, int axis, const float* dy,
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

int eng_unary_fwd_bwd(int which, const float* x, int64_t rows, int64_t cols, const float* dy,
                      float* y, float* dx) {
    return guarded([&] {
        Tensor X = make({size_t(rows), size_t(cols)}, x, true);
        Tensor Y = which == 0 ? X.relu() : X.softmax();
        Y.backward(make({size_t(rows), size_t(cols)}, dy, false));
        put(Y, y);
        put(X.grad(), dx);
    });
}

int eng_sum(const float* x, int64_t n, float* out) {
    return guarded([&] { put(make({size_t(n)}, x, false).sum(), out); });
}

int eng_im2col(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, int64_t kh, int64_t kw,
               int64_t stride, int64_t pad, float* cols) {
    return guarded([&] {
        Tensor X = make({size_t(N), size_t(C), size_t(H), size_t(W)}, x, false);
        put(nn::im2col(X, nn::Window2d(size_t(kh), size_t(kw), size_t(stride), size_t(pad))), cols);
    });
}

int eng_col2im(const float* cols, int64_t N, int64_t C, int64_t H, int64_t W, int64_t kh,
               int64_t kw, int64_t stride, int64_t pad, float* x) {
    return guarded([&] {
        nn::Window2d win{size_t(kh), size_t(kw), size_t(stride), size_t(pad)};
        const size_t rows = size_t(N) * win.out_h(size_t(H)) * win.out_w(size_t(W));
        Tensor Cc = make({rows, size_t(C * kh * kw)}, cols, false);
        put(nn::col2im(Cc, {size_t(N), size_t(C), size_t(H), size_t(W)}, win), x);
    });
}

int eng_conv2d_fwd_bwd(const float* x, const float* w, const float* bias, int64_t N, int64_t C,
                       int64_t H, int64_t W, int64_t out_c, int64_t k, int64_t stride,
                       int64_t pad, const float* dy, float* y, float* dx, float* dw, float* db) {
    return guarded([&] {
        nn::Conv2d conv{size_t(C), size_t(out_c), nn::Window2d{size_t(k), size_t(k), size_t(stride), size_t(pad)}};
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

int eng_maxpool_fwd_bwd(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, int64_t k,
                        int64_t stride, const float* dy, float* y, float* dx) {
    return guarded([&] {
        nn::MaxPool2d pool{size_t(k), size_t(stride)};
        Tensor X = make({size_t(N), size_t(C), size_t(H), size_t(W)}, x, true);
        Tensor Y = pool(X);
        Y.backward(make(Y.shape(), dy, false));
        put(Y, y);
        put(X.grad(), dx);
    });
}

int eng_layernorm_fwd_bwd(const float* x, const float* gamma, const float* beta, int64_t rows,
                          int64_t d, const float* dy, float* y, float* dx, float* dgamma,
                          float* dbeta) {
    return guarded([&] {
        nn::LayerNorm ln{size_t(d)};
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

int eng_cross_entropy(const float* logits, const int64_t* targets, int64_t n, int64_t c,
                      float* loss, float* dlogits) {
    return guarded([&] {
        Tensor L = make({size_t(n), size_t(c)}, logits, true);
        Tensor loss_t = nn::cross_entropy_loss(L, labels_of(targets, n));
        loss_t.backward();
        put(loss_t, loss);
        put(L.grad(), dlogits);
    });
}

int eng_embedding_fwd_bwd(const float* table, int64_t vocab, int64_t d, const float* ids,
                          int64_t batch, int64_t seq, const float* dy, float* y, float* dtable) {
    return guarded([&] {
        nn::Embedding emb{size_t(vocab), size_t(d)};
        std::memcpy(emb.weight().data(), table, size_t(vocab * d) * sizeof(float));
        Tensor Y = emb(make({size_t(batch), size_t(seq)}, ids, false));
        Y.backward(make(Y.shape(), dy, false));
        put(Y, y);
        put(emb.weight().grad(), dtable);
    });
}

int eng_adam_steps(float* p, const float* grads, int64_t n, int64_t steps, float lr, float b1,
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

// nn::Dropout(p) after manual_seed(seed), forward and backward on n values
// (train mode, or eval mode when `eval` is nonzero).
int eng_dropout_fwd_bwd(const float* x, int64_t n, float p, uint64_t seed, int eval,
                        const float* dy, float* y, float* dx) {
    return guarded([&] {
        engine::manual_seed(seed);
        nn::Dropout drop(p);
        drop.train(eval == 0);
        Tensor X = make({size_t(n)}, x, true);
        Tensor Y = drop(X);
        Y.backward(make({size_t(n)}, dy, false));
        put(Y, y);
        put(X.grad(), dx);
    });
}

// clip_grad_norm over `count` parameters: parameter i has |sizes[i]| elements
// and, when sizes[i] > 0, the gradient taken from `grads` (concatenated); a
// negative size is a parameter without a gradient. The clipped gradients are
// written back over `grads` and the norm to *norm.
int eng_clip_grad_norm(float* grads, const int64_t* sizes, int count, float max_norm,
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

int eng_attention_fwd_bwd(const float* q, const float* k, const float* v, const float* mask,
                          int64_t b, int64_t h, int64_t s, int64_t dk, const float* dy, float* y,
                          float* weights, float* dq, float* dkk, float* dv) {
    return guarded([&] {
        std::vector<size_t> sh = {size_t(b), size_t(h), size_t(s), size_t(dk)};
        Tensor Q = make(sh, q, true), K = make(sh, k, true), V = make(sh, v, true);
        Tensor M;
        if (mask != nullptr) M = make({size_t(s), size_t(s)}, mask, false);
        Tensor Wt;
        Tensor Y = nn::scaled_dot_product_attention(Q, K, V, mask ? &M : nullptr, &Wt);
        Y.backward(make(sh, dy, false));
        put(Y, y);
        put(Wt, weights);
        put(Q.grad(), dq);
        put(K.grad(), dkk);
        put(V.grad(), dv);
    });
}

int eng_block_fwd_bwd(const float* x, int64_t b, int64_t s, int64_t d, int64_t heads, int64_t ff,
                      int causal, const float* params, const float* dy, float* y, float* dx,
                      float* dparams) {
    return guarded([&] {
        nn::TransformerBlock block{size_t(d), size_t(heads), size_t(ff)};
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

// nn::Linear forward and backward with given weight (in, out) and bias (1, out);
// x is (rows, in) or (b, s, in) flattened to rows.
// nn::set_fused_nodes: 1 builds the fused nodes (the default), 0 the
// reference's node-by-node graph. Returns the previous setting.
int eng_set_fused_nodes(int on) {
    const bool was = nn::fused_nodes();
    nn::set_fused_nodes(on != 0);
    return was ? 1 : 0;
}

int eng_set_short_attention(int on) {
    const bool was = nn::short_attention();
    nn::set_short_attention(on != 0);
    return was ? 1 : 0;
}

int eng_set_deferred_weight_grads(int on) {
    const bool was = nn::deferred_weight_grads();
    nn::set_deferred_weight_grads(on != 0);
    return was ? 1 : 0;
}

int eng_set_conv_implicit_gemm(int on) {
    const bool was = nn::conv_implicit_gemm();
    nn::set_conv_implicit_gemm(on != 0);
    return was ? 1 : 0;
}

int eng_set_fused_bias_grad(int on) {
    const bool was = nn::fused_bias_grad();
    nn::set_fused_bias_grad(on != 0);
    return was ? 1 : 0;
}

int eng_linear_fwd_bwd(const float* x, int64_t rows, int64_t in, int64_t out, const float* w,
                       const float* bias, const float* dy, float* y, float* dx, float* dw,
                       float* db) {
    return guarded([&] {
        nn::Linear lin{size_t(in), size_t(out)};
        std::memcpy(lin.weight().data(), w, size_t(in * out) * sizeof(float));
        std::memcpy(lin.bias().data(), bias, size_t(out) * sizeof(float));
        Tensor X = make({size_t(rows), size_t(in)}, x, true);
        Tensor Y = lin(X);
        Y.backward(make(Y.shape(), dy, false));
        put(Y, y);
        put(X.grad(), dx);
        put(lin.weight().grad(), dw);
        put(lin.bias().grad(), db);
    });
}

// nn::MultiHeadAttention forward and backward; params in parameters() order
// (wq, bq, wk, bk, wv, bv, wo, bo). mask (s, s) may be NULL; fuse selects the
// in-place attention node or the composed path; weights (b, heads, s, s) may
// be NULL.
int eng_mha_fwd_bwd(const float* x, int64_t b, int64_t s, int64_t d, int64_t heads,
                    const float* params, const float* dy, float* y, float* dx, float* dparams,
                    const float* mask, int fuse, float* weights) {
    return guarded([&] {
        struct Restore {
            bool was = nn::fused_nodes();
            ~Restore() { nn::set_fused_nodes(was); }
        } restore;
        nn::set_fused_nodes(fuse != 0);
        nn::MultiHeadAttention mha{size_t(d), size_t(heads)};
        mha.keep_attention(weights != nullptr);
        load_params(mha.parameters(), params);
        Tensor X = make({size_t(b), size_t(s), size_t(d)}, x, true);
        Tensor M;
        if (mask != nullptr) M = make({size_t(s), size_t(s)}, mask, false);
        Tensor Y = mha.forward(X, mask ? &M : nullptr);
        Y.backward(make(Y.shape(), dy, false));
        if (weights != nullptr) put(mha.last_attention(), weights);
        put(Y, y);
        put(X.grad(), dx);
        size_t off = 0;
        for (const Tensor& p : mha.parameters()) {
            put(p.grad(), dparams + off);
            off += p.size();
        }
    });
}

// Fused MultiHeadAttention forward + backward under a causal mask: tagged != 0
// passes nn::causal_mask(s) (whose products may skip the masked blocks),
// tagged == 0 a copy of the same values made as a plain tensor (every product
// computed in full), so that tests can compare the two.
int eng_mha_causal_fwd_bwd(const float* x, int64_t b, int64_t s, int64_t d, int64_t heads,
                           const float* params, const float* dy, float* y, float* dx,
                           float* dparams, float* weights, int tagged) {
    return guarded([&] {
        nn::MultiHeadAttention mha{size_t(d), size_t(heads)};
        mha.keep_attention(weights != nullptr);
        load_params(mha.parameters(), params);
        Tensor X = make({size_t(b), size_t(s), size_t(d)}, x, true);
        const Tensor causal = nn::causal_mask(size_t(s));
        const Tensor M = tagged ? causal : make({size_t(s), size_t(s)}, causal.data(), false);
        Tensor Y = mha.forward(X, &M);
        Y.backward(make(Y.shape(), dy, false));
        if (weights != nullptr) put(mha.last_attention(), weights);
        put(Y, y);
        put(X.grad(), dx);
        size_t off = 0;
        for (const Tensor& p : mha.parameters()) {
            put(p.grad(), dparams + off);
            off += p.size();
        }
    });
}

// Adam on mse_loss(w, target) for `steps` steps; traj receives w after each
// step (the optimiser replays of the reference's tests/test_reference.cpp:387-422).
int eng_mse_adam(const float* w0, const float* target, int64_t n, int64_t steps, float lr,
                 float* traj) {
    return guarded([&] {
        Tensor W = make({size_t(n)}, w0, true);
        const Tensor T = make({size_t(n)}, target, false);
        optim::Adam opt({W}, lr);
        for (int64_t st = 0; st < steps; ++st) {
            opt.zero_grad();
            Tensor loss = nn::mse_loss(W, T);
            loss.backward();
            opt.step();
            put(W, traj + st * n);
        }
    });
}

int64_t eng_block_num_params(int64_t d, int64_t heads, int64_t ff) {
    return (4 * d) + 4 * (d * d + d) + (d * ff + ff) + (ff * d + d) + 0 * heads;
}

// One forward and backward of the cfg2 CNN; the gradients are read through
// Tensor::grad() (which runs any queued weight sums first), in parameter order.
int eng_cnn_grads(const float* x, const int64_t* labels, int64_t batch, int64_t in_c, int64_t c1,
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
        for (Tensor& p : model->parameters()) {
            put(p.grad(), grads_out + off);
            off += p.size();
        }
    });
}

// Forward and backward of a CNN that is then destroyed without anything
// reading its gradients: the fused convolution blocks' weight sums stay queued
// past the model's lifetime, to be run by whatever engine work comes next.
int eng_cnn_backward_orphan(const float* x, const int64_t* labels, int64_t batch, int64_t in_c,
                            int64_t c1, int64_t c2, int64_t hw, int64_t classes,
                            const float* params) {
    return guarded([&] {
        auto model = cnn_model(size_t(in_c), size_t(c1), size_t(c2), size_t(hw), size_t(classes));
        load_params(model->parameters(), params);
        Tensor X = make({size_t(batch), size_t(in_c), size_t(hw), size_t(hw)}, x, false);
        Tensor loss = nn::cross_entropy_loss((*model)(X), labels_of(labels, batch));
        loss.backward();
    });
}

int eng_cnn_train(const float* x, const int64_t* labels, int64_t batch, int64_t in_c, int64_t c1,
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

// `steps` Adam steps of the character model on one batch: the loss of every
// step, the final parameters and, when grads0 is not NULL, the first step's
// gradients (after backward, before the update; parameter order).
int eng_charlm_train_grads(const float* ids, const int64_t* targets, int64_t batch, int64_t seq,
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
                for (Tensor& p : model.parameters()) {
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

// The character model's gradients summed over `passes` forward and backward
// passes of one batch (gradient accumulation: the second pass adds into
// gradients the first left, some of them still queued).
int eng_charlm_accumulated_grads(const float* ids, const int64_t* targets, int64_t batch,
                                 int64_t seq, int64_t vocab, int64_t d, int64_t heads, int64_t ff,
                                 int64_t layers, const float* params, int64_t passes,
                                 float* grads_out) {
    return guarded([&] {
        CharModel model{size_t(vocab), size_t(seq), size_t(d), size_t(heads), size_t(ff),
                        size_t(layers)};
        load_params(model.parameters(), params);
        const Tensor mask = nn::causal_mask(size_t(seq));
        Tensor X = make({size_t(batch), size_t(seq)}, ids, false);
        const std::vector<size_t> y = labels_of(targets, batch * seq);
        for (int64_t p = 0; p < passes; ++p) {
            Tensor logits = model.forward(X, mask).reshape({size_t(batch * seq), size_t(vocab)});
            nn::cross_entropy_loss(logits, y).backward();
        }
        size_t off = 0;
        for (Tensor& p : model.parameters()) {
            put(p.grad(), grads_out + off);
            off += p.size();
        }
    });
}

// Forward and backward of a character model that is then destroyed without
// anything reading its gradients: the queued weight-gradient products (and
// LayerNorm sums) outlive the model, to be run by the next engine work.
int eng_charlm_backward_orphan(const float* ids, const int64_t* targets, int64_t batch,
                               int64_t seq, int64_t vocab, int64_t d, int64_t heads, int64_t ff,
                               int64_t layers, const float* params) {
    return guarded([&] {
        CharModel model{size_t(vocab), size_t(seq), size_t(d), size_t(heads), size_t(ff),
                        size_t(layers)};
        load_params(model.parameters(), params);
        const Tensor mask = nn::causal_mask(size_t(seq));
        Tensor X = make({size_t(batch), size_t(seq)}, ids, false);
        Tensor logits = model.forward(X, mask).reshape({size_t(batch * seq), size_t(vocab)});
        nn::cross_entropy_loss(logits, labels_of(targets, batch * seq)).backward();
    });
}

int eng_charlm_train(const float* ids, const int64_t* targets, int64_t batch, int64_t seq,
                     int64_t vocab, int64_t d, int64_t heads, int64_t ff, int64_t layers,
                     const float* params, int64_t steps, float lr, float* losses,
                     float* params_out) {
    return eng_charlm_train_grads(ids, targets, batch, seq, vocab, d, heads, ff, layers, params,
                                  steps, lr, losses, nullptr, params_out);
}

int64_t eng_charlm_num_params(int64_t vocab, int64_t seq, int64_t d, int64_t heads, int64_t ff,
                              int64_t layers) {
    return vocab * d + layers * eng_block_num_params(d, heads, ff) + d * vocab + vocab + 0 * seq;
}

// ------------------------------------------------------------------ timing

// Enqueues `reps` back-to-back ehip_gemm_f32 calls on `stream` (device pointers,
// the arguments of ehip_gemm_f32), so that a caller can time one kernel with
// events around the whole batch without host launch overhead between calls.
int eng_repeat_gemm(int trans_a, int trans_b, int64_t batch, int64_t m, int64_t n, int64_t k,
                    const float* a, int64_t lda, int64_t stride_a, const float* b, int64_t ldb,
                    int64_t stride_b, float beta, float* c, int64_t ldc, int64_t stride_c,
                    void* stream, int reps) {
    return guarded([&] {
        for (int r = 0; r < reps; ++r)
            engine::hip::check(ehip_gemm_f32(trans_a, trans_b, batch, m, n, k, a, lda, stride_a, b,
                                             ldb, stride_b, beta, c, ldc, stride_c, stream),
                               "gemm");
    });
}

// Enqueues `reps` back-to-back calls of one bandwidth-bound entry point on
// `stream`, so that events around the batch time the kernels without host
// launch gaps. p holds the device pointers and n the extents, in the entry
// point's argument order:
//   0 ehip_layernorm_f32          p: x gamma beta out xhat inv    n: rows cols   f: eps
//   1 ehip_layernorm_backward_f32 p: dy xhat gamma inv dx dg db   n: rows cols
//   2 ehip_sum_axis_f32           p: x out                        n: outer axis inner
//   3 ehip_softmax_f32            p: x y                          n: rows cols
//   4 ehip_softmax_backward_f32   p: y g dx                       n: rows cols
//   5 ehip_maxpool_f32            p: x y argmax                   w: the window
//   6 ehip_maxpool_backward_f32   p: argmax g dx                  w: the window
//   7 ehip_layernorm_backward_partials_f32 p: dy xhat gamma inv dx partials
//                                            n: rows cols groups
int eng_repeat_bandwidth(int op, void* const* p, const int64_t* n, float f, const ehip_window_t* w,
                         void* stream, int reps) {
    return guarded([&] {
        const auto F = [&](int i) { return static_cast<float*>(p[i]); };
        for (int r = 0; r < reps; ++r) {
            int rc = EHIP_EINVAL;
            switch (op) {
                case 0: rc = ehip_layernorm_f32(F(0), F(1), F(2), F(3), F(4), F(5), n[0], n[1], f,
                                                stream); break;
                case 1: rc = ehip_layernorm_backward_f32(F(0), F(1), F(2), F(3), F(4), F(5), F(6),
                                                         n[0], n[1], stream); break;
                case 2: rc = ehip_sum_axis_f32(F(0), F(1), n[0], n[1], n[2], stream); break;
                case 3: rc = ehip_softmax_f32(F(0), F(1), n[0], n[1], stream); break;
                case 4: rc = ehip_softmax_backward_f32(F(0), F(1), F(2), n[0], n[1], stream); break;
                case 5: rc = ehip_maxpool_f32(F(0), F(1), static_cast<int32_t*>(p[2]), w, stream);
                        break;
                case 6: rc = ehip_maxpool_backward_f32(static_cast<const int32_t*>(p[0]), F(1),
                                                       F(2), w, stream); break;
                case 7:
                case 8: rc = ehip_layernorm_backward_partials_f32(F(0), F(1), F(2), F(3), F(4),
                                                                  F(5), n[2], n[0], n[1],
                                                                  op == 8 ? 1 : 0, stream);
                        break;
                default: throw std::invalid_argument("repeat_bandwidth: unknown op");
            }
            engine::hip::check(rc, "repeat_bandwidth");
        }
    });
}

// Enqueues `reps` back-to-back ehip_matmul_backward_f32 calls on `stream`
// (device pointers, contiguous 2-D operands): the backward of C = A B.
int eng_repeat_matmul_backward(int64_t m, int64_t k, int64_t n, const float* a, const float* b,
                               const float* dc, float* da, float* db, void* stream, int reps) {
    return guarded([&] {
        for (int r = 0; r < reps; ++r)
            engine::hip::check(ehip_matmul_backward_f32(m, k, n, a, k, b, n, dc, n, da, k, 0.0f, db,
                                                        n, 0.0f, stream),
                               "matmul backward");
    });
}

// Enqueues `reps` back-to-back ehip_conv2d_relu_maxpool_backward_f32 calls on
// `stream` (device pointers; the windows are the entry point's), for timing
// the fused block's backward kernels with events around the batch.
int eng_repeat_conv_relu_pool_backward(const float* x, const float* weight, const float* grad_out,
                                       const float* out, const int32_t* argmax, float* dx,
                                       float* dweight, float* dbias, const ehip_window_t* conv,
                                       int64_t out_channels, const ehip_window_t* pool,
                                       void* stream, int reps) {
    return guarded([&] {
        for (int r = 0; r < reps; ++r)
            engine::hip::check(
                ehip_conv2d_relu_maxpool_backward_f32(x, weight, grad_out, out, argmax, dx,
                                                      dweight, dbias, conv, out_channels, pool,
                                                      stream),
                "conv2d_relu_maxpool backward");
    });
}

// ------------------------------------------------------------------ trainers

void* eng_trainer_cnn(const float* x, const int64_t* labels, int64_t batch, int64_t in_c,
                      int64_t c1, int64_t c2, int64_t hw, int64_t classes, const float* params,
                      float lr) {
    Trainer* t = nullptr;
    const int rc = guarded([&] {
        auto tr = std::make_unique<Trainer>();
        tr->cnn = cnn_model(size_t(in_c), size_t(c1), size_t(c2), size_t(hw), size_t(classes));
        if (params) load_params(tr->cnn->parameters(), params);
        tr->opt = std::make_unique<optim::Adam>(tr->cnn->parameters(), lr);
        tr->x = make({size_t(batch), size_t(in_c), size_t(hw), size_t(hw)}, x, false);
        (void)tr->x.storage().device();
        tr->labels = labels_of(labels, batch);
        tr->device_labels = nn::Labels(tr->labels);
        tr->rows = size_t(batch);
        tr->classes = size_t(classes);
        t = tr.release();
    });
    return rc == 0 ? t : nullptr;
}

void* eng_trainer_charlm(const float* ids, const int64_t* targets, int64_t batch, int64_t seq,
                         int64_t vocab, int64_t d, int64_t heads, int64_t ff, int64_t layers,
                         const float* params, float lr) {
    Trainer* t = nullptr;
    const int rc = guarded([&] {
        auto tr = std::make_unique<Trainer>();
        tr->lm = std::make_unique<CharModel>(size_t(vocab), size_t(seq), size_t(d), size_t(heads),
                                             size_t(ff), size_t(layers));
        if (params) load_params(tr->lm->parameters(), params);
        tr->opt = std::make_unique<optim::Adam>(tr->lm->parameters(), lr);
        tr->x = make({size_t(batch), size_t(seq)}, ids, false);
        tr->mask = nn::causal_mask(size_t(seq));
        (void)tr->mask.storage().device();
        (void)tr->lm->positions.storage().device();
        tr->labels = labels_of(targets, batch * seq);
        tr->device_labels = nn::Labels(tr->labels);
        tr->rows = size_t(batch * seq);
        tr->classes = size_t(vocab);
        t = tr.release();
    });
    return rc == 0 ? t : nullptr;
}

// Checkpoints of a trainer: the model's parameters in the reference's weight
// format at params_path, and (when opt_path is not NULL) the Adam state.
int eng_trainer_save(void* h, const char* params_path, const char* opt_path) {
    return guarded([&] {
        Trainer* t = static_cast<Trainer*>(h);
        if (t->cnn)
            engine::save_parameters(*t->cnn, params_path);
        else
            engine::save_parameters(t->lm->named_parameters(), params_path);
        if (opt_path) engine::save_optimizer(*t->opt, opt_path);
    });
}

int eng_trainer_load(void* h, const char* params_path, const char* opt_path) {
    return guarded([&] {
        Trainer* t = static_cast<Trainer*>(h);
        // New values may come in new buffers: a captured step is taken again.
        if (t->graph.ready()) t->drop_graph();
        if (t->cnn) {
            engine::load_parameters(*t->cnn, params_path, true);
        } else {
            engine::NamedTensors named = t->lm->named_parameters();
            engine::load_parameters(named, params_path, true);
        }
        if (opt_path) engine::load_optimizer(*t->opt, opt_path);
    });
}

int eng_trainer_step(void* h) {
    return guarded([&] { static_cast<Trainer*>(h)->step(); });
}

// Graph mode on (1) or off (0): see Trainer::step. Off drops the captured step.
int eng_trainer_set_graph(void* h, int on) {
    return guarded([&] { static_cast<Trainer*>(h)->set_graph(on != 0); });
}

int eng_trainer_loss(void* h, float* loss) {
    return guarded([&] { *loss = static_cast<Trainer*>(h)->loss.data()[0]; });
}

int64_t eng_trainer_num_params(void* h) {
    int64_t n = 0;
    for (const Tensor& p : static_cast<Trainer*>(h)->parameters()) n += int64_t(p.size());
    return n;
}

int eng_trainer_params(void* h, float* out) {
    return guarded([&] { store_params(static_cast<Trainer*>(h)->parameters(), out); });
}

void eng_trainer_destroy(void* h) { delete static_cast<Trainer*>(h); }

}  // extern "C"
