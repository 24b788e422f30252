// transformer.cpp -- LayerNorm, Embedding, the constant tensors, attention and
// the pre-LN block (the reference's src/transformer.cpp).
#include "engine/transformer.hpp"

#include <cmath>
#include <stdexcept>

#include "detail.hpp"

namespace engine {
namespace nn {

using namespace detail;

LayerNorm::LayerNorm(size_t normalized_size, float eps)
    : normalized_size_(normalized_size), eps_(eps) {
    if (normalized_size == 0) throw std::invalid_argument("LayerNorm requires a size greater than zero.");
    if (eps <= 0.0f) throw std::invalid_argument("LayerNorm requires a positive epsilon.");
    autograd::NoGradGuard no_grad;
    gamma_ = Tensor({normalized_size}, 1.0f, true);
    beta_ = Tensor({normalized_size}, 0.0f, true);
}

// One fused node: the forward saves xhat and inv_std, the backward produces dx,
// dgamma and dbeta in two kernels (src/transformer.cpp:82-179).
Tensor LayerNorm::forward(const Tensor& input) {
    if (input.ndim() < 1 || input.shape().back() != normalized_size_)
        throw std::invalid_argument("LayerNorm of size " + std::to_string(normalized_size_) +
                                    " received an input " + input.shape_str() + ".");
    const size_t D = normalized_size_;
    const size_t rows = input.size() / D;
    Tensor out(input.shape(), 0.0f, false);
    Tensor xhat(input.shape(), 0.0f, false);
    Tensor inv_std({rows}, 0.0f, false);
    hip::check(ehip_layernorm_f32(dptr(input), dptr(gamma_), dptr(beta_), dout(out), dout(xhat),
                                  dout(inv_std), int64_t(rows), int64_t(D), eps_, nullptr),
               "layernorm");
    const bool req_g = autograd::grad_enabled() &&
                       (input.requires_grad() || gamma_.requires_grad() || beta_.requires_grad());
    if (!req_g) return out;
    out.set_requires_grad(true);
    out.get_impl()->parents = {input.get_impl(), gamma_.get_impl(), beta_.get_impl()};
    Tensor input_copy = input, gamma_copy = gamma_, beta_copy = beta_;
    out.get_impl()->backward_fn = [input_copy, gamma_copy, beta_copy, xhat, inv_std, rows,
                                   D](const Tensor& g) mutable {
        Tensor dgamma(gamma_copy.shape(), 0.0f, false);
        Tensor dbeta(beta_copy.shape(), 0.0f, false);
        Tensor dX(input_copy.shape(), 0.0f, false);
        hip::check(ehip_layernorm_backward_f32(dptr(g), dptr(xhat), dptr(gamma_copy),
                                               dptr(inv_std), dout(dX), dout(dgamma), dout(dbeta),
                                               int64_t(rows), int64_t(D), nullptr),
                   "layernorm backward");
        if (input_copy.requires_grad()) input_copy.add_grad(dX);
        if (gamma_copy.requires_grad()) gamma_copy.add_grad(dgamma);
        if (beta_copy.requires_grad()) beta_copy.add_grad(dbeta);
    };
    return out;
}

std::vector<Tensor> LayerNorm::parameters() { return {gamma_, beta_}; }

std::vector<std::pair<std::string, Tensor>> LayerNorm::named_parameters(const std::string& prefix) {
    return {{prefix + "layernorm.gamma", gamma_}, {prefix + "layernorm.beta", beta_}};
}

std::string LayerNorm::name() const { return "LayerNorm(" + std::to_string(normalized_size_) + ")"; }

Embedding::Embedding(size_t num_embeddings, size_t dim) : num_embeddings_(num_embeddings), dim_(dim) {
    if (num_embeddings == 0 || dim == 0)
        throw std::invalid_argument("Embedding requires a positive vocabulary and dimension.");
    autograd::NoGradGuard no_grad;
    weight_ = Tensor::randn({num_embeddings, dim}, 0.0f, 0.02f, true);
}

// ids arrive as floats (batch, seq) and are rounded with llround
// (src/transformer.cpp:206-231); the gather runs on the device.
Tensor Embedding::forward(const Tensor& ids) {
    if (ids.ndim() != 2)
        throw std::invalid_argument("Embedding expects indices (batch, sequence), received " +
                                    ids.shape_str() + ".");
    const size_t batch = ids.shape()[0], seq = ids.shape()[1];
    std::vector<size_t> indices;
    indices.reserve(ids.size());
    const float* v = ids.data();
    for (size_t i = 0; i < ids.size(); ++i) {
        const long long id = std::llround(v[i]);
        if (id < 0 || static_cast<size_t>(id) >= num_embeddings_)
            throw std::out_of_range("Embedding: token " + std::to_string(id) +
                                    " is outside a vocabulary of " +
                                    std::to_string(num_embeddings_) + ".");
        indices.push_back(static_cast<size_t>(id));
    }
    return weight_.select_rows(indices).reshape({batch, seq, dim_});
}

std::vector<Tensor> Embedding::parameters() { return {weight_}; }

std::vector<std::pair<std::string, Tensor>> Embedding::named_parameters(const std::string& prefix) {
    return {{prefix + "embedding.weight", weight_}};
}

std::string Embedding::name() const {
    return "Embedding(" + std::to_string(num_embeddings_) + " x " + std::to_string(dim_) + ")";
}

// Sinusoidal table, float std::pow/sin/cos on the host (src/transformer.cpp:249-267).
Tensor positional_encoding(size_t seq_len, size_t d_model) {
    std::vector<float> pe(seq_len * d_model);
    for (size_t pos = 0; pos < seq_len; ++pos)
        for (size_t i = 0; i < d_model; ++i) {
            const size_t pair = i / 2;
            const float exponent = 2.0f * static_cast<float>(pair) / static_cast<float>(d_model);
            const float angle = static_cast<float>(pos) / std::pow(10000.0f, exponent);
            pe[pos * d_model + i] = (i % 2 == 0) ? std::sin(angle) : std::cos(angle);
        }
    return Tensor({seq_len, d_model}, pe, false);
}

Tensor causal_mask(size_t seq_len, float masked_value) {
    std::vector<float> m(seq_len * seq_len, 0.0f);
    for (size_t i = 0; i < seq_len; ++i)
        for (size_t j = i + 1; j < seq_len; ++j) m[i * seq_len + j] = masked_value;
    return Tensor({seq_len, seq_len}, m, false);
}

// softmax(Q K^T / sqrt(d_k) + mask) V, composed as in src/transformer.cpp:279-304;
// Q K^T reads K in place (no materialised transpose).
Tensor scaled_dot_product_attention(const Tensor& query, const Tensor& key, const Tensor& value,
                                    const Tensor* mask, Tensor* attention_weights) {
    if (query.ndim() < 2 || key.ndim() < 2 || value.ndim() < 2)
        throw std::invalid_argument("Attention needs at least 2 dimensions (seq, d_k).");
    const size_t d_k = query.shape().back();
    if (key.shape().back() != d_k)
        throw std::invalid_argument("Query and key must share d_k: " + query.shape_str() + " and " +
                                    key.shape_str() + ".");
    const float scale = 1.0f / std::sqrt(static_cast<float>(d_k));
    Tensor scores = ops::matmul_nt(query, key) * scale;
    if (mask != nullptr) scores = scores + *mask;
    Tensor weights = scores.softmax();
    if (attention_weights != nullptr) *attention_weights = weights.detach();
    return weights.matmul(value);
}

MultiHeadAttention::MultiHeadAttention(size_t d_model, size_t num_heads)
    : d_model_(d_model),
      num_heads_(num_heads),
      head_dim_(num_heads == 0 ? 0 : d_model / num_heads),
      w_query_(d_model, d_model),
      w_key_(d_model, d_model),
      w_value_(d_model, d_model),
      w_out_(d_model, d_model) {
    if (num_heads == 0) throw std::invalid_argument("MultiHeadAttention requires at least one head.");
    if (d_model % num_heads != 0)
        throw std::invalid_argument("d_model (" + std::to_string(d_model) +
                                    ") must be divisible by num_heads (" +
                                    std::to_string(num_heads) + ").");
}

Tensor MultiHeadAttention::forward(const Tensor& input) { return forward(input, nullptr); }

Tensor MultiHeadAttention::forward(const Tensor& input, const Tensor* mask) {
    if (input.ndim() != 3 || input.shape()[2] != d_model_)
        throw std::invalid_argument("MultiHeadAttention expects (batch, seq, " +
                                    std::to_string(d_model_) + "), received " + input.shape_str() + ".");
    const size_t batch = input.shape()[0], seq = input.shape()[1];
    auto split_heads = [&](const Tensor& projected) {
        return projected.reshape({batch, seq, num_heads_, head_dim_}).permute({0, 2, 1, 3});
    };
    Tensor q = split_heads(w_query_(input));
    Tensor k = split_heads(w_key_(input));
    Tensor v = split_heads(w_value_(input));
    Tensor attended =
        scaled_dot_product_attention(q, k, v, mask, keep_attention_ ? &last_attention_ : nullptr);
    Tensor merged = attended.permute({0, 2, 1, 3}).reshape({batch, seq, d_model_});
    return w_out_(merged);
}

std::vector<Tensor> MultiHeadAttention::parameters() {
    std::vector<Tensor> params;
    for (Linear* layer : {&w_query_, &w_key_, &w_value_, &w_out_})
        for (const Tensor& p : layer->parameters()) params.push_back(p);
    return params;
}

std::vector<std::pair<std::string, Tensor>> MultiHeadAttention::named_parameters(
    const std::string& prefix) {
    std::vector<std::pair<std::string, Tensor>> out;
    const char* names[] = {"query.", "key.", "value.", "out."};
    Linear* layers[] = {&w_query_, &w_key_, &w_value_, &w_out_};
    for (int i = 0; i < 4; ++i)
        for (auto& np : layers[i]->named_parameters(prefix + "attn." + names[i])) out.push_back(np);
    return out;
}

std::string MultiHeadAttention::name() const {
    return "MultiHeadAttention(d_model=" + std::to_string(d_model_) + ", heads=" +
           std::to_string(num_heads_) + ", head_dim=" + std::to_string(d_model_ / num_heads_) +
           ")";
}

TransformerBlock::TransformerBlock(size_t d_model, size_t num_heads, size_t ff_hidden)
    : d_model_(d_model),
      ff_hidden_(ff_hidden),
      norm1_(d_model),
      norm2_(d_model),
      attention_(d_model, num_heads),
      ff1_(d_model, ff_hidden),
      ff2_(ff_hidden, d_model) {
    if (ff_hidden == 0) throw std::invalid_argument("TransformerBlock requires a positive hidden layer.");
}

Tensor TransformerBlock::forward(const Tensor& input) { return forward(input, nullptr); }

// Pre-LN: h = x + MHA(LN1(x)); out = h + FF2(ReLU(FF1(LN2(h)))) (src/transformer.cpp:409-414).
Tensor TransformerBlock::forward(const Tensor& input, const Tensor* mask) {
    Tensor h = input + attention_.forward(norm1_(input), mask);
    return h + ff2_(ff1_(norm2_(h)).relu());
}

std::vector<Tensor> TransformerBlock::parameters() {
    std::vector<Tensor> params;
    for (Module* layer : {static_cast<Module*>(&norm1_), static_cast<Module*>(&norm2_),
                          static_cast<Module*>(&attention_), static_cast<Module*>(&ff1_),
                          static_cast<Module*>(&ff2_)})
        for (const Tensor& p : layer->parameters()) params.push_back(p);
    return params;
}

std::vector<std::pair<std::string, Tensor>> TransformerBlock::named_parameters(
    const std::string& prefix) {
    std::vector<std::pair<std::string, Tensor>> out;
    for (auto& np : norm1_.named_parameters(prefix + "norm1.")) out.push_back(np);
    for (auto& np : norm2_.named_parameters(prefix + "norm2.")) out.push_back(np);
    for (auto& np : attention_.named_parameters(prefix)) out.push_back(np);
    for (auto& np : ff1_.named_parameters(prefix + "ff1.")) out.push_back(np);
    for (auto& np : ff2_.named_parameters(prefix + "ff2.")) out.push_back(np);
    return out;
}

void TransformerBlock::train(bool mode) { Module::train(mode); }

std::string TransformerBlock::name() const {
    return "TransformerBlock(d_model=" + std::to_string(d_model_) + ", ff=" +
           std::to_string(ff_hidden_) + ")";
}

}  // namespace nn
}  // namespace engine
