// transformer.hpp -- LayerNorm, Embedding, attention and the pre-LN block,
// mirroring the reference's include/engine/transformer.hpp.
#ifndef ENGINE_TRANSFORMER_HPP
#define ENGINE_TRANSFORMER_HPP

#include <cstdint>
#include <memory>
#include <utility>
#include <vector>

#include "engine/nn.hpp"

namespace engine {
namespace detail {
struct RowGather;
}  // namespace detail

namespace nn {

class LayerNorm : public Module {
public:
    explicit LayerNorm(size_t normalized_size, float eps = 1e-5f);
    Tensor forward(const Tensor& input) override;
    std::vector<Tensor> parameters() override;
    std::vector<std::pair<std::string, Tensor>> named_parameters(
        const std::string& prefix = "") override;
    std::string name() const override;
    Tensor& gamma() { return gamma_; }
    Tensor& beta() { return beta_; }

private:
    size_t normalized_size_;
    float eps_;
    Tensor gamma_;
    Tensor beta_;
};

class Embedding : public Module {
public:
    Embedding(size_t num_embeddings, size_t dim);
    Tensor forward(const Tensor& ids) override;
    std::vector<Tensor> parameters() override;
    std::vector<std::pair<std::string, Tensor>> named_parameters(
        const std::string& prefix = "") override;
    std::string name() const override;
    Tensor& weight() { return weight_; }
    size_t dim() const noexcept { return dim_; }

private:
    size_t num_embeddings_;
    size_t dim_;
    Tensor weight_;
    // The device index of the last ids tensor seen, reused while the same
    // buffer comes back unmodified (a resident batch uploads it once).
    Storage ids_seen_;
    uint64_t ids_version_ = 0;
    std::shared_ptr<const detail::RowGather> gather_;
};

Tensor positional_encoding(size_t seq_len, size_t d_model);
Tensor causal_mask(size_t seq_len, float masked_value = -1e9f);
Tensor scaled_dot_product_attention(const Tensor& query, const Tensor& key, const Tensor& value,
                                    const Tensor* mask = nullptr,
                                    Tensor* attention_weights = nullptr);

// The attention of MultiHeadAttention on projected activations, heads read
// and written in place: query, key and value are (batch, seq, heads * dim)
// and the result is the merged (batch, seq, heads * dim) tensor. Equal bit
// for bit to splitting the heads, scaled_dot_product_attention and merging
// them back, with one autograd node, no permuted copies and the scale and
// mask applied inside the score product. `mask` must suffix-broadcast over
// (batch, heads, seq, seq) and take no gradient (attention_heads_supported).
bool attention_heads_supported(const Tensor& query, size_t heads, const Tensor* mask);
Tensor attention_heads(const Tensor& query, const Tensor& key, const Tensor& value, size_t heads,
                       const Tensor* mask = nullptr, Tensor* attention_weights = nullptr);

class MultiHeadAttention : public Module {
public:
    MultiHeadAttention(size_t d_model, size_t num_heads);
    Tensor forward(const Tensor& input) override;
    Tensor forward(const Tensor& input, const Tensor* mask);
    // residual + forward(input, mask), the add folded into the output
    // projection on the fused path; residual is (batch, seq, d_model).
    Tensor forward(const Tensor& input, const Tensor* mask, const Tensor* residual);
    std::vector<Tensor> parameters() override;
    std::vector<std::pair<std::string, Tensor>> named_parameters(
        const std::string& prefix = "") override;
    std::string name() const override;
    const Tensor& last_attention() const noexcept { return last_attention_; }
    void keep_attention(bool keep) { keep_attention_ = keep; }
    bool keeps_attention() const noexcept { return keep_attention_; }

private:
    size_t d_model_;
    size_t num_heads_;
    size_t head_dim_;
    Linear w_query_;
    Linear w_key_;
    Linear w_value_;
    Linear w_out_;
    Tensor last_attention_;
    bool keep_attention_ = false;
};

class TransformerBlock : public Module {
public:
    TransformerBlock(size_t d_model, size_t num_heads, size_t ff_hidden);
    Tensor forward(const Tensor& input) override;
    Tensor forward(const Tensor& input, const Tensor* mask);
    std::vector<Tensor> parameters() override;
    std::vector<std::pair<std::string, Tensor>> named_parameters(
        const std::string& prefix = "") override;
    void train(bool mode = true) override;
    std::string name() const override;
    MultiHeadAttention& attention() { return attention_; }

private:
    size_t d_model_;
    size_t ff_hidden_;
    LayerNorm norm1_;
    LayerNorm norm2_;
    MultiHeadAttention attention_;
    Linear ff1_;
    Linear ff2_;
};

}  // namespace nn
}  // namespace engine

#endif  // ENGINE_TRANSFORMER_HPP
