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
// dgamma and dbeta in two kernels (src/transformer.cpp:82-179). With fused
// nodes, a large LayerNorm whose dgamma and dbeta add_grad will adopt writes
// only dx and its per-group partials during backward; the sums of every such
// node (and of the fused convolution blocks) run in one launch afterwards, or
// inside Adam's, with the same bits as the two-kernel backward.
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
        int64_t groups = 0;
        const int64_t nparts =
            nn::fused_nodes() && gamma_copy.requires_grad() && beta_copy.requires_grad() &&
                    detail::grad_adoptable(gamma_copy) && detail::grad_adoptable(beta_copy)
                ? ehip_layernorm_backward_partials(int64_t(rows), int64_t(D), &groups)
                : 0;
        if (nparts > 0) {
            Tensor part({size_t(nparts)}, 0.0f, false);
            // The input's gradient already held (the residual branch's) takes dx
            // added in the row kernel itself: the add_grad below, folded in (rows
            // of at most 1024 columns, the kernel's accumulating form).
            float* acc_dx = input_copy.requires_grad() && D <= 1024
                                ? detail::grad_in_place(input_copy)
                                : nullptr;
            hip::check(ehip_layernorm_backward_partials_f32(
                           dptr(g), dptr(xhat), dptr(gamma_copy), dptr(inv_std),
                           acc_dx ? acc_dx : dout(dX), dout(part), groups, int64_t(rows),
                           int64_t(D), acc_dx ? 1 : 0, nullptr),
                       "layernorm backward");
            const ehip_conv_reduce_t job{dptr(part), groups, int64_t(D), 1, dout(dgamma),
                                         dout(dbeta)};
            detail::defer_conv_reduce(job, part);
            if (input_copy.requires_grad() && acc_dx == nullptr) input_copy.add_grad(dX);
            gamma_copy.add_grad(dgamma);
            beta_copy.add_grad(dbeta);
            detail::defer_conv_output(gamma_copy, dgamma);
            detail::defer_conv_output(beta_copy, dbeta);
            return;
        }
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
// (src/transformer.cpp:206-231); the gather runs on the device. The rounded,
// validated indices and the backward's inverse map are uploaded once per ids
// buffer: while the same buffer comes back with its contents untouched
// (Storage::version), they are reused and the step moves nothing to the
// device.
Tensor Embedding::forward(const Tensor& ids) {
    if (ids.ndim() != 2)
        throw std::invalid_argument("Embedding expects indices (batch, sequence), received " +
                                    ids.shape_str() + ".");
    const size_t batch = ids.shape()[0], seq = ids.shape()[1];
    const bool need_inverse = detail::track(weight_.requires_grad());
    const bool reuse = gather_ && ids.storage().same_buffer(ids_seen_) &&
                       ids.storage().version() == ids_version_ && gather_->n == ids.size() &&
                       (gather_->inverse || !need_inverse);
    if (!reuse) {
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
        if (indices.empty())
            throw std::invalid_argument("select_rows received an empty index list.");
        gather_ = detail::make_row_gather(indices, num_embeddings_, weight_.shape_str(),
                                          need_inverse);
        ids_seen_ = ids.storage().share();
        ids_version_ = ids.storage().version();
    }
    return detail::gather_rows(weight_, gather_).reshape({batch, seq, dim_});
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
    if (seq_len == 0 || d_model == 0)
        throw std::invalid_argument("positional_encoding needs a positive length and dimension.");
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
    Tensor mask({seq_len, seq_len}, m, false);
    mask.get_impl()->causal_value = masked_value;
    mask.get_impl()->causal_version = mask.storage().version();
    return mask;
}

namespace {

// True when `mask` is a causal mask made by causal_mask for S x S scores and
// not written since, with a masked value far enough below any finite score
// that the softmax is exactly 0 above the diagonal (exp underflows to 0 below
// -104): then the attention products may skip what the mask zeroes
// (ehip_gemm_ex_t::causal). The skipped products are exact zeros, so the
// results keep their values while the scores are finite.
bool skippable_causal(const Tensor* mask, size_t S) {
    if (mask == nullptr) return false;
    const auto& impl = mask->get_impl();
    return impl->causal_value <= -1e9f && impl->causal_version == mask->storage().version() &&
           mask->ndim() == 2 && mask->shape()[0] == S && mask->shape()[1] == S;
}

}  // namespace

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

namespace {

// The addend geometry of a mask suffix-broadcast over (batch, heads, S, S):
// its core (leading 1s stripped) is (), (S), (S, S), (heads, S, S) or
// (batch, heads, S, S). False when it is none of these.
struct MaskPlan {
    int64_t ld = 0, stride = 0, period = 1;
};

bool mask_plan(const Tensor& mask, size_t batch, size_t heads, size_t seq, MaskPlan& plan) {
    const std::vector<size_t> full = {batch, heads, seq, seq};
    if (!plan_broadcast(full, mask.shape()).valid) return false;
    size_t first = 0;
    while (first < mask.ndim() && mask.shape()[first] == 1) ++first;
    const size_t core = mask.ndim() - first;
    plan = MaskPlan{};
    if (core >= 2) {
        plan.ld = int64_t(seq);
        plan.stride = int64_t(seq * seq);
    }
    if (core == 3) plan.period = int64_t(heads);
    if (core == 4) plan.period = int64_t(batch * heads);
    return true;
}

// The descriptor of a product over the (sample, head) pairs of heads-major
// operands: z = sample * heads + head.
struct HeadOperand {
    const float* p;
    int64_t ld, stride, stride_inner;
};

ehip_gemm_ex_t head_product(bool ta, bool tb, size_t batch, size_t heads, size_t m, size_t n,
                            size_t k, HeadOperand a, HeadOperand b, float* c, int64_t ldc,
                            int64_t stride_c, int64_t stride_c_inner) {
    ehip_gemm_ex_t d{};
    d.trans_a = ta ? 1 : 0;
    d.trans_b = tb ? 1 : 0;
    d.batch = int64_t(batch * heads);
    d.inner = int64_t(heads);
    d.m = int64_t(m);
    d.n = int64_t(n);
    d.k = int64_t(k);
    d.a = a.p;
    d.lda = a.ld;
    d.stride_a = a.stride;
    d.stride_a_inner = a.stride_inner;
    d.b = b.p;
    d.ldb = b.ld;
    d.stride_b = b.stride;
    d.stride_b_inner = b.stride_inner;
    d.c = c;
    d.ldc = ldc;
    d.stride_c = stride_c;
    d.stride_c_inner = stride_c_inner;
    d.alpha = 1.0f;
    d.addend_period = 1;
    return d;
}

}  // namespace

namespace {

// Sequences and heads of at most 64 values: the whole attention of a head in
// one workgroup (ehip_attention_short_f32 / _backward_f32), two launches per
// step instead of eight; the weights are kept for the backward as the product
// path keeps them.
Tensor attention_short(const Tensor& query, const Tensor& key, const Tensor& value, size_t B,
                       size_t S, size_t D, size_t H, size_t hd, float scale, bool causal,
                       Tensor* attention_weights) {
    Tensor weights({B, H, S, S}, 0.0f, false);
    Tensor out({B, S, D}, 0.0f, false);
    hip::check(ehip_attention_short_f32(dptr(query), dptr(key), dptr(value), dout(weights),
                                        dout(out), int64_t(B), int64_t(S), int64_t(D), int64_t(H),
                                        int64_t(hd), scale, causal ? 1 : 0, nullptr),
               "attention");
    if (attention_weights != nullptr) *attention_weights = weights.detach();
    if (!track(query.requires_grad() || key.requires_grad() || value.requires_grad())) return out;
    out.set_requires_grad(true);
    out.get_impl()->parents = {query.get_impl(), key.get_impl(), value.get_impl()};
    Tensor q = query, k = key, v = value;
    out.get_impl()->backward_fn = [q, k, v, weights, B, S, D, H, hd, scale,
                                   causal](const Tensor& g) mutable {
        Tensor dq, dk, dv;
        if (q.requires_grad()) dq = Tensor({B, S, D}, 0.0f, false);
        if (k.requires_grad()) dk = Tensor({B, S, D}, 0.0f, false);
        if (v.requires_grad()) dv = Tensor({B, S, D}, 0.0f, false);
        hip::check(ehip_attention_short_backward_f32(
                       dptr(q), dptr(k), dptr(v), dptr(weights), dptr(g),
                       q.requires_grad() ? dout(dq) : nullptr,
                       k.requires_grad() ? dout(dk) : nullptr,
                       v.requires_grad() ? dout(dv) : nullptr, int64_t(B), int64_t(S), int64_t(D),
                       int64_t(H), int64_t(hd), scale, causal ? 1 : 0, nullptr),
                   "attention backward");
        // The product path's order of the three hand-overs.
        if (v.requires_grad()) v.add_grad(dv);
        if (q.requires_grad()) q.add_grad(dq);
        if (k.requires_grad()) k.add_grad(dk);
    };
    return out;
}

}  // namespace

bool attention_heads_supported(const Tensor& query, size_t heads, const Tensor* mask) {
    if (query.ndim() != 3 || heads == 0 || query.shape()[2] % heads != 0) return false;
    if (mask == nullptr) return true;
    if (track(mask->requires_grad())) return false;
    MaskPlan plan;
    return mask_plan(*mask, query.shape()[0], heads, query.shape()[1], plan);
}

// One node for softmax(Q K^T / sqrt(d) + mask) V over every head
// (src/transformer.cpp:279-304 under the head split and merge of
// src/transformer.cpp:320-349). Forward: the score product with the scale and
// mask in its epilogue, the row softmax, the product with V written straight
// into the merged layout. Backward: dW = g V^T, dV = W^T g, the softmax
// derivative with the scale's backward folded in (in place over dW), then
// dQ = dS K and dK = dS^T Q -- the composed path's products, operand for
// operand, with each head addressed in place.
Tensor attention_heads(const Tensor& query, const Tensor& key, const Tensor& value, size_t heads,
                       const Tensor* mask, Tensor* attention_weights) {
    if (!attention_heads_supported(query, heads, mask))
        throw std::invalid_argument("attention_heads: query " + query.shape_str() + " with " +
                                    std::to_string(heads) + " heads" +
                                    (mask ? " and mask " + mask->shape_str() : std::string()) +
                                    " is not supported.");
    if (key.shape() != query.shape() || value.shape() != query.shape())
        throw std::invalid_argument("attention_heads: query, key and value differ: " +
                                    query.shape_str() + ", " + key.shape_str() + ", " +
                                    value.shape_str() + ".");
    const size_t B = query.shape()[0], S = query.shape()[1], D = query.shape()[2];
    const size_t H = heads, hd = D / heads;
    const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
    const int64_t sd = int64_t(S * D), ss = int64_t(S * S), hss = int64_t(H * S * S);
    const auto act = [&](const Tensor& t) { return HeadOperand{dptr(t), int64_t(D), sd, int64_t(hd)}; };

    // With a causal mask: score tiles wholly above the diagonal are neither
    // computed nor stored (the softmax reads each row up to the diagonal only
    // and stores 0 past it), and the products with the weights skip the zero
    // blocks above it.
    const bool causal = skippable_causal(mask, S);
    if (nn::short_attention() && (mask == nullptr || causal) &&
        ehip_attention_short_supported(int64_t(S), int64_t(hd)))
        return attention_short(query, key, value, B, S, D, H, hd, scale, causal,
                               attention_weights);
    Tensor scores({B, H, S, S}, 0.0f, false);
    ehip_gemm_ex_t d = head_product(false, true, B, H, S, S, hd, act(query), act(key),
                                    dout(scores), int64_t(S), hss, ss);
    d.alpha = scale;
    d.causal = causal ? 4 : 0;
    if (mask != nullptr) {
        MaskPlan plan;
        mask_plan(*mask, B, H, S, plan);
        d.addend = dptr(*mask);
        d.ld_addend = plan.ld;
        d.stride_addend = plan.stride;
        d.addend_period = plan.period;
    }
    hip::check(ehip_gemm_ex_f32(&d, nullptr), "attention scores");
    Tensor weights({B, H, S, S}, 0.0f, false);
    hip::check(causal ? ehip_softmax_causal_f32(dptr(scores), dout(weights), int64_t(B * H * S),
                                                int64_t(S), nullptr)
                      : ehip_softmax_f32(dptr(scores), dout(weights), int64_t(B * H * S),
                                         int64_t(S), nullptr),
               "attention softmax");
    scores = Tensor();
    if (attention_weights != nullptr) *attention_weights = weights.detach();

    Tensor out({B, S, D}, 0.0f, false);
    d = head_product(false, false, B, H, S, hd, S, HeadOperand{dptr(weights), int64_t(S), hss, ss},
                     act(value), dout(out), int64_t(D), sd, int64_t(hd));
    d.causal = causal ? 2 : 0;  // W(i, k) = 0 for k > i
    hip::check(ehip_gemm_ex_f32(&d, nullptr), "attention output");

    if (!track(query.requires_grad() || key.requires_grad() || value.requires_grad())) return out;
    out.set_requires_grad(true);
    out.get_impl()->parents = {query.get_impl(), key.get_impl(), value.get_impl()};
    Tensor q = query, k = key, v = value;
    out.get_impl()->backward_fn = [q, k, v, weights, B, S, D, H, hd, scale, sd, ss, hss,
                                   causal](const Tensor& g) mutable {
        const auto head = [&](const Tensor& t) {
            return HeadOperand{dptr(t), int64_t(D), sd, int64_t(hd)};
        };
        const HeadOperand w{dptr(weights), int64_t(S), hss, ss};
        if (v.requires_grad()) {  // dV = W^T g
            Tensor dv({B, S, D}, 0.0f, false);
            ehip_gemm_ex_t d = head_product(true, false, B, H, S, hd, S, w, head(g), dout(dv),
                                            int64_t(D), sd, int64_t(hd));
            d.causal = causal ? 3 : 0;  // W^T(i, k) = W(k, i) = 0 for k < i
            hip::check(ehip_gemm_ex_f32(&d, nullptr), "attention dV");
            v.add_grad(dv);
        }
        if (!q.requires_grad() && !k.requires_grad()) return;
        Tensor ds({B, H, S, S}, 0.0f, false);  // dW, then dS in place
        ehip_gemm_ex_t d = head_product(false, true, B, H, S, S, hd, head(g), head(v), dout(ds),
                                        int64_t(S), hss, ss);
        // Above the diagonal dW only meets W = 0 in the softmax backward,
        // which reads each row up to the diagonal and stores all of dS: whole
        // tiles there are neither computed nor stored.
        d.causal = causal ? 4 : 0;
        hip::check(ehip_gemm_ex_f32(&d, nullptr), "attention dW");
        hip::check(causal ? ehip_softmax_backward_scaled_causal_f32(dptr(weights), dptr(ds),
                                                                    dout(ds), int64_t(B * H * S),
                                                                    int64_t(S), scale, nullptr)
                          : ehip_softmax_backward_scaled_f32(dptr(weights), dptr(ds), dout(ds),
                                                             int64_t(B * H * S), int64_t(S),
                                                             scale, nullptr),
                   "attention softmax backward");
        const HeadOperand dsh{dptr(ds), int64_t(S), hss, ss};
        if (q.requires_grad()) {  // dQ = dS K
            Tensor dq({B, S, D}, 0.0f, false);
            d = head_product(false, false, B, H, S, hd, S, dsh, head(k), dout(dq), int64_t(D), sd,
                             int64_t(hd));
            d.causal = causal ? 2 : 0;  // dS(i, k) = 0 for k > i
            hip::check(ehip_gemm_ex_f32(&d, nullptr), "attention dQ");
            q.add_grad(dq);
        }
        if (k.requires_grad()) {  // dK = dS^T Q
            Tensor dk({B, S, D}, 0.0f, false);
            d = head_product(true, false, B, H, S, hd, S, dsh, head(q), dout(dk), int64_t(D), sd,
                             int64_t(hd));
            d.causal = causal ? 3 : 0;  // dS^T(i, k) = dS(k, i) = 0 for k < i
            hip::check(ehip_gemm_ex_f32(&d, nullptr), "attention dK");
            k.add_grad(dk);
        }
    };
    return out;
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
    return forward(input, mask, nullptr);
}

Tensor MultiHeadAttention::forward(const Tensor& input, const Tensor* mask,
                                   const Tensor* residual) {
    if (input.ndim() != 3 || input.shape()[2] != d_model_)
        throw std::invalid_argument("MultiHeadAttention expects (batch, seq, " +
                                    std::to_string(d_model_) + "), received " + input.shape_str() + ".");
    const size_t batch = input.shape()[0], seq = input.shape()[1];
    if (fused_nodes() && attention_heads_supported(input, num_heads_, mask)) {
        // One (batch * seq, d_model) view feeds the three projections, so their
        // input gradients meet in one buffer (the second and third products add
        // into it in place) before a single reshape hands it to `input`.
        const Tensor flat = input.reshape({batch * seq, d_model_});
        const auto bias = [](Linear& layer) { return layer.has_bias() ? &layer.bias() : nullptr; };
        const std::vector<Tensor> qkv = ops::linear_many(
            flat, {&w_query_.weight(), &w_key_.weight(), &w_value_.weight()},
            {bias(w_query_), bias(w_key_), bias(w_value_)});
        const auto heads = [&](const Tensor& t) { return t.reshape({batch, seq, d_model_}); };
        Tensor attended = attention_heads(heads(qkv[0]), heads(qkv[1]), heads(qkv[2]), num_heads_,
                                          mask, keep_attention_ ? &last_attention_ : nullptr);
        if (residual == nullptr) return w_out_(attended);
        if (residual->shape() != input.shape()) return *residual + w_out_(attended);
        // residual + attended w_out + b_out, the add in the product's epilogue.
        return ops::linear(attended.reshape({batch * seq, d_model_}), w_out_.weight(),
                           w_out_.has_bias() ? &w_out_.bias() : nullptr, residual);
    }
    auto split_heads = [&](const Tensor& projected) {
        return projected.reshape({batch, seq, num_heads_, head_dim_}).permute({0, 2, 1, 3});
    };
    Tensor q = split_heads(w_query_(input));
    Tensor k = split_heads(w_key_(input));
    Tensor v = split_heads(w_value_(input));
    Tensor attended =
        scaled_dot_product_attention(q, k, v, mask, keep_attention_ ? &last_attention_ : nullptr);
    Tensor merged = attended.permute({0, 2, 1, 3}).reshape({batch, seq, d_model_});
    return residual ? *residual + w_out_(merged) : w_out_(merged);
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
// With fused nodes both residual adds run in the epilogues of the products
// that end their branches (the output projection, the second feed-forward
// layer).
Tensor TransformerBlock::forward(const Tensor& input, const Tensor* mask) {
    Tensor h = attention_.forward(norm1_(input), mask, &input);
    Tensor n2 = norm2_(h);
    if (fused_nodes() && ff1_.has_bias() && ff2_.has_bias()) {
        const size_t cols = n2.shape().back();
        return ops::feed_forward_relu(n2.reshape({n2.size() / cols, cols}), ff1_.weight(),
                                      ff1_.bias(), ff2_.weight(), ff2_.bias(), &h);
    }
    return h + ff2_(ff1_(n2).relu());
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
