// nn.cpp -- Module plumbing, Linear, Sequential, the losses and the accuracy
// helpers (the reference's src/nn.cpp).
#include "engine/nn.hpp"
#include "engine/conv.hpp"

#include <atomic>
#include <cmath>
#include <cstdio>
#include <stdexcept>

#include "detail.hpp"

namespace engine {
namespace nn {

namespace {
std::atomic<bool> g_fused_nodes{true};
std::atomic<bool> g_short_attention{true};
std::atomic<bool> g_deferred_weight_grads{true};
}  // namespace

void set_fused_nodes(bool on) { g_fused_nodes.store(on); }
bool fused_nodes() { return g_fused_nodes.load(); }
void set_short_attention(bool on) { g_short_attention.store(on); }
bool short_attention() { return g_short_attention.load(); }
void set_deferred_weight_grads(bool on) { g_deferred_weight_grads.store(on); }
bool deferred_weight_grads() { return g_deferred_weight_grads.load(); }
void set_fused_bias_grad(bool on) { ehip_linear_bias_from_dw(on ? 1 : 0); }
bool fused_bias_grad() { return ehip_linear_bias_from_dw(-1) != 0; }


using namespace detail;

std::vector<std::pair<std::string, Tensor>> Module::named_parameters(const std::string& prefix) {
    std::vector<std::pair<std::string, Tensor>> out;
    const std::vector<Tensor> params = parameters();
    for (size_t i = 0; i < params.size(); ++i)
        out.emplace_back(prefix + name() + "." + std::to_string(i), params[i]);
    return out;
}

void Module::zero_grad() {
    for (Tensor& p : parameters()) p.zero_grad();
}

size_t Module::num_parameters() {
    size_t total = 0;
    for (const Tensor& p : parameters()) total += p.size();
    return total;
}

// Xavier-uniform weight (in, out), zero bias (1, out): src/nn.cpp:85-99.
Linear::Linear(size_t in_features, size_t out_features, bool use_bias)
    : in_features_(in_features), out_features_(out_features), use_bias_(use_bias) {
    if (in_features == 0 || out_features == 0)
        throw std::invalid_argument("Linear requires in_features and out_features greater than zero.");
    const float limit = std::sqrt(6.0f / static_cast<float>(in_features + out_features));
    autograd::NoGradGuard no_grad;
    weight_ = Tensor::rand({in_features, out_features}, -limit, limit, true);
    bias_ = Tensor({1, out_features}, 0.0f, use_bias);
}

Tensor Linear::forward(const Tensor& input) {
    if (input.ndim() < 2)
        throw std::invalid_argument("Linear expects at least 2 dimensions (..., in_features), received " +
                                    input.shape_str() + ".");
    if (input.shape().back() != in_features_)
        throw std::invalid_argument("Linear with in_features=" + std::to_string(in_features_) +
                                    " received an input " + input.shape_str() + ".");
    const bool needs_reshape = input.ndim() > 2;
    Tensor flat = needs_reshape ? input.reshape({input.size() / in_features_, in_features_}) : input;
    Tensor out;
    if (fused_nodes()) {
        out = ops::linear(flat, weight_, use_bias_ ? &bias_ : nullptr);
    } else {
        out = flat.matmul(weight_);
        if (use_bias_) out = out + bias_;
    }
    if (needs_reshape) {
        std::vector<size_t> out_shape = input.shape();
        out_shape.back() = out_features_;
        out = out.reshape(out_shape);
    }
    return out;
}

std::vector<Tensor> Linear::parameters() {
    if (use_bias_) return {weight_, bias_};
    return {weight_};
}

std::string Linear::name() const {
    return "Linear(" + std::to_string(in_features_) + " -> " + std::to_string(out_features_) +
           (use_bias_ ? ", bias=true)" : ", bias=false)");
}

Sequential& Sequential::add(std::unique_ptr<Module> layer) {
    if (!layer) throw std::invalid_argument("Sequential::add received a null layer.");
    layers_.push_back(std::move(layer));
    return *this;
}

Dropout::Dropout(float p) : p_(p) {
    if (!(p >= 0.0f && p < 1.0f))
        throw std::invalid_argument("Dropout needs a probability in [0, 1).");
}

// src/nn.cpp:206-244 with the mask drawn on the device; the backward
// multiplies by the same mask.
namespace {

// y = f(x) on the device; backward dx = g * f'(x, y) (the reference's
// unary_with_grad, src/nn.cpp:27-48, with its derivatives of src/nn.cpp:154-198).
Tensor activation(const Tensor& input, int kind) {
    Tensor out(input.shape(), 0.0f, false);
    hip::check(ehip_activation_f32(kind, dptr(input), dout(out), int64_t(input.size()), nullptr),
               "activation");
    if (!track(input.requires_grad())) return out;
    out.set_requires_grad(true);
    out.get_impl()->parents = {input.get_impl()};
    Tensor input_copy = input;
    Tensor saved = out.detach();
    out.get_impl()->backward_fn = [input_copy, saved, kind](const Tensor& g) mutable {
        Tensor dX(input_copy.shape(), 0.0f, false);
        hip::check(ehip_activation_backward_f32(kind, dptr(input_copy), dptr(saved), dptr(g),
                                                dout(dX), int64_t(dX.size()), nullptr),
                   "activation backward");
        input_copy.add_grad(dX);
    };
    return out;
}

}  // namespace

Tensor Sigmoid::forward(const Tensor& input) { return activation(input, EHIP_SIGMOID); }
Tensor Tanh::forward(const Tensor& input) { return activation(input, EHIP_TANH); }
Tensor GELU::forward(const Tensor& input) { return activation(input, EHIP_GELU); }

Tensor Dropout::forward(const Tensor& input) {
    if (!is_training() || p_ == 0.0f) return input;
    Tensor out(input.shape(), 0.0f, false);
    Tensor mask(input.shape(), 0.0f, false);
    const DeviceRng draw = device_rng_take(input.size());
    hip::check(ehip_dropout_f32(dptr(input), dout(out), dout(mask), int64_t(input.size()), p_,
                                draw.seed, draw.offset, nullptr),
               "dropout");
    if (track(input.requires_grad())) {
        out.set_requires_grad(true);
        out.get_impl()->parents = {input.get_impl()};
        Tensor input_copy = input;
        out.get_impl()->backward_fn = [input_copy, mask](const Tensor& g) mutable {
            Tensor dx(input_copy.shape(), 0.0f, false);
            hip::check(ehip_binary_f32(EHIP_MUL, dptr(g), dptr(mask), dout(dx),
                                       int64_t(dx.size()), 1, nullptr),
                       "dropout backward");
            input_copy.add_grad(dx);
        };
    }
    return out;
}

std::string Dropout::name() const { return "Dropout(p=" + std::to_string(p_).substr(0, 4) + ")"; }

// Layer by layer, as the reference does (src/nn.cpp); a Conv2d -> ReLU ->
// MaxPool2d run is handed to the fused node when it qualifies (same values,
// one forward launch instead of three, the pool and ReLU backward folded into
// the convolution's).
Tensor Sequential::forward(const Tensor& input) {
    Tensor x = input;
    for (size_t i = 0; i < layers_.size(); ++i) {
        if (i + 2 < layers_.size()) {
            auto* conv = dynamic_cast<Conv2d*>(layers_[i].get());
            auto* relu = dynamic_cast<ReLU*>(layers_[i + 1].get());
            auto* pool = dynamic_cast<MaxPool2d*>(layers_[i + 2].get());
            Tensor fused;
            if (conv && relu && pool && conv2d_relu_maxpool(x, *conv, *pool, fused)) {
                x = fused;
                i += 2;
                continue;
            }
        }
        x = layers_[i]->forward(x);
    }
    return x;
}

std::vector<Tensor> Sequential::parameters() {
    std::vector<Tensor> out;
    for (auto& layer : layers_)
        for (const Tensor& p : layer->parameters()) out.push_back(p);
    return out;
}

std::vector<std::pair<std::string, Tensor>> Sequential::named_parameters(const std::string& prefix) {
    std::vector<std::pair<std::string, Tensor>> out;
    for (size_t i = 0; i < layers_.size(); ++i)
        for (auto& np : layers_[i]->named_parameters(prefix + std::to_string(i) + "."))
            out.push_back(np);
    return out;
}

void Sequential::train(bool mode) {
    Module::train(mode);
    for (auto& layer : layers_) layer->train(mode);
}

// The reference's console format (src/nn.cpp:303-313), wording included, so
// that programs print the same text.
void Sequential::summary() const {
    std::printf("Sequential (%zu layers)\n", layers_.size());
    size_t total = 0;
    for (size_t i = 0; i < layers_.size(); ++i) {
        const size_t n = layers_[i]->num_parameters();
        total += n;
        std::printf("  [%zu] %-32s%10zu parametros\n", i, layers_[i]->name().c_str(), n);
    }
    std::printf("  Total entrenable: %zu parametros\n", total);
}

Module& Sequential::at(size_t index) {
    if (index >= layers_.size()) throw std::out_of_range("Sequential::at: index out of range.");
    return *layers_[index];
}

Tensor mse_loss(const Tensor& prediction, const Tensor& target) {
    if (prediction.shape() != target.shape())
        throw std::invalid_argument("mse_loss: shapes " + prediction.shape_str() + " and " +
                                    target.shape_str() + " differ.");
    Tensor diff = prediction - target;
    return (diff * diff).mean();
}

// Probabilities, per-row losses and their mean are computed on the device
// (the reference computes them serially on the host, src/nn.cpp:346-380);
// the loss is read back only when host code asks for it.
namespace {

// With fused nodes on and a small head, the forward launch also writes the
// logits' gradient for an upstream gradient of 1; backward hands it over when
// the loss is the root of backward (its seed is a pending fill of ones, known
// on the host), saving the seed's fill and the backward launch. Any other
// upstream gradient takes the backward kernel; the bits are the same.
Tensor cross_entropy_device(const Tensor& logits, std::shared_ptr<DeviceInts> d_t) {
    const size_t N = logits.shape()[0], C = logits.shape()[1];
    Tensor probs(logits.shape(), 0.0f, false);
    const bool req_g = logits.requires_grad() && autograd::grad_enabled();
    Tensor loss({1}, 0.0f, false);
    Tensor d_unit;
    bool unit = false;
    if (req_g && fused_nodes() && ehip_cross_entropy_fused_supported(int64_t(N), int64_t(C))) {
        d_unit = Tensor(logits.shape(), 0.0f, false);
        unit = true;
        hip::check(ehip_cross_entropy_fused_f32(dptr(logits), d_t->get(), dout(probs), dout(loss),
                                                dout(d_unit), int64_t(N), int64_t(C), nullptr),
                   "cross_entropy_loss");
    } else {
        hip::check(ehip_cross_entropy_f32(dptr(logits), d_t->get(), dout(probs), dout(loss),
                                          int64_t(N), int64_t(C), nullptr),
                   "cross_entropy_loss");
    }
    if (req_g) {
        loss.set_requires_grad(true);
        loss.get_impl()->parents = {logits.get_impl()};
        Tensor logits_copy = logits;
        loss.get_impl()->backward_fn = [logits_copy, probs, d_t, N, C, d_unit,
                                        unit](const Tensor& g) mutable {
            float seed = 0.0f;
            if (unit && g.storage().pending_constant(&seed) && seed == 1.0f) {
                // Handed over (not shared), so add_grad can adopt the buffer; a
                // second backward over the graph takes the kernel below.
                Tensor d = std::move(d_unit);
                d_unit = Tensor();
                unit = false;
                logits_copy.add_grad(d);
                return;
            }
            Tensor dX(logits_copy.shape(), 0.0f, false);
            hip::check(ehip_cross_entropy_backward_f32(dptr(probs), d_t->get(), dout(dX),
                                                       int64_t(N), int64_t(C), dptr(g), nullptr),
                       "cross_entropy_loss backward");
            logits_copy.add_grad(dX);
        };
    }
    return loss;
}

void check_logits(const Tensor& logits, size_t n_targets) {
    if (logits.ndim() != 2)
        throw std::invalid_argument("cross_entropy_loss expects 2D logits (batch, classes), received " +
                                    logits.shape_str() + ".");
    const size_t N = logits.shape()[0];
    if (n_targets != N)
        throw std::invalid_argument("cross_entropy_loss received " + std::to_string(n_targets) +
                                    " labels for a batch of " + std::to_string(N) + ".");
    if (N == 0) throw std::invalid_argument("cross_entropy_loss received an empty batch.");
}

}  // namespace

Tensor cross_entropy_loss(const Tensor& logits, const std::vector<size_t>& targets) {
    check_logits(logits, targets.size());
    const size_t N = logits.shape()[0], C = logits.shape()[1];
    std::vector<int32_t> t(N);
    for (size_t i = 0; i < N; ++i) {
        if (targets[i] >= C)
            throw std::out_of_range("Label " + std::to_string(targets[i]) +
                                    " outside the range of " + std::to_string(C) + " classes.");
        t[i] = static_cast<int32_t>(targets[i]);
    }
    return cross_entropy_device(logits, std::make_shared<DeviceInts>(t));
}

Labels::Labels(const std::vector<size_t>& targets) : n_(targets.size()) {
    std::vector<int32_t> t(targets.size());
    for (size_t i = 0; i < targets.size(); ++i) {
        if (targets[i] > size_t(INT32_MAX))
            throw std::out_of_range("Label " + std::to_string(targets[i]) + " beyond int32.");
        t[i] = static_cast<int32_t>(targets[i]);
        if (targets[i] > max_) max_ = targets[i];
    }
    dev_ = DeviceInts(t);
}

Tensor cross_entropy_loss(const Tensor& logits, const Labels& targets) {
    check_logits(logits, targets.size());
    const size_t C = logits.shape()[1];
    if (targets.size() > 0 && targets.max_label() >= C)
        throw std::out_of_range("Label " + std::to_string(targets.max_label()) +
                                " outside the range of " + std::to_string(C) + " classes.");
    return cross_entropy_device(logits, std::make_shared<DeviceInts>(targets.device()));
}

std::vector<size_t> argmax_rows(const Tensor& logits) {
    if (logits.ndim() != 2) throw std::invalid_argument("argmax_rows expects 2D logits.");
    const size_t N = logits.shape()[0], C = logits.shape()[1];
    const float* v = logits.data();
    std::vector<size_t> out(N, 0);
    for (size_t i = 0; i < N; ++i)
        for (size_t j = 1; j < C; ++j)
            if (v[i * C + j] > v[i * C + out[i]]) out[i] = j;
    return out;
}

float accuracy(const Tensor& logits, const std::vector<size_t>& targets) {
    const std::vector<size_t> pred = argmax_rows(logits);
    if (pred.size() != targets.size()) throw std::invalid_argument("accuracy: size mismatch.");
    if (pred.empty()) return 0.0f;
    size_t hit = 0;
    for (size_t i = 0; i < pred.size(); ++i) hit += pred[i] == targets[i];
    return static_cast<float>(hit) / static_cast<float>(pred.size());
}

}  // namespace nn
}  // namespace engine
