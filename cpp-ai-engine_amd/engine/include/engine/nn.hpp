// nn.hpp -- modules and losses of the training path, mirroring the
// reference's include/engine/nn.hpp (Module, Linear, ReLU, Softmax,
// Sequential, make, mse_loss, cross_entropy_loss, argmax_rows, accuracy).
// Sigmoid, Tanh, GELU and Dropout are not provided: no configuration of this
// backend trains through them.
#ifndef ENGINE_NN_HPP
#define ENGINE_NN_HPP

#include <memory>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "engine/tensor.hpp"

namespace engine {
namespace nn {

// Fused graph nodes, on by default: Linear's product and bias add as one
// node (the add in the GEMM epilogue), TransformerBlock's feed-forward as one
// node, MultiHeadAttention's heads read and written in place. Switched off,
// the modules build the reference's node-by-node graph instead; the values
// are the same bit for bit either way. Process-wide; set it between steps.
void set_fused_nodes(bool on);
bool fused_nodes();

// Short attention, on by default: the fused attention node takes one launch
// per direction (ehip_attention_short_f32 and its backward: a workgroup per
// batch and head, scores, softmax and products in LDS, each sum in the
// reference's loop order) for sequences and heads of at most 64 values, with
// no mask or nn::causal_mask's. Off, those take the batched products and
// softmax kernels as longer sequences do; the values agree to the reference's
// tolerance, not bit for bit. Process-wide; set it between steps.
void set_short_attention(bool on);
bool short_attention();

// Queued weight gradients, on by default: the Linear and feed-forward nodes of
// narrow layers (whose dW = X^T dY takes the panel kernel with the bias
// gradient as its column sums) queue that product instead of launching it,
// and the queue runs them together (ehip_gemm_batch_f32) when a gradient is
// first read, before an in-place add into a buffer they read, or before
// Adam's launch: the same bits, fewer launches per backward. Process-wide;
// set it between steps.
void set_deferred_weight_grads(bool on);
bool deferred_weight_grads();

// Bias gradients from the weight-gradient product, on by default: Linear and
// the feed-forward node take db of a mid-sized layer (more than 64 rows, dY of
// at most 2^21 elements) from the column sums of dY that the dW = X^T dY
// product forms from the tiles it stages, instead of a separate two-pass
// column sum (ehip_linear_backward_f32). The sums are the same mathematically,
// added in another order; the char-Transformer's 10-step trajectory stays
// within 3e-6 of the reference's loss either way, and the step gets faster
// (two launch-bound launches fewer per layer). Off, every bias gradient takes
// the separate column sum. Process-wide (it switches the library's setting);
// set it between steps.
void set_fused_bias_grad(bool on);
bool fused_bias_grad();

class Module {
public:
    virtual ~Module() = default;
    virtual Tensor forward(const Tensor& input) = 0;
    Tensor operator()(const Tensor& input) { return forward(input); }
    virtual std::vector<Tensor> parameters() { return {}; }
    virtual std::vector<std::pair<std::string, Tensor>> named_parameters(
        const std::string& prefix = "");
    virtual void train(bool mode = true) { training_ = mode; }
    void eval() { train(false); }
    bool is_training() const noexcept { return training_; }
    virtual std::string name() const { return "Module"; }
    void zero_grad();
    size_t num_parameters();

protected:
    bool training_ = true;
};

// y = x W + b with W of shape (in, out), Xavier-uniform, b (1, out) zero
// (the reference's src/nn.cpp:85-130); inputs of more than two dimensions are
// viewed as rows.
class Linear : public Module {
public:
    Linear(size_t in_features, size_t out_features, bool use_bias = true);
    Tensor forward(const Tensor& input) override;
    std::vector<Tensor> parameters() override;
    std::string name() const override;
    Tensor& weight() { return weight_; }
    Tensor& bias() { return bias_; }
    bool has_bias() const noexcept { return use_bias_; }
    size_t in_features() const noexcept { return in_features_; }
    size_t out_features() const noexcept { return out_features_; }

private:
    size_t in_features_;
    size_t out_features_;
    bool use_bias_;
    Tensor weight_;
    Tensor bias_;
};

class ReLU : public Module {
public:
    Tensor forward(const Tensor& input) override { return input.relu(); }
    std::string name() const override { return "ReLU"; }
};

// Inverted dropout (the reference's include/engine/nn.hpp Dropout): in
// training, each element is kept with probability 1 - p and scaled by
// 1 / (1 - p); in evaluation it is the identity. Masks come from the device
// generator (Philox, keyed by the engine seed, advanced by a running element
// counter): reproducible after manual_seed(), but not the reference's host
// mt19937 stream.
class Dropout : public Module {
public:
    explicit Dropout(float p = 0.5f);
    Tensor forward(const Tensor& input) override;
    std::string name() const override;
    float probability() const noexcept { return p_; }

private:
    float p_;
};

class Softmax : public Module {
public:
    Tensor forward(const Tensor& input) override { return input.softmax(); }
    std::string name() const override { return "Softmax"; }
};

// The smooth activations (the reference's include/engine/nn.hpp:97-116):
// element-wise kernels on the device, forward and backward.
class Sigmoid : public Module {
public:
    Tensor forward(const Tensor& input) override;
    std::string name() const override { return "Sigmoid"; }
};

class Tanh : public Module {
public:
    Tensor forward(const Tensor& input) override;
    std::string name() const override { return "Tanh"; }
};

// GELU in its hyperbolic-tangent approximation.
class GELU : public Module {
public:
    Tensor forward(const Tensor& input) override;
    std::string name() const override { return "GELU"; }
};

class Sequential : public Module {
public:
    Sequential() = default;
    template <typename... Layers,
              typename =
                  std::enable_if_t<(std::is_convertible_v<Layers, std::unique_ptr<Module>> && ...)>>
    explicit Sequential(Layers&&... layers) {
        (add(std::forward<Layers>(layers)), ...);
    }
    Sequential& add(std::unique_ptr<Module> layer);
    Tensor forward(const Tensor& input) override;
    std::vector<Tensor> parameters() override;
    std::vector<std::pair<std::string, Tensor>> named_parameters(
        const std::string& prefix = "") override;
    void train(bool mode = true) override;
    std::string name() const override { return "Sequential"; }
    // Prints each layer's name and parameter count and the total to stdout
    // (src/nn.cpp:303-313 of the reference).
    void summary() const;
    size_t size() const noexcept { return layers_.size(); }
    Module& at(size_t index);

private:
    std::vector<std::unique_ptr<Module>> layers_;
};

template <typename T, typename... Args>
std::unique_ptr<T> make(Args&&... args) {
    return std::make_unique<T>(std::forward<Args>(args)...);
}

Tensor mse_loss(const Tensor& prediction, const Tensor& target);

// Fused log-softmax + NLL over (N, C) logits (the reference's
// src/nn.cpp:324-408), computed on the device; the loss stays on the device
// until read.
Tensor cross_entropy_loss(const Tensor& logits, const std::vector<size_t>& targets);

// Class labels uploaded once and kept on the device, for a batch that is
// reused (a resident batch, or labels produced on the device).
class Labels {
public:
    Labels() = default;
    explicit Labels(const std::vector<size_t>& targets);
    size_t size() const noexcept { return n_; }
    size_t max_label() const noexcept { return max_; }
    const DeviceInts& device() const noexcept { return dev_; }

private:
    DeviceInts dev_;
    size_t n_ = 0, max_ = 0;
};

// The same loss with device-resident labels: no upload per call.
Tensor cross_entropy_loss(const Tensor& logits, const Labels& targets);

class CrossEntropyLoss {
public:
    Tensor forward(const Tensor& logits, const std::vector<size_t>& targets) const {
        return cross_entropy_loss(logits, targets);
    }
    Tensor operator()(const Tensor& logits, const std::vector<size_t>& targets) const {
        return forward(logits, targets);
    }
};

std::vector<size_t> argmax_rows(const Tensor& logits);
float accuracy(const Tensor& logits, const std::vector<size_t>& targets);

}  // namespace nn
}  // namespace engine

#endif  // ENGINE_NN_HPP
