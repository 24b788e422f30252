// conv.hpp -- convolution through im2col and max pooling, mirroring the
// reference's include/engine/conv.hpp.
#ifndef ENGINE_CONV_HPP
#define ENGINE_CONV_HPP

#include <vector>

#include "engine/nn.hpp"

namespace engine {
namespace nn {

struct Window2d {
    size_t kernel_h;
    size_t kernel_w;
    size_t stride = 1;
    size_t padding = 0;

    Window2d(size_t k) : kernel_h(k), kernel_w(k) {}  // NOLINT: implicit, as in the reference
    Window2d(size_t kh, size_t kw, size_t s = 1, size_t p = 0)
        : kernel_h(kh), kernel_w(kw), stride(s), padding(p) {}

    size_t out_h(size_t in_h) const;
    size_t out_w(size_t in_w) const;
    void validate(size_t in_h, size_t in_w) const;
};

Tensor im2col(const Tensor& input, const Window2d& window);
Tensor col2im(const Tensor& cols, const std::vector<size_t>& input_shape, const Window2d& window);

// Wide convolutions (the direct kernels refuse them) run as implicit GEMMs by
// default: the forward, weight-gradient and input-gradient products on MFMA
// with the column operand gathered from the tensors, no column matrix in
// memory. Off, they compose as the reference does (im2col, the product with
// the transposed weight, the bias add, the permute). The values agree within
// the products' K-term tolerance. Process-wide; set it between steps.
void set_conv_implicit_gemm(bool on);
bool conv_implicit_gemm();

class Conv2d : public Module {
public:
    Conv2d(size_t in_channels, size_t out_channels, const Window2d& window, bool use_bias = true);
    Tensor forward(const Tensor& input) override;
    std::vector<Tensor> parameters() override;
    std::string name() const override;
    Tensor& weight() { return weight_; }
    Tensor& bias() { return bias_; }
    bool has_bias() const { return use_bias_; }
    size_t out_channels() const { return out_channels_; }
    const Window2d& window() const { return window_; }

private:
    size_t in_channels_;
    size_t out_channels_;
    Window2d window_;
    bool use_bias_;
    Tensor weight_;  // (out_channels, in_channels, kernel_h, kernel_w)
    Tensor bias_;    // (out_channels)
};

class MaxPool2d : public Module {
public:
    explicit MaxPool2d(const Window2d& window);
    MaxPool2d(size_t kernel, size_t stride);
    Tensor forward(const Tensor& input) override;
    std::string name() const override;
    const Window2d& window() const { return window_; }

private:
    Window2d window_;
};

// Conv2d -> ReLU -> MaxPool2d as one node when the layers allow it (a narrow
// convolution, a pool with kernel == stride and no padding): the values of the
// three separate nodes, without the convolution output in HBM. Returns false
// (and leaves `out` alone) when the layers must run one by one. Sequential
// uses it for that layer pattern.
bool conv2d_relu_maxpool(const Tensor& input, Conv2d& conv, const MaxPool2d& pool, Tensor& out);

class Flatten : public Module {
public:
    Tensor forward(const Tensor& input) override;
    std::string name() const override { return "Flatten"; }
};

}  // namespace nn
}  // namespace engine

#endif  // ENGINE_CONV_HPP
