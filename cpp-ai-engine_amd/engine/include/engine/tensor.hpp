// tensor.hpp -- the engine's N-d fp32 Tensor, device-resident on MI355X.
//
// The public API mirrors the reference's include/engine/tensor.hpp:28-203
// (same names, argument meaning and exceptions) so that models written
// against the reference compile against this engine. Every operation runs as
// a HIP kernel through the C ABI of include/ehip.h; there is no CPU compute
// path, and an operation the device refuses throws std::runtime_error.
// data() is the door to the host copy: it downloads when the host copy is
// stale.
//
// Not provided (not on the training path of any configuration this backend
// serves): slice, concat, stack and max(axis).
#ifndef ENGINE_TENSOR_HPP
#define ENGINE_TENSOR_HPP

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "engine/detail/tensor_impl.hpp"

namespace engine {

// Seeds the global std::mt19937 used by rand()/randn() and layer
// initialisation (the reference's src/tensor.cpp:24-31).
void manual_seed(uint64_t seed);

// The device generator behind Dropout: its seed (set by manual_seed, 5489
// until then) and the counter offset of the next draw; device_rng_take(n)
// returns the offset for n values and advances it past them (rounded up to a
// whole Philox block of four).
struct DeviceRng {
    uint64_t seed;
    uint64_t offset;
};
DeviceRng device_rng_take(size_t n);

class Tensor {
private:
    std::shared_ptr<TensorImpl> impl_;
    explicit Tensor(std::shared_ptr<TensorImpl> impl);

public:
    Tensor();
    explicit Tensor(const std::vector<size_t>& shape, float fill_value = 0.0f,
                    bool requires_grad = false);
    Tensor(const std::vector<size_t>& shape, const std::vector<float>& data,
           bool requires_grad = false);

    static Tensor from_impl(std::shared_ptr<TensorImpl> impl);

    static Tensor zeros(const std::vector<size_t>& shape, bool requires_grad = false);
    static Tensor ones(const std::vector<size_t>& shape, bool requires_grad = false);
    static Tensor rand(const std::vector<size_t>& shape, float min_val = -1.0f,
                       float max_val = 1.0f, bool requires_grad = false);
    static Tensor randn(const std::vector<size_t>& shape, float mean = 0.0f, float stddev = 1.0f,
                        bool requires_grad = false);

    [[nodiscard]] bool requires_grad() const;
    void set_requires_grad(bool requires_grad);
    [[nodiscard]] Tensor grad() const;
    [[nodiscard]] bool has_grad() const;
    void zero_grad();
    void add_grad(const Tensor& g);
    void backward();
    void backward(const Tensor& grad_output);

    [[nodiscard]] Storage& storage() noexcept { return impl_->storage; }
    [[nodiscard]] const Storage& storage() const noexcept { return impl_->storage; }
    [[nodiscard]] const std::shared_ptr<TensorImpl>& get_impl() const noexcept { return impl_; }

    [[nodiscard]] size_t get_flat_index(const std::vector<size_t>& indices) const;
    float& operator()(const std::vector<size_t>& indices);
    [[nodiscard]] const float& operator()(const std::vector<size_t>& indices) const;
    float& operator()(size_t row, size_t col);
    [[nodiscard]] const float& operator()(size_t row, size_t col) const;
    float& at(size_t flat_index);
    [[nodiscard]] const float& at(size_t flat_index) const;

    [[nodiscard]] const std::vector<size_t>& shape() const;
    [[nodiscard]] const std::vector<size_t>& strides() const;
    [[nodiscard]] const float* data() const;
    [[nodiscard]] float* data();
    [[nodiscard]] std::vector<float> to_vector() const;
    [[nodiscard]] size_t size() const;
    [[nodiscard]] size_t ndim() const;
    [[nodiscard]] std::string shape_str() const;

    // Element-wise with suffix broadcast of the right operand.
    [[nodiscard]] Tensor operator+(const Tensor& other) const;
    [[nodiscard]] Tensor operator-(const Tensor& other) const;
    [[nodiscard]] Tensor operator*(const Tensor& other) const;
    [[nodiscard]] Tensor operator/(const Tensor& other) const;

    [[nodiscard]] Tensor operator+(float scalar) const;
    [[nodiscard]] Tensor operator-(float scalar) const;
    [[nodiscard]] Tensor operator*(float scalar) const;
    [[nodiscard]] Tensor operator/(float scalar) const;

    [[nodiscard]] Tensor matmul(const Tensor& other) const;
    [[nodiscard]] Tensor transpose() const;
    [[nodiscard]] Tensor permute(const std::vector<size_t>& order) const;
    [[nodiscard]] Tensor relu() const;
    [[nodiscard]] Tensor softmax() const;
    [[nodiscard]] Tensor reshape(const std::vector<size_t>& new_shape) const;
    [[nodiscard]] Tensor sum() const;
    [[nodiscard]] Tensor mean() const;
    [[nodiscard]] Tensor sum(size_t axis, bool keepdim = false) const;
    [[nodiscard]] Tensor mean(size_t axis, bool keepdim = false) const;
    [[nodiscard]] Tensor max(size_t axis, bool keepdim = false) const;

    // Contiguous sub-tensor along an axis: [start, start + count).
    [[nodiscard]] Tensor slice(size_t axis, size_t start, size_t count) const;
    // Concatenates along an axis (every other dimension must match); stacks
    // along a new axis.
    [[nodiscard]] static Tensor concat(const std::vector<Tensor>& parts, size_t axis);
    [[nodiscard]] static Tensor stack(const std::vector<Tensor>& parts, size_t axis = 0);

    [[nodiscard]] Tensor select_rows(const std::vector<size_t>& indices) const;
    [[nodiscard]] Tensor detach() const;

    void print(const std::string& name = "") const;
};

[[nodiscard]] Tensor operator+(float scalar, const Tensor& t);
[[nodiscard]] Tensor operator-(float scalar, const Tensor& t);
[[nodiscard]] Tensor operator*(float scalar, const Tensor& t);

namespace ops {

// Products the backward passes and attention use without materialising a
// transpose: A^T B, A B^T (both operands 2-D or batched like matmul). They
// are graph nodes with their own derivatives, equal in value to
// a.transpose().matmul(b) and a.matmul(b.transpose()).
Tensor matmul_tn(const Tensor& a, const Tensor& b);
Tensor matmul_nt(const Tensor& a, const Tensor& b);

// x (rows, in) . w (in, out) + bias as one node: the broadcast bias add runs
// in the product's epilogue. Equal bit for bit to x.matmul(w) + bias (the
// reference's Linear::forward, src/nn.cpp:119-122). bias is (out) or
// (1, out), or null for no bias. With a residual (any shape of rows * out
// elements), the node is residual + (x w + bias) under the residual's shape,
// the add in the same epilogue: equal bit for bit to
// residual + linear(x, w, bias).reshape(residual.shape()).
Tensor linear(const Tensor& x, const Tensor& w, const Tensor* bias,
              const Tensor* residual = nullptr);

// linear(x, w[i], bias[i]) for several layers over one input (attention's
// query, key and value projections), the products in one launch where the
// library groups them (ehip_gemm_batch_f32); each output is linear()'s node
// with linear()'s bits. bias[i] may be null.
std::vector<Tensor> linear_many(const Tensor& x, const std::vector<const Tensor*>& w,
                                const std::vector<const Tensor*>& bias);

// relu(x w1 + b1) w2 + b2 as one node (TransformerBlock's feed-forward,
// src/transformer.cpp:409-414): the biases and the ReLU in the products'
// epilogues, only the ReLU output kept (its backward reads the mask from
// it). Equal bit for bit to the composed nodes. x is 2-D. A residual is
// added as in linear().
Tensor feed_forward_relu(const Tensor& x, const Tensor& w1, const Tensor& b1, const Tensor& w2,
                         const Tensor& b2, const Tensor* residual = nullptr);

}  // namespace ops

}  // namespace engine

#endif  // ENGINE_TENSOR_HPP
