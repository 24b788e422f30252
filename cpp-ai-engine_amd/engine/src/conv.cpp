// conv.cpp -- im2col/col2im, Conv2d (direct kernels for narrow layers, im2col +
// one GEMM otherwise), MaxPool2d and Flatten (the reference's src/conv.cpp).
#include "engine/conv.hpp"

#include <atomic>
#include <cmath>
#include <stdexcept>

#include "detail.hpp"

namespace engine {
namespace nn {

using namespace detail;

namespace {

size_t output_size(size_t in_size, size_t kernel, size_t stride, size_t padding) {
    const size_t padded = in_size + 2 * padding;
    if (kernel > padded)
        throw std::invalid_argument("The kernel (" + std::to_string(kernel) +
                                    ") does not fit the padded input dimension (" +
                                    std::to_string(padded) + ").");
    return (padded - kernel) / stride + 1;
}

ehip_window_t window_of(const std::vector<size_t>& shape, const Window2d& w) {
    ehip_window_t s;
    s.batch = int64_t(shape[0]);
    s.channels = int64_t(shape[1]);
    s.height = int64_t(shape[2]);
    s.width = int64_t(shape[3]);
    s.kernel_h = int64_t(w.kernel_h);
    s.kernel_w = int64_t(w.kernel_w);
    s.stride = int64_t(w.stride);
    s.padding = int64_t(w.padding);
    s.out_h = int64_t(w.out_h(shape[2]));
    s.out_w = int64_t(w.out_w(shape[3]));
    return s;
}

// im2col as a graph node: its derivative is col2im (src/conv.cpp:234-253).
Tensor im2col_node(const Tensor& input, const Window2d& window) {
    Tensor cols = im2col(input, window);
    if (!autograd::grad_enabled() || !input.requires_grad()) return cols;
    cols.set_requires_grad(true);
    cols.get_impl()->parents = {input.get_impl()};
    Tensor input_copy = input;
    const std::vector<size_t> in_shape = input.shape();
    const Window2d win = window;
    cols.get_impl()->backward_fn = [input_copy, in_shape, win](const Tensor& g) mutable {
        input_copy.add_grad(col2im(g, in_shape, win));
    };
    return cols;
}

// The direct convolution node (narrow layers): one forward kernel, and a
// backward that makes the input gradient (when the input needs one) and the
// weight and bias gradients (one fused pass plus an ordered reduction). The
// values are those of the reference's composition (src/conv.cpp:280-338):
// forward and input gradient bit for bit, weight and bias gradients within
// the tolerance of their long sums.
Tensor conv2d_direct(const Tensor& input, const Tensor& weight, const Tensor& bias,
                     bool use_bias, const ehip_window_t& w) {
    const size_t co = weight.shape()[0];
    Tensor out({size_t(w.batch), co, size_t(w.out_h), size_t(w.out_w)}, 0.0f, false);
    hip::check(ehip_conv2d_forward_f32(dptr(input), dptr(weight), use_bias ? dptr(bias) : nullptr,
                                       dout(out), &w, int64_t(co), nullptr),
               "conv2d");
    const bool need_x = input.requires_grad();
    const bool need_w = weight.requires_grad();
    const bool need_b = use_bias && bias.requires_grad();
    if (!track(need_x || need_w || need_b)) return out;
    out.set_requires_grad(true);
    auto& parents = out.get_impl()->parents;
    if (need_x) parents.push_back(input.get_impl());
    if (need_w) parents.push_back(weight.get_impl());
    if (need_b) parents.push_back(bias.get_impl());
    Tensor x_copy = input, w_copy = weight, b_copy = bias;
    out.get_impl()->backward_fn = [x_copy, w_copy, b_copy, need_x, need_w, need_b,
                                   w](const Tensor& g) mutable {
        const int64_t co = int64_t(w_copy.shape()[0]);
        if (need_x) {
            Tensor dx(x_copy.shape(), 0.0f, false);
            hip::check(ehip_conv2d_backward_input_f32(dptr(g), dptr(w_copy), dout(dx), &w, co,
                                                      nullptr),
                       "conv2d backward input");
            x_copy.add_grad(dx);
        }
        if (need_w || need_b) {
            Tensor dw(w_copy.shape(), 0.0f, false);
            Tensor db;
            if (need_b) db = Tensor({size_t(co)}, 0.0f, false);
            hip::check(ehip_conv2d_backward_weight_f32(dptr(x_copy), dptr(g), dout(dw),
                                                       need_b ? dout(db) : nullptr, &w, co,
                                                       nullptr),
                       "conv2d backward weight");
            if (need_w) w_copy.add_grad(dw);
            if (need_b) b_copy.add_grad(db);
        }
    };
    return out;
}

std::atomic<bool> g_conv_igemm{true};

// The implicit-GEMM convolution node (wide layers): one forward launch (the
// bias in its epilogue) and one backward call making the input gradient and
// the weight and bias gradients that are needed. Same mathematics as the
// reference's composition (src/conv.cpp:280-338), summed in another order:
// within the K-term tolerance of its values.
Tensor conv2d_igemm(const Tensor& input, const Tensor& weight, const Tensor& bias, bool use_bias,
                    const ehip_window_t& w) {
    const size_t co = weight.shape()[0];
    Tensor out({size_t(w.batch), co, size_t(w.out_h), size_t(w.out_w)}, 0.0f, false);
    hip::check(ehip_conv2d_igemm_f32(dptr(input), dptr(weight), use_bias ? dptr(bias) : nullptr,
                                     dout(out), &w, int64_t(co), nullptr),
               "conv2d (implicit GEMM)");
    const bool need_x = input.requires_grad();
    const bool need_w = weight.requires_grad();
    const bool need_b = use_bias && bias.requires_grad();
    if (!track(need_x || need_w || need_b)) return out;
    out.set_requires_grad(true);
    auto& parents = out.get_impl()->parents;
    if (need_x) parents.push_back(input.get_impl());
    if (need_w) parents.push_back(weight.get_impl());
    if (need_b) parents.push_back(bias.get_impl());
    Tensor x_copy = input, w_copy = weight, b_copy = bias;
    out.get_impl()->backward_fn = [x_copy, w_copy, b_copy, need_x, need_w, need_b,
                                   w](const Tensor& g) mutable {
        Tensor dx, dw, db;
        if (need_x) dx = Tensor(x_copy.shape(), 0.0f, false);
        if (need_w) dw = Tensor(w_copy.shape(), 0.0f, false);
        if (need_b) db = Tensor({w_copy.shape()[0]}, 0.0f, false);
        hip::check(ehip_conv2d_igemm_backward_f32(
                       dptr(x_copy), dptr(w_copy), dptr(g), need_x ? dout(dx) : nullptr,
                       need_w ? dout(dw) : nullptr, need_b ? dout(db) : nullptr, &w,
                       int64_t(w_copy.shape()[0]), nullptr),
                   "conv2d backward (implicit GEMM)");
        if (need_x) x_copy.add_grad(dx);
        if (need_w) w_copy.add_grad(dw);
        if (need_b) b_copy.add_grad(db);
    };
    return out;
}

}  // namespace

void set_conv_implicit_gemm(bool on) { g_conv_igemm.store(on); }
bool conv_implicit_gemm() { return g_conv_igemm.load(); }

size_t Window2d::out_h(size_t in_h) const { return output_size(in_h, kernel_h, stride, padding); }
size_t Window2d::out_w(size_t in_w) const { return output_size(in_w, kernel_w, stride, padding); }

void Window2d::validate(size_t in_h, size_t in_w) const {
    if (kernel_h == 0 || kernel_w == 0 || stride == 0)
        throw std::invalid_argument("The window needs a kernel and a stride greater than zero.");
    (void)out_h(in_h);
    (void)out_w(in_w);
}

Tensor im2col(const Tensor& input, const Window2d& window) {
    if (input.ndim() != 4)
        throw std::invalid_argument("im2col expects (N, C, H, W), received " + input.shape_str() + ".");
    window.validate(input.shape()[2], input.shape()[3]);
    const ehip_window_t w = window_of(input.shape(), window);
    Tensor cols({size_t(w.batch * w.out_h * w.out_w), size_t(w.channels * w.kernel_h * w.kernel_w)},
                0.0f, false);
    hip::check(ehip_im2col_f32(dptr(input), dout(cols), &w, nullptr), "im2col");
    return cols;
}

Tensor col2im(const Tensor& cols, const std::vector<size_t>& input_shape, const Window2d& window) {
    if (input_shape.size() != 4) throw std::invalid_argument("col2im expects a 4D input shape.");
    window.validate(input_shape[2], input_shape[3]);
    const ehip_window_t w = window_of(input_shape, window);
    if (cols.size() != size_t(w.batch * w.out_h * w.out_w * w.channels * w.kernel_h * w.kernel_w))
        throw std::invalid_argument("col2im: columns " + cols.shape_str() +
                                    " do not match the window over the input.");
    Tensor x(input_shape, 0.0f, false);
    hip::check(ehip_col2im_f32(dptr(cols), dout(x), &w, nullptr), "col2im");
    return x;
}

// Xavier-uniform over (fan_in + fan_out) x receptive field, zero bias
// (src/conv.cpp:257-277).
Conv2d::Conv2d(size_t in_channels, size_t out_channels, const Window2d& window, bool use_bias)
    : in_channels_(in_channels), out_channels_(out_channels), window_(window), use_bias_(use_bias) {
    if (in_channels == 0 || out_channels == 0)
        throw std::invalid_argument("Conv2d requires in_channels and out_channels greater than zero.");
    if (window_.kernel_h == 0 || window_.kernel_w == 0 || window_.stride == 0)
        throw std::invalid_argument("Conv2d requires a kernel and a stride greater than zero.");
    const size_t receptive = window_.kernel_h * window_.kernel_w;
    const float fan_in = static_cast<float>(in_channels * receptive);
    const float fan_out = static_cast<float>(out_channels * receptive);
    const float limit = std::sqrt(6.0f / (fan_in + fan_out));
    autograd::NoGradGuard no_grad;
    weight_ = Tensor::rand({out_channels, in_channels, window_.kernel_h, window_.kernel_w}, -limit,
                           limit, true);
    bias_ = Tensor({out_channels}, 0.0f, use_bias);
}

// Narrow layers take the direct kernels, wider ones the implicit GEMM. With
// that switched off, or for a layer beyond the implicit GEMM's 32-bit index
// and batch limits, wide layers compose as the reference does: im2col ->
// cols (W reshaped to (outC, K))^T -> + bias -> (N, outC, oH, oW)
// (src/conv.cpp:280-338), the product on MFMA reading W in place through the
// GEMM's transposed mode, so its derivative needs no transpose either.
Tensor Conv2d::forward(const Tensor& input) {
    if (input.ndim() != 4)
        throw std::invalid_argument("Conv2d expects a 4D volume (N, C, H, W), received " +
                                    input.shape_str() + ".");
    if (input.shape()[1] != in_channels_)
        throw std::invalid_argument("Conv2d with in_channels=" + std::to_string(in_channels_) +
                                    " received an input " + input.shape_str() + ".");
    const size_t N = input.shape()[0], H = input.shape()[2], W = input.shape()[3];
    window_.validate(H, W);
    const size_t oH = window_.out_h(H), oW = window_.out_w(W);
    const size_t K = in_channels_ * window_.kernel_h * window_.kernel_w;
    const ehip_window_t w = window_of(input.shape(), window_);
    if (ehip_conv2d_direct_supported(&w, int64_t(out_channels_)))
        return conv2d_direct(input, weight_, bias_, use_bias_, w);
    if (conv_implicit_gemm() && ehip_conv2d_igemm_supported(&w, int64_t(out_channels_)))
        return conv2d_igemm(input, weight_, bias_, use_bias_, w);
    Tensor cols = im2col_node(input, window_);
    Tensor out = ops::matmul_nt(cols, weight_.reshape({out_channels_, K}));
    if (use_bias_) out = out + bias_;
    return out.reshape({N, oH * oW, out_channels_})
        .permute({0, 2, 1})
        .reshape({N, out_channels_, oH, oW});
}

std::vector<Tensor> Conv2d::parameters() {
    if (use_bias_) return {weight_, bias_};
    return {weight_};
}

std::string Conv2d::name() const {
    return "Conv2d(" + std::to_string(in_channels_) + " -> " + std::to_string(out_channels_) +
           ", k=" + std::to_string(window_.kernel_h) + "x" + std::to_string(window_.kernel_w) +
           ", s=" + std::to_string(window_.stride) + ", p=" + std::to_string(window_.padding) + ")";
}

MaxPool2d::MaxPool2d(const Window2d& window) : window_(window) {
    if (window_.padding >= window_.kernel_h || window_.padding >= window_.kernel_w)
        throw std::invalid_argument("MaxPool2d requires padding smaller than the kernel.");
}

MaxPool2d::MaxPool2d(size_t kernel, size_t stride) : window_(kernel, kernel, stride, 0) {}

// Window max with the int32 index of the first strict maximum; the backward
// gathers per input pixel (src/conv.cpp:367-473).
Tensor MaxPool2d::forward(const Tensor& input) {
    if (input.ndim() != 4)
        throw std::invalid_argument("MaxPool2d expects a 4D volume (N, C, H, W), received " +
                                    input.shape_str() + ".");
    window_.validate(input.shape()[2], input.shape()[3]);
    const ehip_window_t w = window_of(input.shape(), window_);
    Tensor out({size_t(w.batch), size_t(w.channels), size_t(w.out_h), size_t(w.out_w)}, 0.0f, false);
    auto argmax = std::make_shared<DeviceInts>(out.size());
    hip::check(ehip_maxpool_f32(dptr(input), dout(out), argmax->get(), &w, nullptr), "maxpool");
    if (track(input.requires_grad())) {
        out.set_requires_grad(true);
        out.get_impl()->parents = {input.get_impl()};
        Tensor input_copy = input;
        out.get_impl()->backward_fn = [input_copy, argmax, w](const Tensor& g) mutable {
            Tensor dX(input_copy.shape(), 0.0f, false);
            hip::check(ehip_maxpool_backward_f32(argmax->get(), dptr(g), dout(dX), &w, nullptr),
                       "maxpool backward");
            input_copy.add_grad(dX);
        };
    }
    return out;
}

bool conv2d_relu_maxpool(const Tensor& input, Conv2d& conv, const MaxPool2d& pool, Tensor& out) {
    if (input.ndim() != 4 || input.shape()[1] * conv.window().kernel_h * conv.window().kernel_w *
                                     conv.out_channels() !=
                                 conv.weight().size())
        return false;
    const size_t H = input.shape()[2], W = input.shape()[3];
    conv.window().validate(H, W);
    const ehip_window_t cw = window_of(input.shape(), conv.window());
    const size_t co = conv.out_channels();
    const std::vector<size_t> conv_shape{size_t(cw.batch), co, size_t(cw.out_h), size_t(cw.out_w)};
    const Window2d& pwin = pool.window();
    if (pwin.kernel_h != pwin.kernel_w || pwin.kernel_h != pwin.stride || pwin.padding != 0)
        return false;
    if (pwin.kernel_h > conv_shape[2] || pwin.kernel_w > conv_shape[3]) return false;
    const ehip_window_t pw = window_of(conv_shape, pwin);
    if (!ehip_conv2d_relu_maxpool_supported(&cw, int64_t(co), &pw)) return false;
    Tensor& weight = conv.weight();
    Tensor& bias = conv.bias();
    const bool use_bias = conv.has_bias();
    Tensor res({size_t(pw.batch), co, size_t(pw.out_h), size_t(pw.out_w)}, 0.0f, false);
    auto argmax = std::make_shared<DeviceInts>(res.size());
    hip::check(ehip_conv2d_relu_maxpool_f32(dptr(input), dptr(weight),
                                            use_bias ? dptr(bias) : nullptr, dout(res),
                                            argmax->get(), &cw, int64_t(co), &pw, nullptr),
               "conv2d_relu_maxpool");
    const bool need_x = input.requires_grad();
    const bool need_w = weight.requires_grad();
    const bool need_b = use_bias && bias.requires_grad();
    if (track(need_x || need_w || need_b)) {
        res.set_requires_grad(true);
        auto& parents = res.get_impl()->parents;
        if (need_x) parents.push_back(input.get_impl());
        if (need_w) parents.push_back(weight.get_impl());
        if (need_b) parents.push_back(bias.get_impl());
        Tensor x_copy = input, w_copy = weight, b_copy = bias;
        // The pooled values are read through their storage: holding the output
        // tensor itself inside its own backward would keep it alive forever.
        Storage pooled = res.storage().share();
        res.get_impl()->backward_fn = [x_copy, w_copy, b_copy, pooled, argmax, cw, pw, need_x,
                                       need_w, need_b](const Tensor& g) mutable {
            const int64_t co = int64_t(w_copy.shape()[0]);
            Tensor dx, dw, db;
            if (need_x) dx = Tensor(x_copy.shape(), 0.0f, false);
            if (need_w || need_b) dw = Tensor(w_copy.shape(), 0.0f, false);
            if (need_b) db = Tensor({size_t(co)}, 0.0f, false);
            // With fused nodes, a layer whose weight (and bias) gradients will be
            // adopted by add_grad writes only its tile partials now; the sums of
            // every such layer run in one launch at the end of backward (the same
            // bits as the one-call backward below).
            int64_t chunks = 0;
            const int64_t nparts =
                fused_nodes() && need_w && detail::grad_adoptable(w_copy) &&
                        (!need_b || detail::grad_adoptable(b_copy))
                    ? ehip_conv2d_relu_maxpool_partials(&cw, co, &pw, need_x ? 1 : 0, &chunks)
                    : 0;
            if (nparts > 0) {
                Tensor part({size_t(nparts)}, 0.0f, false);
                hip::check(ehip_conv2d_relu_maxpool_backward_partials_f32(
                               dptr(x_copy), dptr(w_copy), dptr(g), pooled.device(),
                               argmax->get(), need_x ? dout(dx) : nullptr, dout(part), chunks,
                               &cw, co, &pw, nullptr),
                           "conv2d_relu_maxpool backward");
                const ehip_conv_reduce_t job{dptr(part), chunks, co,
                                             int64_t(w_copy.size()) / co, dout(dw),
                                             need_b ? dout(db) : nullptr};
                detail::defer_conv_reduce(job, part);
                if (need_x) x_copy.add_grad(dx);
                w_copy.add_grad(dw);
                if (need_b) b_copy.add_grad(db);
                detail::defer_conv_output(w_copy, dw);
                if (need_b) detail::defer_conv_output(b_copy, db);
                return;
            }
            hip::check(ehip_conv2d_relu_maxpool_backward_f32(
                           dptr(x_copy), dptr(w_copy), dptr(g), pooled.device(), argmax->get(),
                           need_x ? dout(dx) : nullptr, (need_w || need_b) ? dout(dw) : nullptr,
                           need_b ? dout(db) : nullptr, &cw, co, &pw, nullptr),
                       "conv2d_relu_maxpool backward");
            if (need_x) x_copy.add_grad(dx);
            if (need_w) w_copy.add_grad(dw);
            if (need_b) b_copy.add_grad(db);
        };
    }
    out = res;
    return true;
}

std::string MaxPool2d::name() const {
    return "MaxPool2d(k=" + std::to_string(window_.kernel_h) + "x" +
           std::to_string(window_.kernel_w) + ", s=" + std::to_string(window_.stride) + ")";
}

Tensor Flatten::forward(const Tensor& input) {
    if (input.ndim() < 2)
        throw std::invalid_argument("Flatten expects at least 2 dimensions, received " +
                                    input.shape_str() + ".");
    const size_t N = input.shape()[0];
    if (N == 0) throw std::invalid_argument("Flatten received an empty batch.");
    return input.reshape({N, input.size() / N});
}

}  // namespace nn
}  // namespace engine
