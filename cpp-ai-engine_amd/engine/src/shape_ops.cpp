// shape_ops.cpp -- Tensor::max(axis), slice, concat and stack on the device
// (the reference's src/tensor.cpp:383-552): the moves are ehip_copy_rows_f32
// runs of count x inner floats per outer index, the maximum and its gradient
// route are ehip_max_axis_f32 / _backward_f32. Every result is a move or a
// comparison, so it equals the reference's bit for bit.
#include <stdexcept>
#include <string>

#include "detail.hpp"

namespace engine {

using namespace detail;

namespace {

void check_axis(size_t axis, size_t ndim, const char* what, const std::string& shape_txt) {
    if (axis >= ndim)
        throw std::out_of_range(std::string(what) + ": axis " + std::to_string(axis) +
                                " does not exist in a tensor " + shape_txt + ".");
}

// (outer, axis_len, inner) of a shape around `axis`.
struct AxisView {
    size_t outer = 1, axis_len = 1, inner = 1;
};

AxisView axis_view(const std::vector<size_t>& shape, size_t axis) {
    AxisView v;
    for (size_t i = 0; i < axis; ++i) v.outer *= shape[i];
    v.axis_len = shape[axis];
    for (size_t i = axis + 1; i < shape.size(); ++i) v.inner *= shape[i];
    return v;
}

void copy_rows(const float* src, size_t src_pitch, float* dst, size_t dst_pitch, size_t rows,
               size_t len, const char* what) {
    hip::check(ehip_copy_rows_f32(src, int64_t(src_pitch), dst, int64_t(dst_pitch), int64_t(rows),
                                  int64_t(len), nullptr),
               what);
}

}  // namespace

Tensor Tensor::max(size_t axis, bool keepdim) const {
    check_axis(axis, ndim(), "max", shape_str());
    if (size() == 0) throw std::invalid_argument("max over an empty tensor.");
    const AxisView v = axis_view(shape(), axis);
    std::vector<size_t> out_shape = shape();
    if (keepdim) {
        out_shape[axis] = 1;
    } else {
        out_shape.erase(out_shape.begin() + static_cast<long>(axis));
        if (out_shape.empty()) out_shape.push_back(1);
    }
    const bool req_g = track(requires_grad());
    Tensor res(out_shape, 0.0f, req_g);
    DeviceInts argmax(v.outer * v.inner);
    hip::check(ehip_max_axis_f32(dptr(*this), dout(res), argmax.get(), int64_t(v.outer),
                                 int64_t(v.axis_len), int64_t(v.inner), nullptr),
               "max(axis)");
    if (req_g) {
        res.impl_->parents = {impl_};
        Tensor self_copy = *this;
        res.impl_->backward_fn = [self_copy, argmax, v](const Tensor& grad_out) mutable {
            // Only the maximum influenced the output.
            Tensor dX(self_copy.shape(), 0.0f, false);
            hip::check(ehip_max_axis_backward_f32(dptr(grad_out), argmax.get(), dout(dX),
                                                  int64_t(v.outer), int64_t(v.axis_len),
                                                  int64_t(v.inner), nullptr),
                       "max(axis) backward");
            self_copy.add_grad(dX);
        };
    }
    return res;
}

Tensor Tensor::slice(size_t axis, size_t start, size_t count) const {
    check_axis(axis, ndim(), "slice", shape_str());
    if (count == 0) throw std::invalid_argument("slice needs at least one element.");
    if (start + count > shape()[axis])
        throw std::out_of_range("slice [" + std::to_string(start) + ", " +
                                std::to_string(start + count) + ") runs off axis " +
                                std::to_string(axis) + " of a tensor " + shape_str() + ".");
    const AxisView v = axis_view(shape(), axis);
    std::vector<size_t> out_shape = shape();
    out_shape[axis] = count;
    const bool req_g = track(requires_grad());
    Tensor res(out_shape, 0.0f, req_g);
    copy_rows(dptr(*this) + start * v.inner, v.axis_len * v.inner, dout(res), count * v.inner,
              v.outer, count * v.inner, "slice");
    if (req_g) {
        res.impl_->parents = {impl_};
        Tensor self_copy = *this;
        res.impl_->backward_fn = [self_copy, v, start, count](const Tensor& grad_out) mutable {
            // The gradient goes back to its slot; the rest of the tensor gets zero.
            Tensor dX(self_copy.shape(), 0.0f, false);
            float* d = dX.storage().device_mut();  // the zeros, then the slot
            copy_rows(dptr(grad_out), count * v.inner, d + start * v.inner,
                      v.axis_len * v.inner, v.outer, count * v.inner, "slice backward");
            self_copy.add_grad(dX);
        };
    }
    return res;
}

Tensor Tensor::concat(const std::vector<Tensor>& parts, size_t axis) {
    if (parts.empty()) throw std::invalid_argument("concat needs at least one tensor.");
    const std::vector<size_t>& first = parts[0].shape();
    check_axis(axis, first.size(), "concat", parts[0].shape_str());
    size_t total_axis = 0;
    bool req_g = false;
    for (const Tensor& t : parts) {
        if (t.ndim() != first.size())
            throw std::invalid_argument("concat needs the same number of axes in every part.");
        for (size_t d = 0; d < first.size(); ++d)
            if (d != axis && t.shape()[d] != first[d])
                throw std::invalid_argument("concat: the parts may only differ along axis " +
                                            std::to_string(axis) + "; " + parts[0].shape_str() +
                                            " against " + t.shape_str() + ".");
        total_axis += t.shape()[axis];
        req_g = req_g || t.requires_grad();
    }
    req_g = track(req_g);
    std::vector<size_t> out_shape = first;
    out_shape[axis] = total_axis;
    Tensor res(out_shape, 0.0f, req_g);
    const AxisView out_view = axis_view(out_shape, axis);
    float* out = dout(res);
    size_t offset = 0;
    for (const Tensor& t : parts) {
        const size_t len = t.shape()[axis];
        copy_rows(dptr(t), len * out_view.inner, out + offset * out_view.inner,
                  out_view.axis_len * out_view.inner, out_view.outer, len * out_view.inner,
                  "concat");
        offset += len;
    }
    if (req_g) {
        std::vector<std::shared_ptr<TensorImpl>> parents;
        parents.reserve(parts.size());
        for (const Tensor& t : parts) parents.push_back(t.get_impl());
        res.impl_->parents = parents;
        std::vector<Tensor> copies = parts;
        res.impl_->backward_fn = [copies, axis, out_view](const Tensor& grad_out) mutable {
            // Each part receives the band of the gradient it contributed.
            size_t off = 0;
            for (Tensor& t : copies) {
                const size_t len = t.shape()[axis];
                if (t.requires_grad()) {
                    Tensor d(t.shape(), 0.0f, false);
                    copy_rows(dptr(grad_out) + off * out_view.inner,
                              out_view.axis_len * out_view.inner, dout(d), len * out_view.inner,
                              out_view.outer, len * out_view.inner, "concat backward");
                    t.add_grad(d);
                }
                off += len;
            }
        };
    }
    return res;
}

Tensor Tensor::stack(const std::vector<Tensor>& parts, size_t axis) {
    if (parts.empty()) throw std::invalid_argument("stack needs at least one tensor.");
    if (axis > parts[0].ndim())
        throw std::out_of_range("stack: axis " + std::to_string(axis) +
                                " does not fit in a tensor " + parts[0].shape_str() + ".");
    // Stacking is concatenating after inserting a size-1 axis into each part.
    std::vector<Tensor> expanded;
    expanded.reserve(parts.size());
    for (const Tensor& t : parts) {
        if (t.shape() != parts[0].shape())
            throw std::invalid_argument("stack needs every part to have the same shape: " +
                                        parts[0].shape_str() + " against " + t.shape_str() + ".");
        std::vector<size_t> s = t.shape();
        s.insert(s.begin() + static_cast<long>(axis), 1);
        expanded.push_back(t.reshape(s));
    }
    return concat(expanded, axis);
}

}  // namespace engine
