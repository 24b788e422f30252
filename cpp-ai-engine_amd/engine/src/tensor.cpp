// tensor.cpp -- Tensor construction, gradients, host access, reductions and
// the row gather (the reference's src/tensor.cpp). Arithmetic and layout
// operations live in tensor_ops.cpp.
#include <algorithm>
#include <cmath>
#include <iomanip>
#include <iostream>
#include <random>
#include <sstream>
#include <stdexcept>

#include "detail.hpp"
#include "engine/autograd.hpp"
#include "engine/tensor.hpp"

namespace engine {

using namespace detail;

std::mt19937& global_rng() {
    static std::mt19937 gen(std::random_device{}());
    return gen;
}

namespace {
DeviceRng& device_rng() {
    static DeviceRng g{5489u, 0u};
    return g;
}
}  // namespace

DeviceRng device_rng_take(size_t n) {
    DeviceRng& g = device_rng();
    const DeviceRng now = g;
    g.offset += (uint64_t(n) + 3) / 4 * 4;
    return now;
}

void manual_seed(uint64_t seed) {
    device_rng() = DeviceRng{seed, 0u};
    global_rng().seed(static_cast<std::mt19937::result_type>(seed));
}

// ------------------------------------------------------------------ impl

TensorImpl::TensorImpl(const std::vector<size_t>& s, float fill_val, bool req_grad)
    : shape(s), requires_grad(req_grad) {
    compute_strides();
    storage = Storage(product(shape), fill_val);
}

TensorImpl::TensorImpl(const std::vector<size_t>& s, const std::vector<float>& d, bool req_grad)
    : shape(s), requires_grad(req_grad) {
    compute_strides();
    if (d.size() != product(shape))
        throw std::invalid_argument("Data size (" + std::to_string(d.size()) +
                                    ") does not match the shape's element count (" +
                                    std::to_string(product(shape)) + ").");
    storage = Storage(d);
}

void TensorImpl::compute_strides() {
    strides.assign(shape.size(), 1);
    for (size_t i = shape.size(); i-- > 1;) strides[i - 1] = strides[i] * shape[i];
}

size_t TensorImpl::get_flat_index(const std::vector<size_t>& indices) const {
    if (indices.size() != shape.size())
        throw std::invalid_argument("Wrong number of indices for the tensor.");
    size_t flat = 0;
    for (size_t i = 0; i < indices.size(); ++i) {
        if (indices[i] >= shape[i]) throw std::out_of_range("Index out of range.");
        flat += indices[i] * strides[i];
    }
    return flat;
}

// ------------------------------------------------------------------ construction

Tensor::Tensor() : impl_(std::make_shared<TensorImpl>(std::vector<size_t>{0}, 0.0f, false)) {}

Tensor::Tensor(std::shared_ptr<TensorImpl> impl) : impl_(std::move(impl)) {
    if (!impl_) throw std::invalid_argument("Cannot construct a Tensor over a null implementation.");
}

Tensor::Tensor(const std::vector<size_t>& shape, float fill_value, bool requires_grad)
    : impl_(std::make_shared<TensorImpl>(shape, fill_value, requires_grad)) {}

Tensor::Tensor(const std::vector<size_t>& shape, const std::vector<float>& data, bool requires_grad)
    : impl_(std::make_shared<TensorImpl>(shape, data, requires_grad)) {}

Tensor Tensor::from_impl(std::shared_ptr<TensorImpl> impl) { return Tensor(std::move(impl)); }

Tensor Tensor::zeros(const std::vector<size_t>& shape, bool requires_grad) {
    return Tensor(shape, 0.0f, requires_grad);
}

Tensor Tensor::ones(const std::vector<size_t>& shape, bool requires_grad) {
    return Tensor(shape, 1.0f, requires_grad);
}

// Drawn on the host from the global generator, in element order, exactly as
// the reference does (src/tensor.cpp:117-136), so seeded initialisations match.
Tensor Tensor::rand(const std::vector<size_t>& shape, float min_val, float max_val,
                    bool requires_grad) {
    std::vector<float> v(product(shape));
    std::uniform_real_distribution<float> dis(min_val, max_val);
    for (float& x : v) x = dis(global_rng());
    return Tensor(shape, v, requires_grad);
}

Tensor Tensor::randn(const std::vector<size_t>& shape, float mean, float stddev,
                     bool requires_grad) {
    std::vector<float> v(product(shape));
    std::normal_distribution<float> dis(mean, stddev);
    for (float& x : v) x = dis(global_rng());
    return Tensor(shape, v, requires_grad);
}

// ------------------------------------------------------------------ gradients

bool Tensor::requires_grad() const { return impl_->requires_grad; }
void Tensor::set_requires_grad(bool req_grad) { impl_->requires_grad = req_grad; }

Tensor Tensor::grad() const {
    if (!impl_->grad) throw std::runtime_error("The tensor has no computed gradient.");
    if (deferred_pending()) flush_deferred();
    return Tensor(impl_->grad);
}

bool Tensor::has_grad() const { return impl_->grad != nullptr; }

// Lazy: the next add_grad initialises the zeroed gradient without a fill
// (src/tensor.cpp:157-166 assigns zeros without copying either). A shared
// gradient buffer is replaced rather than zeroed, so no other holder sees it.
void Tensor::zero_grad() {
    if (!impl_->grad) return;
    // A queued sum may still write this buffer: run it before the buffer can
    // be released or reused.
    if (deferred_pending()) flush_deferred();
    Storage& s = impl_->grad->storage;
    if (s.exclusive())
        s.assign(0.0f);
    else
        s = Storage(s.size(), 0.0f);
}

// The first write is 0 + g, later writes grad += g (src/tensor.cpp:168-203).
//
// A first write from a temporary that nothing else references adopts its
// buffer instead of copying it (every gradient edge of the backward pass is
// such a temporary); the only difference from 0 + g is that a -0.0 element
// stays -0.0. Accumulating into a buffer that is still shared writes the sum
// into a fresh buffer (copy on write), so adopted buffers are never mutated
// under another holder.
void Tensor::add_grad(const Tensor& g) {
    if (!requires_grad()) return;
    if (g.shape() != shape())
        throw std::invalid_argument("Gradient shape " + g.shape_str() +
                                    " incompatible with the tensor's " + shape_str() + ".");
    detail::add_grad_reshaped(*this, g);
}

void detail::add_grad_reshaped(Tensor& target, const Tensor& g) {
    const std::shared_ptr<TensorImpl>& impl_ = target.get_impl();
    if (!impl_->requires_grad) return;
    if (g.size() != target.size())
        throw std::invalid_argument("Gradient of " + std::to_string(g.size()) +
                                    " elements for a tensor of " + std::to_string(target.size()) +
                                    ".");
    const std::vector<size_t>& shape = impl_->shape;
    const size_t n = target.size();
    const bool initialize = !impl_->grad || impl_->grad->storage.pending_zero();
    if (initialize && g.get_impl().use_count() == 1 && g.storage().exclusive() &&
        g.storage().resident_on_device()) {
        if (!impl_->grad) {
            impl_->grad = std::make_shared<TensorImpl>();
            impl_->grad->shape = shape;
            impl_->grad->compute_strides();
        }
        impl_->grad->storage = g.storage().share();
        return;
    }
    // Accumulating reads the existing gradient and g and writes the gradient:
    // finish first queued work that writes either, or reads the gradient.
    if (impl_->grad) settle_deferred(impl_->grad->storage);
    if (deferred_pending() && deferred_writes(g.storage())) flush_deferred();
    if (!impl_->grad) impl_->grad = std::make_shared<TensorImpl>(shape, 0.0f, false);
    Storage& acc = impl_->grad->storage;
    const float* src = g.storage().device();
    if (!initialize && !acc.exclusive()) {
        Storage sum(acc.size(), 0.0f);
        hip::check(ehip_binary_f32(EHIP_ADD, acc.device(), src, sum.device_write(), int64_t(n), 1,
                                   nullptr),
                   "add_grad");
        acc = sum;
        return;
    }
    float* dst = initialize ? acc.device_write() : acc.device_mut();
    hip::check(ehip_accumulate_grad_f32(dst, src, int64_t(n), initialize ? 1 : 0, nullptr),
               "add_grad");
}

float* detail::grad_in_place(Tensor& target) {
    const std::shared_ptr<TensorImpl>& impl_ = target.get_impl();
    if (!impl_ || !impl_->requires_grad || !impl_->grad) return nullptr;
    // The product reads the existing gradient and adds into it: finish first
    // queued work that writes or reads it (the queue holds a view of those
    // buffers, so their exclusivity test below is only meaningful once it has
    // run).
    settle_deferred(impl_->grad->storage);
    Storage& acc = impl_->grad->storage;
    if (acc.pending_zero() || !acc.exclusive() || acc.size() != target.size()) return nullptr;
    return acc.device_mut();
}

void Tensor::backward() { autograd::backward(*this); }

void Tensor::backward(const Tensor& grad_output) {
    if (grad_output.shape() != shape())
        throw std::invalid_argument("Initial gradient shape " + grad_output.shape_str() +
                                    " incompatible with the root's " + shape_str() + ".");
    auto g = std::make_shared<TensorImpl>();
    g->shape = shape();
    g->compute_strides();
    g->storage = grad_output.storage().clone();
    impl_->grad = g;
    autograd::backward(*this);
}

// ------------------------------------------------------------------ host access

size_t Tensor::get_flat_index(const std::vector<size_t>& indices) const {
    return impl_->get_flat_index(indices);
}
float& Tensor::operator()(const std::vector<size_t>& indices) {
    return impl_->storage.host_mut()[get_flat_index(indices)];
}
const float& Tensor::operator()(const std::vector<size_t>& indices) const {
    return impl_->storage.host()[get_flat_index(indices)];
}
float& Tensor::operator()(size_t row, size_t col) { return (*this)({row, col}); }
const float& Tensor::operator()(size_t row, size_t col) const { return (*this)({row, col}); }
float& Tensor::at(size_t i) {
    if (i >= size()) throw std::out_of_range("Flat index out of range.");
    return impl_->storage.host_mut()[i];
}
const float& Tensor::at(size_t i) const {
    if (i >= size()) throw std::out_of_range("Flat index out of range.");
    return impl_->storage.host()[i];
}

const std::vector<size_t>& Tensor::shape() const { return impl_->shape; }
const std::vector<size_t>& Tensor::strides() const { return impl_->strides; }
const float* Tensor::data() const { return impl_->storage.host().data(); }
float* Tensor::data() { return impl_->storage.host_mut().data(); }
std::vector<float> Tensor::to_vector() const { return impl_->storage.host(); }
size_t Tensor::size() const { return impl_->storage.size(); }
size_t Tensor::ndim() const { return impl_->shape.size(); }

std::string Tensor::shape_str() const {
    std::ostringstream os;
    os << "(";
    for (size_t i = 0; i < shape().size(); ++i) os << shape()[i] << (i + 1 < ndim() ? ", " : "");
    os << ")";
    return os.str();
}

// The reference's console format (src/tensor_ops.cpp:762-805), so programs
// that print tensors print the same text: the shape in brackets, then 1-D as
// one bracketed row, 2-D as bracketed rows, higher ranks as one block broken
// at the last axis, values in width 8 with 4 decimals; the gradient follows
// when there is one.
void Tensor::print(const std::string& name) const {
    if (!name.empty()) std::cout << name << " = ";
    std::cout << "Tensor(shape=[";
    const std::vector<size_t>& sh = shape();
    for (size_t i = 0; i < sh.size(); ++i) std::cout << (i ? ", " : "") << sh[i];
    std::cout << "], requires_grad=" << (requires_grad() ? "true" : "false") << ")\n";
    const float* v = data();
    const auto value = [&](size_t i) -> std::ostream& {
        return std::cout << std::setw(8) << std::fixed << std::setprecision(4) << v[i];
    };
    if (sh.size() == 1) {
        std::cout << "[";
        for (size_t i = 0; i < sh[0]; ++i) value(i) << (i + 1 < sh[0] ? ", " : "");
        std::cout << "]\n";
    } else if (sh.size() == 2) {
        std::cout << "[\n";
        for (size_t r = 0; r < sh[0]; ++r) {
            std::cout << "  [";
            for (size_t c = 0; c < sh[1]; ++c) value(r * sh[1] + c) << (c + 1 < sh[1] ? ", " : "");
            std::cout << "]\n";
        }
        std::cout << "]\n";
    } else if (size() > 0) {
        std::cout << "[ ";
        for (size_t i = 0; i < size(); ++i) {
            value(i) << " ";
            if ((i + 1) % sh.back() == 0 && i + 1 < size()) std::cout << "\n  ";
        }
        std::cout << "]\n";
    } else {
        std::cout << "[]\n";
    }
    if (has_grad()) {
        std::cout << "  grad = \n";
        grad().print("  gradientes");
    }
    std::cout << "\n";
}

// ------------------------------------------------------------------ reductions

// Sum in double over the whole buffer (src/tensor_ops.cpp:679-703); the float
// cast is written on the device, so nothing synchronises here.
Tensor Tensor::sum() const {
    const bool req_g = track(requires_grad());
    Tensor res({1}, 0.0f, req_g);
    hip::check(ehip_reduce_sum_f32(dptr(*this), int64_t(size()), 0, nullptr, dout(res), nullptr),
               "sum");
    if (req_g) {
        res.impl_->parents = {impl_};
        Tensor self_copy = *this;
        res.impl_->backward_fn = [self_copy](const Tensor& grad_out) mutable {
            self_copy.add_grad(broadcast_middle(grad_out, self_copy.shape(), 1, self_copy.size(), 1));
        };
    }
    return res;
}

Tensor Tensor::mean() const {
    if (size() == 0) throw std::invalid_argument("Cannot take the mean of an empty tensor.");
    return sum() * (1.0f / static_cast<float>(size()));
}

Tensor Tensor::sum(size_t axis, bool keepdim) const {
    if (axis >= ndim())
        throw std::invalid_argument("sum: axis " + std::to_string(axis) + " out of range for " +
                                    shape_str() + ".");
    size_t outer = 1, inner = 1;
    for (size_t i = 0; i < axis; ++i) outer *= shape()[i];
    for (size_t i = axis + 1; i < ndim(); ++i) inner *= shape()[i];
    const size_t axis_len = shape()[axis];
    std::vector<size_t> out_shape;
    for (size_t i = 0; i < ndim(); ++i) {
        if (i != axis)
            out_shape.push_back(shape()[i]);
        else if (keepdim)
            out_shape.push_back(1);
    }
    if (out_shape.empty()) out_shape.push_back(1);
    const bool req_g = track(requires_grad());
    Tensor res(out_shape, 0.0f, req_g);
    hip::check(ehip_sum_axis_f32(dptr(*this), dout(res), int64_t(outer), int64_t(axis_len),
                                 int64_t(inner), nullptr),
               "sum(axis)");
    if (req_g) {
        res.impl_->parents = {impl_};
        Tensor self_copy = *this;
        res.impl_->backward_fn = [self_copy, outer, axis_len,
                                  inner](const Tensor& grad_out) mutable {
            self_copy.add_grad(broadcast_middle(grad_out, self_copy.shape(), outer, axis_len, inner));
        };
    }
    return res;
}

Tensor Tensor::mean(size_t axis, bool keepdim) const {
    if (axis >= ndim())
        throw std::invalid_argument("mean: axis " + std::to_string(axis) + " out of range for " +
                                    shape_str() + ".");
    return sum(axis, keepdim) * (1.0f / static_cast<float>(shape()[axis]));
}

// ------------------------------------------------------------------ gather

// Rows of the first axis (src/tensor.cpp:556-604). The backward scatters in
// CSR form: every destination row sums the positions that selected it, in
// ascending order, which is the reference's loop order.
std::shared_ptr<const detail::RowGather> detail::make_row_gather(
    const std::vector<size_t>& indices, size_t rows, const std::string& shape_str,
    bool with_inverse) {
    std::vector<int32_t> idx(indices.size());
    for (size_t i = 0; i < indices.size(); ++i) {
        if (indices[i] >= rows)
            throw std::out_of_range("select_rows: row " + std::to_string(indices[i]) +
                                    " does not exist in a tensor " + shape_str + ".");
        idx[i] = static_cast<int32_t>(indices[i]);
    }
    auto g = std::make_shared<RowGather>();
    g->n = idx.size();
    g->rows = rows;
    g->idx = DeviceInts(idx);
    if (with_inverse) {
        // CSR of the inverse map, built once on the host.
        std::vector<int32_t> row_ptr(rows + 1, 0), pos(idx.size());
        for (int32_t r : idx) ++row_ptr[size_t(r) + 1];
        for (size_t r = 0; r < rows; ++r) row_ptr[r + 1] += row_ptr[r];
        std::vector<int32_t> fill(row_ptr.begin(), row_ptr.end() - 1);
        for (size_t i = 0; i < idx.size(); ++i) pos[size_t(fill[size_t(idx[i])]++)] = int32_t(i);
        g->row_ptr = DeviceInts(row_ptr);
        g->pos = DeviceInts(pos);
        g->inverse = true;
    }
    return g;
}

Tensor detail::gather_rows(const Tensor& table, const std::shared_ptr<const RowGather>& g) {
    const size_t rows = table.shape()[0];
    const size_t row_size = rows == 0 ? 0 : table.size() / rows;
    if (g->rows != rows) throw std::logic_error("gather_rows: index built for another table");
    std::vector<size_t> out_shape = table.shape();
    out_shape[0] = g->n;
    const bool req_g = track(table.requires_grad());
    if (req_g && !g->inverse) throw std::logic_error("gather_rows: index has no inverse map");
    Tensor res(out_shape, 0.0f, req_g);
    hip::check(ehip_select_rows_f32(dptr(table), g->idx.get(), dout(res), int64_t(g->n),
                                    int64_t(row_size), int64_t(rows), nullptr),
               "select_rows");
    if (req_g) {
        res.get_impl()->parents = {table.get_impl()};
        Tensor self_copy = table;
        res.get_impl()->backward_fn = [self_copy, g, rows, row_size](const Tensor& grad_out) mutable {
            Tensor dX(self_copy.shape(), 0.0f, false);
            hip::check(ehip_scatter_add_rows_f32(dptr(grad_out), g->row_ptr.get(), g->pos.get(),
                                                 dout(dX), int64_t(rows), int64_t(row_size),
                                                 int64_t(g->n), 0, nullptr),
                       "select_rows backward");
            self_copy.add_grad(dX);
        };
    }
    return res;
}

Tensor Tensor::select_rows(const std::vector<size_t>& indices) const {
    if (ndim() < 2)
        throw std::invalid_argument("select_rows requires at least 2 dimensions; this tensor is " +
                                    shape_str() + ".");
    if (indices.empty()) throw std::invalid_argument("select_rows received an empty index list.");
    return detail::gather_rows(
        *this, detail::make_row_gather(indices, shape()[0], shape_str(), track(requires_grad())));
}

Tensor Tensor::detach() const {
    auto impl = std::make_shared<TensorImpl>();
    impl->storage = impl_->storage.clone();
    impl->shape = shape();
    impl->compute_strides();
    return Tensor::from_impl(impl);
}

}  // namespace engine
