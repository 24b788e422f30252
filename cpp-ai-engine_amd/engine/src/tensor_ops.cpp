// tensor_ops.cpp -- arithmetic with suffix broadcast, scalar ops, matmul and
// its transposed-operand forms, transpose/permute/reshape, ReLU and softmax,
// each with its derivative (the reference's src/tensor_ops.cpp). Every value
// is computed by a kernel of libehip on the engine's stream.
#include <cmath>
#include <stdexcept>
#include <string>

#include "detail.hpp"
#include "engine/nn.hpp"
#include "engine/tensor.hpp"

namespace engine {

using namespace detail;

namespace {

// out = a op b with the suffix broadcast of b.
Tensor binary_values(int op, const Tensor& a, const Tensor& b, const char* what) {
    const bool broadcast = a.shape() != b.shape();
    size_t inner = a.size(), repeat = 1;
    if (broadcast) {
        const BroadcastPlan plan = plan_broadcast(a.shape(), b.shape());
        if (!plan.valid)
            throw std::invalid_argument(std::string("Incompatible shapes for tensor ") + what +
                                        ": " + a.shape_str() + " and " + b.shape_str() + ".");
        inner = plan.inner;
        repeat = plan.repeat;
    }
    Tensor res(a.shape(), 0.0f, false);
    if (inner > 0)
        hip::check(ehip_binary_f32(op, dptr(a), dptr(b), dout(res), int64_t(inner),
                                   int64_t(repeat), nullptr),
                   what);
    return res;
}

void attach(Tensor& res, std::vector<std::shared_ptr<TensorImpl>> parents,
            std::function<void(const Tensor&)> fn) {
    res.set_requires_grad(true);
    res.get_impl()->parents = std::move(parents);
    res.get_impl()->backward_fn = std::move(fn);
}

// By value, so that a temporary passed in is moved through and stays the only
// handle on its buffer (add_grad then adopts it instead of copying).
Tensor reduce_to(Tensor d, const Tensor& target) {
    if (d.shape() == target.shape()) return d;
    return fold_leading(d, target.shape());
}

// The batch geometry of a product: 2-D operands are shared across the batch.
struct Batch {
    std::vector<size_t> dims;
    size_t count = 1;
    bool a_batched = false, b_batched = false;
};

Batch batch_of(const Tensor& a, const Tensor& b) {
    if (a.ndim() < 2 || b.ndim() < 2)
        throw std::invalid_argument("MatMul requires at least 2 dimensions in both operands.");
    const std::vector<size_t> ba(a.shape().begin(), a.shape().end() - 2);
    const std::vector<size_t> bb(b.shape().begin(), b.shape().end() - 2);
    Batch r;
    r.a_batched = !ba.empty();
    r.b_batched = !bb.empty();
    if (r.a_batched && r.b_batched && ba != bb)
        throw std::invalid_argument("Batched MatMul needs identical batch axes: " + a.shape_str() +
                                    " and " + b.shape_str() + ".");
    r.dims = r.a_batched ? ba : bb;
    r.count = product(r.dims);
    return r;
}

// C = op(A) op(B), batched; returns a fresh tensor of shape dims + (m, n).
Tensor gemm(bool ta, bool tb, const Tensor& a, const Tensor& b, const Batch& bt, size_t m,
            size_t n, size_t k) {
    std::vector<size_t> shape = bt.dims;
    shape.push_back(m);
    shape.push_back(n);
    Tensor c(shape, 0.0f, false);
    const size_t a_rows = a.shape()[a.ndim() - 2], a_cols = a.shape()[a.ndim() - 1];
    const size_t b_rows = b.shape()[b.ndim() - 2], b_cols = b.shape()[b.ndim() - 1];
    hip::check(ehip_gemm_f32(ta ? 1 : 0, tb ? 1 : 0, int64_t(bt.count), int64_t(m), int64_t(n),
                             int64_t(k), dptr(a), int64_t(a_cols),
                             bt.a_batched ? int64_t(a_rows * a_cols) : 0, dptr(b), int64_t(b_cols),
                             bt.b_batched ? int64_t(b_rows * b_cols) : 0, 0.0f, dout(c),
                             int64_t(n), int64_t(m * n), nullptr),
               "matmul");
    return c;
}

}  // namespace

// ------------------------------------------------------------------ element-wise

Tensor Tensor::operator+(const Tensor& other) const {
    Tensor res = binary_values(EHIP_ADD, *this, other, "addition");
    if (track(requires_grad() || other.requires_grad())) {
        Tensor self_copy = *this, other_copy = other;
        attach(res, {impl_, other.impl_}, [self_copy, other_copy](const Tensor& g) mutable {
            // When g's buffer can be adopted, the first operand takes it and the
            // second gets a copy (8 bytes per element). Otherwise, for two
            // same-shape operands, one fused pass writes both (12 bytes per
            // element instead of 16); it equals two add_grad calls bit for bit.
            const bool same = self_copy.shape() == other_copy.shape();
            auto& sg = self_copy.get_impl()->grad;
            auto& og = other_copy.get_impl()->grad;
            const bool init_a = !sg || sg->storage.pending_zero();
            const bool init_b = !og || og->storage.pending_zero();
            const bool adoptable = g.get_impl().use_count() == 1 && g.storage().exclusive() &&
                                   init_a && self_copy.requires_grad();
            if (!adoptable && same && self_copy.requires_grad() && other_copy.requires_grad() &&
                self_copy.get_impl() != other_copy.get_impl() &&
                (init_a || sg->storage.exclusive()) && (init_b || og->storage.exclusive())) {
                if (!sg) sg = std::make_shared<TensorImpl>(self_copy.shape(), 0.0f, false);
                if (!og) og = std::make_shared<TensorImpl>(other_copy.shape(), 0.0f, false);
                const float* src = dptr(g);
                float* da = init_a ? sg->storage.device_write() : sg->storage.device_mut();
                float* db = init_b ? og->storage.device_write() : og->storage.device_mut();
                hip::check(ehip_add_backward_f32(src, da, db, int64_t(g.size()), init_a ? 0 : 1,
                                                 init_b ? 0 : 1, nullptr),
                           "add backward");
                return;
            }
            if (self_copy.requires_grad()) self_copy.add_grad(g);
            if (other_copy.requires_grad()) other_copy.add_grad(reduce_to(g, other_copy));
        });
    }
    return res;
}

Tensor Tensor::operator-(const Tensor& other) const {
    Tensor res = binary_values(EHIP_SUB, *this, other, "subtraction");
    if (track(requires_grad() || other.requires_grad())) {
        Tensor self_copy = *this, other_copy = other;
        attach(res, {impl_, other.impl_}, [self_copy, other_copy](const Tensor& g) mutable {
            if (self_copy.requires_grad()) self_copy.add_grad(g);
            if (other_copy.requires_grad()) other_copy.add_grad(reduce_to(g * -1.0f, other_copy));
        });
    }
    return res;
}

Tensor Tensor::operator*(const Tensor& other) const {
    Tensor res = binary_values(EHIP_MUL, *this, other, "multiplication");
    if (track(requires_grad() || other.requires_grad())) {
        Tensor self_copy = *this, other_copy = other;
        attach(res, {impl_, other.impl_}, [self_copy, other_copy](const Tensor& g) mutable {
            const bool na = self_copy.requires_grad(), nb = other_copy.requires_grad();
            if (self_copy.shape() == other_copy.shape() &&
                self_copy.get_impl() != other_copy.get_impl() && g.size() > 0) {
                // Same shapes: both products in one launch, added in place into a
                // gradient that already holds values (add_grad's sum), otherwise
                // written to a fresh buffer that add_grad then takes over.
                float* acc_a = na ? grad_in_place(self_copy) : nullptr;
                float* acc_b = nb ? grad_in_place(other_copy) : nullptr;
                Tensor ta = na && !acc_a ? Tensor(self_copy.shape(), 0.0f, false) : Tensor();
                Tensor tb = nb && !acc_b ? Tensor(other_copy.shape(), 0.0f, false) : Tensor();
                hip::check(ehip_mul_backward_f32(dptr(g), dptr(self_copy), dptr(other_copy),
                                                 na ? (acc_a ? acc_a : dout(ta)) : nullptr,
                                                 nb ? (acc_b ? acc_b : dout(tb)) : nullptr,
                                                 int64_t(g.size()), acc_a != nullptr,
                                                 acc_b != nullptr, nullptr),
                           "mul backward");
                if (na && !acc_a) self_copy.add_grad(ta);
                if (nb && !acc_b) other_copy.add_grad(tb);
                return;
            }
            // g * expand(other) is the broadcast product itself.
            if (self_copy.requires_grad()) self_copy.add_grad(binary_values(EHIP_MUL, g, other_copy, "mul"));
            if (other_copy.requires_grad())
                other_copy.add_grad(reduce_to(binary_values(EHIP_MUL, g, self_copy, "mul"), other_copy));
        });
    }
    return res;
}

Tensor Tensor::operator/(const Tensor& other) const {
    Tensor res = binary_values(EHIP_DIV, *this, other, "division");
    if (track(requires_grad() || other.requires_grad())) {
        Tensor self_copy = *this, other_copy = other;
        attach(res, {impl_, other.impl_}, [self_copy, other_copy](const Tensor& g) mutable {
            if (self_copy.requires_grad()) self_copy.add_grad(binary_values(EHIP_DIV, g, other_copy, "div"));
            if (other_copy.requires_grad()) {
                // (g * x * -1) / (rhs * rhs), rhs broadcast (src/tensor_ops.cpp:251-256).
                Tensor num = binary_values(EHIP_MUL, g, self_copy, "mul") * -1.0f;
                Tensor r2 = binary_values(EHIP_MUL, other_copy, other_copy, "mul");
                other_copy.add_grad(reduce_to(binary_values(EHIP_DIV, num, r2, "div"), other_copy));
            }
        });
    }
    return res;
}

Tensor Tensor::operator+(float scalar) const {
    Tensor res(shape(), 0.0f, false);
    hip::check(ehip_scalar_f32(dptr(*this), dout(res), int64_t(size()), 1.0f, scalar, nullptr),
               "scalar add");
    if (track(requires_grad())) {
        Tensor self_copy = *this;
        attach(res, {impl_}, [self_copy](const Tensor& g) mutable { self_copy.add_grad(g); });
    }
    return res;
}

Tensor Tensor::operator-(float scalar) const { return (*this) + (-scalar); }

Tensor Tensor::operator*(float scalar) const {
    Tensor res(shape(), 0.0f, false);
    if (scalar == 1.0f) {  // x * 1 is x exactly (ehip_scalar_f32 would add 0)
        if (size() > 0)
            hip::check(ehip_memcpy_d2d(dout(res), dptr(*this), size() * sizeof(float), nullptr),
                       "copy");
    } else {
        hip::check(ehip_scalar_f32(dptr(*this), dout(res), int64_t(size()), scalar, 0.0f, nullptr),
                   "scalar mul");
    }
    if (track(requires_grad())) {
        Tensor self_copy = *this;
        attach(res, {impl_},
               [self_copy, scalar](const Tensor& g) mutable { self_copy.add_grad(g * scalar); });
    }
    return res;
}

Tensor Tensor::operator/(float scalar) const {
    if (scalar == 0.0f) throw std::invalid_argument("Division by zero.");
    return (*this) * (1.0f / scalar);
}

Tensor operator+(float scalar, const Tensor& t) { return t + scalar; }
Tensor operator*(float scalar, const Tensor& t) { return t * scalar; }
Tensor operator-(float scalar, const Tensor& t) { return (t * -1.0f) + scalar; }

// ------------------------------------------------------------------ products

// src/tensor_ops.cpp:475-588. The backward products read the operands in
// place through the GEMM's transposed modes instead of materialising B^T and
// A^T; a shared operand's gradient is folded over the batch.
Tensor Tensor::matmul(const Tensor& B) const {
    const Batch bt = batch_of(*this, B);
    const size_t M = shape()[ndim() - 2], K = shape()[ndim() - 1];
    const size_t K2 = B.shape()[B.ndim() - 2], N = B.shape()[B.ndim() - 1];
    if (K != K2)
        throw std::invalid_argument("Incompatible dimensions for MatMul: " + shape_str() + " and " +
                                    B.shape_str() + ".");
    Tensor C = gemm(false, false, *this, B, bt, M, N, K);
    if (track(requires_grad() || B.requires_grad())) {
        Tensor a = *this, b = B;
        attach(C, {impl_, B.impl_}, [a, b, bt, M, N, K](const Tensor& g) mutable {
            if (bt.dims.empty() && a.requires_grad() && b.requires_grad() && M > 0 && N > 0 &&
                K > 0) {
                // Plain 2-D operands: both products from one entry point (one launch
                // when both take the K-sliced tiles; the same bits as two calls).
                Tensor da({M, K}, 0.0f, false), db({K, N}, 0.0f, false);
                hip::check(ehip_matmul_backward_f32(int64_t(M), int64_t(K), int64_t(N), dptr(a),
                                                    int64_t(K), dptr(b), int64_t(N), dptr(g),
                                                    int64_t(N), dout(da), int64_t(K), 0.0f,
                                                    dout(db), int64_t(N), 0.0f, nullptr),
                           "matmul backward");
                a.add_grad(da);
                b.add_grad(db);
                return;
            }
            Batch gb = bt;
            gb.a_batched = true;  // g always carries the batch
            if (a.requires_grad()) {
                Batch db = gb;
                db.b_batched = bt.b_batched;
                a.add_grad(reduce_to(gemm(false, true, g, b, db, M, K, N), a));  // g B^T
            }
            if (b.requires_grad()) {
                Batch db;
                db.dims = bt.dims;
                db.count = bt.count;
                db.a_batched = bt.a_batched;
                db.b_batched = true;
                b.add_grad(reduce_to(gemm(true, false, a, g, db, K, N, M), b));  // A^T g
            }
        });
    }
    return C;
}

namespace ops {

// C = A B^T: A (.., m, k), B (.., n, k).
Tensor matmul_nt(const Tensor& A, const Tensor& B) {
    const Batch bt = batch_of(A, B);
    const size_t M = A.shape()[A.ndim() - 2], K = A.shape()[A.ndim() - 1];
    const size_t N = B.shape()[B.ndim() - 2];
    if (B.shape()[B.ndim() - 1] != K)
        throw std::invalid_argument("Incompatible dimensions for A B^T: " + A.shape_str() + " and " +
                                    B.shape_str() + ".");
    Tensor C = gemm(false, true, A, B, bt, M, N, K);
    if (track(A.requires_grad() || B.requires_grad())) {
        Tensor a = A, b = B;
        attach(C, {A.get_impl(), B.get_impl()}, [a, b, bt, M, N, K](const Tensor& g) mutable {
            if (a.requires_grad()) {  // dA = g B
                Batch db = bt;
                db.a_batched = true;
                a.add_grad(reduce_to(gemm(false, false, g, b, db, M, K, N), a));
            }
            if (b.requires_grad()) {  // dB = g^T A
                Batch db = bt;
                db.a_batched = true;
                db.b_batched = bt.a_batched;
                b.add_grad(reduce_to(gemm(true, false, g, a, db, N, K, M), b));
            }
        });
    }
    return C;
}

namespace {

// out (m, n) = op(a) op(b) over plain 2-D operands, then + bias (a row),
// + residual (an (m, n) array) and ReLU, each rounded on its own.
ehip_gemm_ex_t gemm_2d_desc(bool ta, bool tb, size_t m, size_t n, size_t k, const float* a,
                            const float* b, float* c, const float* bias, bool relu,
                            const float* residual) {
    ehip_gemm_ex_t d{};
    d.trans_a = ta ? 1 : 0;
    d.trans_b = tb ? 1 : 0;
    d.batch = 1;
    d.inner = 1;
    d.m = int64_t(m);
    d.n = int64_t(n);
    d.k = int64_t(k);
    d.a = a;
    d.lda = int64_t(ta ? m : k);
    d.b = b;
    d.ldb = int64_t(tb ? k : n);
    d.c = c;
    d.ldc = int64_t(n);
    d.alpha = 1.0f;
    d.addend = bias;
    d.addend_period = 1;  // ld_addend 0: one row over every row
    d.relu = relu ? 1 : 0;
    d.residual = residual;
    d.ld_residual = int64_t(n);
    return d;
}

void gemm_2d(bool ta, bool tb, size_t m, size_t n, size_t k, const float* a, const float* b,
             float* c, const float* bias, bool relu, const char* what,
             const float* residual = nullptr) {
    const ehip_gemm_ex_t d = gemm_2d_desc(ta, tb, m, n, k, a, b, c, bias, relu, residual);
    hip::check(ehip_gemm_ex_f32(&d, nullptr), what);
}

bool row_bias(const Tensor* bias, size_t n) {
    if (bias == nullptr) return true;
    return bias->size() == n && (bias->ndim() == 1 || (bias->ndim() == 2 && bias->shape()[0] == 1));
}

Tensor empty_2d(size_t rows, size_t cols) { return Tensor({rows, cols}, 0.0f, false); }

// A residual added in a product's epilogue: any shape holding the (m, n)
// result's elements in row-major order; the node's output takes its shape.
void check_residual(const Tensor* residual, size_t m, size_t n, const char* what) {
    if (residual != nullptr && residual->size() != m * n)
        throw std::invalid_argument(std::string(what) + ": residual " + residual->shape_str() +
                                    " does not hold the (" + std::to_string(m) + ", " +
                                    std::to_string(n) + ") result.");
}

// dW = X^T dY (X rows x in, dY rows x out) with db = the column sums of dY,
// the descriptor ehip_linear_backward_f32 launches for a layer whose bias
// gradient comes from the product.
ehip_gemm_ex_t weight_grad_desc(const float* x, const float* dy, float* dw, float* db,
                                size_t rows, size_t in, size_t out) {
    ehip_gemm_ex_t d{};
    d.trans_a = 1;
    d.batch = 1;
    d.inner = 1;
    d.m = int64_t(in);
    d.n = int64_t(out);
    d.k = int64_t(rows);
    d.a = x;
    d.lda = int64_t(in);
    d.b = dy;
    d.ldb = int64_t(out);
    d.c = dw;
    d.ldc = int64_t(out);
    d.alpha = 1.0f;
    d.addend_period = 1;
    d.colsum_b = db;
    return d;
}

// Queues dW and db of a narrow layer (see nn::set_deferred_weight_grads) when
// both are fresh gradients and the library would form db from the product
// and run it as a panel product (what ehip_gemm_batch_f32 groups); returns
// false, having done nothing, otherwise. x and dy are kept until it runs.
bool queue_weight_grads(const Tensor& x, const Tensor& dy, const Tensor& w, const Tensor& b,
                        Tensor& dw, Tensor& db, size_t rows, size_t in, size_t out) {
    if (!nn::deferred_weight_grads() || !w.requires_grad() || !b.requires_grad() ||
        !grad_adoptable(w) || !grad_adoptable(b) ||
        ehip_linear_backward_plan(int64_t(rows), int64_t(in), int64_t(out)) != 1)
        return false;
    const ehip_gemm_ex_t d = weight_grad_desc(dptr(x), dptr(dy), dout(dw), dout(db), rows, in, out);
    if (!ehip_gemm_groupable(&d)) return false;
    defer_product(d, {x, dy});
    return true;
}

// Multiply-adds of g w^T above which Linear's backward no longer runs as one
// launch (csrc/gemm.hip's thread-per-output limit), so that adding dx into
// x's gradient in place saves a pass instead of splitting a launch in two.
constexpr double kInPlaceWork = double(1 << 21);

bool linear_fusable(const Tensor& x, const Tensor& w, const Tensor* bias) {
    return x.ndim() == 2 && w.ndim() == 2 && x.shape()[1] == w.shape()[0] &&
           row_bias(bias, w.shape()[1]);
}

// The node of out = [residual +] x w + bias, already computed: linear()'s
// backward attached.
Tensor linear_node(Tensor out, const Tensor& x, const Tensor& w, const Tensor* bias,
                   const Tensor* residual) {
    const size_t M = x.shape()[0], K = x.shape()[1], N = w.shape()[1];
    const bool bias_grad = bias != nullptr && bias->requires_grad();
    const bool res_grad = residual != nullptr && residual->requires_grad();
    if (!track(x.requires_grad() || w.requires_grad() || bias_grad || res_grad)) return out;
    Tensor xc = x, wc = w, bc = bias ? *bias : Tensor(), rc = residual ? *residual : Tensor();
    std::vector<std::shared_ptr<TensorImpl>> parents = {x.get_impl(), w.get_impl()};
    if (bias) parents.push_back(bias->get_impl());
    if (residual) parents.push_back(residual->get_impl());
    attach(out, std::move(parents), [xc, wc, bc, rc, M, N, K](const Tensor& g) mutable {
        // The residual add's node comes last in the composed graph, so its
        // gradient goes first; the product reads g itself instead of the copy
        // the add's backward would hand it.
        if (rc.get_impl() && rc.requires_grad()) rc.add_grad(g);
        const bool want_db = bc.get_impl() && bc.requires_grad();
        if (M > 0 && K > 0 && N > 0) {
            // The same three results as the composed graph's add and product
            // backward (one launch for small layers), added in its order: the
            // bias, then x, then w. Past the one-launch sizes, g w^T adds
            // straight into an existing gradient of x (beta = 1, the same sum
            // as add_grad's, without the separate accumulation pass).
            float* dx_acc = xc.requires_grad() && double(M) * double(K) * double(N) > kInPlaceWork
                                ? grad_in_place(xc)
                                : nullptr;
            const bool want_dx = xc.requires_grad() && dx_acc == nullptr;
            Tensor dx = want_dx ? empty_2d(M, K) : Tensor();
            Tensor dw = wc.requires_grad() ? empty_2d(K, N) : Tensor();
            Tensor db = want_db ? Tensor(bc.shape(), 0.0f, false) : Tensor();
            if (dx_acc)
                hip::check(ehip_gemm_f32(0, 1, 1, int64_t(M), int64_t(K), int64_t(N), dptr(g),
                                         int64_t(N), 0, dptr(wc), int64_t(N), 0, 1.0f, dx_acc,
                                         int64_t(K), 0, nullptr),
                           "linear backward dx");
            // dW and db queued (g may be the residual's gradient by now: an
            // in-place add into it first runs the queue).
            if (want_db && queue_weight_grads(xc, g, wc, bc, dw, db, M, K, N)) {
                // dx as ehip_linear_backward_f32 forms it for such a layer.
                if (want_dx)
                    hip::check(ehip_gemm_f32(0, 1, 1, int64_t(M), int64_t(K), int64_t(N),
                                             dptr(g), int64_t(N), 0, dptr(wc), int64_t(N), 0,
                                             0.0f, dout(dx), int64_t(K), 0, nullptr),
                               "linear backward dx");
                bc.add_grad(db);
                if (want_dx) xc.add_grad(dx);
                wc.add_grad(dw);
                defer_conv_output(wc, dw);
                defer_conv_output(bc, db);
                return;
            }
            hip::check(ehip_linear_backward_f32(dptr(xc), dptr(wc), dptr(g),
                                                want_dx ? dout(dx) : nullptr,
                                                wc.requires_grad() ? dout(dw) : nullptr,
                                                want_db ? dout(db) : nullptr, int64_t(M),
                                                int64_t(K), int64_t(N), nullptr),
                       "linear backward");
            if (want_db) bc.add_grad(db);
            if (want_dx) xc.add_grad(dx);
            if (wc.requires_grad()) wc.add_grad(dw);
            return;
        }
        // The composed graph's order: the bias add's node, then the product's.
        if (want_db) bc.add_grad(reduce_to(g, bc));
        if (xc.requires_grad()) {  // g w^T
            Tensor dx = empty_2d(M, K);
            if (M > 0 && K > 0) gemm_2d(false, true, M, K, N, dptr(g), dptr(wc), dout(dx), nullptr,
                                        false, "linear dx");
            xc.add_grad(dx);
        }
        if (wc.requires_grad()) {  // x^T g
            Tensor dw = empty_2d(K, N);
            if (K > 0 && N > 0) gemm_2d(true, false, K, N, M, dptr(xc), dptr(g), dout(dw), nullptr,
                                        false, "linear dw");
            wc.add_grad(dw);
        }
    });
    return out;
}

}  // namespace

Tensor linear(const Tensor& x, const Tensor& w, const Tensor* bias, const Tensor* residual) {
    if (!linear_fusable(x, w, bias)) {
        Tensor out = x.matmul(w);
        if (bias) out = out + *bias;
        return residual ? *residual + out.reshape(residual->shape()) : out;
    }
    const size_t M = x.shape()[0], K = x.shape()[1], N = w.shape()[1];
    check_residual(residual, M, N, "linear");
    Tensor out = residual ? Tensor(residual->shape(), 0.0f, false) : empty_2d(M, N);
    if (M > 0 && N > 0)
        gemm_2d(false, false, M, N, K, dptr(x), dptr(w), dout(out), bias ? dptr(*bias) : nullptr,
                false, "linear", residual ? dptr(*residual) : nullptr);
    return linear_node(out, x, w, bias, residual);
}

std::vector<Tensor> linear_many(const Tensor& x, const std::vector<const Tensor*>& w,
                                const std::vector<const Tensor*>& bias) {
    if (w.size() != bias.size())
        throw std::invalid_argument("linear_many: " + std::to_string(w.size()) + " weights and " +
                                    std::to_string(bias.size()) + " biases.");
    bool fusable = true;
    for (size_t i = 0; i < w.size(); ++i) fusable = fusable && linear_fusable(x, *w[i], bias[i]);
    std::vector<Tensor> outs;
    if (!fusable) {
        for (size_t i = 0; i < w.size(); ++i) outs.push_back(linear(x, *w[i], bias[i]));
        return outs;
    }
    const size_t M = x.shape()[0], K = x.shape()[1];
    std::vector<ehip_gemm_ex_t> descs;
    for (size_t i = 0; i < w.size(); ++i) {
        const size_t N = w[i]->shape()[1];
        outs.push_back(empty_2d(M, N));
        if (M > 0 && N > 0)
            descs.push_back(gemm_2d_desc(false, false, M, N, K, dptr(x), dptr(*w[i]),
                                         dout(outs.back()), bias[i] ? dptr(*bias[i]) : nullptr,
                                         false, nullptr));
    }
    if (!descs.empty())
        hip::check(ehip_gemm_batch_f32(descs.data(), int(descs.size()), nullptr), "linear_many");
    for (size_t i = 0; i < w.size(); ++i) outs[i] = linear_node(outs[i], x, *w[i], bias[i], nullptr);
    return outs;
}

Tensor feed_forward_relu(const Tensor& x, const Tensor& w1, const Tensor& b1, const Tensor& w2,
                         const Tensor& b2, const Tensor* residual) {
    const bool plain = x.ndim() == 2 && w1.ndim() == 2 && w2.ndim() == 2 &&
                       x.shape()[1] == w1.shape()[0] && w1.shape()[1] == w2.shape()[0] &&
                       row_bias(&b1, w1.shape()[1]) && row_bias(&b2, w2.shape()[1]);
    if (!plain) return linear(linear(x, w1, &b1).relu(), w2, &b2, residual);
    const size_t M = x.shape()[0], D = x.shape()[1], F = w1.shape()[1], N = w2.shape()[1];
    check_residual(residual, M, N, "feed-forward");
    Tensor h = empty_2d(M, F);  // relu(x w1 + b1)
    if (M > 0 && F > 0)
        gemm_2d(false, false, M, F, D, dptr(x), dptr(w1), dout(h), dptr(b1), true,
                "feed-forward 1");
    Tensor out = residual ? Tensor(residual->shape(), 0.0f, false) : empty_2d(M, N);
    if (M > 0 && N > 0)
        gemm_2d(false, false, M, N, F, dptr(h), dptr(w2), dout(out), dptr(b2), false,
                "feed-forward 2", residual ? dptr(*residual) : nullptr);
    const bool res_grad = residual != nullptr && residual->requires_grad();
    if (!track(x.requires_grad() || w1.requires_grad() || b1.requires_grad() ||
               w2.requires_grad() || b2.requires_grad() || res_grad))
        return out;
    Tensor xc = x, w1c = w1, b1c = b1, w2c = w2, b2c = b2, rc = residual ? *residual : Tensor();
    std::vector<std::shared_ptr<TensorImpl>> parents = {x.get_impl(), w1.get_impl(), b1.get_impl(),
                                                        w2.get_impl(), b2.get_impl()};
    if (residual) parents.push_back(residual->get_impl());
    attach(out, std::move(parents),
           [xc, w1c, b1c, w2c, b2c, rc, h, M, D, F, N](const Tensor& g) mutable {
               // The composed graph's order: the residual add, second bias,
               // second product (h, then w2), ReLU, first bias, first product
               // (x, then w1). A bias and its weight both trained take one
               // ehip_linear_backward_f32 call (db from the dW product where
               // that pays, as in Linear).
               if (rc.get_impl() && rc.requires_grad()) rc.add_grad(g);
               Tensor dw2;
               bool queued2 = false;
               if (b2c.requires_grad() && w2c.requires_grad() && F > 0 && N > 0) {
                   dw2 = empty_2d(F, N);
                   Tensor db2(b2c.shape(), 0.0f, false);
                   queued2 = queue_weight_grads(h, g, w2c, b2c, dw2, db2, M, F, N);
                   if (!queued2)
                       hip::check(ehip_linear_backward_f32(dptr(h), dptr(w2c), dptr(g), nullptr,
                                                           dout(dw2), dout(db2), int64_t(M),
                                                           int64_t(F), int64_t(N), nullptr),
                                  "feed-forward dw2 and db2");
                   b2c.add_grad(db2);
                   if (queued2) defer_conv_output(b2c, db2);
               } else if (b2c.requires_grad()) {
                   b2c.add_grad(reduce_to(g, b2c));
               }
               const bool need_dh = xc.requires_grad() || w1c.requires_grad() || b1c.requires_grad();
               Tensor dh;
               if (need_dh) {  // g w2^T
                   dh = empty_2d(M, F);
                   if (M > 0 && F > 0)
                       gemm_2d(false, true, M, F, N, dptr(g), dptr(w2c), dout(dh), nullptr, false,
                               "feed-forward dh");
               }
               if (w2c.requires_grad()) {  // h^T g
                   if (!dw2.get_impl()) {
                       dw2 = empty_2d(F, N);
                       if (F > 0 && N > 0)
                           gemm_2d(true, false, F, N, M, dptr(h), dptr(g), dout(dw2), nullptr,
                                   false, "feed-forward dw2");
                   }
                   w2c.add_grad(dw2);
                   if (queued2) defer_conv_output(w2c, dw2);
               }
               if (!need_dh) return;
               // ReLU's backward from its output: h > 0 exactly where the
               // pre-activation was positive.
               Tensor dpre = empty_2d(M, F);
               if (M > 0 && F > 0)
                   hip::check(ehip_relu_backward_f32(dptr(h), dptr(dh), dout(dpre),
                                                     int64_t(M * F), nullptr),
                              "feed-forward relu backward");
               dh = Tensor();
               Tensor dw1;
               bool queued1 = false;
               if (b1c.requires_grad() && w1c.requires_grad() && D > 0 && F > 0) {
                   dw1 = empty_2d(D, F);
                   Tensor db1(b1c.shape(), 0.0f, false);
                   queued1 = queue_weight_grads(xc, dpre, w1c, b1c, dw1, db1, M, D, F);
                   if (!queued1)
                       hip::check(ehip_linear_backward_f32(dptr(xc), dptr(w1c), dptr(dpre),
                                                           nullptr, dout(dw1), dout(db1),
                                                           int64_t(M), int64_t(D), int64_t(F),
                                                           nullptr),
                                  "feed-forward dw1 and db1");
                   b1c.add_grad(db1);
                   if (queued1) defer_conv_output(b1c, db1);
               } else if (b1c.requires_grad()) {
                   b1c.add_grad(reduce_to(dpre, b1c));
               }
               if (xc.requires_grad()) {  // dpre w1^T
                   Tensor dx = empty_2d(M, D);
                   if (M > 0 && D > 0)
                       gemm_2d(false, true, M, D, F, dptr(dpre), dptr(w1c), dout(dx), nullptr,
                               false, "feed-forward dx");
                   xc.add_grad(dx);
               }
               if (w1c.requires_grad()) {  // x^T dpre
                   if (!dw1.get_impl()) {
                       dw1 = empty_2d(D, F);
                       if (D > 0 && F > 0)
                           gemm_2d(true, false, D, F, M, dptr(xc), dptr(dpre), dout(dw1), nullptr,
                                   false, "feed-forward dw1");
                   }
                   w1c.add_grad(dw1);
                   if (queued1) defer_conv_output(w1c, dw1);
               }
           });
    return out;
}

// C = A^T B: A (.., k, m), B (.., k, n).
Tensor matmul_tn(const Tensor& A, const Tensor& B) {
    const Batch bt = batch_of(A, B);
    const size_t K = A.shape()[A.ndim() - 2], M = A.shape()[A.ndim() - 1];
    const size_t N = B.shape()[B.ndim() - 1];
    if (B.shape()[B.ndim() - 2] != K)
        throw std::invalid_argument("Incompatible dimensions for A^T B: " + A.shape_str() + " and " +
                                    B.shape_str() + ".");
    Tensor C = gemm(true, false, A, B, bt, M, N, K);
    if (track(A.requires_grad() || B.requires_grad())) {
        Tensor a = A, b = B;
        attach(C, {A.get_impl(), B.get_impl()}, [a, b, bt, M, N, K](const Tensor& g) mutable {
            if (a.requires_grad()) {  // dA = B g^T
                Batch db = bt;
                db.a_batched = bt.b_batched;
                db.b_batched = true;
                a.add_grad(reduce_to(gemm(false, true, b, g, db, K, M, N), a));
            }
            if (b.requires_grad()) {  // dB = A g
                Batch db = bt;
                db.b_batched = true;
                b.add_grad(reduce_to(gemm(false, false, a, g, db, K, N, M), b));
            }
        });
    }
    return C;
}

}  // namespace ops

// ------------------------------------------------------------------ layout

Tensor Tensor::transpose() const {
    if (ndim() < 2)
        throw std::invalid_argument("Transpose requires at least 2 dimensions; this tensor is " +
                                    shape_str() + ".");
    const size_t rows = shape()[ndim() - 2], cols = shape()[ndim() - 1];
    const size_t batch = rows * cols == 0 ? 0 : size() / (rows * cols);
    std::vector<size_t> out_shape = shape();
    std::swap(out_shape[ndim() - 2], out_shape[ndim() - 1]);
    Tensor res(out_shape, 0.0f, false);
    if (size() > 0)
        hip::check(ehip_transpose_f32(dptr(*this), dout(res), int64_t(batch), int64_t(rows),
                                      int64_t(cols), nullptr),
                   "transpose");
    if (track(requires_grad())) {
        Tensor self_copy = *this;
        attach(res, {impl_},
               [self_copy](const Tensor& g) mutable { self_copy.add_grad(g.transpose()); });
    }
    return res;
}

Tensor Tensor::permute(const std::vector<size_t>& order) const {
    const size_t nd = ndim();
    if (order.size() != nd)
        throw std::invalid_argument("permute needs an order of " + std::to_string(nd) +
                                    " axes for a tensor " + shape_str() + ".");
    std::vector<bool> seen(nd, false);
    for (size_t axis : order) {
        if (axis >= nd || seen[axis])
            throw std::invalid_argument("permute needs a valid permutation of the axes.");
        seen[axis] = true;
    }
    std::vector<size_t> out_shape(nd);
    std::vector<int64_t> oshape(nd), src(nd);
    for (size_t i = 0; i < nd; ++i) {
        out_shape[i] = shape()[order[i]];
        oshape[i] = int64_t(out_shape[i]);
        src[i] = int64_t(strides()[order[i]]);
    }
    Tensor res(out_shape, 0.0f, false);
    if (size() > 0)
        hip::check(ehip_permute_f32(dptr(*this), dout(res), int(nd), oshape.data(), src.data(),
                                    nullptr),
                   "permute");
    if (track(requires_grad())) {
        Tensor self_copy = *this;
        std::vector<size_t> inverse(nd);
        for (size_t i = 0; i < nd; ++i) inverse[order[i]] = i;
        attach(res, {impl_}, [self_copy, inverse](const Tensor& g) mutable {
            self_copy.add_grad(g.permute(inverse));
        });
    }
    return res;
}

Tensor Tensor::reshape(const std::vector<size_t>& new_shape) const {
    if (product(new_shape) != size())
        throw std::invalid_argument("Incompatible element count for Reshape.");
    const bool req_g = track(requires_grad());
    Tensor res = view_with_shape(impl_->storage, new_shape, false);
    if (req_g) {
        Tensor self_copy = *this;
        attach(res, {impl_},
               [self_copy](const Tensor& g) mutable { add_grad_reshaped(self_copy, g); });
    }
    return res;
}

// ------------------------------------------------------------------ activations

Tensor Tensor::relu() const {
    Tensor res(shape(), 0.0f, false);
    hip::check(ehip_relu_f32(dptr(*this), dout(res), int64_t(size()), nullptr), "relu");
    if (track(requires_grad())) {
        Tensor self_copy = *this;
        attach(res, {impl_}, [self_copy](const Tensor& g) mutable {
            Tensor dX(self_copy.shape(), 0.0f, false);
            hip::check(ehip_relu_backward_f32(dptr(self_copy), dptr(g), dout(dX),
                                              int64_t(self_copy.size()), nullptr),
                       "relu backward");
            self_copy.add_grad(dX);
        });
    }
    return res;
}

// Row softmax over the last axis. The backward keeps a view of the output
// (the reference keeps a detached copy, src/tensor_ops.cpp:652-654; nothing
// writes into an op's output, so the view holds the same values).
Tensor Tensor::softmax() const {
    if (ndim() == 0 || size() == 0) throw std::invalid_argument("Softmax needs a non-empty tensor.");
    const size_t cols = shape().back();
    const size_t rows = size() / cols;
    Tensor res(shape(), 0.0f, false);
    hip::check(ehip_softmax_f32(dptr(*this), dout(res), int64_t(rows), int64_t(cols), nullptr),
               "softmax");
    if (track(requires_grad())) {
        Tensor self_copy = *this;
        Tensor saved = view_with_shape(res.storage(), res.shape(), false);
        attach(res, {impl_}, [self_copy, saved, rows, cols](const Tensor& g) mutable {
            Tensor dX(self_copy.shape(), 0.0f, false);
            hip::check(ehip_softmax_backward_f32(dptr(saved), dptr(g), dout(dX), int64_t(rows),
                                                 int64_t(cols), nullptr),
                       "softmax backward");
            self_copy.add_grad(dX);
        });
    }
    return res;
}

}  // namespace engine
