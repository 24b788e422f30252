// deferred.cpp -- gradient work queued during backward: the weight-gradient
// sums of fused convolution blocks and the parameter sums of large LayerNorms,
// reduced for every queued node in one launch (ehip_conv_weight_reduce_f32)
// instead of one launch per node; and the weight-gradient products of narrow
// Linear layers (with their bias sums), run together by ehip_gemm_batch_f32.
#include <memory>
#include <utility>
#include <vector>

#include "detail.hpp"

namespace engine {
namespace detail {

namespace {

struct Pending {
    std::vector<ehip_conv_reduce_t> jobs;
    std::vector<ehip_gemm_ex_t> products;
    std::vector<Tensor> product_inputs;  // the operands the products read
    DeferredKeep keep;
};

thread_local Pending g_pending;

}  // namespace

void DeferredKeep::reset_outputs() {
    for (auto& out : outputs) {
        const std::shared_ptr<TensorImpl> param = out.first.lock();
        if (param && param->grad && param->grad->storage.same_buffer(out.second))
            param->grad->storage = Storage(out.second.size(), 0.0f);
    }
    outputs.clear();
}

void defer_conv_reduce(const ehip_conv_reduce_t& job, const Tensor& partials) {
    g_pending.jobs.push_back(job);
    g_pending.keep.partials.push_back(partials);
}

void defer_conv_output(const Tensor& param, const Tensor& grad) {
    // An add_grad between the job and this call may have flushed the queue, and
    // with it the job that writes `grad`: then there is nothing left to own.
    if (g_pending.jobs.empty() && g_pending.products.empty()) return;
    g_pending.keep.outputs.emplace_back(param.get_impl(), grad.storage().share());
}

void defer_product(const ehip_gemm_ex_t& desc, std::initializer_list<Tensor> inputs) {
    g_pending.products.push_back(desc);
    for (const Tensor& t : inputs) g_pending.product_inputs.push_back(t);
}

bool deferred_pending() { return !g_pending.jobs.empty() || !g_pending.products.empty(); }

namespace {

// Runs the queued products (before anything reads their outputs or the
// reductions that follow them in the queue's order).
void run_products() {
    if (g_pending.products.empty()) return;
    std::vector<ehip_gemm_ex_t> products;
    std::vector<Tensor> inputs;
    std::swap(products, g_pending.products);
    std::swap(inputs, g_pending.product_inputs);
    const int rc = ehip_gemm_batch_f32(products.data(), int(products.size()), nullptr);
    if (rc != EHIP_OK) {
        g_pending.keep.reset_outputs();
        g_pending.jobs.clear();
        g_pending.keep = DeferredKeep{};
    }
    hip::check(rc, "queued weight-gradient products");
}

}  // namespace

bool deferred_writes(const Storage& s) {
    for (const auto& out : g_pending.keep.outputs)
        if (out.second.same_buffer(s)) return true;
    return false;
}

void settle_deferred(const Storage& s) {
    if (!deferred_pending()) return;
    if (deferred_writes(s)) {
        flush_deferred();
        return;
    }
    for (const Tensor& t : g_pending.product_inputs)
        if (t.storage().same_buffer(s)) {
            run_products();  // the sums stay queued for Adam's launch
            return;
        }
}

void flush_deferred() {
    run_products();
    if (g_pending.jobs.empty()) {
        g_pending.keep = DeferredKeep{};
        return;
    }
    Pending p;
    std::swap(p, g_pending);
    const int rc = ehip_conv_weight_reduce_f32(p.jobs.data(), int(p.jobs.size()), nullptr);
    if (rc != EHIP_OK) p.keep.reset_outputs();
    hip::check(rc, "conv weight-gradient reduction");
    // The buffers return to the arena here; later work on the same stream is
    // ordered after the launch that reads and writes them.
}

void take_deferred(std::vector<ehip_conv_reduce_t>& jobs, DeferredKeep& keep) {
    run_products();  // their outputs are gradients the caller's launch reads
    jobs = std::move(g_pending.jobs);
    keep = std::move(g_pending.keep);
    g_pending.jobs.clear();
    g_pending.keep = DeferredKeep{};
}

void drop_deferred() {
    g_pending.keep.reset_outputs();
    g_pending.jobs.clear();
    g_pending.products.clear();
    g_pending.product_inputs.clear();
    g_pending.keep = DeferredKeep{};
}

bool grad_adoptable(const Tensor& target) {
    const auto& impl = target.get_impl();
    return impl->requires_grad && (!impl->grad || impl->grad->storage.pending_zero());
}

float* grad_in_place(const Tensor& target) {
    const auto& impl = target.get_impl();
    if (!impl->requires_grad || !impl->grad) return nullptr;
    Storage& acc = impl->grad->storage;
    // Queued work that writes or reads the gradient runs first (it holds a
    // view of the buffer, so the exclusivity test is only meaningful after).
    settle_deferred(acc);
    if (acc.pending_zero() || !acc.exclusive() || acc.size() != target.size()) return nullptr;
    return acc.device_mut();
}

}  // namespace detail
}  // namespace engine
