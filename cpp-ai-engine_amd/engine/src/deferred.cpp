// deferred.cpp -- gradient work queued during backward: the weight-gradient
// sums of fused convolution blocks, reduced for every layer in one launch
// (ehip_conv_weight_reduce_f32) instead of one launch per layer.
#include <vector>

#include "detail.hpp"

namespace engine {
namespace detail {

namespace {

struct Pending {
    std::vector<ehip_conv_reduce_t> jobs;
    std::vector<Tensor> keep;  // the partial buffers, alive until the launch
};

thread_local Pending g_pending;

}  // namespace

void defer_conv_reduce(const ehip_conv_reduce_t& job, const Tensor& partials) {
    g_pending.jobs.push_back(job);
    g_pending.keep.push_back(partials);
}

bool deferred_pending() { return !g_pending.jobs.empty(); }

void flush_deferred() {
    if (g_pending.jobs.empty()) return;
    Pending p;
    std::swap(p, g_pending);
    hip::check(ehip_conv_weight_reduce_f32(p.jobs.data(), int(p.jobs.size()), nullptr),
               "conv weight-gradient reduction");
    // The partial buffers return to the arena here; later work on the same
    // stream is ordered after the launch that reads them.
}

void take_deferred(std::vector<ehip_conv_reduce_t>& jobs, std::vector<Tensor>& keep) {
    jobs = std::move(g_pending.jobs);
    keep = std::move(g_pending.keep);
    g_pending.jobs.clear();
    g_pending.keep.clear();
}

void drop_deferred() {
    g_pending.jobs.clear();
    g_pending.keep.clear();
}

bool grad_adoptable(const Tensor& target) {
    const auto& impl = target.get_impl();
    return impl->requires_grad && (!impl->grad || impl->grad->storage.pending_zero());
}

}  // namespace detail
}  // namespace engine
