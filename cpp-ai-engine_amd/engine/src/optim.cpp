// optim.cpp -- SGD and Adam as one fused kernel per parameter, and
// clip_grad_norm over the device reductions (the reference's src/optim.cpp).
#include "engine/optim.hpp"

#include <algorithm>
#include <cmath>
#include <stdexcept>

#include "detail.hpp"

namespace engine {
namespace optim {

using namespace detail;

Optimizer::Optimizer(std::vector<Tensor> parameters) : params_(std::move(parameters)) {}

void Optimizer::zero_grad() {
    for (Tensor& p : params_) p.zero_grad();
}

SGD::SGD(std::vector<Tensor> parameters, float lr, float momentum, float weight_decay)
    : Optimizer(std::move(parameters)), momentum_(momentum), weight_decay_(weight_decay) {
    if (lr <= 0.0f) throw std::invalid_argument("SGD requires a positive learning rate.");
    if (momentum < 0.0f) throw std::invalid_argument("SGD requires a non-negative momentum.");
    lr_ = lr;
    if (momentum_ != 0.0f)
        for (const Tensor& p : params_) velocity_.emplace_back(p.size(), 0.0f);
}

void SGD::step() {
    autograd::NoGradGuard no_grad;
    for (size_t i = 0; i < params_.size(); ++i) {
        Tensor& p = params_[i];
        if (!p.requires_grad() || !p.has_grad()) continue;
        const Tensor g = p.grad();
        float* vel = momentum_ != 0.0f ? velocity_[i].device_mut() : nullptr;
        hip::check(ehip_sgd_f32(p.storage().device_mut(), dptr(g), vel, int64_t(p.size()), lr_,
                                momentum_, weight_decay_, nullptr),
                   "sgd step");
    }
}

Adam::Adam(std::vector<Tensor> parameters, float lr, float beta1, float beta2, float eps,
           float weight_decay)
    : Optimizer(std::move(parameters)), beta1_(beta1), beta2_(beta2), eps_(eps),
      weight_decay_(weight_decay) {
    if (lr <= 0.0f) throw std::invalid_argument("Adam requires a positive learning rate.");
    if (beta1 < 0.0f || beta1 >= 1.0f || beta2 < 0.0f || beta2 >= 1.0f)
        throw std::invalid_argument("Adam requires beta1 and beta2 in the interval [0, 1).");
    lr_ = lr;
    for (const Tensor& p : params_) {
        m_.emplace_back(p.size(), 0.0f);
        v_.emplace_back(p.size(), 0.0f);
    }
}

// Bias corrections in float with std::pow on the host, then one fused update
// per parameter (src/optim.cpp:113-162).
void Adam::step() {
    autograd::NoGradGuard no_grad;
    // The step count advances only once the update has been launched, so a
    // step whose launch fails leaves the optimiser exactly as it was.
    const size_t t = t_ + 1;
    const float bias_c1 = 1.0f - std::pow(beta1_, static_cast<float>(t));
    const float bias_c2 = 1.0f - std::pow(beta2_, static_cast<float>(t));
    // Every parameter in one multi-tensor launch; the arithmetic per element is
    // the single-tensor update's.
    std::vector<ehip_adam_tensor_t> table;
    table.reserve(params_.size());
    // Weight sums still queued from backward run in the same launch as the
    // update (their gradients are read from the buffers the sums fill, without
    // flushing them first through grad()).
    std::vector<ehip_conv_reduce_t> jobs;
    DeferredKeep keep;
    take_deferred(jobs, keep);
    for (size_t i = 0; i < params_.size(); ++i) {
        Tensor& p = params_[i];
        if (!p.requires_grad() || !p.has_grad()) continue;
        const float* g = p.get_impl()->grad->storage.device();
        table.push_back({p.storage().device_mut(), g, m_[i].device_mut(), v_[i].device_mut(),
                         int64_t(p.size())});
    }
    int rc;
    if (device_scalars_) {
        const float* h = hyper_.device();
        rc = jobs.empty()
                 ? ehip_adam_multi_dev_f32(table.data(), int(table.size()), h, beta1_, beta2_,
                                           eps_, weight_decay_, nullptr)
                 : ehip_adam_multi_reduce_dev_f32(table.data(), int(table.size()), jobs.data(),
                                                  int(jobs.size()), h, beta1_, beta2_, eps_,
                                                  weight_decay_, nullptr);
    } else {
        rc = jobs.empty()
                 ? ehip_adam_multi_f32(table.data(), int(table.size()), lr_, beta1_, beta2_, eps_,
                                       weight_decay_, bias_c1, bias_c2, nullptr)
                 : ehip_adam_multi_reduce_f32(table.data(), int(table.size()), jobs.data(),
                                              int(jobs.size()), lr_, beta1_, beta2_, eps_,
                                              weight_decay_, bias_c1, bias_c2, nullptr);
    }
    if (rc != EHIP_OK) keep.reset_outputs();
    hip::check(rc, "adam step");
    if (!device_scalars_) t_ = t;
}

void Adam::set_device_scalars(bool on) {
    if (on && hyper_.size() != 3) {
        hyper_ = Storage(3, 0.0f);
        (void)hyper_.device_write();
    }
    device_scalars_ = on;
}

void Adam::prepare_replay() {
    if (!device_scalars_) throw std::logic_error("Adam::prepare_replay: device scalars are off");
    const size_t t = t_ + 1;
    const float vals[3] = {lr_, 1.0f - std::pow(beta1_, static_cast<float>(t)),
                           1.0f - std::pow(beta2_, static_cast<float>(t))};
    hip::check(ehip_store_f32(hyper_.device_write(), vals, 3, nullptr), "adam scalars");
    // The launch that follows rewrites the moments on the device.
    for (size_t i = 0; i < m_.size(); ++i) {
        if (m_[i].resident_on_device()) (void)m_[i].device_write();
        if (v_[i].resident_on_device()) (void)v_[i].device_write();
    }
    t_ = t;
}

std::vector<Tensor> Adam::state_tensors() const {
    std::vector<Tensor> out;
    out.reserve(2 * m_.size());
    for (size_t i = 0; i < m_.size(); ++i) {
        out.push_back(view_with_shape(m_[i], {m_[i].size()}, false));
        out.push_back(view_with_shape(v_[i], {v_[i].size()}, false));
    }
    return out;
}

void Adam::set_state(size_t t, const std::vector<Tensor>& moments) {
    if (moments.size() != 2 * m_.size())
        throw std::invalid_argument("Adam::set_state: " + std::to_string(moments.size()) +
                                    " moment tensors for " + std::to_string(m_.size()) +
                                    " parameters.");
    for (size_t i = 0; i < moments.size(); ++i) {
        Storage& dst = (i % 2 == 0) ? m_[i / 2] : v_[i / 2];
        if (moments[i].size() != dst.size())
            throw std::invalid_argument("Adam::set_state: moment " + std::to_string(i) +
                                        " has " + std::to_string(moments[i].size()) +
                                        " values, the optimizer " + std::to_string(dst.size()) +
                                        ".");
        if (dst.size() > 0)
            hip::check(ehip_memcpy_d2d(dst.device_write(), dptr(moments[i]),
                                       dst.size() * sizeof(float), nullptr),
                       "Adam::set_state");
    }
    t_ = t;
}

// src/optim.cpp:168-208: the norm needs one host read (it decides whether to scale).
float clip_grad_norm(const std::vector<Tensor>& parameters, float max_norm) {
    if (max_norm <= 0.0f) throw std::invalid_argument("clip_grad_norm needs a positive max_norm.");
    autograd::NoGradGuard no_grad;
    void* block = nullptr;
    hip::check(ehip_arena_alloc(parameters.size() * sizeof(double) + 8, &block), "clip alloc");
    double* d = static_cast<double*>(block);
    size_t k = 0;
    for (const Tensor& p : parameters) {
        if (!p.has_grad()) continue;
        const Tensor g = p.grad();
        hip::check(ehip_reduce_sum_f32(dptr(g), int64_t(g.size()), 1, d + k, nullptr, nullptr),
                   "clip norm");
        ++k;
    }
    std::vector<double> host(k);
    if (k > 0) hip::check(ehip_memcpy_d2h(host.data(), d, k * sizeof(double), nullptr), "clip read");
    ehip_arena_free(block);
    double total = 0.0;
    for (double v : host) total += v;
    const float norm = static_cast<float>(std::sqrt(total));
    if (norm > max_norm) {
        const float scale = max_norm / (norm + 1e-6f);
        for (const Tensor& p : parameters) {
            if (!p.has_grad()) continue;
            Tensor g = p.grad();
            if (!g.storage().exclusive()) g.storage() = g.storage().clone();
            hip::check(ehip_scale_f32(g.storage().device_mut(), int64_t(g.size()), scale, nullptr),
                       "clip scale");
        }
    }
    return norm;
}

}  // namespace optim
}  // namespace engine

namespace engine {
namespace optim {

// ------------------------------------------------------------------ schedulers
// The reference's src/optim.cpp:214-275; each rate is the same float
// expression, so a schedule matches it value for value.

Scheduler::Scheduler(Optimizer& optimizer)
    : optimizer_(optimizer), base_lr_(optimizer.learning_rate()) {}

void Scheduler::step() {
    ++epoch_;
    optimizer_.set_learning_rate(compute(epoch_));
}

StepLR::StepLR(Optimizer& optimizer, size_t step_size, float gamma)
    : Scheduler(optimizer), step_size_(step_size), gamma_(gamma) {
    if (step_size == 0) throw std::invalid_argument("StepLR needs a positive step_size.");
    if (gamma <= 0.0f) throw std::invalid_argument("StepLR needs a positive gamma.");
}

float StepLR::compute(size_t epoch) const {
    const size_t drops = epoch / step_size_;  // the rate falls in whole steps
    return base_lr_ * std::pow(gamma_, static_cast<float>(drops));
}

CosineAnnealingLR::CosineAnnealingLR(Optimizer& optimizer, size_t total_epochs, float min_lr)
    : Scheduler(optimizer), total_epochs_(total_epochs), min_lr_(min_lr) {
    if (total_epochs == 0) throw std::invalid_argument("CosineAnnealingLR needs at least one epoch.");
    if (min_lr < 0.0f) throw std::invalid_argument("CosineAnnealingLR needs min_lr >= 0.");
}

namespace {
constexpr float kPi = 3.14159265358979f;
float half_cosine(float t) { return 0.5f * (1.0f + std::cos(kPi * t)); }
}  // namespace

float CosineAnnealingLR::compute(size_t epoch) const {
    const float t = std::min(static_cast<float>(epoch) / static_cast<float>(total_epochs_), 1.0f);
    return min_lr_ + (base_lr_ - min_lr_) * half_cosine(t);
}

WarmupCosineLR::WarmupCosineLR(Optimizer& optimizer, size_t warmup_epochs, size_t total_epochs,
                               float min_lr)
    : Scheduler(optimizer),
      warmup_epochs_(warmup_epochs),
      total_epochs_(total_epochs),
      min_lr_(min_lr) {
    if (total_epochs == 0) throw std::invalid_argument("WarmupCosineLR needs at least one epoch.");
    if (warmup_epochs >= total_epochs)
        throw std::invalid_argument("The warm-up must be shorter than the total number of epochs.");
}

float WarmupCosineLR::compute(size_t epoch) const {
    if (epoch < warmup_epochs_)
        return base_lr_ * static_cast<float>(epoch) / static_cast<float>(warmup_epochs_);
    const float t = static_cast<float>(epoch - warmup_epochs_) /
                    static_cast<float>(total_epochs_ - warmup_epochs_);
    return min_lr_ + (base_lr_ - min_lr_) * half_cosine(std::min(t, 1.0f));
}

}  // namespace optim
}  // namespace engine
