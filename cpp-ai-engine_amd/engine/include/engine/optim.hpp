// optim.hpp -- optimisers of the training path, mirroring the reference's
// include/engine/optim.hpp (Optimizer, SGD, Adam, clip_grad_norm). The
// learning-rate schedulers are not provided (no configuration uses them).
#ifndef ENGINE_OPTIM_HPP
#define ENGINE_OPTIM_HPP

#include <vector>

#include "engine/detail/storage.hpp"
#include "engine/tensor.hpp"

namespace engine {
namespace optim {

class Optimizer {
public:
    explicit Optimizer(std::vector<Tensor> parameters);
    virtual ~Optimizer() = default;
    virtual void step() = 0;
    void zero_grad();
    float learning_rate() const noexcept { return lr_; }
    void set_learning_rate(float lr) { lr_ = lr; }
    const std::vector<Tensor>& parameters() const noexcept { return params_; }

protected:
    std::vector<Tensor> params_;
    float lr_ = 0.01f;
};

class SGD : public Optimizer {
public:
    SGD(std::vector<Tensor> parameters, float lr = 0.01f, float momentum = 0.0f,
        float weight_decay = 0.0f);
    void step() override;

private:
    float momentum_;
    float weight_decay_;
    std::vector<Storage> velocity_;
};

class Adam : public Optimizer {
public:
    Adam(std::vector<Tensor> parameters, float lr = 0.001f, float beta1 = 0.9f,
         float beta2 = 0.999f, float eps = 1e-8f, float weight_decay = 0.0f);
    void step() override;
    size_t steps() const noexcept { return t_; }
    // Moments and step count for a checkpoint: state_tensors() holds the
    // first and second moments of parameter i at 2i and 2i + 1 (views of the
    // optimizer's buffers); set_state() copies them back (shapes must match).
    std::vector<Tensor> state_tensors() const;
    void set_state(size_t t, const std::vector<Tensor>& moments);
    // For a step captured into a hip::Graph (an engine extension): while on,
    // step() launches an update that reads the step size and both bias
    // corrections from a device array and leaves the step count alone;
    // prepare_replay() computes the next step's three values on the host with
    // step()'s own arithmetic, uploads them and advances the count, before
    // each launch of the captured step. The moments are device-resident after
    // it, as after step().
    void set_device_scalars(bool on);
    void prepare_replay();

private:
    float beta1_;
    float beta2_;
    float eps_;
    float weight_decay_;
    size_t t_ = 0;
    std::vector<Storage> m_;
    std::vector<Storage> v_;
    bool device_scalars_ = false;
    Storage hyper_;  // {lr, bias_c1, bias_c2} on the device
};

// Scales every gradient by max_norm / total_norm when the global L2 norm
// exceeds max_norm; returns the norm (the reference's src/optim.cpp:168-208).
float clip_grad_norm(const std::vector<Tensor>& parameters, float max_norm);

// Learning-rate schedulers (the reference's include/engine/optim.hpp:102-170):
// step() once per epoch sets the optimiser's learning rate for the new epoch.
// Host arithmetic only; the next Adam or SGD step takes the new rate.
class Scheduler {
public:
    explicit Scheduler(Optimizer& optimizer);
    virtual ~Scheduler() = default;
    void step();
    size_t epoch() const noexcept { return epoch_; }
    float base_learning_rate() const noexcept { return base_lr_; }

protected:
    virtual float compute(size_t epoch) const = 0;  // epoch 0 is the initial rate
    Optimizer& optimizer_;
    float base_lr_;
    size_t epoch_ = 0;
};

// base_lr * gamma^(epoch / step_size)
class StepLR : public Scheduler {
public:
    StepLR(Optimizer& optimizer, size_t step_size, float gamma = 0.1f);

protected:
    float compute(size_t epoch) const override;

private:
    size_t step_size_;
    float gamma_;
};

// A cosine from base_lr down to min_lr over total_epochs.
class CosineAnnealingLR : public Scheduler {
public:
    CosineAnnealingLR(Optimizer& optimizer, size_t total_epochs, float min_lr = 0.0f);

protected:
    float compute(size_t epoch) const override;

private:
    size_t total_epochs_;
    float min_lr_;
};

// A linear ramp over warmup_epochs, then a cosine to min_lr at total_epochs.
class WarmupCosineLR : public Scheduler {
public:
    WarmupCosineLR(Optimizer& optimizer, size_t warmup_epochs, size_t total_epochs,
                   float min_lr = 0.0f);

protected:
    float compute(size_t epoch) const override;

private:
    size_t warmup_epochs_;
    size_t total_epochs_;
    float min_lr_;
};

}  // namespace optim
}  // namespace engine

#endif  // ENGINE_OPTIM_HPP
