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

}  // namespace optim
}  // namespace engine

#endif  // ENGINE_OPTIM_HPP
