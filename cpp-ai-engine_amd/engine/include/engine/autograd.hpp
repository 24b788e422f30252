// autograd.hpp -- define-by-run reverse mode (the reference's
// include/engine/autograd.hpp:17-36 and src/autograd.cpp:104-157).
#ifndef ENGINE_AUTOGRAD_HPP
#define ENGINE_AUTOGRAD_HPP

namespace engine {

class Tensor;

namespace autograd {

bool grad_enabled();
void set_grad_enabled(bool enabled);

class NoGradGuard {
public:
    NoGradGuard();
    ~NoGradGuard();
    NoGradGuard(const NoGradGuard&) = delete;
    NoGradGuard& operator=(const NoGradGuard&) = delete;

private:
    bool previous_;
};

void backward(Tensor& root_tensor);

}  // namespace autograd
}  // namespace engine

#endif  // ENGINE_AUTOGRAD_HPP
