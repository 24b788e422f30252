// autograd.cpp -- reverse-mode traversal (the reference's src/autograd.cpp:16-157):
// an iterative depth-first topological order, intermediate gradients cleared
// before the traversal and released once consumed, so a node with a single
// consumer always receives its gradient through add_grad's first write.
#include "engine/autograd.hpp"

#include <stdexcept>
#include <unordered_set>
#include <utility>
#include <vector>

#include "detail.hpp"
#include "engine/tensor.hpp"

namespace engine {
namespace autograd {

namespace {

thread_local bool g_grad_enabled = true;

std::vector<std::shared_ptr<TensorImpl>> topological_sort(const std::shared_ptr<TensorImpl>& root) {
    std::vector<std::shared_ptr<TensorImpl>> order;
    std::unordered_set<TensorImpl*> visited;
    std::vector<std::pair<std::shared_ptr<TensorImpl>, size_t>> stack;
    if (!root) return order;
    stack.emplace_back(root, 0);
    visited.insert(root.get());
    while (!stack.empty()) {
        auto& frame = stack.back();
        const auto& parents = frame.first->parents;
        if (frame.second < parents.size()) {
            const auto& parent = parents[frame.second++];
            if (parent && visited.insert(parent.get()).second) stack.emplace_back(parent, 0);
        } else {
            order.push_back(std::move(frame.first));
            stack.pop_back();
        }
    }
    return order;
}

}  // namespace

bool grad_enabled() { return g_grad_enabled; }
void set_grad_enabled(bool enabled) { g_grad_enabled = enabled; }

NoGradGuard::NoGradGuard() : previous_(g_grad_enabled) { g_grad_enabled = false; }
NoGradGuard::~NoGradGuard() { g_grad_enabled = previous_; }

void backward(Tensor& root_tensor) {
    const auto& root = root_tensor.get_impl();
    if (!root) return;
    if (!root->grad) {
        if (root->storage.size() != 1)
            throw std::runtime_error(
                "An implicit backward() is only allowed on a scalar; the root tensor has shape " +
                root_tensor.shape_str() + ". Use backward(grad_output).");
        root->grad = std::make_shared<TensorImpl>(root->shape, 1.0f, false);
    }
    NoGradGuard no_grad;
    detail::flush_deferred();   // sums still queued by an earlier backward
    std::vector<std::shared_ptr<TensorImpl>> order = topological_sort(root);
    for (const auto& node : order)
        if (node != root && node->backward_fn) node->grad = nullptr;
    try {
        for (auto it = order.rbegin(); it != order.rend(); ++it) {
            const auto& node = *it;
            if (!node->backward_fn || !node->grad) continue;
            if (node == root) {
                node->backward_fn(Tensor::from_impl(node->grad));
            } else {
                // The gradient is handed over, not shared: inside backward_fn it is
                // referenced only by the argument, so add_grad can adopt its buffer.
                const Tensor g = Tensor::from_impl(std::move(node->grad));
                node->grad = nullptr;
                node->backward_fn(g);
            }
        }
        // The weight sums the nodes queued stay queued: the next reader of a
        // gradient flushes them in one launch, or Adam::step runs them with
        // its update.
    } catch (...) {
        detail::drop_deferred();
        throw;
    }
}

}  // namespace autograd
}  // namespace engine
