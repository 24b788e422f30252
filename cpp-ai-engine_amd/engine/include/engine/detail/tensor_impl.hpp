// tensor_impl.hpp -- the node shared by Tensor handles: buffer, shape and the
// edges of the autograd graph (the reference's
// include/engine/detail/tensor_impl.hpp:26-47). Parents are held by shared_ptr
// and children never are, so the graph frees itself; backward_fn receives the
// output gradient as an argument for the same reason.
#ifndef ENGINE_DETAIL_TENSOR_IMPL_HPP
#define ENGINE_DETAIL_TENSOR_IMPL_HPP

#include <cstdint>
#include <functional>
#include <memory>
#include <vector>

#include "engine/detail/storage.hpp"

namespace engine {

class Tensor;

struct TensorImpl {
    Storage storage;
    std::vector<size_t> shape;
    std::vector<size_t> strides;

    bool requires_grad = false;
    std::shared_ptr<TensorImpl> grad = nullptr;

    std::vector<std::shared_ptr<TensorImpl>> parents;
    std::function<void(const Tensor&)> backward_fn = nullptr;

    // Set by nn::causal_mask on the tensor it returns: the value above the
    // diagonal, and the storage version it was written with (a mask written
    // since then, through this tensor or a view, no longer counts as one).
    float causal_value = 0.0f;
    uint64_t causal_version = ~uint64_t(0);

    TensorImpl() = default;
    TensorImpl(const std::vector<size_t>& s, float fill_val = 0.0f, bool req_grad = false);
    TensorImpl(const std::vector<size_t>& s, const std::vector<float>& d, bool req_grad = false);

    void compute_strides();
    size_t get_flat_index(const std::vector<size_t>& indices) const;
};

}  // namespace engine

#endif  // ENGINE_DETAIL_TENSOR_IMPL_HPP
