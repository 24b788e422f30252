// detail.hpp -- helpers shared by the engine's translation units: graph
// tracking, shape arithmetic, the suffix-broadcast plan and the fold of a
// broadcast gradient (the reference's src/tensor_detail.hpp:111-262).
#ifndef ENGINE_SRC_DETAIL_HPP
#define ENGINE_SRC_DETAIL_HPP

#include <cstdint>
#include <initializer_list>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "ehip.h"
#include "engine/autograd.hpp"
#include "engine/hip.hpp"
#include "engine/tensor.hpp"

namespace engine {
namespace detail {

inline bool track(bool requires_grad) { return requires_grad && autograd::grad_enabled(); }

inline size_t product(const std::vector<size_t>& dims, size_t from = 0) {
    size_t total = 1;
    for (size_t i = from; i < dims.size(); ++i) total *= dims[i];
    return total;
}

// Suffix broadcast: `other`, stripped of leading 1s, must equal the trailing
// axes of `base`; it then repeats `repeat` times over blocks of `inner`.
struct BroadcastPlan {
    bool valid = false;
    size_t inner = 1;
    size_t repeat = 1;
};

inline BroadcastPlan plan_broadcast(const std::vector<size_t>& base,
                                    const std::vector<size_t>& other) {
    BroadcastPlan plan;
    size_t first = 0;
    while (first < other.size() && other[first] == 1) ++first;
    const size_t core = other.size() - first;
    if (core > base.size()) return plan;
    const size_t offset = base.size() - core;
    for (size_t i = 0; i < core; ++i)
        if (base[offset + i] != other[first + i]) return plan;
    plan.valid = true;
    plan.inner = product(base, offset);
    plan.repeat = plan.inner == 0 ? 0 : product(base) / plan.inner;
    return plan;
}

inline const float* dptr(const Tensor& t) { return t.storage().device(); }

// add_grad of g into `target`, where g has the target's element count but may
// carry another shape (the backward of a reshape): g's buffer is adopted under
// the target's shape when nothing else references it. Defined in tensor.cpp.
void add_grad_reshaped(Tensor& target, const Tensor& g);
// The device buffer of target's gradient when a product can add into it in
// place (beta = 1: grad + product, the sum add_grad would form, bit for bit):
// the gradient exists, holds values (not a pending zero) and is referenced by
// nothing else. Otherwise nullptr, and the caller goes through add_grad.
float* grad_in_place(Tensor& target);
inline float* dout(Tensor& t) { return t.storage().device_write(); }

// A row gather in device form (the forward of select_rows and Embedding): the
// source row of every output row and, for the backward's ordered scatter, the
// inverse map in CSR form (row_ptr over the table's rows, positions ascending
// within each row). Built on the host from validated indices, then only read,
// so one index can serve every step of a resident batch.
struct RowGather {
    DeviceInts idx, row_ptr, pos;
    size_t n = 0, rows = 0;
    bool inverse = false;
};
std::shared_ptr<const RowGather> make_row_gather(const std::vector<size_t>& indices, size_t rows,
                                                 const std::string& shape_str, bool with_inverse);
Tensor gather_rows(const Tensor& table, const std::shared_ptr<const RowGather>& g);

// Gradient work queued during backward: the weight-gradient sums of fused
// convolution blocks and the dgamma / dbeta sums of large LayerNorms
// (deferred.cpp). The queue is flushed -- one launch for every queued job --
// before anything can read or change a queued gradient: Tensor::grad(),
// zero_grad(), the start of autograd::backward, add_grad when it accumulates
// into or from a buffer a queued job writes, and a product that adds in place
// into such a buffer; Adam::step instead takes the jobs into its own launch. A
// gradient may be queued only when add_grad will adopt its buffer
// (grad_adoptable).
//
// The queue owns everything its launch touches: the partials it reads (given
// to defer_conv_reduce) and the buffers it writes (registered by
// defer_conv_output after add_grad has adopted them, with the parameter that
// holds each). So a model destroyed before the flush leaves the sums writing
// into buffers that are still alive, never into released arena blocks. When
// queued work is abandoned (an exception in backward, or a failed Adam
// launch), every gradient it would have written that is still the parameter's
// gradient goes back to a pending zero -- the state it had before the
// backward, since only a gradient that was absent or a pending zero is queued.
struct DeferredKeep {
    std::vector<Tensor> partials;
    std::vector<std::pair<std::weak_ptr<TensorImpl>, Storage>> outputs;
    void reset_outputs();
};
void defer_conv_reduce(const ehip_conv_reduce_t& job, const Tensor& partials);
void defer_conv_output(const Tensor& param, const Tensor& grad);
// Queues a product (a narrow weight gradient and its bias sum: a descriptor
// ehip_gemm_groupable accepts) whose operands `inputs` hold; its outputs are
// registered with defer_conv_output like a reduction's. Queued products run
// before the queued reductions, all in as few launches as ehip_gemm_batch_f32
// allows.
void defer_product(const ehip_gemm_ex_t& desc, std::initializer_list<Tensor> inputs);
bool deferred_pending();
// True when a queued job writes the buffer of `s` (a registered output).
bool deferred_writes(const Storage& s);
// Before an in-place write into the buffer: runs the queue when queued work
// writes it, or only the queued products when one reads it.
void settle_deferred(const Storage& s);
void flush_deferred();
void drop_deferred();
// Moves the queued jobs (and the buffers they touch) to the caller, which must
// launch them before releasing `keep` (and call keep.reset_outputs() if the
// launch fails).
void take_deferred(std::vector<ehip_conv_reduce_t>& jobs, DeferredKeep& keep);
// True when add_grad of a fresh, unshared gradient buffer into `target` adopts
// that buffer (no gradient yet, or a pending zero).
bool grad_adoptable(const Tensor& target);
// The device buffer of `target`'s gradient when add_grad of a gradient into it
// would add in place (a gradient is held, not a pending zero, and not shared),
// after finishing any queued sum that writes it; else nullptr. A kernel that
// adds its result into this buffer replaces the add_grad call.
float* grad_in_place(const Tensor& target);

// A tensor viewing `src` with a new shape (no copy).
inline Tensor view_with_shape(const Storage& src, const std::vector<size_t>& shape, bool req) {
    auto impl = std::make_shared<TensorImpl>();
    impl->storage = src.share();
    impl->shape = shape;
    impl->compute_strides();
    impl->requires_grad = req;
    return Tensor::from_impl(impl);
}

// Sum of `full` over its leading blocks down to `target` (src/tensor_detail.hpp:182-206).
inline Tensor fold_leading(const Tensor& full, const std::vector<size_t>& target) {
    const size_t inner = product(target);
    const size_t repeat = inner == 0 ? 0 : full.size() / inner;
    Tensor folded(target, 0.0f, false);
    hip::check(ehip_sum_axis_f32(dptr(full), dout(folded), 1, int64_t(repeat), int64_t(inner),
                                 nullptr),
               "fold_leading");
    return folded;
}

// out[o][a][i] = g[o][i]: the gradient of a sum over the middle axis, as a
// strided move (stride 0 over the summed axis).
inline Tensor broadcast_middle(const Tensor& g, const std::vector<size_t>& out_shape,
                               size_t outer, size_t axis_len, size_t inner) {
    Tensor out(out_shape, 0.0f, false);
    const int64_t shape[3] = {int64_t(outer), int64_t(axis_len), int64_t(inner)};
    const int64_t strides[3] = {int64_t(inner), 0, 1};
    hip::check(ehip_permute_f32(dptr(g), dout(out), 3, shape, strides, nullptr), "broadcast");
    return out;
}

}  // namespace detail
}  // namespace engine

#endif  // ENGINE_SRC_DETAIL_HPP
