/*
 * ehip.h -- the C ABI of the MI355X (gfx950) backend for cpp-ai-engine's fp32
 * training path.
 *
 * This is the drop-in boundary. It replaces the reference's device seam
 * `engine::cuda::ops` (include/engine/detail/cuda_ops.hpp:25-203), its runtime
 * control API (include/engine/cuda.hpp:23-218) and its memory primitives
 * (include/engine/cuda.hpp:229-236). Paths in citations are relative to the
 * reference repository root.
 *
 * Conventions
 *   - Every pointer argument named like a tensor is a DEVICE pointer to fp32
 *     (or int32 where stated), row-major and contiguous unless a leading
 *     dimension says otherwise. Shape and geometry arguments are host values.
 *   - `stream` is a hipStream_t passed as void*; NULL is the null stream. Work
 *     is ordered on that stream; nothing here synchronises unless stated.
 *   - Every entry point returns an int status: EHIP_OK (0) when the work was
 *     enqueued, nonzero when it was refused (bad geometry, backend disabled)
 *     or failed to launch. No C++ exception crosses this boundary.
 *     ehip_last_error() gives the message of the last failure on the calling
 *     thread. This is the reference's bool contract (true = the device took the
 *     work, cuda_ops.hpp:14-23) with the reason kept.
 *   - Results that the reference CPU path produces bit-for-bit (moves, index
 *     maps, ordered sums, element-wise arithmetic without fused multiply-add,
 *     the optimiser updates) are produced bit-for-bit here; the comment of each
 *     entry point says which it is.
 */
#ifndef EHIP_H
#define EHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ----------------------------------------------------------------- status */

enum {
    EHIP_OK = 0,
    EHIP_EINVAL = 1,   /* refused: bad geometry, null pointer, size limit  */
    EHIP_ELAUNCH = 2,  /* the kernel launch failed                         */
    EHIP_ENODEV = 3,   /* no usable gfx950 device                          */
    EHIP_ENOMEM = 4,   /* device allocation failed                         */
    EHIP_EDISABLED = 5 /* the backend was switched off (ehip_set_enabled)  */
};

/* Message of the last nonzero status returned on this thread ("" if none). */
const char* ehip_last_error(void);

/* ---------------------------------------------------------------- runtime */

/* Selects device 0, checks that it is gfx950 and builds the context. Called
 * implicitly by every other entry point. Replaces cuda::available()
 * (include/engine/cuda.hpp:23; src/cuda/runtime.cu:77-151). */
int ehip_init(void);
int ehip_available(void);

/* Runtime switch: when off, every kernel entry point returns EHIP_EDISABLED
 * without launching (cuda::enabled/set_enabled, include/engine/cuda.hpp:28-29).
 * The environment variable ENGINE_HIP=0 starts the process switched off. */
int ehip_enabled(void);
void ehip_set_enabled(int on);

typedef struct {
    char name[256];
    char arch[64];              /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int compute_units;
    int clock_khz;              /* peak engine clock                          */
    int memory_clock_khz;
    int memory_bus_width_bits;
    size_t total_memory;
    size_t lds_per_block;
    int l2_bytes;
    double peak_fp32_mfma_gflops; /* CUs x 256 FLOP/clk x clock            */
    double peak_hbm_gbs;          /* 2 x memory clock x bus width / 8      */
} ehip_device_info_t;

/* cuda::device_info, peak_fp32_gflops, peak_bandwidth_gbs
 * (include/engine/cuda.hpp:49, 93-95). */
int ehip_device_info(ehip_device_info_t* out);

/* The HIP versions in play, in HIP's encoding (major * 10000000 + minor *
 * 100000 + patch): the headers this library was compiled with, the runtime
 * and the driver it runs on (cuda::compiled_version / runtime_version /
 * driver_version, include/engine/cuda.hpp:67-69). A query the runtime cannot
 * answer leaves 0 there and returns its error. */
int ehip_version_info(int* compiled, int* runtime, int* driver);

/* The static occupancy of the library's main kernels on this device
 * (cuda::kernel_occupancy, include/engine/cuda.hpp:100-125): for each, the block
 * size it is launched with, VGPRs per lane, static LDS per block, the blocks
 * that fit on one CU at once (hipOccupancyMaxActiveBlocksPerMultiprocessor),
 * the resident waves that makes as a fraction of the CU's maximum, and the
 * resource that runs out first ("registers", "lds" or "waves"). The ceiling,
 * not the achieved occupancy. Writes at most `capacity` entries and the number
 * available to *count. */
typedef struct {
    char name[96];
    int block_threads;
    int registers;
    int64_t lds_bytes;
    int blocks_per_cu;
    double occupancy;
    char limiter[16];
} ehip_kernel_occupancy_t;
int ehip_kernel_occupancy(ehip_kernel_occupancy_t* out, int capacity, int* count);

/* Waits for all work on the device (cuda::synchronize, include/engine/cuda.hpp:53). */
int ehip_synchronize(void);
/* Waits for one stream. */
int ehip_stream_synchronize(void* stream);

/* Launch counters (cuda::kernels_launched/failed/reset_kernel_counters,
 * include/engine/cuda.hpp:79-81). */
uint64_t ehip_kernels_launched(void);
uint64_t ehip_kernels_failed(void);
void ehip_reset_counters(void);

/* Failure injection for tests: the n-th kernel launch counted from this call
 * (n >= 1) is refused with EHIP_ELAUNCH and counted as failed, as
 * ENGINE_HIP_FAIL_LAUNCH=n does from process start; n = 0 turns it off. The
 * run-time form of the reference's launch-failure path (launch_ok,
 * src/cuda/kernels.cu:81-157), which its parity tests reach by refusing a
 * kernel configuration. */
void ehip_fail_launch_after(int64_t n);

typedef struct {
    uint64_t to_device_bytes, to_host_bytes, device_to_device_bytes;
    uint64_t to_device_count, to_host_count, device_to_device_count;
    double to_device_seconds, to_host_seconds;
} ehip_transfer_stats_t;

/* cuda::transfer_stats / reset_transfer_stats (include/engine/cuda.hpp:209-218). */
void ehip_transfer_stats(ehip_transfer_stats_t* out);
void ehip_reset_transfer_stats(void);

/* ------------------------------------------------------- HBM arena, copies */

/* Pooled device allocator: sizes are rounded up to a size class (256-byte
 * granules, then quarter-powers of two), freed blocks are cached per class
 * and reused, and nothing goes back to the driver until ehip_arena_trim().
 * Freeing is stream-ordered with respect to the engine's one stream: a block
 * freed while queued kernels still use it is only handed to later work on the
 * same stream. Replaces cuda::detail::device_alloc/device_free
 * (include/engine/cuda.hpp:229-230; src/cuda/runtime.cu:137-143, 352-387) and
 * the host BufferPool (src/storage.cpp:44-128). */
int ehip_arena_alloc(size_t bytes, void** out);
void ehip_arena_free(void* ptr);
int ehip_arena_trim(void);

typedef struct {
    uint64_t bytes_in_use;     /* rounded sizes of live blocks      */
    uint64_t bytes_cached;     /* rounded sizes of cached free blocks */
    uint64_t bytes_reserved;   /* everything obtained from the driver */
    uint64_t allocations;      /* ehip_arena_alloc calls              */
    uint64_t driver_allocations; /* misses that reached hipMalloc    */
    uint64_t bytes_graph_held; /* part of bytes_cached held for graphs */
} ehip_arena_stats_t;
void ehip_arena_stats(ehip_arena_stats_t* out);

/* ------------------------------------------------------------ graph capture */

/* Captures a sequence of library calls as one HIP graph and replays it with a
 * single launch. No counterpart in the reference, whose training step is a
 * host loop of launches (src/optim.cpp:113-162, src/autograd.cpp): these are
 * for launch-bound steps (a small model's forward, backward and update).
 *
 * ehip_graph_begin() starts recording on a non-blocking stream of the calling
 * thread: from then on every call of this thread made with a NULL stream is
 * recorded into the graph instead of being run (calls naming a stream of
 * their own still go to it). Refused while capturing: host-to-device and
 * device-to-host copies on the capture, ehip_synchronize, ehip_arena_trim and
 * nested captures (each returns EHIP_EINVAL and leaves the capture going).
 * ehip_graph_end() stops recording and instantiates the graph into *graph;
 * ehip_graph_abort() drops a capture. ehip_graph_launch() replays it on
 * `stream` (NULL: the null stream, ordered with the library's other work), and
 * ehip_graph_destroy() waits for the device and frees it.
 *
 * Kernel arguments (pointers, sizes, scalars) are fixed at capture time: a
 * replay reads and writes the same buffers. The arena keeps those buffers
 * valid: a block live when the capture began, or handed out during it, is
 * held for the graph once freed (not handed to anyone else) until the graph
 * is destroyed. Values a replay must see change (Adam's step size and bias
 * corrections) are read from device memory instead (ehip_adam_multi_dev_f32).
 */
int ehip_graph_begin(void);
int ehip_graph_end(void** graph);
int ehip_graph_abort(void);
int ehip_capturing(void);
int ehip_graph_launch(void* graph, void* stream);
int ehip_graph_destroy(void* graph);

/* Copies of `bytes` bytes (cuda::detail::copy_to_device/copy_to_host/
 * copy_device_to_device, include/engine/cuda.hpp:231-236). All three are
 * ordered on `stream`. Host-to-device returns once the host buffer may be
 * reused: uploads up to 16 MiB are staged through a pinned ring and complete
 * asynchronously; larger ones wait for the stream. Device-to-host waits for
 * the stream and returns with the data in place. Device-to-device is
 * asynchronous. */
int ehip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int ehip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int ehip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);

/* ------------------------------------------------------------ dense GEMM */

/* C[b] = op(A[b]) . op(B[b]) + beta * C[b], b in [0, batch).
 * op(A) is m x k: A is m x k (lda >= k) when trans_a == 0, or k x m (lda >= m)
 * when trans_a != 0; likewise op(B) is k x n. stride_* is the element distance
 * between batch matrices; 0 shares one matrix across the batch (the reference's
 * unbatched operand). beta == 0 overwrites C without reading it.
 * fp32 MFMA (v_mfma_f32_32x32x2f32) with LDS-staged tiles; deterministic (a
 * fixed summation order per shape), not bit-equal to the CPU's serial sums.
 * Replaces cuda::ops::matmul (include/engine/detail/cuda_ops.hpp:46-47); the
 * transposed modes replace the materialised transposes of the backward pass
 * (src/tensor_ops.cpp:570-585). */
int ehip_gemm_f32(int trans_a, int trans_b, int64_t batch, int64_t m, int64_t n, int64_t k,
                  const float* a, int64_t lda, int64_t stride_a, const float* b, int64_t ldb,
                  int64_t stride_b, float beta, float* c, int64_t ldc, int64_t stride_c,
                  void* stream);

/* The backward of C = A . B for 2-D operands (A m x k, B k x n, dC m x n):
 * dA = dC . B^T + beta_a * dA (m x k) when da is not NULL, and
 * dB = A^T . dC + beta_b * dB (k x n) when db is not NULL. When both products
 * take the K-sliced 32 x 32 tiles they run as two block ranges of one launch,
 * which halves the fixed cost of a kernel boundary (the cache write-back and
 * invalidation, the first loads' latency) for small products; otherwise they
 * are ehip_gemm_f32's two calls. Same bits as those calls either way.
 * Replaces the two products of the matmul backward lambda
 * (src/tensor_ops.cpp:565-586), without its materialised transposes. */
int ehip_matmul_backward_f32(int64_t m, int64_t k, int64_t n, const float* a, int64_t lda,
                             const float* b, int64_t ldb, const float* dc, int64_t lddc, float* da,
                             int64_t ldda, float beta_a, float* db, int64_t lddb, float beta_b,
                             void* stream);

/* ehip_gemm_f32 without any device allocation: the same arguments, the same
 * kernels and tile plan (so the same bits), with the split-K partials kept in
 * a fixed 32 MiB device array that the library holds on each GPU it runs on
 * until the process ends, instead of the library's grow-only scratch. No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). A product whose split-K plan needs more than 32 MiB of
 * partials is refused with EHIP_EINVAL before anything is launched. Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller. */
int ehip_gemm_f32_noalloc(int trans_a, int trans_b, int64_t batch, int64_t m, int64_t n,
                          int64_t k, const float* a, int64_t lda, int64_t stride_a,
                          const float* b, int64_t ldb, int64_t stride_b, float beta, float* c,
                          int64_t ldc, int64_t stride_c, void* stream);

/* ehip_gemm_f32 with two-level batch strides and an epilogue, for products
 * that read and write attention heads in place. Product z in [0, batch) uses
 *   A at a + (z / inner) * stride_a + (z % inner) * stride_a_inner
 * (likewise B and C), so that z = (sample, head) walks the heads of a
 * (batch, seq, heads * head_dim) activation with ld = heads * head_dim and no
 * permuted copy (the reshape + permute({0, 2, 1, 3}) of
 * src/transformer.cpp:320-349). The result is stored as
 *   c = acc;  c = c * alpha (alpha != 1);  c = c + addend[z % addend_period]
 *   [i * ld_addend + j] (addend != NULL);  c = c + beta * c_old (beta != 0),
 * each step rounded to fp32 on its own -- the separate `scores * scale` and
 * `scores + mask` nodes of src/transformer.cpp:285-291, bit for bit; an
 * addend with ld_addend 0 is Linear's broadcast bias add (src/nn.cpp:119-122).
 * Then, with residual != NULL (batch 1), c = c + residual[i * ld_residual + j]:
 * the residual add that follows a block's output projection or feed-forward
 * (src/transformer.cpp:409-414; the add commutes, so the same bits). Then,
 * when relu != 0, c = (0 < c) ? c : 0, std::max(0.0f, c) of Tensor::relu
 * (src/tensor_ops.cpp:591-600).
 * colsum_b, when not NULL (batch 1, trans_b 0), receives the n column sums
 * of B over its k rows -- for dW = X^T dY the bias gradient sum_rows(dY) of
 * Linear's broadcast add (src/tensor_ops.cpp:81-102 through fold_leading,
 * src/tensor_detail.hpp:182-206) -- made from the B tiles the product stages
 * anyway: fixed order (k within each K step, the steps, then the K splits),
 * deterministic, within the K-term tolerance of the reference's serial sum.
 * addend_period >= 1; consecutive addend matrices are stride_addend apart
 * (stride_addend 0 broadcasts one mask over every product, ld_addend 0 one
 * row over every row). inner >= 1. With k == 0, acc is 0 and the epilogue
 * still runs.
 * causal lets the caller of a causal-attention product skip work whose
 * result it does not need or knows to be zero; each mode holds per product
 * matrix, with i the row and j the column of C, and k the reduction index:
 *   1  elements with j > i are don't-cares: tiles lying wholly above the
 *      diagonal skip their products and store the epilogue of acc = 0 (the
 *      addend where there is one, else 0);
 *   2  op(A)(i, k) = 0 whenever k > i: products past a tile's last row are
 *      skipped;
 *   3  op(A)(i, k) = 0 whenever k < i: products before a tile's first row are
 *      skipped;
 *   4  as 1, but tiles lying wholly above the diagonal are not stored at all
 *      (their C elements keep whatever they held; where another kernel or a
 *      split K computes the product they are stored as in mode 1), for a
 *      consumer that never reads j > i: the causal softmax pair below.
 * Skipped products are exact zeros, so every result keeps its value (its bits,
 * but for the sign of a sum that is exactly zero) as long as the operands are
 * finite; 0 computes everything. Honoured by the staged MFMA tiles; the other
 * kernels compute everything. (No counterpart in the reference, which
 * computes and then masks: src/transformer.cpp:279-304.) */
typedef struct {
    int trans_a, trans_b;
    int64_t batch, inner;
    int64_t m, n, k;
    const float* a;
    int64_t lda, stride_a, stride_a_inner;
    const float* b;
    int64_t ldb, stride_b, stride_b_inner;
    float* c;
    int64_t ldc, stride_c, stride_c_inner;
    float alpha;
    const float* addend;
    int64_t ld_addend, stride_addend, addend_period;
    float beta;
    int relu;
    float* colsum_b;
    int causal;
    const float* residual;  /* batch 1: v += residual[i * ld_residual + j], after beta C */
    int64_t ld_residual;
} ehip_gemm_ex_t;

int ehip_gemm_ex_f32(const ehip_gemm_ex_t* desc, void* stream);

/* Independent products in as few launches as their kernels allow: the narrow
 * weight-gradient products (the A^T B panel kernel: trans_a, batch 1, few 16 x
 * 16 output tiles over a long K; ehip_gemm_groupable says 1) run together,
 * up to 12 per launch, and so do untransposed batch-1 products small enough
 * for the K-sliced 32 x 32 tiles (several projections of one input), up to
 * 12 of one kernel form per launch; every other descriptor runs as its own
 * ehip_gemm_ex_f32 call. Each product's result, column sums included, has the
 * bits of its own ehip_gemm_ex_f32 call. The products must be independent (no
 * output read or written by another of the list). For engines that queue the
 * weight gradients of a backward and run them together (launch-bound small
 * models); no counterpart in the reference. */
int ehip_gemm_groupable(const ehip_gemm_ex_t* desc);
int ehip_gemm_batch_f32(const ehip_gemm_ex_t* descs, int count, void* stream);

/* Timing probe for chosen products inside a real workload (measurement only; no
 * counterpart in the reference). ehip_gemm_probe_arm: from now on, every product
 * of batch 1 with these trans_a / trans_b and (m, n, k) among `count` triples of
 * `shapes` is bracketed by a pair of events recorded on its own stream -- the
 * tile kernel and its split-K reduction inside -- for up to max_products
 * products (events created here, on the host; refused while armed).
 * ehip_gemm_probe_read waits for the last event, returns the summed GPU time in
 * ms, the number of products and their 2 m n k FLOPs, and disarms. Event
 * records ride the products' streams, so calls made under stream capture
 * record them into the graph: arm only around eager work. */
int ehip_gemm_probe_arm(int trans_a, int trans_b, const int64_t* shapes, int count,
                        int max_products);
int ehip_gemm_probe_read(double* ms, int64_t* products, double* flop);

/* The three gradients of Linear, y = x . w + b with x (rows, in), w (in,
 * out), dy (rows, out): dx = dy . w^T, dw = x^T . dy, db = the column sums of
 * dy -- the matmul backward and the broadcast add's backward through
 * fold_leading (src/tensor_ops.cpp:565-586, 81-102; src/tensor_detail.hpp:
 * 182-206). dx and dw equal what ehip_gemm_f32 computes for them bit for
 * bit; when all requested parts are small (thread-per-output products, a
 * serial column sum) they run in one launch. db is ehip_sum_axis_f32's, except
 * for mid-sized layers (more than 64 rows, dy of at most 2^21 elements, fewer
 * than 16384 columns, dw requested too, and a dw product that takes staged
 * MFMA tiles either way), where it is the column sums of dy that the dw
 * product forms from the tiles it stages (ehip_gemm_ex_f32's colsum_b): the
 * same sums in another order, two launches fewer. dx, dw and db may each be
 * NULL. */
int ehip_linear_backward_f32(const float* x, const float* w, const float* dy, float* dx,
                             float* dw, float* db, int64_t rows, int64_t in, int64_t out,
                             void* stream);

/* Switches the mid-sized-layer bias gradients of ehip_linear_backward_f32
 * between the dw product's column sums (on = 1, the default) and the separate
 * column sum (on = 0); on < 0 only queries. Returns the previous setting.
 * Process-wide; no counterpart in the reference (its fold is always separate,
 * src/tensor_detail.hpp:196-204). */
int ehip_linear_bias_from_dw(int on);
/* 1 when ehip_linear_backward_f32 of rows x in -> out takes db from the dW
 * product's column sums (ehip_gemm_ex_t.colsum_b), 0 when it sums dy apart. */
int ehip_linear_backward_plan(int64_t rows, int64_t in, int64_t out);

/* --------------------------------------------------------- element-wise */

enum { EHIP_ADD = 0, EHIP_SUB = 1, EHIP_MUL = 2, EHIP_DIV = 3 };

/* out[r*inner + j] = a[r*inner + j] op b[j], r < repeat (suffix broadcast).
 * Bit-exact. cuda::ops::binary (cuda_ops.hpp:30-31). */
int ehip_binary_f32(int op, const float* a, const float* b, float* out, int64_t inner,
                    int64_t repeat, void* stream);

/* out = x * mul + add (two roundings, no fma). Bit-exact.
 * cuda::ops::scalar (cuda_ops.hpp:67). */
int ehip_scalar_f32(const float* x, float* out, int64_t n, float mul, float add, void* stream);

/* y = (0 < x) ? x : 0 and dx = (x > 0) ? g : 0. Bit-exact.
 * cuda::ops::relu / relu_backward (cuda_ops.hpp:49-50). */
int ehip_relu_f32(const float* x, float* y, int64_t n, void* stream);
int ehip_relu_backward_f32(const float* x, const float* g, float* dx, int64_t n, void* stream);

/* y = f(x) and dx = g * f'(x, y) for the smooth activations of nn::Sigmoid,
 * nn::Tanh and nn::GELU (src/nn.cpp:154-198 of the reference, which runs
 * them on the host only): sigmoid in the reference's two-branch stable form,
 * tanh, and GELU's tanh approximation 0.5 x (1 + tanh(sqrt(2/pi) (x +
 * 0.044715 x^3))), each evaluated in the reference's order; exp and tanh are
 * the device library's (a few ulp from the host's). */
enum { EHIP_SIGMOID = 0, EHIP_TANH = 1, EHIP_GELU = 2 };
int ehip_activation_f32(int kind, const float* x, float* y, int64_t n, void* stream);
int ehip_activation_backward_f32(int kind, const float* x, const float* y, const float* g,
                                 float* dx, int64_t n, void* stream);

/* For r < rows: dst[r * dst_pitch + j] = src[r * src_pitch + j], j < len. The
 * moves of Tensor::slice, concat and stack and of their backward passes
 * (src/tensor.cpp:428-552: per outer index, a run of count x inner floats).
 * Bit-exact. */
int ehip_copy_rows_f32(const float* src, int64_t src_pitch, float* dst, int64_t dst_pitch,
                       int64_t rows, int64_t len, void* stream);

/* Tensor::max(axis) over x viewed as (outer, axis_len, inner)
 * (src/tensor.cpp:383-424): y[o][i] = the first maximum along the axis
 * (strict >, in axis order, so a leading NaN stays), argmax[o][i] its axis
 * index; backward dx = 0 + g at the winning position, 0 elsewhere. Bit-exact. */
int ehip_max_axis_f32(const float* x, float* y, int32_t* argmax, int64_t outer, int64_t axis_len,
                      int64_t inner, void* stream);
int ehip_max_axis_backward_f32(const float* g, const int32_t* argmax, float* dx, int64_t outer,
                               int64_t axis_len, int64_t inner, void* stream);

/* grad = g (initialize != 0) or grad += g. Bit-exact.
 * cuda::ops::accumulate_grad (cuda_ops.hpp:61). */
int ehip_accumulate_grad_f32(float* grad, const float* g, int64_t n, int initialize,
                             void* stream);

/* The backward of y = a * b (same shapes) in one pass: da = g * b and db = g * a,
 * each product rounded, then added to the existing gradient when accumulate_*
 * is set (otherwise written); either of da / db may be NULL. Replaces the two
 * products and two add_grad calls of the multiply node's backward
 * (src/tensor_ops.cpp:199-213): the same bits, one launch. */
int ehip_mul_backward_f32(const float* g, const float* a, const float* b, float* da, float* db,
                          int64_t n, int accumulate_a, int accumulate_b, void* stream);

/* The backward of out = a + b for same-shape operands, fused: the upstream
 * gradient g goes to both operand gradients in one pass, each either
 * initialised (accumulate_* == 0: da = g) or accumulated (da += g).
 * Bit-exact. Replaces the two accumulate_grad launches of the add node
 * (src/tensor_ops.cpp:81-102 -> src/tensor.cpp:168-203). */
int ehip_add_backward_f32(const float* g, float* da, float* db, int64_t n, int accumulate_a,
                          int accumulate_b, void* stream);

/* x[i] = value. A kernel, not a memset, so it is safe inside graph capture. */
int ehip_fill_f32(float* x, int64_t n, float value, void* stream);

/* dst[i] = values[i] for i < count <= 16, `values` a HOST array whose floats
 * travel in the kernel's arguments: a handful of values stored with one
 * launch and no host-to-device transfer, so also recordable into a graph.
 * No counterpart in the reference; it sets the device scalars of a captured
 * step (Adam's step size and bias corrections) before each replay. */
int ehip_store_f32(float* dst, const float* values, int count, void* stream);

/* x *= factor in place. cuda::ops::scale_in_place (cuda_ops.hpp:144). */
int ehip_scale_f32(float* x, int64_t n, float factor, void* stream);

/* ------------------------------------------------------------- optimisers */

/* SGD with optional momentum and weight decay, in place; velocity may be NULL
 * when momentum == 0. Bit-exact with src/optim.cpp:71-84.
 * cuda::ops::sgd_step (cuda_ops.hpp:165-166). */
int ehip_sgd_f32(float* p, const float* g, float* velocity, int64_t n, float lr, float momentum,
                 float weight_decay, void* stream);

/* Adam in place: m = b1 m + (1-b1) g; v = b2 v + (1-b2) g g;
 * p -= lr (m/c1) / (sqrt(v/c2) + eps). bias_c1/bias_c2 come from the host
 * (1 - pow(beta, t) in float, src/optim.cpp:119-120). Bit-exact with
 * src/optim.cpp:147-160. cuda::ops::adam_step (cuda_ops.hpp:167-168). */
int ehip_adam_f32(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1,
                  float beta2, float eps, float weight_decay, float bias_c1, float bias_c2,
                  void* stream);

/* One parameter tensor of a multi-tensor Adam step (DEVICE pointers). */
typedef struct {
    float* p;
    const float* g;
    float* m;
    float* v;
    int64_t n;
} ehip_adam_tensor_t;

/* The Adam update of ehip_adam_f32 applied to `count` tensors in ONE launch:
 * `tensors` is a HOST array (copied to the device, stream-ordered, before the
 * call returns). Element for element the same arithmetic as ehip_adam_f32,
 * so bit-exact with src/optim.cpp:147-160. Replaces the per-parameter loop of
 * Adam::step (src/optim.cpp:122-161), which launches once per parameter. */
int ehip_adam_multi_f32(const ehip_adam_tensor_t* tensors, int count, float lr, float beta1,
                        float beta2, float eps, float weight_decay, float bias_c1,
                        float bias_c2, void* stream);

/* ehip_adam_multi_f32 with lr, bias_c1 and bias_c2 read by the kernel from the
 * DEVICE array hyper[3] = {lr, bias_c1, bias_c2} when it runs, so that a
 * captured graph (ehip_graph_begin) takes each replay's values from memory the
 * host refreshes before the launch. The same bits as ehip_adam_multi_f32 given
 * the same three values. No counterpart in the reference (whose Adam::step,
 * src/optim.cpp:113-162, passes them by value); for captured training steps.
 * Tables beyond 48 tensors are written by kernels whose arguments carry them,
 * so a capture records no host transfer. */
int ehip_adam_multi_dev_f32(const ehip_adam_tensor_t* tensors, int count, const float* hyper,
                            float beta1, float beta2, float eps, float weight_decay,
                            void* stream);

/* ------------------------------------------------------ layout and index maps */

/* out[flat] = x[sum_d coord_d(flat, out_shape) * src_strides[d]], ndim <= 8.
 * out_shape and src_strides are HOST arrays. A pure move: bit-exact.
 * cuda::ops::permute (cuda_ops.hpp:75-76). */
int ehip_permute_f32(const float* x, float* out, int ndim, const int64_t* out_shape,
                     const int64_t* src_strides, void* stream);

/* out[b][j][i] = x[b][i][j]: the last-two-axes transpose, LDS-tiled.
 * Bit-exact (src/tensor_ops.cpp:335-370). */
int ehip_transpose_f32(const float* x, float* out, int64_t batch, int64_t rows, int64_t cols,
                       void* stream);

/* Window geometry: the fields of cuda::ops::WindowShape (cuda_ops.hpp:86-90). */
typedef struct {
    int64_t batch, channels, height, width;
    int64_t kernel_h, kernel_w, stride, padding;
    int64_t out_h, out_w;
} ehip_window_t;

/* im2col: (N,C,H,W) -> (N*oH*oW, C*kH*kW), zero in the padding. Bit-exact.
 * col2im: the adjoint; each pixel sums its covering windows in (oh, ow)
 * ascending order from zero, as src/conv.cpp:183-214 does: bit-exact.
 * cuda::ops::im2col / col2im (cuda_ops.hpp:99-100). */
int ehip_im2col_f32(const float* x, float* cols, const ehip_window_t* w, void* stream);
int ehip_col2im_f32(const float* cols, float* x, const ehip_window_t* w, void* stream);

/* Max pooling with the flat input index of the first strict maximum as int32
 * (src/conv.cpp:410-442); backward sums, per input pixel, the gradients of the
 * windows that chose it in output order (src/conv.cpp:461-469). Bit-exact.
 * cuda::ops::maxpool / maxpool_backward (cuda_ops.hpp:116-118); the argmax is
 * int32 here where the reference's device path stores it as float. */
int ehip_maxpool_f32(const float* x, float* y, int32_t* argmax, const ehip_window_t* w,
                     void* stream);
int ehip_maxpool_backward_f32(const int32_t* argmax, const float* g, float* dx,
                              const ehip_window_t* w, void* stream);
/* The same pair with the argmax stored as float, the layout of the reference's
 * device path (a float Storage holding flat input indices: maxpool_windows and
 * maxpool_windows_grad, src/cuda/kernels.cu:482-549, behind
 * cuda_ops.hpp:116-118), so an
 * adapter can hand over the reference's argmax Storage as is. Indices are
 * exact below 2^24; larger inputs are refused with EHIP_EINVAL, as the
 * reference's admission rule refuses inputs beyond 2^24 elements
 * (src/cuda/kernels.cu:1100-1103). Bit-exact. */
int ehip_maxpool_fidx_f32(const float* x, float* y, float* argmax, const ehip_window_t* w,
                          void* stream);
int ehip_maxpool_backward_fidx_f32(const float* argmax, const float* g, float* dx,
                                   const ehip_window_t* w, void* stream);

/* Direct convolution for narrow layers (out_channels * C_in * kH * kW <= 8192,
 * ehip_conv2d_direct_supported() says 1): x (N, C_in, H, W), weight
 * (out_channels, C_in, kH, kW), output (N, out_channels, oH, oW), all dense
 * row-major; the window's channels field is C_in. Together the three replace
 * the node chain Conv2d::forward builds -- im2col, the product with the
 * transposed weight, the broadcast bias add, the (N, oH*oW, C) -> (N, C, oH*oW)
 * permute -- and its autograd backward (src/conv.cpp:280-338; im2col/col2im
 * src/conv.cpp:61-217), with no columns in HBM and no permute.
 *   forward: out = sum_k x_col[k] w[co][k] in k order from zero, zero inputs
 *     skipped, then + bias[co] (bias may be NULL): the reference's i-k-j loop
 *     (src/tensor_ops.cpp:553-560) and bias add, bit-exact.
 *   backward_input: dx = col2im of (grad_out . w), each column entry a co-order
 *     sum with zero gradients skipped and the windows of a pixel added in
 *     (oh, ow) order from zero: bit-exact with the reference's two steps.
 *     dx is overwritten.
 *   backward_weight: dweight[co][k] = sum over pixels of grad_out . x_col[k],
 *     dbias[co] = sum over pixels of grad_out (dbias may be NULL), overwritten;
 *     chunked partials reduced in a fixed order: deterministic, within the
 *     K-term tolerance of the reference's serial sums.
 * Wider layers are refused with EHIP_EINVAL (use im2col + ehip_gemm_f32). */
int ehip_conv2d_direct_supported(const ehip_window_t* w, int64_t out_channels);
int ehip_conv2d_forward_f32(const float* x, const float* weight, const float* bias, float* out,
                            const ehip_window_t* w, int64_t out_channels, void* stream);
int ehip_conv2d_backward_input_f32(const float* grad_out, const float* weight, float* dx,
                                   const ehip_window_t* w, int64_t out_channels, void* stream);
int ehip_conv2d_backward_weight_f32(const float* x, const float* grad_out, float* dweight,
                                    float* dbias, const ehip_window_t* w, int64_t out_channels,
                                    void* stream);

/* Implicit-GEMM convolution for layers of any width, on the fp32 MFMA tiles:
 * the products of the reference's wide composition -- im2col, the product with
 * the transposed weight, the bias add and the permute to (N, C_out, oH, oW)
 * (src/conv.cpp:280-338, im2col/col2im src/conv.cpp:61-217) -- with the column
 * operand gathered from x (forward, weight gradient) or from grad_out (input
 * gradient, col2im's adjoint as a gather), never written to HBM. Layouts as
 * for the direct kernels above: x (N, C_in, H, W), weight (C_out, C_in, kH, kW),
 * out and grad_out (N, C_out, oH, oW), dense row-major.
 *   forward: out = weight . cols + bias[co] (bias may be NULL).
 *   backward: dx = sum over (co, i, j) of weight . grad_out at the window that
 *     covers the pixel; dweight = sum over images and pixels of grad_out .
 *     cols; dbias = sum of grad_out per channel. Each output may be NULL to
 *     skip it; the ones given are overwritten.
 * Fixed-order sums (K split into fixed chunks on small grids): deterministic,
 * within the K-term tolerance of the reference's serial loops. Layers with
 * more than 2^31 - 1 elements in one image's input, output or weight rows, or
 * more than 65535 images, are refused with EHIP_EINVAL;
 * ehip_conv2d_igemm_supported() says 1 for a layer inside those limits (a
 * query without side effects: the caller composes im2col + ehip_gemm_f32 for
 * the others, as Conv2d::forward does in src/conv.cpp:280-338). */
int ehip_conv2d_igemm_supported(const ehip_window_t* w, int64_t out_channels);
int ehip_conv2d_igemm_f32(const float* x, const float* weight, const float* bias, float* out,
                          const ehip_window_t* w, int64_t out_channels, void* stream);
int ehip_conv2d_igemm_backward_f32(const float* x, const float* weight, const float* grad_out,
                                   float* dx, float* dweight, float* dbias,
                                   const ehip_window_t* w, int64_t out_channels, void* stream);

/* Conv2d -> ReLU -> MaxPool2d fused, for a narrow convolution followed by a
 * max pool with disjoint square windows (kernel == stride, no padding): the
 * Sequential pattern of the reference's CNN (conv, ReLU, pool, twice). `conv`
 * is the convolution's window over x; `pool` is the pool's window over the
 * convolution output (batch, channels = out_channels, height = conv out_h,
 * width = conv out_w). ehip_conv2d_relu_maxpool_supported() says whether a
 * layer qualifies (1) or must run unfused (0).
 *   forward: out = the pooled ReLU of the convolution, argmax = the flat index
 *     into the (N, out_channels, oH, oW) convolution output of each window's
 *     first strict maximum -- bit-exact with the three reference nodes
 *     (src/conv.cpp:280-338, src/tensor_ops.cpp:591-600, src/conv.cpp:367-442).
 *     The convolution output never reaches HBM.
 *   backward: from the pooled gradient grad_out, the saved out and argmax:
 *     dx (NULL to skip; bit-exact, as ehip_conv2d_backward_input_f32) and
 *     dweight/dbias (NULL to skip; as ehip_conv2d_backward_weight_f32), the
 *     pool and ReLU backward (src/conv.cpp:454-472, src/tensor_ops.cpp:603-615)
 *     folded into the gradient the two read. All outputs are overwritten. */
int ehip_conv2d_relu_maxpool_supported(const ehip_window_t* conv, int64_t out_channels,
                                       const ehip_window_t* pool);
int ehip_conv2d_relu_maxpool_f32(const float* x, const float* weight, const float* bias,
                                 float* out, int32_t* argmax, const ehip_window_t* conv,
                                 int64_t out_channels, const ehip_window_t* pool, void* stream);
int ehip_conv2d_relu_maxpool_backward_f32(const float* x, const float* weight,
                                          const float* grad_out, const float* out,
                                          const int32_t* argmax, float* dx, float* dweight,
                                          float* dbias, const ehip_window_t* conv,
                                          int64_t out_channels, const ehip_window_t* pool,
                                          void* stream);

/* The fused block's backward in two parts, so that a caller can reduce the
 * weight gradients of several layers in one launch (the engine does so at the
 * end of backward). Together they replace what the entry point above
 * replaces, with the weight-gradient sums -- the product A^T dC of
 * src/tensor_ops.cpp:565-586 and the bias fold of src/tensor_detail.hpp:196-204
 * for the conv node of src/conv.cpp:280-338 -- finished by a separate call.
 *
 * ehip_conv2d_relu_maxpool_partials returns the number of floats of weight
 * partials the layer's tile kernel writes (chunks * out_channels * (K + 1), K =
 * C_in kH kW; *chunks receives the chunk count), or 0 when the layer has no
 * tile path (then use ehip_conv2d_relu_maxpool_backward_f32). want_dx says
 * whether dx will be requested: it can change the tiling.
 * ehip_conv2d_relu_maxpool_backward_partials_f32 writes dx (may be NULL) and
 * the partials. ehip_conv_weight_reduce_f32 reduces `count` layers' partials
 * into dweight / dbias (dbias may be NULL) in one launch; the values are the
 * bits ehip_conv2d_relu_maxpool_backward_f32 gives. */
typedef struct ehip_conv_reduce {
    const float* partials;
    int64_t chunks;
    int64_t out_channels;
    int64_t k;               /* C_in * kH * kW */
    float* dweight;          /* (out_channels, k) */
    float* dbias;            /* (out_channels) or NULL */
} ehip_conv_reduce_t;

int64_t ehip_conv2d_relu_maxpool_partials(const ehip_window_t* conv, int64_t out_channels,
                                          const ehip_window_t* pool, int want_dx,
                                          int64_t* chunks);
int ehip_conv2d_relu_maxpool_backward_partials_f32(
    const float* x, const float* weight, const float* grad_out, const float* out,
    const int32_t* argmax, float* dx, float* partials, int64_t chunks, const ehip_window_t* conv,
    int64_t out_channels, const ehip_window_t* pool, void* stream);
int ehip_conv_weight_reduce_f32(const ehip_conv_reduce_t* jobs, int count, void* stream);

/* The convolution weight-gradient sums of ehip_conv_weight_reduce_f32 and the
 * Adam step of ehip_adam_multi_f32 in one launch: each job's sums are stored
 * into its dweight / dbias, and a tensor whose g is one of those buffers (same
 * size) is updated right there with the sum; the other tensors take the
 * multi-tensor update. The same bits as the two calls one after the other
 * (which it makes itself for more than 8 jobs or a model beyond 2^20
 * parameters). Replaces the bias and weight folds of the conv nodes
 * (src/tensor_detail.hpp:196-204, src/tensor_ops.cpp:565-586) followed by
 * Adam::step (src/optim.cpp:113-162). */
int ehip_adam_multi_reduce_f32(const ehip_adam_tensor_t* tensors, int count,
                               const ehip_conv_reduce_t* jobs, int njobs, float lr, float beta1,
                               float beta2, float eps, float weight_decay, float bias_c1,
                               float bias_c2, void* stream);
/* ehip_adam_multi_reduce_f32 with lr, bias_c1 and bias_c2 read from the
 * DEVICE array hyper[3], as ehip_adam_multi_dev_f32 (for captured steps; no
 * counterpart in the reference). */
int ehip_adam_multi_reduce_dev_f32(const ehip_adam_tensor_t* tensors, int count,
                                   const ehip_conv_reduce_t* jobs, int njobs, const float* hyper,
                                   float beta1, float beta2, float eps, float weight_decay,
                                   void* stream);

/* out[i] = x[idx[i]] row by row (rows of row_size floats); an index outside
 * [0, n_rows) yields a row of NaN instead of a read out of bounds.
 * Tensor::select_rows forward (src/tensor.cpp:556-585). Bit-exact. */
int ehip_select_rows_f32(const float* x, const int32_t* idx, float* out, int64_t n_idx,
                         int64_t row_size, int64_t n_rows, void* stream);

/* Scatter-add adjoint of select_rows in CSR form: for every destination row r,
 * S = sum of g rows pos[p] for p in [row_ptr[r], row_ptr[r+1]) taken in that
 * order from zero, and dx[r] = S (accumulate == 0) or dx[r] + S. g has n_src
 * rows; a position outside [0, n_src) makes the row NaN instead of a wild read.
 * With pos listing each row's source positions in ascending order this is the
 * reference's zeroed `dX[idx[i]] += g[i]` for i ascending followed by add_grad
 * (src/tensor.cpp:593-601): bit-exact. */
int ehip_scatter_add_rows_f32(const float* g, const int32_t* row_ptr, const int32_t* pos,
                              float* dx, int64_t n_rows, int64_t row_size, int64_t n_src,
                              int accumulate, void* stream);

/* Dropout: y = x * m with m = 1 / (1 - p) where element i is kept, else 0;
 * mask (may be NULL) receives m for the backward (dx = g * m, ehip_binary_f32
 * EHIP_MUL). Element i is kept when the 24-bit uniform drawn for counter value
 * offset + i by Philox4x32-10 keyed by `seed` (word (offset + i) % 4 of block
 * (offset + i) / 4) is below 1 - p: reproducible from (seed, offset) on any
 * device and launch shape. Replaces the mask loop of Dropout::forward
 * (src/nn.cpp:206-244), whose sequential mt19937 stream it does not reproduce;
 * the kept values use the reference's arithmetic (x * (1 / keep)). */
int ehip_dropout_f32(const float* x, float* y, float* mask, int64_t n, float p, uint64_t seed,
                     uint64_t offset, void* stream);

/* ------------------------------------------------------------- reductions */

/* Sum over the middle axis of an (outer, axis_len, inner) view.
 * Bit-exact (a ascending from zero, src/tensor.cpp:347-356) when
 * axis_len <= 64 or outer * inner >= 16384; above that, a deterministic
 * two-stage sum over fixed chunks of the axis (the same result on every run,
 * within fp32 rounding of the serial sum). cuda::ops::sum_axis (cuda_ops.hpp:80). */
int ehip_sum_axis_f32(const float* x, float* out, int64_t outer, int64_t axis_len, int64_t inner,
                      void* stream);

/* Whole-buffer sum of x (squares == 0) or of x*x, accumulated in double over a
 * fixed partition (deterministic). Writes the double to out_d and its float
 * cast to out_f (either may be NULL): both DEVICE pointers, so no
 * synchronisation. cuda::ops::reduce_sum / reduce_sum_squares
 * (cuda_ops.hpp:137-138). */
int ehip_reduce_sum_f32(const float* x, int64_t n, int squares, double* out_d, float* out_f,
                        void* stream);

/* ---------------------------------------------------------------- row ops */

/* Row softmax over `cols` contiguous values and its derivative from the saved
 * output y: dx = y (g - sum(g y)). cuda::ops::softmax / softmax_backward
 * (cuda_ops.hpp:200-203). */
int ehip_softmax_f32(const float* x, float* y, int64_t rows, int64_t cols, void* stream);
int ehip_softmax_backward_f32(const float* y, const float* g, float* dx, int64_t rows,
                              int64_t cols, void* stream);

/* dx = (y (g - sum(g y))) * scale, the product rounded before the scale: the
 * softmax derivative followed by the backward of a `scores * scale` node
 * (src/transformer.cpp:285-289 under src/tensor_ops.cpp's scalar multiply),
 * in one pass. dx may alias g (each element is read before it is written). */
int ehip_softmax_backward_scaled_f32(const float* y, const float* g, float* dx, int64_t rows,
                                     int64_t cols, float scale, void* stream);

/* The softmax forward and scaled backward of a causal attention's scores:
 * rows are stacked cols x cols matrices, and entries right of the diagonal
 * (column j > row i within a matrix) are masked -- in the forward at least
 * 104 below the row's maximum (their exponential is 0), in the backward with
 * y = 0. Masked entries are not used -- any values there, NaN included, leave
 * the results as they are (the 16-byte vector that straddles the diagonal is
 * loaded whole, its masked lanes discarded; whole vectors past it are never
 * loaded) -- and they are stored as 0. Every other output
 * equals ehip_softmax_f32's / ehip_softmax_backward_scaled_f32's bit for bit,
 * and a masked one by value (its sign of zero may differ). rows must be a
 * multiple of cols. (The reference reads and computes the masked entries:
 * src/transformer.cpp:279-304 through src/tensor_ops.cpp:621-676.) */
int ehip_softmax_causal_f32(const float* x, float* y, int64_t rows, int64_t cols, void* stream);
int ehip_softmax_backward_scaled_causal_f32(const float* y, const float* g, float* dx,
                                            int64_t rows, int64_t cols, float scale,
                                            void* stream);

/* Scaled dot-product attention of short sequences in one launch per direction
 * (one workgroup per batch and head, everything in LDS): the reference's
 * scaled_dot_product_attention under its multi-head split and merge
 * (src/transformer.cpp:279-304, 320-349) -- weights = softmax(Q K^T * scale
 * [+ causal mask]), out = weights V -- and its autograd backward, each sum in
 * the reference CPU loops' order (ascending index from zero, zero A operands
 * skipped; the softmax's denominator and the backward's row dot serial), so
 * that only the device exp separates the values from the reference's. q, k,
 * v, out, grad, dq, dk, dv are (batch, seq, width) activations holding head h
 * at columns [h head_dim, (h + 1) head_dim); weights is (batch, heads, seq,
 * seq). causal = 1 masks entries right of the diagonal, as nn::causal_mask's
 * -1e9 addend does (those weights are 0; masked entries are not read or
 * computed). The backward takes the forward's weights and writes (does not
 * accumulate) each of dq, dk, dv that is not NULL. seq and head_dim at most 64
 * (ehip_attention_short_supported says 1); others are refused with EHIP_EINVAL
 * and take the batched products and softmax kernels above. */
int ehip_attention_short_supported(int64_t seq, int64_t head_dim);
int ehip_attention_short_f32(const float* q, const float* k, const float* v, float* weights,
                             float* out, int64_t batch, int64_t seq, int64_t width, int64_t heads,
                             int64_t head_dim, float scale, int causal, void* stream);
int ehip_attention_short_backward_f32(const float* q, const float* k, const float* v,
                                      const float* weights, const float* grad, float* dq,
                                      float* dk, float* dv, int64_t batch, int64_t seq,
                                      int64_t width, int64_t heads, int64_t head_dim, float scale,
                                      int causal, void* stream);

/* LayerNorm over the last axis (two-pass mean and variance, eps inside the
 * square root) saving xhat and inv_std, and its derivative; dgamma and dbeta
 * are summed over rows in a fixed order (deterministic, no atomics). Rows of
 * up to 8192 columns are held in registers; wider ones take looped kernels
 * with the same expressions (up to 4,194,240 columns: 65535 column tiles of
 * the parameter sums).
 * cuda::ops::layernorm / layernorm_backward (cuda_ops.hpp:193-197). */
int ehip_layernorm_f32(const float* x, const float* gamma, const float* beta, float* out,
                       float* xhat, float* inv_std, int64_t rows, int64_t cols, float eps,
                       void* stream);
int ehip_layernorm_backward_f32(const float* dy, const float* xhat, const float* gamma,
                                const float* inv_std, float* dx, float* dgamma, float* dbeta,
                                int64_t rows, int64_t cols, void* stream);

/* The LayerNorm backward with its parameter sums left for later, for callers
 * that run several of them into one reduction (the engine sums every
 * LayerNorm's dgamma / dbeta of a backward in the launch of the conv weight
 * sums, or inside Adam's). ehip_layernorm_backward_partials returns the floats
 * of the partial buffer for rows x cols and the group count through *groups,
 * or 0 when that shape is summed in one call only (fewer than 2^17 elements,
 * or more than 2048 columns). ehip_layernorm_backward_partials_f32 writes dx
 * and partials[group][c][2] = (dgamma, dbeta) of each row group; the job
 * {partials, groups, out_channels = cols, k = 1, dweight = dgamma,
 * dbias = dbeta} of ehip_conv_weight_reduce_f32 or ehip_adam_multi_reduce_f32
 * then forms dgamma and dbeta with the same bits as
 * ehip_layernorm_backward_f32. Refuses a group count other than the one
 * returned. With accumulate != 0 (rows of at most 1024 columns; wider ones are
 * refused), dx receives dx + (the input gradient), one add per element: the
 * bits of writing it and then accumulating it into dx with
 * ehip_accumulate_grad_f32, in one pass. The backward of the reference's
 * LayerNorm node (src/transformer.cpp:123-150) with the parameter folds
 * deferred, and its add_grad into the input's gradient (src/tensor.cpp:168-203). */
int64_t ehip_layernorm_backward_partials(int64_t rows, int64_t cols, int64_t* groups);
int ehip_layernorm_backward_partials_f32(const float* dy, const float* xhat, const float* gamma,
                                         const float* inv_std, float* dx, float* partials,
                                         int64_t groups, int64_t rows, int64_t cols,
                                         int accumulate, void* stream);

/* Fused log-softmax + NLL over (rows, cols) logits with int32 targets: probs
 * receives the row softmax and loss[0] the mean of -log p[target] (summed in
 * double over a fixed partition). A target outside [0, cols) makes loss NaN.
 * The reference has no device kernel for this: it replaces the host loop of
 * nn::cross_entropy_loss (src/nn.cpp:324-380). */
int ehip_cross_entropy_f32(const float* logits, const int32_t* targets, float* probs, float* loss,
                           int64_t rows, int64_t cols, void* stream);

/* ehip_cross_entropy_f32 plus the logits' gradient for an upstream gradient
 * of 1 (the loss as the root of backward): dlogits = (probs - onehot(target))
 * / rows, the same bits as ehip_cross_entropy_backward_f32 with grad[0] = 1,
 * written by the same launch. The forward and backward of
 * nn::cross_entropy_loss (src/nn.cpp:324-405) for a classifier head; only
 * shapes ehip_cross_entropy_fused_supported accepts (rows <= 1024, cols <= 128,
 * one block), others are refused with EHIP_EINVAL. */
int ehip_cross_entropy_fused_supported(int64_t rows, int64_t cols);
int ehip_cross_entropy_fused_f32(const float* logits, const int32_t* targets, float* probs,
                                 float* loss, float* dlogits, int64_t rows, int64_t cols,
                                 void* stream);

/* dx = (probs - onehot(target)) * (grad[0] / rows), grad a DEVICE scalar (the
 * upstream gradient of the loss). src/nn.cpp:386-405. Bit-exact given probs. */
int ehip_cross_entropy_backward_f32(const float* probs, const int32_t* targets, float* dx,
                                    int64_t rows, int64_t cols, const float* grad, void* stream);

/* The softmax-cross-entropy backward straight from the logits, one pass:
 * recomputes each row's softmax in registers and writes
 * (softmax - onehot) * (grad[0] / rows). Reads 4 and writes 4 bytes per
 * element; equal bit-for-bit to ehip_cross_entropy_f32 followed by
 * ehip_cross_entropy_backward_f32. Replaces src/nn.cpp:352-405 for the
 * backward pass. */
int ehip_softmax_xent_backward_f32(const float* logits, const int32_t* targets, float* dx,
                                   int64_t rows, int64_t cols, const float* grad, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EHIP_H */
