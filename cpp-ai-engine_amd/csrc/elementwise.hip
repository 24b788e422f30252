// elementwise.hip -- the HBM-bound element-wise kernels: binary ops with
// suffix broadcast, scalar affine, ReLU and its derivative, gradient
// accumulation, the fused add backward, fill/scale, and the SGD and Adam
// updates.
//
// Every kernel streams 128-bit vectors: a thread issues all U of its loads
// before any store (so U * inputs loads are in flight per thread), and the
// vectors of one unrolled step are 256 threads apart, so each wavefront
// touches 1 KiB contiguous per load instruction. Built with
// -ffp-contract=off and correctly rounded division and square root, so the
// arithmetic rounds exactly as the reference's CPU loops do
// (src/tensor_ops.cpp, src/tensor.cpp:193-202, src/optim.cpp:71-84, 147-160).

#include "common.hpp"

#include <cstring>
#include <mutex>
#include <vector>

namespace ehip {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;  // float4 vectors per thread per input

// Streams of at least this many elements (64 MiB per operand, far past the L2s
// and a quarter of the 256 MB Infinity Cache) are read and written with
// non-temporal hints: nothing is reused, and keeping the lines out of the
// caches measured 2-7 % faster on 2^28-element streams.
constexpr int64_t kNontemporalMin = int64_t(1) << 24;

typedef float nf4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ float4 ld4(const float* p, int64_t v) {
    if (NT) {
        const nf4 x = __builtin_nontemporal_load(reinterpret_cast<const nf4*>(p) + v);
        return make_float4(x.x, x.y, x.z, x.w);
    }
    return reinterpret_cast<const float4*>(p)[v];
}
template <bool NT>
__device__ __forceinline__ void st4(float* p, int64_t v, float4 x) {
    if (NT) {
        const nf4 y = {x.x, x.y, x.z, x.w};
        __builtin_nontemporal_store(y, reinterpret_cast<nf4*>(p) + v);
    } else {
        reinterpret_cast<float4*>(p)[v] = x;
    }
}

// Applies f component-wise to up to three float4 operands.
template <class F>
__device__ __forceinline__ float4 map4(F f, float4 a, float4 b, float4 c) {
    return make_float4(f(a.x, b.x, c.x), f(a.y, b.y, c.y), f(a.z, b.z, c.z), f(a.w, b.w, c.w));
}

// Generic streaming skeleton. Op supplies:
//   static constexpr int kIn;                  inputs loaded per vector
//   load(v, float4* r)  / store(v, const float4* r)   for vector v (4 elements)
//   scalar(i)                                   for the tail element i
template <class Op, bool NT>
__global__ __launch_bounds__(kThreads) void stream_vec(Op op, int64_t n) {
    const int64_t nv = n >> 2;
    const int64_t base = int64_t(blockIdx.x) * (kThreads * kUnroll) + threadIdx.x;
    float4 r[kUnroll][Op::kIn];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t v = base + int64_t(u) * kThreads;
        if (v < nv) op.template load<NT>(v, r[u]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t v = base + int64_t(u) * kThreads;
        if (v < nv) op.template store<NT>(v, r[u]);
    }
    if (blockIdx.x == gridDim.x - 1)
        for (int64_t i = (nv << 2) + threadIdx.x; i < n; i += kThreads) op.scalar(i);
}

// Unaligned operands: one element per thread, grid-stride.
template <class Op>
__global__ __launch_bounds__(kThreads) void stream_scalar(Op op, int64_t n) {
    const int64_t step = int64_t(gridDim.x) * kThreads;
    for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < n; i += step) op.scalar(i);
}

template <class Op>
int launch_stream(const char* name, const Op& op, int64_t n, bool vec_ok, hipStream_t s) {
    if (n < 0) return fail(EHIP_EINVAL, "%s: negative size", name);
    if (n == 0) return EHIP_OK;
    if (vec_ok) {
        const int64_t nv = n >> 2;
        int64_t grid = ceil_div(nv, int64_t(kThreads) * kUnroll);
        if (grid == 0) grid = 1;
        if (grid > 0x7fffffff) return fail(EHIP_EINVAL, "%s: %lld elements is too many", name,
                                           static_cast<long long>(n));
        if (n >= kNontemporalMin)
            EHIP_LAUNCH(name, (stream_vec<Op, true>), dim3(unsigned(grid)), dim3(kThreads), 0, s,
                        op, n);
        else
            EHIP_LAUNCH(name, (stream_vec<Op, false>), dim3(unsigned(grid)), dim3(kThreads), 0, s,
                        op, n);
    } else {
        int64_t grid = ceil_div(n, kThreads);
        if (grid > 65536) grid = 65536;
        EHIP_LAUNCH(name, stream_scalar<Op>, dim3(unsigned(grid)), dim3(kThreads), 0, s, op, n);
    }
    return EHIP_OK;
}

// ------------------------------------------------------------------ ops

__device__ __forceinline__ float apply_binary(int op, float a, float b) {
    switch (op) {
        case EHIP_ADD: return a + b;
        case EHIP_SUB: return a - b;
        case EHIP_MUL: return a * b;
        default: return a / b;
    }
}

template <int OP>
struct Binary {
    static constexpr int kIn = 2;
    const float* a;
    const float* b;
    float* out;
    int64_t inner;
    template <bool NT>
    __device__ void load(int64_t v, float4* r) const {
        r[0] = ld4<NT>(a, v);
        r[1] = ld4<NT>(b, (v << 2) % inner >> 2);
    }
    template <bool NT>
    __device__ void store(int64_t v, const float4* r) const {
        st4<NT>(out, v, map4([](float x, float y, float) { return apply_binary(OP, x, y); }, r[0],
                         r[1], r[1]));
    }
    __device__ void scalar(int64_t i) const { out[i] = apply_binary(OP, a[i], b[i % inner]); }
};

// The scalar node: `t * k` is (k, 0) and `t + k` is (1, k); each rounds once,
// as on the CPU (src/tensor_ops.cpp:280-285, 307-312).
struct Scalar {
    static constexpr int kIn = 1;
    const float* x;
    float* out;
    float mul, add;
    __device__ float f(float v) const {
        if (mul == 1.0f) return v + add;
        if (add == 0.0f) return v * mul;
        return v * mul + add;
    }
    template <bool NT>
    __device__ void load(int64_t v, float4* r) const { r[0] = ld4<NT>(x, v); }
    template <bool NT>
    __device__ void store(int64_t v, const float4* r) const {
        st4<NT>(out, v, make_float4(f(r[0].x), f(r[0].y), f(r[0].z), f(r[0].w)));
    }
    __device__ void scalar(int64_t i) const { out[i] = f(x[i]); }
};

struct Relu {
    static constexpr int kIn = 1;
    const float* x;
    float* y;
    static __device__ float f(float v, float, float) { return (0.0f < v) ? v : 0.0f; }
    template <bool NT>
    __device__ void load(int64_t v, float4* r) const { r[0] = ld4<NT>(x, v); }
    template <bool NT>
    __device__ void store(int64_t v, const float4* r) const { st4<NT>(y, v, map4(f, r[0], r[0], r[0])); }
    __device__ void scalar(int64_t i) const { y[i] = f(x[i], 0, 0); }
};

// Sigmoid, tanh and the tanh form of GELU, forward and backward, in the
// reference's expressions (src/nn.cpp:154-198), evaluated in the same order;
// expf and tanhf are the device library's, within a few ulp of the host's.
constexpr float kGeluAlpha = 0.7978845608028654f;  // sqrt(2 / pi)
constexpr float kGeluBeta = 0.044715f;

template <int KIND>  // 0 sigmoid, 1 tanh, 2 GELU
__device__ __forceinline__ float act_f(float x) {
    if (KIND == 0) return (x >= 0.0f) ? 1.0f / (1.0f + expf(-x)) : expf(x) / (1.0f + expf(x));
    if (KIND == 1) return tanhf(x);
    return 0.5f * x * (1.0f + tanhf(kGeluAlpha * (x + kGeluBeta * x * x * x)));
}

// The derivative at x, given y = f(x).
template <int KIND>
__device__ __forceinline__ float act_d(float x, float v) {
    if (KIND == 0) return v * (1.0f - v);
    if (KIND == 1) return 1.0f - v * v;
    const float inner = kGeluAlpha * (x + kGeluBeta * x * x * x);
    const float t = tanhf(inner);
    const float dinner = kGeluAlpha * (1.0f + 3.0f * kGeluBeta * x * x);
    return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * dinner;
}

template <int KIND>
struct Activation {
    static constexpr int kIn = 1;
    const float* x;
    float* y;
    static __device__ float f(float v, float, float) { return act_f<KIND>(v); }
    template <bool NT>
    __device__ void load(int64_t v, float4* r) const { r[0] = ld4<NT>(x, v); }
    template <bool NT>
    __device__ void store(int64_t v, const float4* r) const { st4<NT>(y, v, map4(f, r[0], r[0], r[0])); }
    __device__ void scalar(int64_t i) const { y[i] = f(x[i], 0, 0); }
};

// dx = g * f'(x, y)
template <int KIND>
struct ActivationBackward {
    static constexpr int kIn = 3;
    const float* x;
    const float* y;
    const float* g;
    float* dx;
    static __device__ float f(float xv, float yv, float gv) { return gv * act_d<KIND>(xv, yv); }
    template <bool NT>
    __device__ void load(int64_t v, float4* r) const {
        r[0] = ld4<NT>(x, v);
        r[1] = ld4<NT>(y, v);
        r[2] = ld4<NT>(g, v);
    }
    template <bool NT>
    __device__ void store(int64_t v, const float4* r) const {
        st4<NT>(dx, v, map4(f, r[0], r[1], r[2]));
    }
    __device__ void scalar(int64_t i) const { dx[i] = f(x[i], y[i], g[i]); }
};

// rows x len floats from src (row pitch sp) to dst (row pitch dp): the moves of
// slice, concat and stack and of their backward passes. One workgroup per
// (row, 1024-float chunk); float4 where every address allows.
__global__ __launch_bounds__(256) void copy_rows(const float* __restrict__ src, int64_t sp,
                                                 float* __restrict__ dst, int64_t dp, int64_t len,
                                                 int64_t chunks, int vec) {
    const int64_t row = int64_t(blockIdx.x) / chunks, c = int64_t(blockIdx.x) % chunks;
    const float* s = src + row * sp;
    float* d = dst + row * dp;
    const int64_t begin = c * 1024, end = min(begin + 1024, len);
    if (vec) {
        const int64_t i = begin + 4 * int64_t(threadIdx.x);
        if (i + 3 < end)
            *reinterpret_cast<float4*>(d + i) = *reinterpret_cast<const float4*>(s + i);
        else
            for (int64_t j = i; j < end; ++j) d[j] = s[j];
    } else {
        for (int64_t i = begin + threadIdx.x; i < end; i += 256) d[i] = s[i];
    }
}

// Maximum over the middle axis of (outer, axis_len, inner) and the axis index
// of the first maximum, scanning in axis order with a strict > as the
// reference does (src/tensor.cpp:383-424): a NaN first element stays the
// maximum, a later NaN is never taken.
__global__ __launch_bounds__(256) void max_axis(const float* __restrict__ x, float* __restrict__ y,
                                                int32_t* __restrict__ arg, int64_t outer,
                                                int64_t axis_len, int64_t inner) {
    const int64_t k = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (k >= outer * inner) return;
    const int64_t o = k / inner, i = k % inner;
    const float* p = x + o * axis_len * inner + i;
    float best = p[0];
    int32_t best_a = 0;
    for (int64_t a = 1; a < axis_len; ++a) {
        const float v = p[a * inner];
        if (v > best) {
            best = v;
            best_a = int32_t(a);
        }
    }
    y[k] = best;
    arg[k] = best_a;
}

// dx of max_axis: 0 + g at each winning position, 0 elsewhere.
__global__ __launch_bounds__(256) void max_axis_backward(const float* __restrict__ g,
                                                         const int32_t* __restrict__ arg,
                                                         float* __restrict__ dx, int64_t outer,
                                                         int64_t axis_len, int64_t inner) {
    const int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (e >= outer * axis_len * inner) return;
    const int64_t i = e % inner, a = (e / inner) % axis_len, o = e / (inner * axis_len);
    const int64_t k = o * inner + i;
    dx[e] = (arg[k] == a) ? 0.0f + g[k] : 0.0f;
}

struct ReluBackward {
    static constexpr int kIn = 2;
    const float* x;
    const float* g;
    float* dx;
    static __device__ float f(float v, float gv, float) { return (v > 0.0f) ? gv : 0.0f; }
    template <bool NT>
    __device__ void load(int64_t v, float4* r) const {
        r[0] = ld4<NT>(x, v);
        r[1] = ld4<NT>(g, v);
    }
    template <bool NT>
    __device__ void store(int64_t v, const float4* r) const {
        st4<NT>(dx, v, map4(f, r[0], r[1], r[1]));
    }
    __device__ void scalar(int64_t i) const { dx[i] = f(x[i], g[i], 0); }
};

template <bool INIT>
struct Accumulate {
    static constexpr int kIn = INIT ? 1 : 2;
    float* grad;
    const float* g;
    template <bool NT>
    __device__ void load(int64_t v, float4* r) const {
        r[0] = ld4<NT>(g, v);
        if (!INIT) r[kIn - 1] = ld4<NT>(grad, v);
    }
    // The first write is 0 + g, not a copy: the reference adds into a zeroed
    // buffer (src/tensor.cpp:177-202), which turns -0 into +0.
    template <bool NT>
    __device__ void store(int64_t v, const float4* r) const {
        if (INIT)
            st4<NT>(grad, v, map4([](float a, float, float) { return 0.0f + a; }, r[0], r[0], r[0]));
        else
            st4<NT>(grad, v, map4([](float a, float b, float) { return b + a; }, r[0], r[kIn - 1],
                              r[0]));
    }
    __device__ void scalar(int64_t i) const { grad[i] = INIT ? 0.0f + g[i] : grad[i] + g[i]; }
};

// The add node's backward: g goes to both operands in one pass.
template <bool ACC_A, bool ACC_B>
struct AddBackward {
    static constexpr int kIn = 1 + int(ACC_A) + int(ACC_B);
    const float* g;
    float* da;
    float* db;
    template <bool NT>
    __device__ void load(int64_t v, float4* r) const {
        r[0] = ld4<NT>(g, v);
        if (ACC_A) r[1] = ld4<NT>(da, v);
        if (ACC_B) r[kIn - 1] = ld4<NT>(db, v);
    }
    template <bool NT>
    __device__ void store(int64_t v, const float4* r) const {
        const auto add = [](float a, float b, float) { return a + b; };
        const float4 first = map4(add, make_float4(0.0f, 0.0f, 0.0f, 0.0f), r[0], r[0]);
        st4<NT>(da, v, ACC_A ? map4(add, r[1], r[0], r[0]) : first);
        st4<NT>(db, v, ACC_B ? map4(add, r[kIn - 1], r[0], r[0]) : first);
    }
    __device__ void scalar(int64_t i) const {
        const float gv = g[i];
        da[i] = ACC_A ? da[i] + gv : 0.0f + gv;
        db[i] = ACC_B ? db[i] + gv : 0.0f + gv;
    }
};

// The multiply node's backward in one pass (src/tensor_ops.cpp:199-213, same
// shapes): da = g * b, db = g * a, each product rounded, then, when the
// gradient already holds values, added to it (the composed graph's product
// node followed by add_grad's accumulation, bit for bit). MA / MB: 0 the
// operand needs no gradient, 1 write the product, 2 add it to the gradient.
template <int MA, int MB>
struct MulBackward {
    static constexpr int kA = MB != 0, kB = MA != 0;  // a feeds db, b feeds da
    static constexpr int kIn = 1 + kA + kB + (MA == 2) + (MB == 2);
    const float* g;
    const float* a;
    const float* b;
    float* da;
    float* db;
    template <bool NT>
    __device__ void load(int64_t v, float4* r) const {
        int q = 0;
        r[q++] = ld4<NT>(g, v);
        if (kA) r[q++] = ld4<NT>(a, v);
        if (kB) r[q++] = ld4<NT>(b, v);
        if (MA == 2) r[q++] = ld4<NT>(da, v);
        if (MB == 2) r[q++] = ld4<NT>(db, v);
    }
    template <bool NT>
    __device__ void store(int64_t v, const float4* r) const {
        const auto mul = [](float x, float y, float) { return x * y; };
        const auto add = [](float x, float y, float) { return x + y; };
        const float4 gv = r[0];
        const int ia = 1, ib = 1 + kA, ida = 1 + kA + kB, idb = ida + (MA == 2);
        if (MA != 0) {
            const float4 p = map4(mul, gv, r[ib], gv);
            st4<NT>(da, v, MA == 2 ? map4(add, r[ida], p, p) : p);
        }
        if (MB != 0) {
            const float4 p = map4(mul, gv, r[ia], gv);
            st4<NT>(db, v, MB == 2 ? map4(add, r[idb], p, p) : p);
        }
    }
    __device__ void scalar(int64_t i) const {
        const float gv = g[i];
        if (MA != 0) {
            const float p = gv * b[i];
            da[i] = MA == 2 ? da[i] + p : p;
        }
        if (MB != 0) {
            const float p = gv * a[i];
            db[i] = MB == 2 ? db[i] + p : p;
        }
    }
};

struct Fill {
    static constexpr int kIn = 1;
    float* x;
    float value;
    template <bool NT>
    __device__ void load(int64_t, float4*) const {}
    template <bool NT>
    __device__ void store(int64_t v, const float4*) const {
        st4<NT>(x, v, make_float4(value, value, value, value));
    }
    __device__ void scalar(int64_t i) const { x[i] = value; }
};

struct Scale {
    static constexpr int kIn = 1;
    float* x;
    float factor;
    template <bool NT>
    __device__ void load(int64_t v, float4* r) const { r[0] = ld4<NT>(x, v); }
    template <bool NT>
    __device__ void store(int64_t v, const float4* r) const {
        st4<NT>(x, v, make_float4(r[0].x * factor, r[0].y * factor, r[0].z * factor,
                              r[0].w * factor));
    }
    __device__ void scalar(int64_t i) const { x[i] = x[i] * factor; }
};

// src/optim.cpp:71-84, term for term.
template <bool MOMENTUM>
struct Sgd {
    static constexpr int kIn = MOMENTUM ? 3 : 2;
    float* p;
    const float* g;
    float* vel;
    float lr, momentum, wd;
    __device__ void one(float& pv, float gv, float& vv) const {
        float grad = gv;
        if (wd != 0.0f) grad += wd * pv;
        if (MOMENTUM) {
            vv = momentum * vv + grad;
            grad = vv;
        }
        pv -= lr * grad;
    }
    template <bool NT>
    __device__ void load(int64_t v, float4* r) const {
        r[0] = ld4<NT>(p, v);
        r[1] = ld4<NT>(g, v);
        if (MOMENTUM) r[kIn - 1] = ld4<NT>(vel, v);
    }
    template <bool NT>
    __device__ void store(int64_t v, const float4* r) const {
        float4 pv = r[0], vv = r[kIn - 1];
        one(pv.x, r[1].x, vv.x);
        one(pv.y, r[1].y, vv.y);
        one(pv.z, r[1].z, vv.z);
        one(pv.w, r[1].w, vv.w);
        st4<NT>(p, v, pv);
        if (MOMENTUM) st4<NT>(vel, v, vv);
    }
    __device__ void scalar(int64_t i) const {
        float pv = p[i], vv = MOMENTUM ? vel[i] : 0.0f;
        one(pv, g[i], vv);
        p[i] = pv;
        if (MOMENTUM) vel[i] = vv;
    }
};

// src/optim.cpp:147-160, term for term and in the same association order.
struct Adam {
    static constexpr int kIn = 4;
    float* p;
    const float* g;
    float* m;
    float* v;
    float lr, b1, b2, eps, wd, c1, c2;
    __device__ void one(float& pv, float gv, float& mv, float& vv) const {
        float grad = gv;
        if (wd != 0.0f) grad += wd * pv;
        mv = b1 * mv + (1.0f - b1) * grad;
        vv = b2 * vv + (1.0f - b2) * grad * grad;
        const float m_hat = mv / c1;
        const float v_hat = vv / c2;
        pv -= lr * m_hat / (sqrtf(v_hat) + eps);
    }
    template <bool NT>
    __device__ void load(int64_t i, float4* r) const {
        r[0] = ld4<NT>(p, i);
        r[1] = ld4<NT>(g, i);
        r[2] = ld4<NT>(m, i);
        r[3] = ld4<NT>(v, i);
    }
    template <bool NT>
    __device__ void store(int64_t i, const float4* r) const {
        float4 pv = r[0], mv = r[2], vv = r[3];
        one(pv.x, r[1].x, mv.x, vv.x);
        one(pv.y, r[1].y, mv.y, vv.y);
        one(pv.z, r[1].z, mv.z, vv.z);
        one(pv.w, r[1].w, mv.w, vv.w);
        st4<NT>(p, i, pv);
        st4<NT>(m, i, mv);
        st4<NT>(v, i, vv);
    }
    __device__ void scalar(int64_t i) const {
        float pv = p[i], mv = m[i], vv = v[i];
        one(pv, g[i], mv, vv);
        p[i] = pv;
        m[i] = mv;
        v[i] = vv;
    }
};

// Multi-tensor Adam: the tensors are cut into chunks of U float4 per thread
// (one chunk per workgroup: kAdamChunk elements with U = kUnroll, a quarter of
// that for small models, whose few workgroups would otherwise each update
// sixteen elements per thread one after another); a workgroup finds its tensor
// by binary search over the chunk prefix of the slot table. Every element's
// update is the same whatever the chunking.
struct AdamSlot {
    float* p;
    const float* g;
    float* m;
    float* v;
    int64_t n;
    int64_t first_chunk;
};
constexpr int64_t kAdamChunk = int64_t(kThreads) * kUnroll * 4;

// Up to this many tensors travel in the kernel arguments (48 slots of 48
// bytes), so a model whose gradient buffers change from step to step (the
// first gradient write adopts a fresh buffer) needs no table upload per step.
constexpr int kInlineSlots = 48;
struct AdamInline {
    AdamSlot s[kInlineSlots];
};

// The slot whose chunks include chunk b (slots ordered by first_chunk).
template <class Slots>
__device__ __forceinline__ AdamSlot find_slot(const Slots& slots, int count, int64_t b) {
    int lo = 0, hi = count - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (slots[mid].first_chunk <= b)
            lo = mid;
        else
            hi = mid - 1;
    }
    return slots[lo];
}

template <bool NT, int U>
__device__ __forceinline__ void adam_chunk(const AdamSlot& s, int64_t b, float lr, float b1,
                                           float b2, float eps, float wd, float c1, float c2) {
    const Adam op{s.p, s.g, s.m, s.v, lr, b1, b2, eps, wd, c1, c2};
    constexpr int64_t kChunk = int64_t(kThreads) * U * 4;
    const int64_t begin = (b - s.first_chunk) * kChunk;
    const int64_t end = min(begin + kChunk, s.n);
    const bool vec = aligned16(s.p) && aligned16(s.g) && aligned16(s.m) && aligned16(s.v);
    int64_t tail = begin;
    if (vec) {
        const int64_t v0 = begin >> 2, v1 = end >> 2;  // whole float4 vectors in the chunk
        float4 r[U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t v = v0 + int64_t(u) * kThreads + threadIdx.x;
            if (v < v1) op.template load<NT>(v, r[u]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t v = v0 + int64_t(u) * kThreads + threadIdx.x;
            if (v < v1) op.template store<NT>(v, r[u]);
        }
        tail = v1 << 2;
    }
    for (int64_t i = tail + threadIdx.x; i < end; i += kThreads) op.scalar(i);
}

// lr, c1 and c2 come from the arguments, or from hyper[0..2] in device memory
// when hyper is not null (a captured step whose replays change them).
__device__ __forceinline__ void read_hyper(const float* hyper, float& lr, float& c1, float& c2) {
    if (hyper != nullptr) {
        lr = hyper[0];
        c1 = hyper[1];
        c2 = hyper[2];
    }
}

template <bool NT>
__global__ __launch_bounds__(kThreads) void adam_multi(const AdamSlot* __restrict__ slots,
                                                       int count, float lr, float b1, float b2,
                                                       float eps, float wd, float c1, float c2,
                                                       const float* __restrict__ hyper) {
    read_hyper(hyper, lr, c1, c2);
    const int64_t b = blockIdx.x;
    adam_chunk<NT, kUnroll>(find_slot(slots, count, b), b, lr, b1, b2, eps, wd, c1, c2);
}

template <bool NT, int U>
__global__ __launch_bounds__(kThreads) void adam_multi_inline(AdamInline table, int count,
                                                              float lr, float b1, float b2,
                                                              float eps, float wd, float c1,
                                                              float c2,
                                                              const float* __restrict__ hyper) {
    read_hyper(hyper, lr, c1, c2);
    const int64_t b = blockIdx.x;
    adam_chunk<NT, U>(find_slot(table.s, count, b), b, lr, b1, b2, eps, wd, c1, c2);
}

// Copies one argument-borne piece of a slot table to device memory (one
// thread per slot): the table upload of a captured step, which can record no
// host transfer.
__global__ __launch_bounds__(kInlineSlots) void write_slots(AdamInline piece, int count,
                                                            AdamSlot* __restrict__ dst) {
    const int i = int(threadIdx.x);
    if (i < count) dst[i] = piece.s[i];
}

// Adam over the multi-tensor table, launched together with the ordered sums
// of convolution weight-gradient partials: blocks [0, rb.blocks) each sum a
// few outputs of one job (partial_sums, the order of conv_weight_reduce), store
// the gradient and, when the gradient belongs to a parameter of this step,
// update that element with the same arithmetic as the table's blocks, which
// take the remaining blocks.
constexpr int kMaxReduceAdam = 8;

struct ReduceAdamJob {
    const float* partial;
    float* grad[2];           // dweight, dbias (or null)
    float* p[2];              // the parameters those gradients belong to (or null)
    float* m[2];
    float* v[2];
    int cout, k, chunks, rl, first;
};

struct ReduceAdamBatch {
    ReduceAdamJob job[kMaxReduceAdam];
    int count, blocks;
};

template <bool NT, int U>
__global__ __launch_bounds__(kThreads) void adam_multi_reduce(ReduceAdamBatch rb, AdamInline table,
                                                              int count, float lr, float b1,
                                                              float b2, float eps, float wd,
                                                              float c1, float c2,
                                                              const float* __restrict__ hyper) {
    read_hyper(hyper, lr, c1, c2);
    __shared__ float lanes[256];
    if (int(blockIdx.x) < rb.blocks) {
        int j = 0;
        while (j + 1 < rb.count && int(blockIdx.x) >= rb.job[j + 1].first) ++j;
        const ReduceAdamJob& r = rb.job[j];
        float sum;
        int o;
        const int outs = r.cout * (r.k + 1), nb = (outs + 256 / r.rl - 1) / (256 / r.rl);
        if (!partial_sums(r.partial, outs, r.chunks, r.rl,
                          xcd_paired_block(int(blockIdx.x) - r.first, nb), lanes, sum, o))
            return;
        const int co = o / (r.k + 1), kk = o % (r.k + 1);
        const int which = kk < r.k ? 0 : 1;
        if (r.grad[which] == nullptr) return;
        const int64_t e = which == 0 ? int64_t(co) * r.k + kk : co;
        r.grad[which][e] = sum;
        if (r.p[which] != nullptr) {
            const Adam op{r.p[which], r.grad[which], r.m[which], r.v[which], lr, b1, b2, eps, wd,
                          c1, c2};
            float pv = r.p[which][e], mv = r.m[which][e], vv = r.v[which][e];
            op.one(pv, sum, mv, vv);
            r.p[which][e] = pv;
            r.m[which][e] = mv;
            r.v[which][e] = vv;
        }
        return;
    }
    if (count == 0) return;
    const int64_t b = int64_t(blockIdx.x) - rb.blocks;
    adam_chunk<NT, U>(find_slot(table.s, count, b), b, lr, b1, b2, eps, wd, c1, c2);
}

// Up to kStoreMax floats carried in the kernel arguments, stored by one thread
// each: a few values reach the device with one launch and no DMA transfer.
constexpr int kStoreMax = 16;
struct StoreValues {
    float v[kStoreMax];
};
__global__ __launch_bounds__(64) void store_values(StoreValues vals, int count,
                                                   float* __restrict__ dst) {
    const int i = int(threadIdx.x);
    if (i < count) dst[i] = vals.v[i];
}

int launch_write_slots(const AdamInline& piece, int n, AdamSlot* dst, hipStream_t s) {
    EHIP_LAUNCH("adam_table", write_slots, dim3(1), dim3(kInlineSlots), 0, s, piece, n, dst);
    return EHIP_OK;
}

// The table-driven update over `chunks` chunks of kAdamChunk elements.
int launch_adam_table(const AdamSlot* table, int count, int64_t chunks, bool nt, float lr,
                      float b1, float b2, float eps, float wd, float c1, float c2,
                      const float* hyper, hipStream_t s) {
    if (nt)
        EHIP_LAUNCH("adam_multi", adam_multi<true>, dim3(unsigned(chunks)), dim3(kThreads), 0, s,
                    table, count, lr, b1, b2, eps, wd, c1, c2, hyper);
    else
        EHIP_LAUNCH("adam_multi", adam_multi<false>, dim3(unsigned(chunks)), dim3(kThreads), 0, s,
                    table, count, lr, b1, b2, eps, wd, c1, c2, hyper);
    return EHIP_OK;
}

template <int OP>
int binary_op(const float* a, const float* b, float* out, int64_t inner, int64_t repeat,
              hipStream_t s) {
    const bool vec = aligned16(a) && aligned16(b) && aligned16(out) && inner % 4 == 0;
    return launch_stream("binary", Binary<OP>{a, b, out, inner}, inner * repeat, vec, s);
}

const OccupancyKernel kElementwiseKernels[] = {
    {"stream_vec<ReluBackward>", reinterpret_cast<const void*>(&stream_vec<ReluBackward, true>), kThreads},
    {"stream_vec<Adam>", reinterpret_cast<const void*>(&stream_vec<Adam, true>), kThreads},
    {"adam_multi", reinterpret_cast<const void*>(&adam_multi<true>), kThreads},
    {"adam_multi_reduce", reinterpret_cast<const void*>(&adam_multi_reduce<true, 1>), kThreads},
};
const OccupancyEntries kElementwiseKernelsReg(kElementwiseKernels);

}  // namespace
}  // namespace ehip

using namespace ehip;

extern "C" {

int ehip_binary_f32(int op, const float* a, const float* b, float* out, int64_t inner,
                    int64_t repeat, void* stream) {
    EHIP_READY();
    if (inner <= 0 || repeat < 0) return fail(EHIP_EINVAL, "binary: bad shape");
    if (!a || !b || !out) return fail(EHIP_EINVAL, "binary: null pointer");
    hipStream_t s = as_stream(stream);
    switch (op) {
        case EHIP_ADD: return binary_op<EHIP_ADD>(a, b, out, inner, repeat, s);
        case EHIP_SUB: return binary_op<EHIP_SUB>(a, b, out, inner, repeat, s);
        case EHIP_MUL: return binary_op<EHIP_MUL>(a, b, out, inner, repeat, s);
        case EHIP_DIV: return binary_op<EHIP_DIV>(a, b, out, inner, repeat, s);
        default: return fail(EHIP_EINVAL, "binary: unknown op %d", op);
    }
}

int ehip_scalar_f32(const float* x, float* out, int64_t n, float mul, float add, void* stream) {
    EHIP_READY();
    if (!x || !out) return fail(EHIP_EINVAL, "scalar: null pointer");
    return launch_stream("scalar", Scalar{x, out, mul, add}, n, aligned16(x) && aligned16(out),
                         as_stream(stream));
}

int ehip_relu_f32(const float* x, float* y, int64_t n, void* stream) {
    EHIP_READY();
    if (!x || !y) return fail(EHIP_EINVAL, "relu: null pointer");
    return launch_stream("relu", Relu{x, y}, n, aligned16(x) && aligned16(y), as_stream(stream));
}

int ehip_activation_f32(int kind, const float* x, float* y, int64_t n, void* stream) {
    EHIP_READY();
    if (!x || !y) return fail(EHIP_EINVAL, "activation: null pointer");
    const bool vec = aligned16(x) && aligned16(y);
    hipStream_t s = as_stream(stream);
    switch (kind) {
        case EHIP_SIGMOID: return launch_stream("sigmoid", Activation<0>{x, y}, n, vec, s);
        case EHIP_TANH: return launch_stream("tanh", Activation<1>{x, y}, n, vec, s);
        case EHIP_GELU: return launch_stream("gelu", Activation<2>{x, y}, n, vec, s);
        default: return fail(EHIP_EINVAL, "activation: kind %d", kind);
    }
}

int ehip_activation_backward_f32(int kind, const float* x, const float* y, const float* g,
                                 float* dx, int64_t n, void* stream) {
    EHIP_READY();
    if (!x || !y || !g || !dx) return fail(EHIP_EINVAL, "activation_backward: null pointer");
    const bool vec = aligned16(x) && aligned16(y) && aligned16(g) && aligned16(dx);
    hipStream_t s = as_stream(stream);
    switch (kind) {
        case EHIP_SIGMOID:
            return launch_stream("sigmoid_backward", ActivationBackward<0>{x, y, g, dx}, n, vec, s);
        case EHIP_TANH:
            return launch_stream("tanh_backward", ActivationBackward<1>{x, y, g, dx}, n, vec, s);
        case EHIP_GELU:
            return launch_stream("gelu_backward", ActivationBackward<2>{x, y, g, dx}, n, vec, s);
        default: return fail(EHIP_EINVAL, "activation_backward: kind %d", kind);
    }
}

int ehip_copy_rows_f32(const float* src, int64_t src_pitch, float* dst, int64_t dst_pitch,
                       int64_t rows, int64_t len, void* stream) {
    EHIP_READY();
    if (rows < 0 || len < 0 || src_pitch < len || dst_pitch < len)
        return fail(EHIP_EINVAL, "copy_rows: bad geometry");
    if (rows == 0 || len == 0) return EHIP_OK;
    if (!src || !dst) return fail(EHIP_EINVAL, "copy_rows: null pointer");
    const int64_t chunks = ceil_div(len, 1024);
    if (rows * chunks > 0x7fffffff) return fail(EHIP_EINVAL, "copy_rows: too large");
    const int vec = aligned16(src) && aligned16(dst) && src_pitch % 4 == 0 && dst_pitch % 4 == 0;
    EHIP_LAUNCH("copy_rows", copy_rows, dim3(unsigned(rows * chunks)), dim3(256), 0,
                as_stream(stream), src, src_pitch, dst, dst_pitch, len, chunks, vec);
    return EHIP_OK;
}

int ehip_max_axis_f32(const float* x, float* y, int32_t* argmax, int64_t outer, int64_t axis_len,
                      int64_t inner, void* stream) {
    EHIP_READY();
    if (outer < 0 || axis_len < 1 || inner < 0 || axis_len > 0x7fffffff)
        return fail(EHIP_EINVAL, "max_axis: bad shape");
    const int64_t n = outer * inner;
    if (n == 0) return EHIP_OK;
    if (!x || !y || !argmax) return fail(EHIP_EINVAL, "max_axis: null pointer");
    if (ceil_div(n, 256) > 0x7fffffff) return fail(EHIP_EINVAL, "max_axis: too large");
    EHIP_LAUNCH("max_axis", max_axis, dim3(unsigned(ceil_div(n, 256))), dim3(256), 0,
                as_stream(stream), x, y, argmax, outer, axis_len, inner);
    return EHIP_OK;
}

int ehip_max_axis_backward_f32(const float* g, const int32_t* argmax, float* dx, int64_t outer,
                               int64_t axis_len, int64_t inner, void* stream) {
    EHIP_READY();
    if (outer < 0 || axis_len < 1 || inner < 0) return fail(EHIP_EINVAL, "max_axis_backward: bad shape");
    const int64_t n = outer * axis_len * inner;
    if (n == 0) return EHIP_OK;
    if (!g || !argmax || !dx) return fail(EHIP_EINVAL, "max_axis_backward: null pointer");
    if (ceil_div(n, 256) > 0x7fffffff) return fail(EHIP_EINVAL, "max_axis_backward: too large");
    EHIP_LAUNCH("max_axis_backward", max_axis_backward, dim3(unsigned(ceil_div(n, 256))), dim3(256),
                0, as_stream(stream), g, argmax, dx, outer, axis_len, inner);
    return EHIP_OK;
}

int ehip_relu_backward_f32(const float* x, const float* g, float* dx, int64_t n, void* stream) {
    EHIP_READY();
    if (!x || !g || !dx) return fail(EHIP_EINVAL, "relu_backward: null pointer");
    return launch_stream("relu_backward", ReluBackward{x, g, dx}, n,
                         aligned16(x) && aligned16(g) && aligned16(dx), as_stream(stream));
}

int ehip_accumulate_grad_f32(float* grad, const float* g, int64_t n, int initialize,
                             void* stream) {
    EHIP_READY();
    if (!grad || !g) return fail(EHIP_EINVAL, "accumulate_grad: null pointer");
    const bool vec = aligned16(grad) && aligned16(g);
    if (initialize)
        return launch_stream("accumulate_grad", Accumulate<true>{grad, g}, n, vec,
                             as_stream(stream));
    return launch_stream("accumulate_grad", Accumulate<false>{grad, g}, n, vec, as_stream(stream));
}

int ehip_add_backward_f32(const float* g, float* da, float* db, int64_t n, int accumulate_a,
                          int accumulate_b, void* stream) {
    EHIP_READY();
    if (!g || !da || !db) return fail(EHIP_EINVAL, "add_backward: null pointer");
    if (da == db) return fail(EHIP_EINVAL, "add_backward: da and db alias");
    const bool vec = aligned16(g) && aligned16(da) && aligned16(db);
    hipStream_t s = as_stream(stream);
    if (accumulate_a && accumulate_b)
        return launch_stream("add_backward", AddBackward<true, true>{g, da, db}, n, vec, s);
    if (accumulate_a)
        return launch_stream("add_backward", AddBackward<true, false>{g, da, db}, n, vec, s);
    if (accumulate_b)
        return launch_stream("add_backward", AddBackward<false, true>{g, da, db}, n, vec, s);
    return launch_stream("add_backward", AddBackward<false, false>{g, da, db}, n, vec, s);
}

int ehip_mul_backward_f32(const float* g, const float* a, const float* b, float* da, float* db,
                          int64_t n, int accumulate_a, int accumulate_b, void* stream) {
    EHIP_READY();
    if (!g || (da && !b) || (db && !a)) return fail(EHIP_EINVAL, "mul_backward: null pointer");
    if (da && da == db) return fail(EHIP_EINVAL, "mul_backward: da and db alias");
    const int ma = da ? (accumulate_a ? 2 : 1) : 0, mb = db ? (accumulate_b ? 2 : 1) : 0;
    const bool vec = aligned16(g) && (!a || aligned16(a)) && (!b || aligned16(b)) &&
                     (!da || aligned16(da)) && (!db || aligned16(db));
    hipStream_t s = as_stream(stream);
#define EHIP_MULB(A, B)                                                                            \
    if (ma == A && mb == B)                                                                        \
        return launch_stream("mul_backward", MulBackward<A, B>{g, a, b, da, db}, n, vec, s)
    EHIP_MULB(1, 1);
    EHIP_MULB(2, 2);
    EHIP_MULB(1, 2);
    EHIP_MULB(2, 1);
    EHIP_MULB(1, 0);
    EHIP_MULB(2, 0);
    EHIP_MULB(0, 1);
    EHIP_MULB(0, 2);
#undef EHIP_MULB
    return EHIP_OK;  // neither gradient requested
}

int ehip_fill_f32(float* x, int64_t n, float value, void* stream) {
    EHIP_READY();
    if (!x && n > 0) return fail(EHIP_EINVAL, "fill: null pointer");
    return launch_stream("fill", Fill{x, value}, n, aligned16(x), as_stream(stream));
}

int ehip_store_f32(float* dst, const float* values, int count, void* stream) {
    EHIP_READY();
    if (count < 0 || count > kStoreMax)
        return fail(EHIP_EINVAL, "store: %d values (at most %d)", count, kStoreMax);
    if (count == 0) return EHIP_OK;
    if (!dst || !values) return fail(EHIP_EINVAL, "store: null pointer");
    StoreValues vals{};
    std::memcpy(vals.v, values, size_t(count) * sizeof(float));
    EHIP_LAUNCH("store", store_values, dim3(1), dim3(64), 0, as_stream(stream), vals, count, dst);
    return EHIP_OK;
}

int ehip_scale_f32(float* x, int64_t n, float factor, void* stream) {
    EHIP_READY();
    if (!x && n > 0) return fail(EHIP_EINVAL, "scale: null pointer");
    return launch_stream("scale", Scale{x, factor}, n, aligned16(x), as_stream(stream));
}

int ehip_sgd_f32(float* p, const float* g, float* velocity, int64_t n, float lr, float momentum,
                 float weight_decay, void* stream) {
    EHIP_READY();
    if (!p || !g) return fail(EHIP_EINVAL, "sgd: null pointer");
    hipStream_t s = as_stream(stream);
    if (momentum != 0.0f) {
        if (!velocity) return fail(EHIP_EINVAL, "sgd: momentum needs a velocity buffer");
        return launch_stream("sgd", Sgd<true>{p, g, velocity, lr, momentum, weight_decay}, n,
                             aligned16(p) && aligned16(g) && aligned16(velocity), s);
    }
    return launch_stream("sgd", Sgd<false>{p, g, nullptr, lr, momentum, weight_decay}, n,
                         aligned16(p) && aligned16(g), s);
}

int ehip_adam_f32(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1,
                  float beta2, float eps, float weight_decay, float bias_c1, float bias_c2,
                  void* stream) {
    EHIP_READY();
    if (!p || !g || !m || !v) return fail(EHIP_EINVAL, "adam: null pointer");
    const bool vec = aligned16(p) && aligned16(g) && aligned16(m) && aligned16(v);
    return launch_stream("adam",
                         Adam{p, g, m, v, lr, beta1, beta2, eps, weight_decay, bias_c1, bias_c2},
                         n, vec, as_stream(stream));
}

static int adam_multi_impl(const ehip_adam_tensor_t* tensors, int count, float lr, float beta1,
                           float beta2, float eps, float weight_decay, float bias_c1,
                           float bias_c2, const float* hyper, void* stream) {
    EHIP_READY();
    if (count < 0 || (count > 0 && tensors == nullptr))
        return fail(EHIP_EINVAL, "adam_multi: bad tensor list");
    int64_t total = 0;
    for (int i = 0; i < count; ++i) {
        if (tensors[i].n < 0)
            return fail(EHIP_EINVAL, "adam_multi: tensor %d has a negative size", i);
        total += tensors[i].n;
    }
    // Small models (at most 2^20 parameters in at most kInlineSlots tensors)
    // take chunks of one float4 per thread.
    int nonempty = 0;
    for (int i = 0; i < count; ++i) nonempty += tensors[i].n > 0;
    const bool small = total <= (int64_t(1) << 20) && nonempty <= kInlineSlots;
    const int64_t chunk = small ? int64_t(kThreads) * 4 : kAdamChunk;
    std::vector<AdamSlot> slots;
    slots.reserve(size_t(count));
    int64_t chunks = 0;
    for (int i = 0; i < count; ++i) {
        const ehip_adam_tensor_t& t = tensors[i];
        if (t.n == 0) continue;
        if (!t.p || !t.g || !t.m || !t.v)
            return fail(EHIP_EINVAL, "adam_multi: tensor %d has a null pointer", i);
        slots.push_back({t.p, t.g, t.m, t.v, t.n, chunks});
        chunks += ceil_div(t.n, chunk);
    }
    if (slots.empty()) return EHIP_OK;
    if (chunks > 0x7fffffff) return fail(EHIP_EINVAL, "adam_multi: too many elements");
    hipStream_t s = as_stream(stream);
    const bool nt = chunks * chunk >= kNontemporalMin;
    if (slots.size() <= size_t(kInlineSlots)) {
        AdamInline inline_table{};
        std::memcpy(inline_table.s, slots.data(), slots.size() * sizeof(AdamSlot));
        if (small)
            EHIP_LAUNCH("adam_multi", (adam_multi_inline<false, 1>), dim3(unsigned(chunks)),
                        dim3(kThreads), 0, s, inline_table, int(slots.size()), lr, beta1, beta2,
                        eps, weight_decay, bias_c1, bias_c2, hyper);
        else if (nt)
            EHIP_LAUNCH("adam_multi", (adam_multi_inline<true, kUnroll>), dim3(unsigned(chunks)),
                        dim3(kThreads), 0, s, inline_table, int(slots.size()), lr, beta1, beta2,
                        eps, weight_decay, bias_c1, bias_c2, hyper);
        else
            EHIP_LAUNCH("adam_multi", (adam_multi_inline<false, kUnroll>), dim3(unsigned(chunks)),
                        dim3(kThreads), 0, s, inline_table, int(slots.size()), lr, beta1, beta2,
                        eps, weight_decay, bias_c1, bias_c2, hyper);
        return EHIP_OK;
    }
    if (capturing() && s == t_capture) {
        // A captured step: a table block of the graph's own, written by kernels
        // whose arguments carry the slots; freed at once, the arena holds the
        // block for the graph until it is destroyed.
        const size_t bytes = slots.size() * sizeof(AdamSlot);
        void* p = nullptr;
        if (int rc = ehip_arena_alloc(bytes, &p)) return rc;
        AdamSlot* tab = static_cast<AdamSlot*>(p);
        int rc = EHIP_OK;
        for (size_t at = 0; at < slots.size() && rc == EHIP_OK; at += kInlineSlots) {
            const int n = int(std::min(slots.size() - at, size_t(kInlineSlots)));
            AdamInline piece{};
            std::memcpy(piece.s, slots.data() + at, size_t(n) * sizeof(AdamSlot));
            rc = launch_write_slots(piece, n, tab + at, s);
        }
        if (rc == EHIP_OK)
            rc = launch_adam_table(tab, int(slots.size()), chunks, nt, lr, beta1, beta2, eps,
                                   weight_decay, bias_c1, bias_c2, hyper, s);
        ehip_arena_free(p);
        return rc;
    }
    // The slot table lives in a buffer of its own and is uploaded only when it
    // differs from the previous call's: an optimiser stepping the same
    // parameters every iteration pays no host-to-device copy per step. Work is
    // ordered on one stream, so a new upload lands after the kernels that read
    // the old table.
    static std::mutex table_mu;
    static std::vector<AdamSlot> last;
    static AdamSlot* table = nullptr;
    static size_t table_cap = 0;
    std::lock_guard<std::mutex> lock(table_mu);
    const size_t bytes = slots.size() * sizeof(AdamSlot);
    const bool same = table != nullptr && last.size() == slots.size() &&
                      std::memcmp(last.data(), slots.data(), bytes) == 0;
    if (!same) {
        if (bytes > table_cap) {
            if (table != nullptr) ehip_arena_free(table);
            table = nullptr;
            table_cap = 0;
            void* p = nullptr;
            if (int rc = ehip_arena_alloc(bytes, &p)) return rc;
            table = static_cast<AdamSlot*>(p);
            table_cap = bytes;
        }
        last.clear();  // a failed upload leaves no table marked as current
        if (int rc = ehip_memcpy_h2d(table, slots.data(), bytes, stream)) return rc;
        last = slots;
    }
    return launch_adam_table(table, int(slots.size()), chunks, nt, lr, beta1, beta2, eps,
                             weight_decay, bias_c1, bias_c2, hyper, s);
}

int ehip_adam_multi_f32(const ehip_adam_tensor_t* tensors, int count, float lr, float beta1,
                        float beta2, float eps, float weight_decay, float bias_c1,
                        float bias_c2, void* stream) {
    return adam_multi_impl(tensors, count, lr, beta1, beta2, eps, weight_decay, bias_c1, bias_c2,
                           nullptr, stream);
}

int ehip_adam_multi_dev_f32(const ehip_adam_tensor_t* tensors, int count, const float* hyper,
                            float beta1, float beta2, float eps, float weight_decay,
                            void* stream) {
    if (hyper == nullptr) return fail(EHIP_EINVAL, "adam_multi_dev: null hyper-parameter array");
    return adam_multi_impl(tensors, count, 0.0f, beta1, beta2, eps, weight_decay, 0.0f, 0.0f,
                           hyper, stream);
}


static int adam_multi_reduce_impl(const ehip_adam_tensor_t* tensors, int count,
                                  const ehip_conv_reduce_t* jobs, int njobs, float lr,
                                  float beta1, float beta2, float eps, float weight_decay,
                                  float bias_c1, float bias_c2, const float* hyper,
                                  void* stream) {
    EHIP_READY();
    if (count < 0 || (count > 0 && tensors == nullptr) || njobs < 0 ||
        (njobs > 0 && jobs == nullptr))
        return fail(EHIP_EINVAL, "adam_multi_reduce: bad list");
    hipStream_t s = as_stream(stream);
    // Beyond one launch's job table: the separate reduction, then the step.
    if (njobs > kMaxReduceAdam) {
        if (int rc = ehip_conv_weight_reduce_f32(jobs, njobs, stream)) return rc;
        return adam_multi_impl(tensors, count, lr, beta1, beta2, eps, weight_decay, bias_c1,
                               bias_c2, hyper, stream);
    }
    ReduceAdamBatch rb{};
    std::vector<char> owned(size_t(count), 0);
    int64_t blocks = 0;
    for (int j = 0; j < njobs; ++j) {
        const ehip_conv_reduce_t& q = jobs[j];
        if (!q.partials || !q.dweight || q.chunks <= 0 || q.out_channels <= 0 || q.k <= 0 ||
            q.chunks > 0x7fffffff || q.out_channels * (q.k + 1) > 0x7fffffff)
            return fail(EHIP_EINVAL, "adam_multi_reduce: bad job %d", j);
        ReduceAdamJob& r = rb.job[rb.count++];
        r.partial = q.partials;
        r.grad[0] = q.dweight;
        r.grad[1] = q.dbias;
        const int64_t n[2] = {q.out_channels * q.k, q.out_channels};
        for (int w = 0; w < 2; ++w)
            for (int i = 0; i < count && r.grad[w] != nullptr; ++i)
                if (tensors[i].g == r.grad[w] && tensors[i].n == n[w] && !owned[size_t(i)]) {
                    if (!tensors[i].p || !tensors[i].m || !tensors[i].v)
                        return fail(EHIP_EINVAL, "adam_multi_reduce: tensor %d has a null pointer", i);
                    r.p[w] = tensors[i].p;
                    r.m[w] = tensors[i].m;
                    r.v[w] = tensors[i].v;
                    owned[size_t(i)] = 1;
                    break;
                }
        r.cout = int(q.out_channels);
        r.k = int(q.k);
        r.chunks = int(q.chunks);
        r.rl = reduce_lanes(q.chunks);
        r.first = int(blocks);
        blocks += ceil_div(q.out_channels * (q.k + 1), 256 / r.rl);
    }
    rb.blocks = int(blocks);
    // The other tensors: the small-model chunking of ehip_adam_multi_f32.
    std::vector<AdamSlot> slots;
    int64_t total = 0, chunks = 0;
    for (int i = 0; i < count; ++i) {
        if (tensors[i].n < 0) return fail(EHIP_EINVAL, "adam_multi_reduce: tensor %d has a negative size", i);
        if (!owned[size_t(i)]) total += tensors[i].n;
    }
    for (int i = 0; i < count; ++i) {
        const ehip_adam_tensor_t& t = tensors[i];
        if (owned[size_t(i)] || t.n == 0) continue;
        if (!t.p || !t.g || !t.m || !t.v)
            return fail(EHIP_EINVAL, "adam_multi_reduce: tensor %d has a null pointer", i);
        slots.push_back({t.p, t.g, t.m, t.v, t.n, chunks});
        chunks += ceil_div(t.n, int64_t(kThreads) * 4);
    }
    if (total > (int64_t(1) << 20) || slots.size() > size_t(kInlineSlots)) {
        // A large model: the separate reduction, then the step.
        if (int rc = ehip_conv_weight_reduce_f32(jobs, njobs, stream)) return rc;
        return adam_multi_impl(tensors, count, lr, beta1, beta2, eps, weight_decay, bias_c1,
                               bias_c2, hyper, stream);
    }
    AdamInline inline_table{};
    if (!slots.empty()) std::memcpy(inline_table.s, slots.data(), slots.size() * sizeof(AdamSlot));
    if (blocks + chunks == 0) return EHIP_OK;
    if (blocks + chunks > 0x7fffffff) return fail(EHIP_EINVAL, "adam_multi_reduce: too many blocks");
    EHIP_LAUNCH("adam_multi_reduce", (adam_multi_reduce<false, 1>), dim3(unsigned(blocks + chunks)),
                dim3(kThreads), 0, s, rb, inline_table, int(slots.size()), lr, beta1, beta2, eps,
                weight_decay, bias_c1, bias_c2, hyper);
    return EHIP_OK;
}

int ehip_adam_multi_reduce_f32(const ehip_adam_tensor_t* tensors, int count,
                               const ehip_conv_reduce_t* jobs, int njobs, float lr, float beta1,
                               float beta2, float eps, float weight_decay, float bias_c1,
                               float bias_c2, void* stream) {
    return adam_multi_reduce_impl(tensors, count, jobs, njobs, lr, beta1, beta2, eps,
                                  weight_decay, bias_c1, bias_c2, nullptr, stream);
}

int ehip_adam_multi_reduce_dev_f32(const ehip_adam_tensor_t* tensors, int count,
                                   const ehip_conv_reduce_t* jobs, int njobs, const float* hyper,
                                   float beta1, float beta2, float eps, float weight_decay,
                                   void* stream) {
    if (hyper == nullptr)
        return fail(EHIP_EINVAL, "adam_multi_reduce_dev: null hyper-parameter array");
    return adam_multi_reduce_impl(tensors, count, jobs, njobs, 0.0f, beta1, beta2, eps,
                                  weight_decay, 0.0f, 0.0f, hyper, stream);
}


}  // extern "C"
