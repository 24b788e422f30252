// conv_gemm.hip -- implicit-GEMM convolution for layers too wide for the
// direct kernels: the three products of a Conv2d (forward, weight gradient,
// input gradient) on the MFMA tiles, with the im2col / col2im operand read
// straight from the activation or gradient it is made of, so no column matrix
// is materialised (the reference builds it in memory: src/conv.cpp:61-217,
// 280-338).
//
//   forward   out[n] (C_out x P)  = W (C_out x K) . cols[n] (K x P) + bias
//   dW                (C_out x K) = sum over n, p of dOut[n](co, p) cols[n](k, p)
//   dx        dx[n] (C x H W)     = W' (C x K') . dOut'[n] (K' x H W)
//
// with P = oH oW, K = C kH kW ordered (c, i, j) as the reference's im2col,
// cols[n](k, p) = x[n][c][oh s - pad + i][ow s - pad + j] (0 in the padding),
// K' = C_out kH kW ordered (co, i, j), W'(c, (co, i, j)) = W[co][c][i][j] and
// dOut'[n]((co, i, j), (h, w)) = dOut[n][co][(h + pad - i) / s][(w + pad - j) / s]
// where the division is exact and in range, else 0 (the adjoint of im2col,
// col2im, as a gather). dx thus reduces over C_out kH kW in (co, i, j) order
// instead of col2im's sum over windows.
//
// The tiles are the GEMM's (fp32 MFMA 32x32x2, two LDS buffers, the next K
// step's loads issued before the current MFMAs); only the operand loads
// differ. Each thread decomposes the rows it gathers (output pixel, input
// pixel, kernel tap) once per tile; per K step it decomposes the one reduction
// index it starts from with multiply-shift division by the layer's invariant
// divisors and steps the rest. Dense runs (weight rows, gradient rows of one
// image) load as float4. Sums are fixed-order and deterministic; the results
// are the products' values within the K-term tolerance, not the bits of the
// reference's serial loops (as for the explicit im2col + GEMM path).
#include <algorithm>
#include <climits>

#include "common.hpp"
#include "gemm_kernel.hpp"

namespace ehip {
namespace {

using namespace gemm_detail;

// n / d for 0 <= n < 2^31 by the round-up multiply-shift method of Granlund
// and Montgomery ("Division by invariant integers using multiplication",
// PLDI 1994): s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1,
// n / d = (mulhi(n, m) + n) >> s, the sum taken in 64 bits.
struct FastDiv {
    uint32_t m, s;
    __device__ __forceinline__ int div(int n) const {
        return int((uint64_t(__umulhi(uint32_t(n), m)) + uint32_t(n)) >> s);
    }
};

FastDiv fast_div(int64_t d) {
    FastDiv f{0, 0};
    while ((int64_t(1) << f.s) < d) ++f.s;
    f.m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << f.s) - uint64_t(d))) / uint64_t(d) + 1);
    return f;
}

// One layer's geometry; every index inside an image, and the batch's output
// pixels N oH oW, fit in 32 bits (check_layer).
struct ConvGeo {
    int c, h, w, co, kh, kw, stride, pad, oh, ow;
    int khw, hw, p, k;  // kH kW, H W, oH oW, C kH kW
    int64_t chw;        // C H W
    FastDiv d_khw, d_kw, d_p, d_ow, d_w, d_s;
    const float* x;
    const float* wt;
    const float* dout;
};

ConvGeo geo_of(const ehip_window_t& w, int64_t out_channels) {
    ConvGeo g{};
    g.c = int(w.channels);
    g.h = int(w.height);
    g.w = int(w.width);
    g.co = int(out_channels);
    g.kh = int(w.kernel_h);
    g.kw = int(w.kernel_w);
    g.stride = int(w.stride);
    g.pad = int(w.padding);
    g.oh = int(w.out_h);
    g.ow = int(w.out_w);
    g.khw = g.kh * g.kw;
    g.hw = g.h * g.w;
    g.p = g.oh * g.ow;
    g.k = g.c * g.khw;
    g.chw = int64_t(g.c) * g.hw;
    g.d_khw = fast_div(g.khw);
    g.d_kw = fast_div(g.kw);
    g.d_p = fast_div(g.p);
    g.d_ow = fast_div(g.ow);
    g.d_w = fast_div(g.w);
    g.d_s = fast_div(g.stride);
    return g;
}

// Slot l of a thread in a BR x BK operand tile. Row-major slots (op(A) stored
// rows x K): row q / (BK / 4), four consecutive k from 4 (q % (BK / 4)).
// Transposed slots (stored K x rows): k q / (BR / 4), four consecutive rows
// from 4 (q % (BR / 4)). q = threadIdx.x + l * threads.
template <class C>
__device__ __forceinline__ int slot_q(int l) { return int(threadIdx.x) + l * C::kThreads; }

// ---- forward: A = W (C_out x K, row pitch K), B = cols of one image as (p, k) rows.
template <class C, int BR, int BK>
struct WeightRows {
    static constexpr bool kTrans = false;
    static constexpr int L = BR * BK / 4 / C::kThreads;
    const float* src[L];
    bool vec;
    __device__ WeightRows(const ConvGeo& g, int64_t, int64_t r0, bool v) : vec(v) {
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int q = slot_q<C>(l);
            const int64_t r = r0 + q / (BK / 4);
            src[l] = r < g.co ? g.wt + r * g.k + 4 * (q % (BK / 4)) : nullptr;
        }
    }
    __device__ void load(int64_t k0, int64_t kend, float4* reg) const {
#pragma unroll
        for (int l = 0; l < L; ++l) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            const int64_t kk = k0 + 4 * (slot_q<C>(l) % (BK / 4));
            if (src[l] != nullptr) {
                const float* s = src[l] + k0;
                if (vec && kk + 3 < kend) {
                    v = *reinterpret_cast<const float4*>(s);
                } else {
                    v.x = kk < kend ? s[0] : 0.f;
                    v.y = kk + 1 < kend ? s[1] : 0.f;
                    v.z = kk + 2 < kend ? s[2] : 0.f;
                    v.w = kk + 3 < kend ? s[3] : 0.f;
                }
            }
            reg[l] = v;
        }
    }
};

template <class C, int BR, int BK>
struct ColsByPixel {
    static constexpr bool kTrans = true;
    static constexpr int L = BR * BK / 4 / C::kThreads;
    const ConvGeo& g;
    const float* img;
    int iy[L][4], ix[L][4];
    __device__ ColsByPixel(const ConvGeo& g_, int64_t z, int64_t r0, bool) : g(g_) {
        img = g.x + z * g.chw;
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int64_t p0 = r0 + 4 * (slot_q<C>(l) % (BR / 4));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (p0 + e < g.p) {
                    const int p = int(p0 + e);
                    const int oh = g.d_ow.div(p);
                    iy[l][e] = oh * g.stride - g.pad;
                    ix[l][e] = (p - oh * g.ow) * g.stride - g.pad;
                } else {
                    iy[l][e] = INT_MIN / 2;  // never inside the image
                    ix[l][e] = 0;
                }
            }
        }
    }
    __device__ void load(int64_t k0, int64_t kend, float4* reg) const {
#pragma unroll
        for (int l = 0; l < L; ++l) {
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            const int64_t kk = k0 + slot_q<C>(l) / (BR / 4);
            if (kk < kend) {
                const int k = int(kk);
                const int c = g.d_khw.div(k), r = k - c * g.khw;
                const int i = g.d_kw.div(r), j = r - i * g.kw;
                const float* b = img + int64_t(c) * g.hw;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int y = iy[l][e] + i, xx = ix[l][e] + j;
                    if (unsigned(y) < unsigned(g.h) && unsigned(xx) < unsigned(g.w))
                        v[e] = b[y * g.w + xx];
                }
            }
            reg[l] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
};

// ---- dW: reduction index kr = (n, p). A(co, kr) = dOut[n][co][p];
// B(k, kr) = cols[n](k, p), k = (c, i, j) fixed per slot.
template <class C, int BR, int BK>
struct DoutByChannel {
    static constexpr bool kTrans = false;
    static constexpr int L = BR * BK / 4 / C::kThreads;
    const ConvGeo& g;
    int co[L];
    bool vec;
    __device__ DoutByChannel(const ConvGeo& g_, int64_t, int64_t r0, bool v) : g(g_), vec(v) {
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int64_t r = r0 + slot_q<C>(l) / (BK / 4);
            co[l] = r < g.co ? int(r) : -1;
        }
    }
    __device__ void load(int64_t k0, int64_t kend, float4* reg) const {
#pragma unroll
        for (int l = 0; l < L; ++l) {
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            const int64_t kk = k0 + 4 * (slot_q<C>(l) % (BK / 4));
            if (co[l] >= 0 && kk < kend) {
                const int kr = int(kk);
                int n = g.d_p.div(kr), p = kr - n * g.p;
                if (vec && kk + 3 < kend) {  // p % 4 == 0 and P % 4 == 0: one image
                    const float4 f = *reinterpret_cast<const float4*>(
                        g.dout + (int64_t(n) * g.co + co[l]) * g.p + p);
                    v[0] = f.x;
                    v[1] = f.y;
                    v[2] = f.z;
                    v[3] = f.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (kk + e < kend) v[e] = g.dout[(int64_t(n) * g.co + co[l]) * g.p + p];
                        if (++p == g.p) {
                            p = 0;
                            ++n;
                        }
                    }
                }
            }
            reg[l] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
};

template <class C, int BR, int BK>
struct ColsByTap {
    static constexpr bool kTrans = false;
    static constexpr int L = BR * BK / 4 / C::kThreads;
    const ConvGeo& g;
    int64_t coff[L];  // c H W, or -1 past the last row
    int ti[L], tj[L];
    __device__ ColsByTap(const ConvGeo& g_, int64_t, int64_t r0, bool) : g(g_) {
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int64_t r = r0 + slot_q<C>(l) / (BK / 4);
            if (r < g.k) {
                const int k = int(r);
                const int c = g.d_khw.div(k), t = k - c * g.khw;
                ti[l] = g.d_kw.div(t);
                tj[l] = t - ti[l] * g.kw;
                coff[l] = int64_t(c) * g.hw;
            } else {
                coff[l] = -1;
                ti[l] = tj[l] = 0;
            }
        }
    }
    __device__ void load(int64_t k0, int64_t kend, float4* reg) const {
#pragma unroll
        for (int l = 0; l < L; ++l) {
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            const int64_t kk = k0 + 4 * (slot_q<C>(l) % (BK / 4));
            if (coff[l] >= 0 && kk < kend) {
                const int kr = int(kk);
                int n = g.d_p.div(kr), p = kr - n * g.p;
                int oh = g.d_ow.div(p), ow = p - oh * g.ow;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int y = oh * g.stride - g.pad + ti[l];
                    const int xx = ow * g.stride - g.pad + tj[l];
                    if (kk + e < kend && unsigned(y) < unsigned(g.h) && unsigned(xx) < unsigned(g.w))
                        v[e] = g.x[int64_t(n) * g.chw + coff[l] + y * g.w + xx];
                    if (++ow == g.ow) {
                        ow = 0;
                        if (++oh == g.oh) {
                            oh = 0;
                            ++n;
                        }
                    }
                }
            }
            reg[l] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
};

// ---- dx: reduction index kr = (co, i, j). A(c, kr) = W[co][c][i][j];
// B(q, kr) = dOut of one image at the window (i, j) of input pixel q = (h, w).
template <class C, int BR, int BK>
struct WeightByInput {
    static constexpr bool kTrans = false;
    static constexpr int L = BR * BK / 4 / C::kThreads;
    const ConvGeo& g;
    int ch[L];
    __device__ WeightByInput(const ConvGeo& g_, int64_t, int64_t r0, bool) : g(g_) {
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int64_t r = r0 + slot_q<C>(l) / (BK / 4);
            ch[l] = r < g.c ? int(r) : -1;
        }
    }
    __device__ void load(int64_t k0, int64_t kend, float4* reg) const {
#pragma unroll
        for (int l = 0; l < L; ++l) {
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            const int64_t kk = k0 + 4 * (slot_q<C>(l) % (BK / 4));
            if (ch[l] >= 0 && kk < kend) {
                const int kr = int(kk);
                int o = g.d_khw.div(kr), t = kr - o * g.khw;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (kk + e < kend) v[e] = g.wt[(int64_t(o) * g.c + ch[l]) * g.khw + t];
                    if (++t == g.khw) {
                        t = 0;
                        ++o;
                    }
                }
            }
            reg[l] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
};

template <class C, int BR, int BK, bool STRIDE1>
struct DoutByPixel {
    static constexpr bool kTrans = true;
    static constexpr int L = BR * BK / 4 / C::kThreads;
    const ConvGeo& g;
    const float* img;
    int hp[L][4], wp[L][4];  // h + pad, w + pad
    __device__ DoutByPixel(const ConvGeo& g_, int64_t z, int64_t r0, bool) : g(g_) {
        img = g.dout + z * int64_t(g.co) * g.p;
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int64_t q0 = r0 + 4 * (slot_q<C>(l) % (BR / 4));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (q0 + e < g.hw) {
                    const int q = int(q0 + e);
                    const int h = g.d_w.div(q);
                    hp[l][e] = h + g.pad;
                    wp[l][e] = q - h * g.w + g.pad;
                } else {
                    hp[l][e] = INT_MIN / 2;  // no window covers it
                    wp[l][e] = 0;
                }
            }
        }
    }
    __device__ void load(int64_t k0, int64_t kend, float4* reg) const {
#pragma unroll
        for (int l = 0; l < L; ++l) {
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            const int64_t kk = k0 + slot_q<C>(l) / (BR / 4);
            if (kk < kend) {
                const int kr = int(kk);
                const int o = g.d_khw.div(kr), t = kr - o * g.khw;
                const int i = g.d_kw.div(t), j = t - i * g.kw;
                const float* b = img + int64_t(o) * g.p;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int y = hp[l][e] - i, xx = wp[l][e] - j;
                    if (STRIDE1) {
                        if (unsigned(y) < unsigned(g.oh) && unsigned(xx) < unsigned(g.ow))
                            v[e] = b[y * g.ow + xx];
                    } else if (y >= 0 && xx >= 0) {
                        const int oy = g.d_s.div(y), ox = g.d_s.div(xx);
                        if (oy * g.stride == y && ox * g.stride == xx && oy < g.oh && ox < g.ow)
                            v[e] = b[oy * g.ow + ox];
                    }
                }
            }
            reg[l] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
};

// ---- dx by stride phase (stride 2..4): input pixel (h, w) is reached only by
// the taps i = ph + s t, j = pw + s u with ph = (h + pad) mod s, pw = (w +
// pad) mod s, from output pixel (a - t, b - u) where a = (h + pad) div s,
// b = (w + pad) div s. The pixels of one phase (ph, pw) form a grid
// h = ph - pad + s a (a0 <= a < a0 + hph), w = pw - pad + s b; their product
// reduces over (co, t, u) only -- the taps that reach them -- instead of all
// C_out kH kW, of which all but about one in s^2 would gather a zero.
constexpr int kMaxPhases = 16;
// Largest column gradient a strided layer's dx materialises (beyond it, the
// phase kernels gather in place).
constexpr size_t kStridedColsMax = size_t(1) << 30;

struct Phase {
    int ph, pw, a0, b0, hph, wph, ti, tj;
    FastDiv d_wph, d_tt, d_tj;  // wph, ti tj, tj
};

struct PhaseSet {
    Phase p[kMaxPhases];
};

template <class C, int BR, int BK>
struct PhaseWeight {  // A(c, (co, t, u)) = W[co][c][ph + s t][pw + s u]
    static constexpr bool kTrans = false;
    static constexpr int L = BR * BK / 4 / C::kThreads;
    const ConvGeo& g;
    const Phase& f;
    int ch[L];
    __device__ PhaseWeight(const ConvGeo& g_, const Phase& f_, int64_t, int64_t r0)
        : g(g_), f(f_) {
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int64_t r = r0 + slot_q<C>(l) / (BK / 4);
            ch[l] = r < g.c ? int(r) : -1;
        }
    }
    __device__ void load(int64_t k0, int64_t kend, float4* reg) const {
        const int tt = f.ti * f.tj;
#pragma unroll
        for (int l = 0; l < L; ++l) {
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            const int64_t kk = k0 + 4 * (slot_q<C>(l) % (BK / 4));
            if (ch[l] >= 0 && kk < kend) {
                const int kr = int(kk);
                int o = f.d_tt.div(kr), rem = kr - o * tt;
                int t = f.d_tj.div(rem), u = rem - t * f.tj;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (kk + e < kend)
                        v[e] = g.wt[((int64_t(o) * g.c + ch[l]) * g.kh + f.ph + g.stride * t) * g.kw +
                                    f.pw + g.stride * u];
                    if (++u == f.tj) {
                        u = 0;
                        if (++t == f.ti) {
                            t = 0;
                            ++o;
                        }
                    }
                }
            }
            reg[l] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
};

template <class C, int BR, int BK>
struct PhaseDout {  // B(q, (co, t, u)) = dOut[co][a - t][b - u], q = (a, b) of the phase
    static constexpr bool kTrans = true;
    static constexpr int L = BR * BK / 4 / C::kThreads;
    const ConvGeo& g;
    const Phase& f;
    const float* img;
    int ay[L][4], bx[L][4];
    __device__ PhaseDout(const ConvGeo& g_, const Phase& f_, int64_t image, int64_t r0)
        : g(g_), f(f_) {
        img = g.dout + image * int64_t(g.co) * g.p;
        const int count = f.hph * f.wph;
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int64_t q0 = r0 + 4 * (slot_q<C>(l) % (BR / 4));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (q0 + e < count) {
                    const int q = int(q0 + e);
                    const int a = f.d_wph.div(q);
                    ay[l][e] = f.a0 + a;
                    bx[l][e] = f.b0 + q - a * f.wph;
                } else {
                    ay[l][e] = INT_MIN / 2;  // past the phase's pixels
                    bx[l][e] = 0;
                }
            }
        }
    }
    __device__ void load(int64_t k0, int64_t kend, float4* reg) const {
        const int tt = f.ti * f.tj;
#pragma unroll
        for (int l = 0; l < L; ++l) {
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            const int64_t kk = k0 + slot_q<C>(l) / (BR / 4);
            if (kk < kend) {
                const int kr = int(kk);
                const int o = f.d_tt.div(kr), rem = kr - o * tt;
                const int t = f.d_tj.div(rem), u = rem - t * f.tj;
                const float* b = img + int64_t(o) * g.p;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int oy = ay[l][e] - t, ox = bx[l][e] - u;
                    if (unsigned(oy) < unsigned(g.oh) && unsigned(ox) < unsigned(g.ow))
                        v[e] = b[oy * g.ow + ox];
                }
            }
            reg[l] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
};

// The K loop of one tile: the loaders' registers for step s + 1 are filled
// while the MFMAs of step s run from LDS; acc starts at zero.
template <class C, int BK, class TA, class TB>
__device__ __forceinline__ void conv_mainloop(const TA& la, const TB& lb, int64_t k_begin,
                                              int64_t k_end, float (*lds_a)[BK * C::kLdsA],
                                              float (*lds_b)[BK * C::kLdsB],
                                              floatx16 (&acc)[C::kFM][C::kFN], int wm0, int wn0,
                                              int lane) {
    constexpr int BM = C::kWavesM * (C::kFM * 32), BN = C::kWavesN * (C::kFN * 32);
#pragma unroll
    for (int i = 0; i < C::kFM; ++i)
#pragma unroll
        for (int j = 0; j < C::kFN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    float4 ra[C::kALoads], rb[C::kBLoads];
    const int64_t steps = (k_end - k_begin + BK - 1) / BK;
    if (steps > 0) {
        la.load(k_begin, k_end, ra);
        lb.load(k_begin, k_end, rb);
        store_tile<C, BM, BK, C::kLdsA, TA::kTrans>(lds_a[0], ra, C::kALoads, C::kA4);
        store_tile<C, BN, BK, C::kLdsB, TB::kTrans>(lds_b[0], rb, C::kBLoads, C::kB4);
        __syncthreads();
    }
    for (int64_t s = 0; s < steps; ++s) {
        const int cur = int(s & 1);
        const bool more = s + 1 < steps;
        if (more) {
            const int64_t kn = k_begin + (s + 1) * BK;
            la.load(kn, k_end, ra);
            lb.load(kn, k_end, rb);
        }
        mfma_stage<C, BK>(acc, lds_a[cur], lds_b[cur], wm0, wn0, lane);
        if (more) {
            store_tile<C, BM, BK, C::kLdsA, TA::kTrans>(lds_a[cur ^ 1], ra, C::kALoads, C::kA4);
            store_tile<C, BN, BK, C::kLdsB, TB::kTrans>(lds_b[cur ^ 1], rb, C::kBLoads, C::kB4);
        }
        __syncthreads();
    }
}

// One BM x BN tile of product blockIdx.z of g (m x n, reduction k), K split
// over blockIdx.y as the GEMM splits it. Output: g.c + z * g.stride_c (row
// pitch g.ldc), or the split-K workspace. LA / LB load the A (m x k) and B
// (n x k) operand tiles.
template <class C, int BK, template <class, int, int> class LA, template <class, int, int> class LB,
          bool EPI>
__global__ __launch_bounds__(C::kThreads) void conv_gemm_kernel(GemmArgs g, ConvGeo cg, int vec_a,
                                                                int vec_b) {
    constexpr int BM = C::kWavesM * (C::kFM * 32), BN = C::kWavesN * (C::kFN * 32);
    __shared__ float lds_a[2][BK * C::kLdsA];
    __shared__ float lds_b[2][BK * C::kLdsB];
    const int bid = blockIdx.x;
    const int tm = bid / g.tiles_n, tn = bid % g.tiles_n;
    const int split = blockIdx.y;
    const int64_t z = blockIdx.z;
    const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;
    const int64_t k_begin = int64_t(split) * g.k_chunk;
    int64_t k_end = k_begin + g.k_chunk;
    if (k_end > g.k) k_end = g.k;
    using TA = LA<C, BM, BK>;
    using TB = LB<C, BN, BK>;
    static_assert(TA::L == C::kALoads && TA::L * C::kThreads == C::kA4, "A slots");
    static_assert(TB::L == C::kBLoads && TB::L * C::kThreads == C::kB4, "B slots");
    const TA la(cg, z, m0, vec_a != 0);
    const TB lb(cg, z, n0, vec_b != 0);

    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int wm0 = (wave / C::kWavesN) * (C::kFM * 32), wn0 = (wave % C::kWavesN) * (C::kFN * 32);
    floatx16 acc[C::kFM][C::kFN];
    conv_mainloop<C, BK>(la, lb, k_begin, k_end, lds_a, lds_b, acc, wm0, wn0, lane);
    float* Cp;
    int64_t ldc;
    if (g.splits > 1) {
        Cp = g.c + int64_t(split) * g.ws_stride + z * g.m * g.n;
        ldc = g.n;
    } else {
        Cp = g.c + z * g.stride_c;
        ldc = g.ldc;
    }
    store_acc<C, true, EPI>(g, acc, Cp, ldc, g.add, m0, n0, wm0, wn0, lane);
}

// dx of one stride phase of one image (blockIdx.z = image * phases + phase):
// a C x (hph wph) product over C_out ti tj, stored at the phase's pixels. A
// tile past the phase's pixels has nothing to do and returns as a whole.
template <class C, int BK>
__global__ __launch_bounds__(C::kThreads) void conv_dx_phase_kernel(GemmArgs g, ConvGeo cg,
                                                                    PhaseSet ps, int phases) {
    constexpr int BM = C::kWavesM * (C::kFM * 32), BN = C::kWavesN * (C::kFN * 32);
    __shared__ float lds_a[2][BK * C::kLdsA];
    __shared__ float lds_b[2][BK * C::kLdsB];
    const int64_t image = blockIdx.z / phases;
    const Phase& f = ps.p[blockIdx.z % phases];
    const int count = f.hph * f.wph;
    const int tm = int(blockIdx.x) / g.tiles_n, tn = int(blockIdx.x) % g.tiles_n;
    const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;
    if (n0 >= count) return;
    using TA = PhaseWeight<C, BM, BK>;
    using TB = PhaseDout<C, BN, BK>;
    static_assert(TA::L == C::kALoads && TA::L * C::kThreads == C::kA4, "A slots");
    static_assert(TB::L == C::kBLoads && TB::L * C::kThreads == C::kB4, "B slots");
    const TA la(cg, f, image, m0);
    const TB lb(cg, f, image, n0);
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int wm0 = (wave / C::kWavesN) * (C::kFM * 32), wn0 = (wave % C::kWavesN) * (C::kFN * 32);
    floatx16 acc[C::kFM][C::kFN];
    conv_mainloop<C, BK>(la, lb, 0, int64_t(cg.co) * f.ti * f.tj, lds_a, lds_b, acc, wm0, wn0,
                         lane);
    float* dst = g.c + image * cg.chw;
#pragma unroll
    for (int i = 0; i < C::kFM; ++i)
#pragma unroll
        for (int j = 0; j < C::kFN; ++j) {
            const int64_t col = n0 + wn0 + 32 * j + lane % 32;
            if (col >= count) continue;
            const int a = f.d_wph.div(int(col));
            const int h = f.ph - cg.pad + cg.stride * (f.a0 + a);
            const int w = f.pw - cg.pad + cg.stride * (f.b0 + int(col) - a * f.wph);
            float* px = dst + h * cg.w + w;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm0 + 32 * i + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
                if (row < cg.c) px[row * cg.hw] = acc[i][j][r];
            }
        }
}

// db[co] = sum over images n and positions p of dOut[n][co][p]: one block per
// channel, thread t adding the float4 (or float) runs t, t + 512, ... of each
// image in image order, then the threads by a fixed tree.
template <bool VEC>
__global__ __launch_bounds__(512) void conv_bias_grad(const float* __restrict__ dout,
                                                      float* __restrict__ db, int64_t n,
                                                      int64_t co, int64_t p) {
    __shared__ float sh[512];
    const int64_t c = blockIdx.x;
    float acc = 0.0f;
    for (int64_t img = 0; img < n; ++img) {
        const float* row = dout + (img * co + c) * p;
        if (VEC) {
            for (int64_t q = threadIdx.x; 4 * q < p; q += 512) {
                const float4 f = reinterpret_cast<const float4*>(row)[q];
                acc += f.x;
                acc += f.y;
                acc += f.z;
                acc += f.w;
            }
        } else {
            for (int64_t q = threadIdx.x; q < p; q += 512) acc += row[q];
        }
    }
    sh[threadIdx.x] = acc;
    __syncthreads();
    for (int half = 256; half >= 1; half /= 2) {
        if (int(threadIdx.x) < half) sh[threadIdx.x] = sh[threadIdx.x] + sh[threadIdx.x + half];
        __syncthreads();
    }
    if (threadIdx.x == 0) db[c] = sh[0];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// K splits for a grid of `blocks` tiles: enough for about 512 workgroups
// while each split keeps at least 8 K steps of bk.
int split_count(int64_t blocks, int64_t k, int bk) {
    if (blocks >= 512 || k < 16 * bk) return 1;
    int64_t want = ceil_div(512, blocks);
    const int64_t max_by_k = k / (8 * bk);
    if (want > max_by_k) want = max_by_k;
    if (want > 256) want = 256;
    return want > 1 ? int(want) : 1;
}

// Launches one product with tile config C: m x n per z (`batch` of them),
// reduction k, split when the tile grid is small and the reduction long (as
// the GEMM does), the splits then summed by the GEMM's split-K reduction.
template <class C, int BK, template <class, int, int> class LA, template <class, int, int> class LB,
          bool EPI>
int launch_product(GemmArgs g, int64_t batch, const ConvGeo& cg, bool vec_a, bool vec_b,
                   hipStream_t s) {
    constexpr int BM = C::kWavesM * (C::kFM * 32), BN = C::kWavesN * (C::kFN * 32);
    g.tiles_m = int(ceil_div(g.m, BM));
    g.tiles_n = int(ceil_div(g.n, BN));
    const int64_t tiles = int64_t(g.tiles_m) * g.tiles_n;
    int splits = split_count(tiles * batch, g.k, BK);
    g.k_chunk = ceil_div(ceil_div(g.k, splits), BK) * BK;
    splits = int(ceil_div(g.k, g.k_chunk));
    g.splits = splits;
    float* out = g.c;
    g.ws_stride = batch * g.m * g.n;
    if (splits > 1) {
        float* ws = static_cast<float*>(
            scratch(size_t(splits) * size_t(g.ws_stride) * sizeof(float)));
        if (ws == nullptr) return EHIP_ENOMEM;
        g.c = ws;
    }
    const dim3 grid{unsigned(tiles), unsigned(splits), unsigned(batch)};
    const int va = vec_a ? 1 : 0, vb = vec_b ? 1 : 0;
    if (splits > 1 || !EPI)
        EHIP_LAUNCH("conv_gemm", (conv_gemm_kernel<C, BK, LA, LB, false>), grid, dim3(C::kThreads),
                    0, s, g, cg, va, vb);
    else
        EHIP_LAUNCH("conv_gemm", (conv_gemm_kernel<C, BK, LA, LB, true>), grid, dim3(C::kThreads),
                    0, s, g, cg, va, vb);
    if (splits > 1) {
        GemmArgs gr = g;
        gr.c = out;
        return splitk_finish(g.c, out, gr, batch, splits, s);
    }
    return EHIP_OK;
}

using Small = Cfg<64, 64, 16, 32, 32>;     // 4 waves of 32 x 32
using Large = Cfg<128, 128, 32, 64, 32>;  // 8 waves of 64 x 32

// 128 x 128 tiles for products of at least 128 x 128 that they cover with
// little more padding than 64 x 64 tiles do, when they still make 256 or more
// workgroups (with their K splits); 64 x 64 otherwise. Measured on MI355X
// over ResNet-stage layers: the larger tile is up to 1.6x faster on 128- and
// 256-channel layers, the smaller one up to 1.5x faster on 64-channel layers
// and on short reductions over few tiles.
bool large_tiles(int64_t m, int64_t n, int64_t batch, int64_t k) {
    if (m < 128 || n < 128) return false;
    const auto area = [&](int64_t t) {
        return double(ceil_div(m, t) * t) * double(ceil_div(n, t) * t);
    };
    if (area(128) > 1.15 * area(64)) return false;
    const int64_t blocks = ceil_div(m, 128) * ceil_div(n, 128) * batch;
    return blocks * split_count(blocks, k, 32) >= 256;
}

template <template <class, int, int> class LA, template <class, int, int> class LB, bool EPI>
int run_product(const GemmArgs& g, int64_t batch, const ConvGeo& cg, bool vec_a, bool vec_b,
                hipStream_t s) {
    if (large_tiles(g.m, g.n, batch, g.k))
        return launch_product<Large, 32, LA, LB, EPI>(g, batch, cg, vec_a, vec_b, s);
    return launch_product<Small, 16, LA, LB, EPI>(g, batch, cg, vec_a, vec_b, s);
}

// The stride phases of dx (stride 2..4, N s^2 <= 65535 products); false
// when the layer takes the per-tap gather instead.
bool plan_phases(const ConvGeo& cg, int64_t n, PhaseSet* ps, int* phases, int* max_count) {
    const int s = cg.stride;
    if (s < 2 || s > 4 || n * s * s > 65535) return false;
    *phases = s * s;
    *max_count = 0;
    const auto first = [&](int ph) { return cg.pad > ph ? int(ceil_div(cg.pad - ph, s)) : 0; };
    const auto end = [&](int ph, int size) {
        return size + cg.pad - ph > 0 ? int(ceil_div(size + cg.pad - ph, s)) : 0;
    };
    for (int ph = 0; ph < s; ++ph)
        for (int pw = 0; pw < s; ++pw) {
            Phase& f = ps->p[ph * s + pw];
            f.ph = ph;
            f.pw = pw;
            f.a0 = first(ph);
            f.b0 = first(pw);
            f.hph = std::max(0, end(ph, cg.h) - f.a0);
            f.wph = std::max(0, end(pw, cg.w) - f.b0);
            f.ti = ph < cg.kh ? int(ceil_div(cg.kh - ph, s)) : 0;
            f.tj = pw < cg.kw ? int(ceil_div(cg.kw - pw, s)) : 0;
            f.d_wph = fast_div(std::max(f.wph, 1));
            f.d_tt = fast_div(std::max(f.ti * f.tj, 1));
            f.d_tj = fast_div(std::max(f.tj, 1));
            *max_count = std::max(*max_count, f.hph * f.wph);
        }
    return true;
}

template <class C, int BK>
int launch_dx_phases(GemmArgs g, int64_t n, const ConvGeo& cg, const PhaseSet& ps, int phases,
                     int max_count, hipStream_t s) {
    constexpr int BM = C::kWavesM * (C::kFM * 32), BN = C::kWavesN * (C::kFN * 32);
    g.tiles_m = int(ceil_div(cg.c, BM));
    g.tiles_n = int(ceil_div(max_count, BN));
    const dim3 grid{unsigned(int64_t(g.tiles_m) * g.tiles_n), 1u, unsigned(n * phases)};
    EHIP_LAUNCH("conv_dx_phase", (conv_dx_phase_kernel<C, BK>), grid, dim3(C::kThreads), 0, s, g,
                cg, ps, phases);
    return EHIP_OK;
}

template <class C, int BR, int BK>
using DoutByPixelS1 = DoutByPixel<C, BR, BK, true>;
template <class C, int BR, int BK>
using DoutByPixelStrided = DoutByPixel<C, BR, BK, false>;

// Indices within an image, and the batch's output pixels (the weight
// gradient's reduction index), are 32-bit; the batch is a grid dimension.
bool layer_fits(const ehip_window_t* w, int64_t out_channels) {
    const int64_t lim = 0x7fffffffLL;
    return !(w->channels * w->height * w->width > lim || out_channels * w->out_h * w->out_w > lim ||
             w->channels * w->kernel_h * w->kernel_w > lim ||
             out_channels * w->kernel_h * w->kernel_w > lim ||
             w->batch * w->out_h * w->out_w > lim || w->batch > 65535);
}

int check_layer(const char* name, const ehip_window_t* w, int64_t out_channels) {
    if (int rc = check_window(name, w)) return rc;
    if (out_channels <= 0)
        return fail(EHIP_EINVAL, "%s: out_channels %lld", name, (long long)out_channels);
    if (!layer_fits(w, out_channels)) return fail(EHIP_EINVAL, "%s: layer too large", name);
    return EHIP_OK;
}

}  // namespace
}  // namespace ehip

using namespace ehip;

extern "C" {

int ehip_conv2d_igemm_supported(const ehip_window_t* w, int64_t out_channels) {
    if (w == nullptr || out_channels <= 0 || w->batch < 0 || w->channels <= 0 ||
        w->out_h <= 0 || w->out_w <= 0 || w->kernel_h <= 0 || w->kernel_w <= 0)
        return 0;
    return layer_fits(w, out_channels) ? 1 : 0;
}

int ehip_conv2d_igemm_f32(const float* x, const float* weight, const float* bias, float* out,
                          const ehip_window_t* win, int64_t out_channels, void* stream) {
    EHIP_READY();
    if (int rc = check_layer("conv2d_igemm", win, out_channels)) return rc;
    if (!x || !weight || !out) return fail(EHIP_EINVAL, "conv2d_igemm: null pointer");
    if (win->batch == 0) return EHIP_OK;
    ConvGeo cg = geo_of(*win, out_channels);
    cg.x = x;
    cg.wt = weight;
    GemmArgs g{};
    g.m = cg.co;
    g.n = cg.p;
    g.k = cg.k;
    g.c = out;
    g.ldc = cg.p;
    g.stride_c = int64_t(cg.co) * cg.p;
    g.inner = 1;
    g.alpha = 1.0f;
    g.add = bias;
    g.add_row = 1;
    g.add_period = 1;
    const bool vec_w = cg.k % 4 == 0 && aligned16(weight);
    const hipStream_t s = as_stream(stream);
    if (bias) return run_product<WeightRows, ColsByPixel, true>(g, win->batch, cg, vec_w, false, s);
    return run_product<WeightRows, ColsByPixel, false>(g, win->batch, cg, vec_w, false, s);
}

int ehip_conv2d_igemm_backward_f32(const float* x, const float* weight, const float* grad_out,
                                   float* dx, float* dweight, float* dbias,
                                   const ehip_window_t* win, int64_t out_channels, void* stream) {
    EHIP_READY();
    if (int rc = check_layer("conv2d_igemm_backward", win, out_channels)) return rc;
    if (!grad_out || (dx && !weight) || (dweight && !x))
        return fail(EHIP_EINVAL, "conv2d_igemm_backward: null pointer");
    if (win->batch == 0) return EHIP_OK;
    hipStream_t s = as_stream(stream);
    ConvGeo cg = geo_of(*win, out_channels);
    cg.x = x;
    cg.wt = weight;
    cg.dout = grad_out;
    const int64_t n = win->batch;
    const bool vec_dout = cg.p % 4 == 0 && aligned16(grad_out);
    if (dbias) {
        if (vec_dout)
            EHIP_LAUNCH("conv2d_igemm_bias", conv_bias_grad<true>, dim3(unsigned(cg.co)), dim3(512),
                        0, s, grad_out, dbias, n, int64_t(cg.co), int64_t(cg.p));
        else
            EHIP_LAUNCH("conv2d_igemm_bias", conv_bias_grad<false>, dim3(unsigned(cg.co)),
                        dim3(512), 0, s, grad_out, dbias, n, int64_t(cg.co), int64_t(cg.p));
    }
    if (dweight) {
        GemmArgs g{};
        g.m = cg.co;
        g.n = cg.k;
        g.k = n * cg.p;
        g.c = dweight;
        g.ldc = cg.k;
        g.inner = 1;
        g.alpha = 1.0f;
        g.add_period = 1;
        if (int rc = run_product<DoutByChannel, ColsByTap, false>(g, 1, cg, vec_dout, false, s))
            return rc;
    }
    if (dx) {
        GemmArgs g{};
        g.m = cg.c;
        g.n = cg.hw;
        g.k = int64_t(cg.co) * cg.khw;
        g.c = dx;
        g.ldc = cg.hw;
        g.stride_c = cg.chw;
        g.inner = 1;
        g.alpha = 1.0f;
        g.add_period = 1;
        PhaseSet ps{};
        int phases = 0, max_count = 0;
        int rc;
        // Strided layers: the column gradient as one batched product, dcols[n]
        // (oH oW x C kH kW) = dOut[n]^T W (C_out x C kH kW), then its col2im
        // gather (the reference's own composition, src/conv.cpp:280-338, without
        // the permutes): a dense MFMA product instead of the phase kernels'
        // element gathers (cfg 16x64x56x56 -> 128, stride 2: 93 us for the phase
        // kernel against about 30 for the two launches).
        const size_t dcols_bytes = size_t(n) * size_t(cg.p) * size_t(cg.k) * sizeof(float);
        if (cg.stride > 1 && dcols_bytes <= kStridedColsMax) {
            float* dcols = static_cast<float*>(scratch(dcols_bytes, 1));
            if (dcols == nullptr) return EHIP_ENOMEM;
            ehip_gemm_ex_t d{};
            d.trans_a = 1;
            d.batch = n;
            d.inner = 1;
            d.m = cg.p;
            d.n = cg.k;
            d.k = cg.co;
            d.a = grad_out;
            d.lda = cg.p;
            d.stride_a = int64_t(cg.co) * cg.p;
            d.b = weight;
            d.ldb = cg.k;
            d.c = dcols;
            d.ldc = cg.k;
            d.stride_c = int64_t(cg.p) * cg.k;
            d.alpha = 1.0f;
            d.addend_period = 1;
            if (int rc2 = ehip_gemm_ex_f32(&d, stream)) return rc2;
            return ehip_col2im_f32(dcols, dx, win, stream);
        }
        if (cg.stride == 1)
            rc = run_product<WeightByInput, DoutByPixelS1, false>(g, n, cg, false, false, s);
        else if (!plan_phases(cg, n, &ps, &phases, &max_count))
            rc = run_product<WeightByInput, DoutByPixelStrided, false>(g, n, cg, false, false, s);
        else if (large_tiles(cg.c, max_count, n * phases, 1))
            rc = launch_dx_phases<Large, 32>(g, n, cg, ps, phases, max_count, s);
        else
            rc = launch_dx_phases<Small, 16>(g, n, cg, ps, phases, max_count, s);
        if (rc) return rc;
    }
    return EHIP_OK;
}

}  // extern "C"
