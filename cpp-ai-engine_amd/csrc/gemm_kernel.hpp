// gemm_kernel.hpp -- the fp32 MFMA GEMM kernel templates (tile loaders, the
// main kernel, the split-K reduction), shared by the dispatcher in gemm.hip.
// See gemm.hip for the design.
#ifndef EHIP_GEMM_KERNEL_HPP
#define EHIP_GEMM_KERNEL_HPP

#include "common.hpp"

namespace ehip {
namespace gemm_detail {


typedef float floatx16 __attribute__((ext_vector_type(16)));

struct GemmArgs {
    const float* a;
    const float* b;
    float* c;  // the output, or the split-K workspace
    int64_t m, n, k;
    int64_t lda, ldb, ldc;
    // Product z reads A at a + (z / inner) * stride_a + (z % inner) * stride_a2
    // (likewise B and C): heads inside a (batch, seq, heads * dim) activation.
    int64_t stride_a, stride_b, stride_c;
    int64_t inner;
    int64_t stride_a2, stride_b2, stride_c2;
    // Epilogue: v = acc; v *= alpha (alpha != 1); v += add[z % add_period]
    // [i * ld_add + j] (add != null); v += beta * c (beta != 0); ReLU.
    float alpha;
    const float* add;
    int64_t ld_add, stride_add, add_period;
    int add_row;  // the addend is one value per row: add[i] (a convolution's bias)
    float beta;
    // v += res[i * ld_res + j] (res != null, batch 1): a residual stream added
    // after the product's own epilogue, as the add node after a Linear does.
    const float* res;
    int64_t ld_res;
    int relu;  // then v = max(0, v)
    // colsum[j] = sum over k of op(B)[k][j] (batch 1), made by the first
    // tile-row's workgroups from the B tiles they stage anyway; with split K
    // each split's sums go after its C partials and the reduction adds them.
    float* colsum;
    int64_t ws_stride;  // split-K workspace floats per split
    int tiles_m, tiles_n;
    int splits;        // K is cut into `splits` chunks of k_chunk (a multiple of BK)
    int64_t k_chunk;
    int vec;           // rows 16-byte aligned: checked loads may use float4 inside the edges
    int vec_ab;        // the same per operand: bit 0 A's rows, bit 1 B's (K-sliced checked loads)
    int causal;        // ehip_gemm_ex_t::causal: 0, or the skipping mode 1 to 4
    // The product index of grid z = 0: batches beyond the grid's 65535 z
    // extent run as several launches of consecutive product ranges.
    int64_t batch0;
};

// The element offset of product z's matrix.
__device__ __forceinline__ int64_t batch_offset(int64_t z, int64_t inner, int64_t stride,
                                                int64_t stride2) {
    if (inner == 1) return z * stride;
    const int64_t outer = z / inner;
    return outer * stride + (z - outer * inner) * stride2;
}

// The epilogue's arithmetic on one value: each step rounded on its own, so
// that a fused scale, mask, bias or ReLU equals the separate nodes bit for bit.
__device__ __forceinline__ float finish(const GemmArgs& g, float v, float add, float old,
                                        float res) {
    if (g.alpha != 1.0f) v = v * g.alpha;
    if (g.add != nullptr) v = v + add;
    if (g.beta != 0.0f) v = v + g.beta * old;
    if (g.res != nullptr) v = v + res;
    if (g.relu) v = (0.0f < v) ? v : 0.0f;
    return v;
}

// The stored value of product z's output (row, col); dst is that element.
__device__ __forceinline__ float epilogue(const GemmArgs& g, int64_t z, int64_t row, int64_t col,
                                          float v, const float* dst) {
    const float add = g.add ? g.add[(z % g.add_period) * g.stride_add +
                                    (g.add_row ? row : row * g.ld_add + col)]
                            : 0.0f;
    const float res = g.res ? g.res[row * g.ld_res + col] : 0.0f;
    return finish(g, v, add, g.beta != 0.0f ? *dst : 0.0f, res);
}

// True when the stored value is the accumulator itself.
__host__ __device__ inline bool plain_epilogue(const GemmArgs& g) {
    return g.alpha == 1.0f && g.add == nullptr && g.beta == 0.0f && !g.relu && g.res == nullptr;
}

template <int BM, int BN, int BK, int WM, int WN>
struct Cfg {
    static constexpr int kWavesM = BM / WM, kWavesN = BN / WN;
    static constexpr int kThreads = kWavesM * kWavesN * 64;
    static constexpr int kFM = WM / 32, kFN = WN / 32;
    static constexpr int kLdsA = BM + 4;  // row pitch of the [k][m] A buffer
    static constexpr int kLdsB = BN + 4;
    static constexpr int kA4 = BM * BK / 4;  // float4 loads per tile
    static constexpr int kB4 = BN * BK / 4;
    static constexpr int kALoads = (kA4 + kThreads - 1) / kThreads;
    static constexpr int kBLoads = (kB4 + kThreads - 1) / kThreads;
    static constexpr bool kPrio = BM * BN <= 128 * 128;
    static_assert(BM % WM == 0 && BN % WN == 0 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
    static_assert(BK % 4 == 0, "BK");
};

// Loads a BM x BK tile of op(A) into registers. TA: A is stored K x M.
// CHECK: zero-fill outside the matrix and use scalar loads.
template <class C, int BM, int BK, bool TRANS, bool CHECK>
__device__ __forceinline__ void load_tile(const float* __restrict__ p, int64_t ld, int64_t rows,
                                          int64_t kdim, int64_t r0, int64_t k0, float4* reg,
                                          int loads, int total, bool vec) {
#pragma unroll
    for (int i = 0; i < loads; ++i) {
        const int q = threadIdx.x + i * C::kThreads;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (q < total) {
            int64_t r, kk;
            if (!TRANS) {  // stored rows x K, 4 consecutive k
                r = r0 + q / (BK / 4);
                kk = k0 + 4 * (q % (BK / 4));
                const float* src = p + r * ld + kk;
                if (!CHECK || (vec && r < rows && kk + 3 < kdim)) {
                    v = *reinterpret_cast<const float4*>(src);
                } else if (r < rows) {
                    v.x = kk < kdim ? src[0] : 0.f;
                    v.y = kk + 1 < kdim ? src[1] : 0.f;
                    v.z = kk + 2 < kdim ? src[2] : 0.f;
                    v.w = kk + 3 < kdim ? src[3] : 0.f;
                }
            } else {  // stored K x rows, 4 consecutive rows
                kk = k0 + q / (BM / 4);
                r = r0 + 4 * (q % (BM / 4));
                const float* src = p + kk * ld + r;
                if (!CHECK || (vec && kk < kdim && r + 3 < rows)) {
                    v = *reinterpret_cast<const float4*>(src);
                } else if (kk < kdim) {
                    v.x = r < rows ? src[0] : 0.f;
                    v.y = r + 1 < rows ? src[1] : 0.f;
                    v.z = r + 2 < rows ? src[2] : 0.f;
                    v.w = r + 3 < rows ? src[3] : 0.f;
                }
            }
        }
        reg[i] = v;
    }
}

// Stores the registers of load_tile into an LDS buffer laid out [k][row].
template <class C, int BM, int BK, int LDS, bool TRANS>
__device__ __forceinline__ void store_tile(float* __restrict__ s, const float4* reg, int loads,
                                           int total) {
#pragma unroll
    for (int i = 0; i < loads; ++i) {
        const int q = threadIdx.x + i * C::kThreads;
        if (q < total) {
            if (!TRANS) {
                const int r = q / (BK / 4), kk = 4 * (q % (BK / 4));
                s[(kk + 0) * LDS + r] = reg[i].x;
                s[(kk + 1) * LDS + r] = reg[i].y;
                s[(kk + 2) * LDS + r] = reg[i].z;
                s[(kk + 3) * LDS + r] = reg[i].w;
            } else {
                const int kk = q / (BM / 4), r = 4 * (q % (BM / 4));
                *reinterpret_cast<float4*>(s + kk * LDS + r) = reg[i];
            }
        }
    }
}

// The MFMAs of one staged K step: the fragments of k-pair kk + 2 are read
// from LDS while the MFMAs of kk run (two register sets). Tiles of at most
// 128 x 128 run four or more waves per SIMD: there the wave issuing its MFMAs
// also takes priority over the others' loads and LDS traffic, which keeps the
// matrix pipe fed (measured on MI355X: 5-9% on 8192 x 1024 x K; neither
// change helps the 256 x 256 tile, nor priority alone).
template <class C, int BK>
__device__ __forceinline__ void mfma_stage(floatx16 (&acc)[C::kFM][C::kFN], const float* lds_a,
                                           const float* lds_b, int wm0, int wn0, int lane) {
    const float* sa = lds_a + (lane / 32) * C::kLdsA + wm0 + lane % 32;
    const float* sb = lds_b + (lane / 32) * C::kLdsB + wn0 + lane % 32;
    float fa[2][C::kFM], fb[2][C::kFN];
#pragma unroll
    for (int i = 0; i < C::kFM; ++i) fa[0][i] = sa[32 * i];
#pragma unroll
    for (int j = 0; j < C::kFN; ++j) fb[0][j] = sb[32 * j];
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
        const int f = (kk / 2) & 1;
        if (kk + 2 < BK) {
#pragma unroll
            for (int i = 0; i < C::kFM; ++i) fa[f ^ 1][i] = sa[(kk + 2) * C::kLdsA + 32 * i];
#pragma unroll
            for (int j = 0; j < C::kFN; ++j) fb[f ^ 1][j] = sb[(kk + 2) * C::kLdsB + 32 * j];
        }
        if (C::kPrio) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < C::kFM; ++i)
#pragma unroll
            for (int j = 0; j < C::kFN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[f][i], fb[f][j], acc[i][j], 0,
                                                                 0, 0);
        if (C::kPrio) __builtin_amdgcn_s_setprio(0);
    }
}

// Stores the accumulators of the tile at (m0, n0) into Cp (row pitch ldc):
// as they are, or through the fused epilogue, one 32 x 32 block at a time --
// the block's addend and old C values are loaded together first (the compiler
// cannot move a load above an earlier store to C, which may alias them), then
// stored. The addend is add[i * ld_add + j], or with add_row add[i].
template <class C, bool CHECK, bool EPI>
__device__ __forceinline__ void store_acc(const GemmArgs& g, floatx16 (&acc)[C::kFM][C::kFN],
                                          float* Cp, int64_t ldc, const float* addp, int64_t m0,
                                          int64_t n0, int wm0, int wn0, int lane) {
    if (!EPI) {
#pragma unroll
        for (int i = 0; i < C::kFM; ++i)
#pragma unroll
            for (int j = 0; j < C::kFN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t row = m0 + wm0 + 32 * i + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
                    const int64_t col = n0 + wn0 + 32 * j + lane % 32;
                    if (CHECK && (row >= g.m || col >= g.n)) continue;
                    Cp[row * ldc + col] = acc[i][j][r];
                }
        return;
    }
    const int64_t ld_add = g.add_row ? 1 : g.ld_add;
#pragma unroll
    for (int i = 0; i < C::kFM; ++i)
#pragma unroll
        for (int j = 0; j < C::kFN; ++j) {
            const int64_t row0 = m0 + wm0 + 32 * i + 4 * (lane / 32);
            const int64_t col = n0 + wn0 + 32 * j + lane % 32;
            float* cb = Cp + row0 * ldc + col;
            const float* ab = addp ? addp + row0 * ld_add + (g.add_row ? 0 : col) : nullptr;
            const float* rb = g.res ? g.res + row0 * g.ld_res + col : nullptr;
            float e_add[16], e_old[16], e_res[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int dr = 8 * (r / 4) + (r % 4);
                const bool in = !CHECK || (row0 + dr < g.m && col < g.n);
                e_add[r] = (ab && in) ? ab[dr * ld_add] : 0.0f;
                e_old[r] = (g.beta != 0.0f && in) ? cb[dr * ldc] : 0.0f;
                e_res[r] = (rb && in) ? rb[dr * g.ld_res] : 0.0f;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int dr = 8 * (r / 4) + (r % 4);
                if (CHECK && (row0 + dr >= g.m || col >= g.n)) continue;
                cb[dr * ldc] = finish(g, acc[i][j][r], e_add[r], e_old[r], e_res[r]);
            }
        }
}

// Products with both operands stored k-contiguous (A untransposed, B
// transposed: C = A B^T) keep each operand tile in LDS as [row][k] (row pitch
// BK + 4), written with one float4 per loaded float4 and read back as one
// float4 per lane per 8 k. MFMA order inside a block of 8 k at kb: half h of
// the lanes holds k = kb + 4h + j and instruction j = 0..3 multiplies them.
// The other layouts ([k][row], above) transpose k-contiguous operands with
// four scalar LDS writes that conflict on the banks; measured on MI355X this
// layout runs the NT products of the cfg5 Transformer 8-12 % faster, while
// for operands stored row-contiguous it is no faster than [k][row], which
// therefore stays for them.
template <int BK>
struct KcTile {
    static constexpr int kPitch = BK + 4;
};

// Stores load_tile<..., TRANS = false> registers (row q / (BK / 4), k 4 (q %
// (BK / 4))) into a [row][k] tile.
template <class C, int BR, int BK>
__device__ __forceinline__ void store_tile_kc(float* __restrict__ s, const float4* reg, int loads,
                                              int total) {
#pragma unroll
    for (int i = 0; i < loads; ++i) {
        const int q = threadIdx.x + i * C::kThreads;
        if (q < total) {
            const int r = q / (BK / 4), kk = 4 * (q % (BK / 4));
            *reinterpret_cast<float4*>(s + r * KcTile<BK>::kPitch + kk) = reg[i];
        }
    }
}

template <class C, int BK>
__device__ __forceinline__ void mfma_stage_kc(floatx16 (&acc)[C::kFM][C::kFN], const float* lds_a,
                                              const float* lds_b, int wm0, int wn0, int lane) {
    constexpr int P = KcTile<BK>::kPitch;
    static_assert(BK % 8 == 0, "BK");
    const float* sa = lds_a + (wm0 + lane % 32) * P + 4 * (lane / 32);
    const float* sb = lds_b + (wn0 + lane % 32) * P + 4 * (lane / 32);
    float4 fa[2][C::kFM], fb[2][C::kFN];
#pragma unroll
    for (int i = 0; i < C::kFM; ++i) fa[0][i] = *reinterpret_cast<const float4*>(sa + 32 * i * P);
#pragma unroll
    for (int j = 0; j < C::kFN; ++j) fb[0][j] = *reinterpret_cast<const float4*>(sb + 32 * j * P);
#pragma unroll
    for (int kb = 0; kb < BK; kb += 8) {
        const int f = (kb / 8) & 1;
        if (kb + 8 < BK) {
#pragma unroll
            for (int i = 0; i < C::kFM; ++i)
                fa[f ^ 1][i] = *reinterpret_cast<const float4*>(sa + 32 * i * P + kb + 8);
#pragma unroll
            for (int j = 0; j < C::kFN; ++j)
                fb[f ^ 1][j] = *reinterpret_cast<const float4*>(sb + 32 * j * P + kb + 8);
        }
        if (C::kPrio) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int i = 0; i < C::kFM; ++i)
#pragma unroll
                for (int j = 0; j < C::kFN; ++j) {
                    const float a = q == 0 ? fa[f][i].x : q == 1 ? fa[f][i].y : q == 2 ? fa[f][i].z : fa[f][i].w;
                    const float b = q == 0 ? fb[f][j].x : q == 1 ? fb[f][j].y : q == 2 ? fb[f][j].z : fb[f][j].w;
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[i][j], 0, 0, 0);
                }
        if (C::kPrio) __builtin_amdgcn_s_setprio(0);
    }
}

// EPI: the fused epilogue (alpha, addend, beta, ReLU); without it the
// accumulators are stored as they are (also the split-K partials).
template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, bool CHECK, bool EPI>
__global__ __launch_bounds__((Cfg<BM, BN, BK, WM, WN>::kThreads)) void gemm_kernel(GemmArgs g) {
    using C = Cfg<BM, BN, BK, WM, WN>;
    constexpr bool KC = !TA && TB;  // both operands k-contiguous: [row][k] tiles
    constexpr int kFloatsA = KC ? BM * KcTile<BK>::kPitch : BK * C::kLdsA;
    constexpr int kFloatsB = KC ? BN * KcTile<BK>::kPitch : BK * C::kLdsB;
    __shared__ float lds_a[2][kFloatsA];
    __shared__ float lds_b[2][kFloatsB];

    // Tile coordinates: XCD-contiguous renumbering, then GROUP_M-row groups.
    const int tiles = g.tiles_m * g.tiles_n;
    int tm, tn;
    int64_t batch = g.batch0 + blockIdx.z;
    if (g.causal != 0 && gridDim.y == 1) {
        // Causal skipping makes a tile's work depend on its row band. Workgroups
        // reach the XCDs (and their CUs) in turn in launch order, so the order
        // runs over the products first: every XCD and CU then gets tiles of
        // every band instead of, with few tiles per product, one band only.
        const int64_t lin = int64_t(blockIdx.z) * gridDim.x + blockIdx.x;
        batch = g.batch0 + lin % gridDim.z;
        const int t = int(lin / gridDim.z);
        tm = t / g.tiles_n;
        tn = t % g.tiles_n;
    } else {
        int bid = blockIdx.x;
        if (tiles % 8 == 0) bid = (bid % 8) * (tiles / 8) + bid / 8;
        constexpr int kGroupM = 8;
        const int group = bid / (kGroupM * g.tiles_n);
        const int first_m = group * kGroupM;
        const int gsz = min(g.tiles_m - first_m, kGroupM);
        const int in_group = bid % (kGroupM * g.tiles_n);
        tm = first_m + in_group % gsz;
        tn = in_group / gsz;
    }

    const int split = blockIdx.y;
    const float* A = g.a + batch_offset(batch, g.inner, g.stride_a, g.stride_a2);
    const float* B = g.b + batch_offset(batch, g.inner, g.stride_b, g.stride_b2);
    const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;
    int64_t k_begin = int64_t(split) * g.k_chunk;
    int64_t k_end = k_begin + g.k_chunk;
    if (k_end > g.k) k_end = g.k;
    // Causal skipping (modes of ehip_gemm_ex_t::causal); m0 and m0 + BM are
    // multiples of BK, so the K steps stay aligned.
    if (g.causal == 4 && n0 >= m0 + BM) return;  // wholly above the diagonal: not stored
    if (g.causal == 1 && n0 >= m0 + BM) {
        k_end = k_begin;  // wholly above the diagonal: the epilogue of acc = 0
    } else if (g.causal == 2) {
        if (k_end > m0 + BM) k_end = k_begin > m0 + BM ? k_begin : m0 + BM;
    } else if (g.causal == 3) {
        if (k_begin < m0) k_begin = k_end < m0 ? k_end : m0;
    }

    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int wm0 = (wave / C::kWavesN) * WM, wn0 = (wave % C::kWavesN) * WN;

    floatx16 acc[C::kFM][C::kFN];
#pragma unroll
    for (int i = 0; i < C::kFM; ++i)
#pragma unroll
        for (int j = 0; j < C::kFN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    float4 ra[C::kALoads], rb[C::kBLoads];
    // The step count is the same for the whole workgroup; read as a scalar so
    // that the per-step conditions are scalar branches, not exec masks.
    const int64_t steps = __builtin_amdgcn_readfirstlane(int((k_end - k_begin + BK - 1) / BK));
    const bool colsum_tile = g.colsum != nullptr && tm == 0;
    float csum = 0.0f;
    if (steps > 0) {
        load_tile<C, BM, BK, TA, CHECK>(A, g.lda, g.m, k_end, m0, k_begin, ra, C::kALoads, C::kA4, g.vec);
        load_tile<C, BN, BK, !TB, CHECK>(B, g.ldb, g.n, k_end, n0, k_begin, rb, C::kBLoads, C::kB4, g.vec);
        if constexpr (KC) {
            store_tile_kc<C, BM, BK>(lds_a[0], ra, C::kALoads, C::kA4);
            store_tile_kc<C, BN, BK>(lds_b[0], rb, C::kBLoads, C::kB4);
        } else {
            store_tile<C, BM, BK, C::kLdsA, TA>(lds_a[0], ra, C::kALoads, C::kA4);
            store_tile<C, BN, BK, C::kLdsB, !TB>(lds_b[0], rb, C::kBLoads, C::kB4);
        }
        __syncthreads();
    }
    for (int64_t s = 0; s < steps; ++s) {
        const int cur = int(s & 1);
        const bool more = s + 1 < steps;
        if (more) {
            const int64_t kn = k_begin + (s + 1) * BK;
            load_tile<C, BM, BK, TA, CHECK>(A, g.lda, g.m, k_end, m0, kn, ra, C::kALoads, C::kA4, g.vec);
            load_tile<C, BN, BK, !TB, CHECK>(B, g.ldb, g.n, k_end, n0, kn, rb, C::kBLoads,
                                             C::kB4, g.vec);
        }
        if constexpr (KC)
            mfma_stage_kc<C, BK>(acc, lds_a[cur], lds_b[cur], wm0, wn0, lane);
        else
            mfma_stage<C, BK>(acc, lds_a[cur], lds_b[cur], wm0, wn0, lane);
        // Column sums exist only for a K x N B (the entry point refuses them
        // otherwise), so the k-contiguous tiles carry no code for them.
        if constexpr (!KC) {
            if (colsum_tile && threadIdx.x < BN) {
                // This K step's B rows, in k order, for column n0 + threadIdx.x.
                const float* col = lds_b[cur] + threadIdx.x;
                float part = 0.0f;
#pragma unroll
                for (int kk = 0; kk < BK; ++kk) part += col[kk * C::kLdsB];
                csum = csum + part;
            }
        }
        if (more) {
            if constexpr (KC) {
                store_tile_kc<C, BM, BK>(lds_a[cur ^ 1], ra, C::kALoads, C::kA4);
                store_tile_kc<C, BN, BK>(lds_b[cur ^ 1], rb, C::kBLoads, C::kB4);
            } else {
                store_tile<C, BM, BK, C::kLdsA, TA>(lds_a[cur ^ 1], ra, C::kALoads, C::kA4);
                store_tile<C, BN, BK, C::kLdsB, !TB>(lds_b[cur ^ 1], rb, C::kBLoads, C::kB4);
            }
        }
        __syncthreads();
    }

    if (!KC && colsum_tile && threadIdx.x < BN && n0 + threadIdx.x < g.n) {
        if (g.splits > 1)
            g.c[int64_t(split) * g.ws_stride + g.m * g.n + n0 + threadIdx.x] = csum;
        else
            g.colsum[n0 + threadIdx.x] = csum;
    }

    // Epilogue. With splits > 1, c is the workspace [split][batch][m][n]
    // (ws_stride floats per split) and the epilogue is applied by the
    // reduction kernel.
    float* Cp;
    int64_t ldc;
    if (g.splits > 1) {
        Cp = g.c + int64_t(split) * g.ws_stride + batch * g.m * g.n;
        ldc = g.n;
    } else {
        Cp = g.c + batch_offset(batch, g.inner, g.stride_c, g.stride_c2);
        ldc = g.ldc;
    }
    const float* addp = g.add ? g.add + (int64_t(batch) % g.add_period) * g.stride_add : nullptr;
    store_acc<C, CHECK, EPI>(g, acc, Cp, ldc, addp, m0, n0, wm0, wn0, lane);
}

// ------------------------------------------------------------ NT pipeline
//
// C = A B^T with both operands stored k-contiguous (the input gradients dX =
// dY W^T of Linear layers), whole 128 x 128 tiles, batch 1: four waves of 64 x
// 64 (2 x 2 blocks of 32 x 32) and the loads two K steps ahead of the MFMAs
// -- step s + 1 waits in registers while step s runs, is written into the
// free LDS stage a quarter of the way into step s, and step s + 2's loads are
// issued right after -- instead of the staged kernel's one step ahead with
// eight waves. The [row][k] tiles and the MFMA sequence are the staged
// kernel's (blocks of 8 k ascending, k and k + 4 paired; mfma_stage_kc), and
// the K split is the one launch_cfg gives a 128 x 128 tile, so each output is
// the same chain with the same bits; measured on MI355X 5-7 % faster on the
// cfg5 input-gradient shapes (8192 x 1024 x 1024: 147 against 155 us;
// 8192 x 1024 x 4096: 505 against 543).
constexpr int kNtBK = 32;
typedef float nt4 __attribute__((ext_vector_type(4)));
using NtCfg = Cfg<128, 128, kNtBK, 64, 64>;  // the 2 x 2 wave grid, for store_acc

struct NtTile {
    static constexpr int kPitch = KcTile<kNtBK>::kPitch;
    static constexpr int kFloats = 128 * kPitch;
    static constexpr int kLoads = 128 * kNtBK / 4 / 256;  // float4 per thread per operand
    // float4 q of the tile (row q / 8, k 4 (q % 8)) of rows r0.. at k0.
    __device__ __forceinline__ static void load(const float* p, int64_t ld, int64_t r0,
                                                int64_t k0, nt4 (&r)[kLoads]) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int q = threadIdx.x + 256 * i;
            r[i] = *reinterpret_cast<const nt4*>(p + (r0 + q / (kNtBK / 4)) * ld + k0 +
                                                 4 * (q % (kNtBK / 4)));
        }
    }
    __device__ __forceinline__ static void store(float* s, const nt4 (&r)[kLoads]) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int q = threadIdx.x + 256 * i;
            *reinterpret_cast<nt4*>(s + (q / (kNtBK / 4)) * kPitch + 4 * (q % (kNtBK / 4))) = r[i];
        }
    }
};

template <bool EPI>
__global__ __launch_bounds__(256) void gemm_nt_pipe(GemmArgs g) {
    constexpr int kStage = 2 * NtTile::kFloats;
    __shared__ __align__(16) float lds[2 * kStage];
    const int tiles = g.tiles_m * g.tiles_n;
    int bid = blockIdx.x;
    if (tiles % 8 == 0) bid = (bid % 8) * (tiles / 8) + bid / 8;
    constexpr int kGroupM = 8;
    const int group = bid / (kGroupM * g.tiles_n);
    const int first_m = group * kGroupM;
    const int gsz = min(g.tiles_m - first_m, kGroupM);
    const int in_group = bid % (kGroupM * g.tiles_n);
    const int tm = first_m + in_group % gsz, tn = in_group / gsz;
    const int64_t m0 = int64_t(tm) * 128, n0 = int64_t(tn) * 128;
    const int split = blockIdx.y;
    const int64_t k_begin = int64_t(split) * g.k_chunk;
    const int64_t k_end = min(k_begin + g.k_chunk, g.k);
    const int steps = __builtin_amdgcn_readfirstlane(int((k_end - k_begin) / kNtBK));
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int wm0 = (wave / 2) * 64, wn0 = (wave % 2) * 64;
    constexpr int P = NtTile::kPitch;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    nt4 ra[NtTile::kLoads], rb[NtTile::kLoads];
    if (steps > 0) {
        NtTile::load(g.a, g.lda, m0, k_begin, ra);
        NtTile::load(g.b, g.ldb, n0, k_begin, rb);
        NtTile::store(lds, ra);
        NtTile::store(lds + NtTile::kFloats, rb);
        if (steps > 1) {
            NtTile::load(g.a, g.lda, m0, k_begin + kNtBK, ra);
            NtTile::load(g.b, g.ldb, n0, k_begin + kNtBK, rb);
        }
        __syncthreads();
    }
    for (int s = 0; s < steps; ++s) {
        const float* sa = lds + (s & 1) * kStage;
        const float* sb = sa + NtTile::kFloats;
        const float* pa = sa + (wm0 + lane % 32) * P + 4 * (lane / 32);
        const float* pb = sb + (wn0 + lane % 32) * P + 4 * (lane / 32);
        nt4 fa[2][2], fb[2][2];  // [register set][block]
#pragma unroll
        for (int i = 0; i < 2; ++i) fa[0][i] = *reinterpret_cast<const nt4*>(pa + 32 * i * P);
#pragma unroll
        for (int j = 0; j < 2; ++j) fb[0][j] = *reinterpret_cast<const nt4*>(pb + 32 * j * P);
#pragma unroll
        for (int kb = 0; kb < kNtBK; kb += 8) {
            const int f = (kb / 8) & 1;
            if (kb + 8 < kNtBK) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    fa[f ^ 1][i] = *reinterpret_cast<const nt4*>(pa + 32 * i * P + kb + 8);
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    fb[f ^ 1][j] = *reinterpret_cast<const nt4*>(pb + 32 * j * P + kb + 8);
            }
            if (kb == 8 && s + 1 < steps) {
                // The other stage was last read before the previous barrier.
                float* st = lds + ((s + 1) & 1) * kStage;
                NtTile::store(st, ra);
                NtTile::store(st + NtTile::kFloats, rb);
                if (s + 2 < steps) {
                    const int64_t kn = k_begin + int64_t(s + 2) * kNtBK;
                    NtTile::load(g.a, g.lda, m0, kn, ra);
                    NtTile::load(g.b, g.ldb, n0, kn, rb);
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[f][i][q], fb[f][j][q],
                                                                         acc[i][j], 0, 0, 0);
                    }
        }
        __syncthreads();
    }
    float* Cp = g.splits > 1 ? g.c + int64_t(split) * g.ws_stride : g.c;
    const int64_t ldc = g.splits > 1 ? g.n : g.ldc;
    store_acc<NtCfg, false, EPI>(g, acc, Cp, ldc, g.splits > 1 ? nullptr : g.add, m0, n0, wm0,
                                 wn0, lane);
}

// ------------------------------------------------------------ K-sliced tiles
//
// Products whose output is too small to give every CU a 64 x 64 tile (512^3
// is 64 such tiles; the old plan split K four ways into a workspace and paid a
// second launch to add the splits): a workgroup computes one 32 x 32 tile of
// C, and its W waves each take one contiguous slice of K (k_chunk long, a
// multiple of 8); the waves' accumulators are then added in wave order in LDS,
// in the same launch. With W = 8 a 512^3 product is 256 workgroups of 8
// waves, two per SIMD.
//
// MFMA operand order: for one block of 8 k values at kb, lane l (row or
// column r = l % 32, half h = l / 32) holds the four values k = kb + 4h + j,
// j = 0..3, and instruction j of the block multiplies them, so that across the
// two lane halves the four instructions cover the 8 k values once.
// Tiles with edges read these operands straight from global memory (L2): an
// operand stored with k contiguous (A untransposed, B transposed) is one
// float4 per lane; an operand stored with rows or columns contiguous (A
// transposed, B untransposed) is four dword loads, each 32 lanes reading 128
// contiguous bytes. Blocks are processed four at a time (32 k), and the next
// four are loaded before the current ones are multiplied.
// The pointer is deliberately not __restrict__: a restrict-qualified read-only
// pointer makes the loads invariant, and the compiler then re-issues them at
// their uses instead of keeping the prefetched registers.
template <bool TRANS_K_CONTIG, bool CHECK>
__device__ __forceinline__ float4 load_kblock(const float* p, int64_t ld,
                                              int64_t rows, int64_t kdim, int64_t r, int64_t kb,
                                              bool vec) {
    // TRANS_K_CONTIG: element (r, k) at p[r * ld + k]; otherwise at p[k * ld + r].
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (TRANS_K_CONTIG) {
        const float* src = p + r * ld + kb;
        if (!CHECK || (vec && r < rows && kb + 3 < kdim)) {
            v = *reinterpret_cast<const float4*>(src);
        } else if (r < rows) {
            v.x = kb < kdim ? src[0] : 0.f;
            v.y = kb + 1 < kdim ? src[1] : 0.f;
            v.z = kb + 2 < kdim ? src[2] : 0.f;
            v.w = kb + 3 < kdim ? src[3] : 0.f;
        }
    } else {
        const float* src = p + kb * ld + r;
        if (!CHECK || r < rows) {
            v.x = (!CHECK || kb < kdim) ? src[0] : 0.f;
            v.y = (!CHECK || kb + 1 < kdim) ? src[ld] : 0.f;
            v.z = (!CHECK || kb + 2 < kdim) ? src[2 * ld] : 0.f;
            v.w = (!CHECK || kb + 3 < kdim) ? src[3 * ld] : 0.f;
        }
    }
    return v;
}

// Whole tiles (no edge checks) take a staged path instead: each wave loads
// its own slice, one stage of 16 k at a time, with float4 loads in storage
// order (an operand stored k-contiguous: 16 rows x 64 bytes per instruction;
// stored row- or column-contiguous: 4 k rows x 128 bytes), writes the stage
// to a region of LDS that only it uses, and reads the MFMA operands back in
// the lane order above, so no lane ever touches more lines than the stage
// holds. Loads of the next stage are issued before the current stage's MFMAs.
// The MFMA instructions, their operands and their order are the direct path's,
// so the bits are too (measured at 512^3 in all three transpose modes; 7.4 ->
// 5.1 us per product).
typedef float kvec4 __attribute__((ext_vector_type(4)));
constexpr int kStageK = 16;  // k per stage on the staged path

template <bool KC>  // KC: element (r, k) at p[r * ld + k]; else at p[k * ld + r]
struct KStage {
    // LDS layouts: KC as [32 r][16 k + 4] (row pitch 20: conflict-free 16-byte
    // reads of one k quad by 32 rows), otherwise [16 k][32 r + 8] (pitch 40:
    // the two lane halves' k rows fall on disjoint banks).
    static constexpr int kPitch = KC ? kStageK + 4 : 40;
    static constexpr int kFloats = KC ? 32 * kPitch : kStageK * kPitch;  // 640 either way
    static constexpr int kLoads = 32 * kStageK / 4 / 64;                 // float4s per lane: 2
    static __device__ __forceinline__ void load(kvec4 (&v)[kLoads], const float* p, int64_t ld,
                                                int64_t r0, int64_t kb, int lane) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int f = lane + 64 * i;
            if (KC)
                v[i] = *reinterpret_cast<const kvec4*>(p + (r0 + f / 4) * ld + kb + 4 * (f % 4));
            else
                v[i] = *reinterpret_cast<const kvec4*>(p + (kb + f / 8) * ld + r0 + 4 * (f % 8));
        }
    }
    static __device__ __forceinline__ void store(const kvec4 (&v)[kLoads], float* s, int lane) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int f = lane + 64 * i;
            if (KC)
                *reinterpret_cast<kvec4*>(s + (f / 4) * kPitch + 4 * (f % 4)) = v[i];
            else
                *reinterpret_cast<kvec4*>(s + (f / 8) * kPitch + 4 * (f % 8)) = v[i];
        }
    }
    // Lane (r, h)'s four values k = 8u + 4h + j, j = 0..3, of block u of the stage.
    static __device__ __forceinline__ float4 operand(const float* s, int u, int r, int h) {
        if (KC) {
            const kvec4 v = *reinterpret_cast<const kvec4*>(s + r * kPitch + 8 * u + 4 * h);
            return make_float4(v.x, v.y, v.z, v.w);
        }
        const float* q = s + (8 * u + 4 * h) * kPitch + r;
        return make_float4(q[0], q[kPitch], q[2 * kPitch], q[3 * kPitch]);
    }
};

// LDS floats per wave on the staged path (A's and B's stage), and per
// workgroup of W waves: the larger of the stages and the wave reduction
// (which reuses the same memory after a barrier).
constexpr int kStageWaveFloats = 2 * 640;
template <int W>
struct KsliceLds {
    static constexpr int kStage = W * kStageWaveFloats;
    static constexpr int kRed = (W > 1 ? W : 1) * 16 * 64;
    static constexpr int kFloats = kStage > kRed ? kStage : kRed;
};

// One 32 x 32 tile of product `batch` of g: tile index `bid` before the XCD
// renumbering, `red` the waves' LDS exchange. The first `wn` of the W waves
// hold K slices (g.k_chunk long); any others hold none, contribute +0.0 and so
// change no sum (a sum that starts at +0.0 is never -0.0).
template <int W, bool TA, bool TB, bool CHECK, bool EPI, int KU>
__device__ __forceinline__ void kslice_tile(const GemmArgs& g, int bid, int64_t batch,
                                            float* lds, int wn) {
    constexpr int kU = KU;  // blocks of 8 k per pipeline stage

    // Tile coordinates: XCD-contiguous renumbering, then groups of four tile
    // rows, so that an XCD's 32 consecutive tiles share 4 A and 8 B panels.
    const int tiles = g.tiles_m * g.tiles_n;
    if (tiles % 8 == 0) bid = (bid % 8) * (tiles / 8) + bid / 8;
    constexpr int kGroupM = 4;
    const int group = bid / (kGroupM * g.tiles_n);
    const int first_m = group * kGroupM;
    const int gsz = min(g.tiles_m - first_m, kGroupM);
    const int in_group = bid % (kGroupM * g.tiles_n);
    const int64_t m0 = int64_t(first_m + in_group % gsz) * 32;
    const int64_t n0 = int64_t(in_group / gsz) * 32;

    const float* A = g.a + batch_offset(batch, g.inner, g.stride_a, g.stride_a2);
    const float* B = g.b + batch_offset(batch, g.inner, g.stride_b, g.stride_b2);
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int r = lane % 32, h = lane / 32;
    // Wave w's slice of K. Unchecked kernels need K and k_chunk to be multiples
    // of 8 KU (whole pipeline stages); checked ones zero-fill past the slice.
    const int64_t k_begin = wave < wn ? int64_t(wave) * g.k_chunk : g.k;
    const int64_t k_end = k_begin + g.k_chunk < g.k ? k_begin + g.k_chunk : g.k;

    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;

    const auto mfma_block = [&](const float4& fa, const float4& fb) {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa.x, fb.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa.y, fb.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa.z, fb.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa.w, fb.w, acc, 0, 0, 0);
    };
    if constexpr (!CHECK) {
        // Staged path. A is k-contiguous unless TA, B unless !TB.
        using SA = KStage<!TA>;
        using SB = KStage<TB>;
        constexpr int kL = SA::kLoads;
        float* sa = lds + wave * kStageWaveFloats;
        float* sb = sa + SA::kFloats;
        const int n_st = int((k_end - k_begin) / kStageK);
        // Program order of one wave's LDS accesses is all the ordering the
        // region needs (no other wave touches it); the wave barrier keeps the
        // compiler from moving them across the stage boundaries.
        const auto wave_sync = []() {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        };
        const auto to_operands = [&](const kvec4 (&xa)[kL], const kvec4 (&xb)[kL],
                                     float4 (&fa)[2], float4 (&fb)[2]) {
            SA::store(xa, sa, lane);
            SB::store(xb, sb, lane);
            wave_sync();
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                fa[u] = SA::operand(sa, u, r, h);
                fb[u] = SB::operand(sb, u, r, h);
            }
        };
        if (n_st > 0) {
            kvec4 ga[kL], gb[kL];
            SA::load(ga, A, g.lda, m0, k_begin, lane);
            SB::load(gb, B, g.ldb, n0, k_begin, lane);
            for (int st = 0; st + 1 < n_st; ++st) {
                float4 fa[2], fb[2];
                to_operands(ga, gb, fa, fb);
                const int64_t kb = k_begin + int64_t(st + 1) * kStageK;
                SA::load(ga, A, g.lda, m0, kb, lane);
                SB::load(gb, B, g.ldb, n0, kb, lane);
                __builtin_amdgcn_sched_barrier(0);
                mfma_block(fa[0], fb[0]);
                mfma_block(fa[1], fb[1]);
                wave_sync();
            }
            float4 fa[2], fb[2];
            to_operands(ga, gb, fa, fb);
            mfma_block(fa[0], fb[0]);
            mfma_block(fa[1], fb[1]);
        }
        // The reduction below reuses the stage regions of every wave.
        __syncthreads();
    } else {
        // Operand A: (m0 + r, k); stored M x K (k contiguous) unless TA.
        // Operand B: (k, n0 + r); stored K x N (n contiguous) unless TB.
        const auto load_stage = [&](int64_t kb, float4 (&fa)[kU], float4 (&fb)[kU]) {
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int64_t k = kb + 8 * u + 4 * h;
                fa[u] = load_kblock<!TA, CHECK>(A, g.lda, g.m, k_end, m0 + r, k,
                                                (g.vec_ab & 1) != 0);
                fb[u] = load_kblock<TB, CHECK>(B, g.ldb, g.n, k_end, n0 + r, k,
                                               (g.vec_ab & 2) != 0);
            }
        };
        // Two register buffers alternate: a stage's loads are issued before the
        // previous stage's MFMAs (a scheduling barrier keeps them there). The last
        // stage re-reads its own addresses (L1 hits) instead of branching around
        // the prefetch: on a guarded prefetch the compiler's wait counts, merged
        // over both paths, wait for every load before the MFMAs.
        const auto mfma_stage = [&](const float4 (&fa)[kU], const float4 (&fb)[kU]) {
#pragma unroll
            for (int u = 0; u < kU; ++u) mfma_block(fa[u], fb[u]);
        };
        constexpr int64_t kStage = 8 * kU;
        float4 a0[kU], b0[kU], a1[kU], b1[kU];
        int64_t kb = k_begin;
        if (kb < k_end) load_stage(kb, a0, b0);
        while (kb < k_end) {
            load_stage(kb + kStage < k_end ? kb + kStage : kb, a1, b1);
            __builtin_amdgcn_sched_barrier(0);
            mfma_stage(a0, b0);
            kb += kStage;
            if (kb >= k_end) break;
            load_stage(kb + kStage < k_end ? kb + kStage : kb, a0, b0);
            __builtin_amdgcn_sched_barrier(0);
            mfma_stage(a1, b1);
            kb += kStage;
        }

    }

    // The waves' sums, added in wave order; wave w then finishes registers
    // [w * 16 / W, (w + 1) * 16 / W) of every lane.
    constexpr int kPer = 16 / W;
    float out[kPer];
    if (W > 1) {
        float (*red)[16][64] = reinterpret_cast<float (*)[16][64]>(lds);
#pragma unroll
        for (int i = 0; i < 16; ++i) red[wave][i][lane] = acc[i];
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int i = wave * kPer + q;
            float v = red[0][i][lane];
#pragma unroll
            for (int w = 1; w < W; ++w)
                if (w < wn) v = v + red[w][i][lane];
            out[q] = v;
        }
    } else {
#pragma unroll
        for (int q = 0; q < kPer; ++q) out[q] = acc[q];
    }
    float* Cp = g.c + batch_offset(batch, g.inner, g.stride_c, g.stride_c2);
    const float* addp = g.add ? g.add + (int64_t(batch) % g.add_period) * g.stride_add : nullptr;
    const int64_t col = n0 + r;
    float e_add[kPer], e_old[kPer], e_res[kPer];
    if (EPI) {
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int i = wave * kPer + q;
            const int64_t row = m0 + 8 * (i / 4) + 4 * h + (i % 4);
            const bool in = !CHECK || (row < g.m && col < g.n);
            e_add[q] = (addp && in) ? addp[row * g.ld_add + col] : 0.0f;
            e_old[q] = (g.beta != 0.0f && in) ? Cp[row * g.ldc + col] : 0.0f;
            e_res[q] = (g.res && in) ? g.res[row * g.ld_res + col] : 0.0f;
        }
    }
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const int i = wave * kPer + q;
        const int64_t row = m0 + 8 * (i / 4) + 4 * h + (i % 4);
        if (CHECK && (row >= g.m || col >= g.n)) continue;
        Cp[row * g.ldc + col] = EPI ? finish(g, out[q], e_add[q], e_old[q], e_res[q]) : out[q];
    }
}

template <int W, bool TA, bool TB, bool CHECK, bool EPI, int KU = 4>
__global__ __launch_bounds__(64 * W) void gemm_kslice(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) float lds[KsliceLds<W>::kFloats];
    kslice_tile<W, TA, TB, CHECK, EPI, KU>(g, blockIdx.x, g.batch0 + blockIdx.z, lds, W);
}

// The two products of a matmul's backward in one launch: g0 is dA = dC B^T
// (B read transposed), g1 is dB = A^T dC (A read transposed), one batch each
// of 32 x 32 tiles; blocks [0, tiles0) compute g0's tiles, the rest g1's.
// Each product keeps the K slicing (w0 or w1 waves, its k_chunk) that its own
// launch would use, so the results are that launch's bits. (Linear's
// dx = g W^T and dW = x^T g have the same two orientations.)
template <int W, bool CHECK, bool EPI, int KU = 4>
__global__ __launch_bounds__(64 * W) void gemm_kslice_pair(GemmArgs g0, GemmArgs g1, int w0,
                                                           int w1) {
    __shared__ __attribute__((aligned(16))) float lds[KsliceLds<W>::kFloats];
    const int tiles0 = g0.tiles_m * g0.tiles_n;
    if (int(blockIdx.x) < tiles0)
        kslice_tile<W, false, true, CHECK, EPI, KU>(g0, blockIdx.x, 0, lds, w0);
    else
        kslice_tile<W, true, false, CHECK, EPI, KU>(g1, int(blockIdx.x) - tiles0, 0, lds, w1);
}

// Sums the split-K partials in ws (splits x gr.ws_stride floats: the C
// partials of `batch` products, then the column sums when gr.colsum is set)
// into gr's output `out` through its epilogue, in a fixed order (gemm.hip).
int splitk_finish(const float* ws, float* out, const GemmArgs& gr, int64_t batch, int splits,
                  hipStream_t s);

}  // namespace gemm_detail
}  // namespace ehip

#endif  // EHIP_GEMM_KERNEL_HPP
