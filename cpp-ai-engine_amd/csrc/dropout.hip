// dropout.hip -- Dropout masks from a counter-based generator.
//
// The reference draws its mask from std::bernoulli over one global mt19937,
// element by element in order (src/nn.cpp:206-244): a sequential stream that
// a GPU cannot reproduce in parallel. Here element i of a call is decided by
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
// as 1, 2, 3", SC'11): the 64-bit counter value c = offset + i selects word
// c % 4 of the block philox((c / 4) low, (c / 4) high, 0, 0; seed low, seed
// high), its top 24 bits give u = word >> 8 over 2^24 in [0, 1), and the
// element is kept when u < keep = 1 - p. The mask is a function of (seed,
// offset, i) only -- the same on any device, launch shape or stream -- and
// the kept values are x * (1 / keep), the reference's arithmetic.

#include "common.hpp"

namespace ehip {
namespace {

constexpr int kThreads = 256;

struct U4 {
    uint32_t v[4];
};

__device__ __forceinline__ void mulhilo(uint32_t a, uint32_t b, uint32_t& hi, uint32_t& lo) {
    const uint64_t p = uint64_t(a) * uint64_t(b);
    hi = uint32_t(p >> 32);
    lo = uint32_t(p);
}

// Philox4x32 with 10 rounds; the key is bumped by the Weyl constants between
// rounds.
__device__ __forceinline__ U4 philox4x32_10(uint64_t block, uint64_t seed) {
    uint32_t c0 = uint32_t(block), c1 = uint32_t(block >> 32), c2 = 0, c3 = 0;
    uint32_t k0 = uint32_t(seed), k1 = uint32_t(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r > 0) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        uint32_t hi0, lo0, hi1, lo1;
        mulhilo(0xD2511F53u, c0, hi0, lo0);
        mulhilo(0xCD9E8D57u, c2, hi1, lo1);
        const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
    }
    return U4{{c0, c1, c2, c3}};
}

__device__ __forceinline__ float dropout_mask(uint32_t word, float keep, float scale) {
    const float u = float(word >> 8) * (1.0f / 16777216.0f);
    return u < keep ? scale : 0.0f;
}

// One Philox block (four consecutive counter values) per thread.
__global__ __launch_bounds__(kThreads) void dropout_kernel(const float* __restrict__ x,
                                                           float* __restrict__ y,
                                                           float* __restrict__ mask, int64_t n,
                                                           float keep, float scale, uint64_t seed,
                                                           uint64_t offset) {
    const uint64_t first_block = offset / 4;
    const uint64_t last_block = (offset + uint64_t(n) - 1) / 4;
    const uint64_t step = uint64_t(gridDim.x) * kThreads;
    for (uint64_t b = first_block + uint64_t(blockIdx.x) * kThreads + threadIdx.x;
         b <= last_block; b += step) {
        const U4 r = philox4x32_10(b, seed);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint64_t c = 4 * b + uint64_t(j);
            if (c < offset || c >= offset + uint64_t(n)) continue;
            const int64_t i = int64_t(c - offset);
            const float m = dropout_mask(r.v[j], keep, scale);
            y[i] = x[i] * m;
            if (mask) mask[i] = m;
        }
    }
}

}  // namespace
}  // namespace ehip

using namespace ehip;

extern "C" {

int ehip_dropout_f32(const float* x, float* y, float* mask, int64_t n, float p, uint64_t seed,
                     uint64_t offset, void* stream) {
    EHIP_READY();
    if (n < 0) return fail(EHIP_EINVAL, "dropout: negative size");
    if (!(p >= 0.0f && p < 1.0f)) return fail(EHIP_EINVAL, "dropout: p must be in [0, 1)");
    if (n == 0) return EHIP_OK;
    if (!x || !y) return fail(EHIP_EINVAL, "dropout: null pointer");
    if (offset > UINT64_MAX - uint64_t(n)) return fail(EHIP_EINVAL, "dropout: counter overflow");
    const float keep = 1.0f - p;
    const float scale = 1.0f / keep;
    const uint64_t blocks = (offset + uint64_t(n) - 1) / 4 - offset / 4 + 1;
    uint64_t grid = (blocks + kThreads - 1) / kThreads;
    if (grid > 65536) grid = 65536;
    EHIP_LAUNCH("dropout", dropout_kernel, dim3(unsigned(grid)), dim3(kThreads), 0,
                as_stream(stream), x, y, mask, n, keep, scale, seed, offset);
    return EHIP_OK;
}

}  // extern "C"
