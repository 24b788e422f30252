// Runs every function of the CPU oracle (oracle/oracle.h) once on small inputs whose
// buffers are exactly the sizes the functions are documented to read and write, under
// AddressSanitizer and UndefinedBehaviorSanitizer: an access past a buffer, a misaligned
// or overflowing index computation, or a use of freed memory stops the run.
#include <cmath>
#include <cstdio>
#include <vector>

#include "oracle.h"

static std::vector<float> seq(size_t n, float scale = 0.01f) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = scale * float(int(i * 37 % 101) - 50);
    return v;
}

int main() {
    // GEMM: batched and shared operands.
    {
        const int64_t b = 3, m = 5, k = 7, n = 4;
        auto a = seq(b * m * k), bb = seq(b * k * n);
        std::vector<float> c(b * m * n);
        orc_matmul(a.data(), bb.data(), c.data(), b, m, k, n, 1, 1);
        std::vector<float> b2 = seq(k * n);
        orc_matmul(a.data(), b2.data(), c.data(), b, m, k, n, 1, 0);
    }
    {
        auto x = seq(2 * 3 * 5);
        std::vector<float> y(x.size());
        orc_transpose(x.data(), y.data(), 2, 3, 5);
        const int64_t shape[4] = {2, 3, 4, 5}, order[4] = {0, 2, 1, 3};
        auto x4 = seq(120);
        std::vector<float> y4(120);
        orc_permute(x4.data(), y4.data(), 4, shape, order);
    }
    {
        auto a = seq(4 * 6), b = seq(6, 0.1f);
        for (float& v : b) v += 3.0f;
        std::vector<float> o(24);
        for (int op = 0; op < 4; ++op) orc_binary(op, a.data(), b.data(), o.data(), 6, 4);
        orc_scalar_add(a.data(), o.data(), 24, 1.5f);
        orc_scalar_mul(a.data(), o.data(), 24, -2.0f);
        orc_relu(a.data(), o.data(), 24);
        orc_relu_backward(a.data(), b.data(), o.data(), 6);
        orc_accumulate(o.data(), a.data(), 24);
        std::vector<float> s(4 * 2);
        orc_sum_axis(a.data(), s.data(), 4, 3, 2);
        if (!std::isfinite(orc_sum(a.data(), 24)) || orc_sum_squares(a.data(), 24) < 0) return 1;
    }
    {
        orc_window w{2, 3, 7, 6, 3, 3, 2, 1, 0, 0};
        w.out_h = (w.height + 2 * w.padding - w.kernel_h) / w.stride + 1;
        w.out_w = (w.width + 2 * w.padding - w.kernel_w) / w.stride + 1;
        auto x = seq(w.batch * w.channels * w.height * w.width);
        std::vector<float> cols(w.batch * w.out_h * w.out_w * w.channels * 9), back(x.size());
        orc_im2col(x.data(), cols.data(), &w);
        orc_col2im(cols.data(), back.data(), &w);
        orc_window p{2, 3, 6, 6, 2, 2, 2, 0, 3, 3};
        auto xp = seq(2 * 3 * 36);
        std::vector<float> y(2 * 3 * 9), dx(xp.size());
        std::vector<int32_t> am(y.size());
        orc_maxpool(xp.data(), y.data(), am.data(), &p);
        orc_maxpool_backward(am.data(), y.data(), dx.data(), int64_t(y.size()), int64_t(xp.size()));
    }
    {
        const int64_t r = 6, c = 9;
        auto x = seq(r * c), g = seq(r * c, 0.02f);
        std::vector<float> y(r * c), dx(r * c);
        orc_softmax(x.data(), y.data(), r, c);
        orc_softmax_backward(y.data(), g.data(), dx.data(), r, c);
        auto gamma = seq(c, 0.1f), beta = seq(c, 0.05f);
        std::vector<float> out(r * c), xh(r * c), inv(r), dg(c), db(c);
        orc_layernorm(x.data(), gamma.data(), beta.data(), out.data(), xh.data(), inv.data(), r, c,
                      1e-5f);
        orc_layernorm_backward(g.data(), xh.data(), gamma.data(), inv.data(), dx.data(), dg.data(),
                               db.data(), r, c);
        std::vector<int64_t> t(r);
        for (int64_t i = 0; i < r; ++i) t[i] = (i * 5) % c;
        std::vector<float> probs(r * c);
        if (!std::isfinite(orc_cross_entropy(x.data(), t.data(), probs.data(), r, c))) return 1;
        orc_cross_entropy_backward(probs.data(), t.data(), dx.data(), r, c, 0.5f);
    }
    {
        const int64_t n = 37;
        auto p = seq(n), g = seq(n, 0.02f);
        std::vector<float> m(n), v(n), vel(n);
        for (int64_t t = 1; t <= 3; ++t) {
            float c1, c2;
            orc_adam_bias(0.9f, 0.999f, t, &c1, &c2);
            orc_adam(p.data(), g.data(), m.data(), v.data(), n, 1e-3f, 0.9f, 0.999f, 1e-8f, 0.01f,
                     c1, c2);
            orc_sgd(p.data(), g.data(), vel.data(), n, 1e-2f, 0.9f, 1e-4f);
        }
        orc_sgd(p.data(), g.data(), nullptr, n, 1e-2f, 0.0f, 0.0f);
    }
    {
        const int64_t rows = 5, rs = 4, ni = 7;
        auto table = seq(rows * rs);
        std::vector<int64_t> idx = {0, 4, 4, 1, 3, 0, 2};
        std::vector<float> out(ni * rs), dx(rows * rs);
        orc_select_rows(table.data(), idx.data(), out.data(), ni, rs);
        orc_scatter_add_rows(out.data(), idx.data(), dx.data(), ni, rs);
        std::vector<float> pe(9 * 6), mask(9 * 9);
        orc_positional_encoding(pe.data(), 9, 6);
        orc_causal_mask(mask.data(), 9, -1e9f);
        const uint32_t ctr[4] = {1, 2, 3, 4}, key[2] = {5, 6};
        uint32_t out4[4];
        orc_philox4x32_10(ctr, key, out4);
        auto x = seq(33);
        std::vector<float> y(33), msk(33);
        orc_dropout(x.data(), y.data(), msk.data(), 33, 0.25f, 7, 3);
    }
    std::printf("oracle_driver: ok\n");
    return 0;
}
