"""Pins the CPU restatement bit-for-bit against the reference compiled from its own sources.

oracle/_ref/libref_engine.so is the reference engine's CPU path (built by oracle/Makefile from
the reference checkout, plus a C shim). On seeded inputs, every oracle function and every
composition in _compose must reproduce it exactly: the restatement keeps the reference's
loop and accumulation orders, so any dropped term, swapped index or reordered sum shows up
as a nonzero difference. Also pins the brute-force and closed-form properties the reference's
own tests assert (tests/test_conv.cpp:46-63 adjoint, 332-430 exact im2col).
"""
import numpy as np
import pytest

import _compose as K
from _oracle import oracle_or_skip, ref_or_skip


@pytest.fixture(scope="module")
def orc():
    return oracle_or_skip()


@pytest.fixture(scope="module")
def ref():
    r = ref_or_skip()
    r.set_threads(4)
    return r


def rng(seed):
    return np.random.default_rng(seed)


def exact(got, want):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32)) if got.dtype == np.float32 \
        else np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} elements differ, first at {bad[:5]}: " \
                          f"{got.ravel()[bad[:3]]} vs {want.ravel()[bad[:3]]}"


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 5, 3), (33, 17, 65), (64, 64, 64),
                                   (128, 9, 8), (5, 300, 2)])
def test_matmul_fwd_bwd_bitexact(orc, ref, m, k, n):
    r = rng(m * 1000 + k * 10 + n)
    a = r.standard_normal((m, k), np.float32)
    a[a < -1.0] = 0.0  # exercise the zero skip
    b = r.standard_normal((k, n), np.float32)
    dc = r.standard_normal((m, n), np.float32)
    exact(K.matmul_fwd_bwd(orc, a, b, dc)[0], ref.matmul_fwd_bwd(a, b, dc)[0])
    for got, want in zip(K.matmul_fwd_bwd(orc, a, b, dc), ref.matmul_fwd_bwd(a, b, dc)):
        exact(got, want)


@pytest.mark.parametrize("ab,bb", [(True, True), (True, False), (False, True)])
def test_matmul_batched_shared_bitexact(orc, ref, ab, bb):
    r = rng(7)
    a = r.standard_normal((3, 6, 5) if ab else (6, 5), np.float32)
    b = r.standard_normal((3, 5, 4) if bb else (5, 4), np.float32)
    exact(orc.matmul(a, b), ref.matmul(a, b))


def test_matmul_512_bitexact(orc, ref):
    """cfg 1's shape: C = A.B at 512^3, A, B ~ N(0,1)."""
    r = rng(1)
    a = r.standard_normal((512, 512), np.float32)
    b = r.standard_normal((512, 512), np.float32)
    exact(orc.matmul(a, b), ref.matmul(a, b))


def test_matmul_brute_force(orc):
    """Sequential i-k-j float sums, spelled out per element on a tiny case."""
    r = rng(3)
    a = r.standard_normal((4, 6), np.float32)
    b = r.standard_normal((6, 5), np.float32)
    want = np.zeros((4, 5), np.float32)
    for i in range(4):
        for kk in range(6):
            for j in range(5):
                want[i, j] = np.float32(want[i, j] + np.float32(a[i, kk] * b[kk, j]))
    exact(orc.matmul(a, b), want)


def test_matmul_integer_exact(orc):
    r = rng(4)
    a = r.integers(-8, 8, (40, 30)).astype(np.float32)
    b = r.integers(-8, 8, (30, 20)).astype(np.float32)
    exact(orc.matmul(a, b), (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
@pytest.mark.parametrize("bshape", [(4, 6, 8), (8,), (1, 8), (6, 8)])
def test_binary_bitexact(orc, ref, op, bshape):
    r = rng(11)
    a = r.standard_normal((4, 6, 8), np.float32)
    b = r.standard_normal(bshape, np.float32) + (3.0 if op == "div" else 0.0)
    dy = r.standard_normal(a.shape, np.float32)
    y, da, db = ref.binary_fwd_bwd(op, a, b, dy)
    exact(orc.binary(op, a, b), y)
    if op == "add":
        exact(dy, da)
        exact(orc.fold_leading(dy, b.shape) if b.shape != a.shape else dy, db)


@pytest.mark.parametrize("shape,order", [((3, 4, 5), (0, 2, 1)), ((2, 3, 4, 5), (0, 2, 1, 3)),
                                         ((2, 3, 4, 5), (3, 1, 0, 2)), ((64, 49, 16), (0, 2, 1))])
def test_permute_bitexact(orc, ref, shape, order):
    r = rng(5)
    x = r.standard_normal(shape, np.float32)
    dy = r.standard_normal(tuple(shape[i] for i in order), np.float32)
    y, dx = ref.permute_fwd_bwd(x, order, dy)
    exact(orc.permute(x, order), y)
    exact(orc.permute(x, order), np.transpose(x, order))
    inv = np.argsort(order)
    exact(orc.permute(dy, tuple(inv)), dx)


@pytest.mark.parametrize("shape,axis", [((5, 7), 0), ((5, 7), 1), ((3, 4, 5), 1),
                                        ((300, 16), 0)])
def test_sum_axis_bitexact(orc, ref, shape, axis):
    r = rng(6)
    x = r.standard_normal(shape, np.float32)
    out_shape = shape[:axis] + shape[axis + 1:]
    dy = r.standard_normal(out_shape, np.float32)
    y, dx = ref.sum_axis_fwd_bwd(x, axis, dy)
    exact(orc.sum_axis(x, axis), y)


@pytest.mark.parametrize("which", ["relu", "softmax"])
def test_unary_bitexact(orc, ref, which):
    r = rng(8)
    x = r.standard_normal((37, 61), np.float32) * 3
    x[0, :5] = 0.0
    dy = r.standard_normal(x.shape, np.float32)
    y, dx = ref.unary_fwd_bwd(which, x, dy)
    if which == "relu":
        exact(orc.relu(x), y)
        exact(orc.relu_backward(x, dy), dx)
    else:
        exact(orc.softmax(x), y)
        exact(orc.softmax_backward(y, dy), dx)


WINDOWS = [(2, 3, 7, 9, 3, 3, 1, 1), (1, 1, 28, 28, 3, 3, 1, 1), (3, 2, 8, 8, 3, 3, 2, 0),
           (2, 4, 5, 6, 2, 3, 1, 0), (1, 2, 9, 9, 4, 4, 3, 2), (2, 8, 14, 14, 3, 3, 1, 1)]


@pytest.mark.parametrize("win", WINDOWS)
def test_im2col_col2im_bitexact(orc, ref, win):
    n, c, h, w, kh, kw, s, p = win
    r = rng(sum(win))
    x = r.standard_normal((n, c, h, w), np.float32)
    cols = orc.im2col(x, kh, kw, s, p)
    exact(cols, ref.im2col(x, kh, kw, s, p))
    y = r.standard_normal(cols.shape, np.float32)
    exact(orc.col2im(y, x.shape, kh, kw, s, p), ref.col2im(y, x.shape, kh, kw, s, p))


@pytest.mark.parametrize("win", WINDOWS)
def test_im2col_brute_force_and_adjoint(orc, win):
    """Exact window contents (tests/test_conv.cpp:332-430) and <im2col x, y> = <x, col2im y>
    (tests/test_conv.cpp:46-63), the latter in float64 on integer data so it is exact."""
    n, c, h, w, kh, kw, s, p = win
    r = rng(sum(win) + 1)
    x = r.integers(-5, 6, (n, c, h, w)).astype(np.float32)
    cols = orc.im2col(x, kh, kw, s, p)
    oh = (h + 2 * p - kh) // s + 1
    ow = (w + 2 * p - kw) // s + 1
    xp = np.pad(x, ((0, 0), (0, 0), (p, p), (p, p)))
    row = 0
    for b in range(n):
        for i in range(oh):
            for j in range(ow):
                exact(cols[row], xp[b, :, i * s:i * s + kh, j * s:j * s + kw].ravel())
                row += 1
    y = r.integers(-5, 6, cols.shape).astype(np.float32)
    lhs = float(np.sum(cols.astype(np.float64) * y))
    rhs = float(np.sum(x.astype(np.float64) * orc.col2im(y, x.shape, kh, kw, s, p)))
    assert lhs == rhs


@pytest.mark.parametrize("shape,k,s", [((2, 3, 8, 8), 2, 2), ((64, 8, 28, 28), 2, 2),
                                       ((1, 2, 7, 7), 3, 2), ((2, 1, 6, 6), 3, 1)])
def test_maxpool_bitexact(orc, ref, shape, k, s):
    r = rng(9)
    x = r.standard_normal(shape, np.float32)
    x[0, 0, :3, :3] = 0.5  # ties: the first strict maximum wins
    y, am = orc.maxpool(x, k, s)
    dy = r.standard_normal(y.shape, np.float32)
    ry, rdx = ref.maxpool_fwd_bwd(x, k, s, dy)
    exact(y, ry)
    exact(orc.maxpool_backward(am, dy, x.shape), rdx)
    # argmax is a valid index into its own window and holds the window max
    assert np.array_equal(x.ravel()[am.ravel()], y.ravel())


def test_layernorm_bitexact(orc, ref):
    r = rng(10)
    x = r.standard_normal((48, 96), np.float32) * 2 + 0.5
    g = r.standard_normal(96, np.float32)
    b = r.standard_normal(96, np.float32)
    dy = r.standard_normal(x.shape, np.float32)
    y, dx, dg, db = ref.layernorm_fwd_bwd(x, g, b, dy)
    out, cache = K.layernorm_fwd(orc, x, g, b)
    exact(out, y)
    for got, want in zip(K.layernorm_bwd(orc, dy, cache), (dx, dg, db)):
        exact(got, want)


@pytest.mark.parametrize("n,c", [(8, 5), (64, 10), (333, 121)])
def test_cross_entropy_bitexact(orc, ref, n, c):
    r = rng(n + c)
    logits = r.standard_normal((n, c), np.float32) * 2
    t = r.integers(0, c, n)
    loss, dl = ref.cross_entropy(logits, t)
    oloss, probs = orc.cross_entropy(logits, t)
    assert np.float32(oloss).view(np.uint32) == np.float32(loss).view(np.uint32)
    exact(orc.cross_entropy_backward(probs, t, 1.0), dl)


def test_cross_entropy_bad_label(orc):
    logits = np.zeros((2, 3), np.float32)
    loss, _ = orc.cross_entropy(logits, np.array([0, 3]))
    assert np.isnan(loss)


def test_embedding_bitexact(orc, ref):
    r = rng(12)
    table = r.standard_normal((13, 6), np.float32)
    ids = r.integers(0, 13, (4, 9)).astype(np.float32)
    dy = r.standard_normal((4, 9, 6), np.float32)
    y, dt = ref.embedding_fwd_bwd(table, ids, dy)
    idx = ids.ravel().astype(np.int64)
    exact(orc.select_rows(table, idx).reshape(4, 9, 6), y)
    exact(orc.scatter_add_rows(dy.reshape(36, 6), idx, table.shape), dt)


def test_adam_bitexact(orc, ref):
    r = rng(13)
    p0 = r.standard_normal(1000, np.float32)
    grads = r.standard_normal((10, 1000), np.float32)
    want = ref.adam_steps(p0, grads, 1e-3)
    p = p0.copy()
    opt = K.AdamState([p], 1e-3)
    for s in range(10):
        opt.step(orc, [p], [grads[s]])
    exact(p, want)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_bitexact(orc, ref, causal):
    r = rng(14)
    q, k, v = (r.standard_normal((2, 3, 7, 4), np.float32) for _ in range(3))
    mask = orc.causal_mask(7) if causal else None
    dy = r.standard_normal(q.shape, np.float32)
    y, w, dq, dk, dv = ref.attention_fwd_bwd(q, k, v, mask, dy)
    oy, cache = K.attention_fwd(orc, q, k, v, mask)
    exact(oy, y)
    exact(cache[3], w)
    for got, want in zip(K.attention_bwd(orc, dy, cache), (dq, dk, dv)):
        exact(got, want)


@pytest.mark.parametrize("causal", [False, True])
def test_transformer_block_bitexact(orc, ref, causal):
    d, heads, ff, b, s = 16, 4, 32, 2, 6
    r = rng(15)
    n = ref.block_num_params(d, heads, ff)
    flat = (r.standard_normal(n, np.float32) * 0.3).astype(np.float32)
    p, used = K.block_params(flat, d, ff)
    assert used == n
    x = r.standard_normal((b, s, d), np.float32)
    dy = r.standard_normal(x.shape, np.float32)
    y, dx, dp = ref.block_fwd_bwd(x, heads, ff, causal, flat, dy)
    mask = orc.causal_mask(s) if causal else None
    oy, cache = K.block_fwd(orc, x, p, heads, mask)
    exact(oy, y)
    odx, g = K.block_bwd(orc, dy, cache)
    exact(odx, dx)
    exact(np.concatenate([g[k].ravel() for k in K.BLOCK_KEYS]), dp)


def kaiming_params(r, shapes):
    out = []
    for s in shapes:
        if len(s) > 1 and s != (1, s[-1]):
            fan_in = int(np.prod(s[1:])) if len(s) == 4 else s[0]
            bound = np.sqrt(6.0 / fan_in)
            out.append(r.uniform(-bound, bound, s).astype(np.float32).ravel())
        else:
            out.append(np.zeros(int(np.prod(s)), np.float32))
    return np.concatenate(out)


def test_cnn_train_bitexact(orc, ref):
    """cfg 2 at a reduced batch (8 images), 3 Adam steps: losses and parameters exact."""
    r = rng(16)
    x = r.uniform(0, 1, (8, 1, 28, 28)).astype(np.float32)
    y = r.integers(0, 10, 8)
    flat = kaiming_params(r, K.cnn_param_shapes())
    losses, params = ref.cnn_train(x, y, flat, 3, 1e-3)
    olosses, oparams = K.cnn_train(orc, x, y, flat, 3, 1e-3)
    exact(olosses, losses)
    exact(oparams, params)


def test_charlm_train_bitexact(orc, ref):
    """cfg 3's architecture at reduced size (d 16, 2 heads, FFN 32, 2 blocks, B 2, S 8)."""
    vocab, d, heads, ff, layers, b, s = 11, 16, 2, 32, 2, 2, 8
    r = rng(17)
    n = ref.charlm_num_params(vocab, s, d, heads, ff, layers)
    flat = (r.standard_normal(n, np.float32) * 0.2).astype(np.float32)
    ids = r.integers(0, vocab, (b, s)).astype(np.float32)
    t = r.integers(0, vocab, b * s)
    losses, params = ref.charlm_train(ids, t, vocab, d, heads, ff, layers, flat, 3, 1e-3)
    olosses, oparams = K.charlm_train(orc, ids, t, flat, vocab, d, heads, ff, layers, 3, 1e-3)
    exact(olosses, losses)
    exact(oparams, params)


# ------------------------------------------------------------------ whole-tensor sums, scalars

@pytest.mark.parametrize("n", [1, 1000, 1 << 20])
def test_sum_and_mean_bitexact(orc, ref, n):
    """Tensor::sum() / mean() (src/tensor_ops.cpp:679-712): the oracle's double sum, cast to
    float, is the reference's sum bit for bit; times 1/n in float it is the mean."""
    r = rng(n + 31)
    x = (r.standard_normal(n, np.float32) * 3).astype(np.float32)
    s = np.float32(orc.sum(x))
    exact(np.array([s]), np.array([ref.sum(x)]))
    exact(np.array([s * np.float32(1.0 / n)]), np.array([ref.mean(x)]))


@pytest.mark.parametrize("n", [1, 1000, 1 << 20])
def test_sum_squares_bitexact_through_clip_norm(orc, ref, n):
    """The double sum of squares behind clip_grad_norm (src/optim.cpp:186-193): for one
    gradient tensor, float(sqrt(oracle)) is the reference's returned norm bit for bit."""
    r = rng(n + 57)
    g = r.standard_normal(n, np.float32)
    norm, _ = ref.clip_grad_norm(g, [n], 1e30)
    exact(np.array([np.float32(np.sqrt(orc.sum_squares(g)))]), np.array([np.float32(norm)]))


def test_sum_closed_forms(orc):
    """Mathematics that fixes the double accumulator: integer-valued data sums exactly (the
    total stays below 2^53), and 2^25 followed by a thousand ones keeps every one, which a
    float accumulator would round away (the float spacing at 2^25 is 4)."""
    r = rng(3)
    x = r.integers(-1000, 1001, 1 << 16).astype(np.float32)
    assert orc.sum(x) == float(int(x.astype(np.int64).sum()))
    assert orc.sum_squares(x) == float(int((x.astype(np.int64) ** 2).sum()))
    big = np.concatenate([[np.float32(2 ** 25)], np.ones(1000, np.float32)])
    assert orc.sum(big) == 2 ** 25 + 1000
    sq = np.concatenate([[np.float32(2 ** 12)], np.ones(1000, np.float32)])
    assert orc.sum_squares(sq) == 2 ** 24 + 1000
    assert orc.sum(np.zeros(0, np.float32)) == 0.0
    assert orc.sum(np.array([-3.5], np.float32)) == -3.5


@pytest.mark.parametrize("n", [1, 1000, 1 << 20])
@pytest.mark.parametrize("k", [0.37, -1e-3, 3.0, 0.0, 1e30])
def test_scalar_add_mul_bitexact(orc, ref, n, k):
    """t + k and t * k (src/tensor_ops.cpp:276-322) bit for bit, with -0, +-inf and NaN in
    the input."""
    r = rng(n + 7)
    x = r.standard_normal(n, np.float32)
    x[: min(n, 4)] = np.array([-0.0, np.inf, -np.inf, np.nan], np.float32)[: min(n, 4)]
    exact(orc.scalar_add(x, k), ref.scalar(x, k))
    exact(orc.scalar_mul(x, k), ref.scalar(x, k, mul=True))


def test_scalar_closed_forms(orc):
    """x + 0 turns -0 into +0 (IEEE round-to-nearest), x + k and x * k are the single
    correctly rounded float operations."""
    x = np.array([-0.0, 1.5, -2.25, 3e38, np.float32(1) / 3], np.float32)
    y = orc.scalar_add(x, 0.0)
    assert np.signbit(y[0]) == False  # noqa: E712
    assert np.array_equal(orc.scalar_add(x, 0.25), x + np.float32(0.25))
    assert np.array_equal(orc.scalar_mul(x, 2.0), x * np.float32(2.0))
    assert np.isinf(orc.scalar_add(x, 3e38)[3])


# ------------------------------------------------------------------ the GEMM test bound

def test_gemm_stat_bound_catches_a_dropped_term(orc):
    """The statistical bound the GPU GEMM tests apply (tests/_hip.py gemm_stat_bound) admits
    the reference's own serial fp32 sum at cfg 2's longest weight-gradient length
    (K = 12544) and rejects the same sum with one product left out: the mistake is planted
    in the oracle's operand, on the CPU."""
    from _hip import gemm_stat_bound
    r = rng(12544)
    m, k, n = 16, 12544, 16
    a = r.standard_normal((m, k), np.float32)
    b = r.standard_normal((k, n), np.float32)
    exact64 = a.astype(np.float64) @ b.astype(np.float64)
    bound = gemm_stat_bound(np.linalg.norm(a.astype(np.float64), axis=1),
                            np.linalg.norm(b.astype(np.float64), axis=0), k)
    assert np.all(np.abs(orc.matmul(a, b) - exact64) <= bound)
    planted = a.copy()
    planted[:, 777] = 0.0  # one product per output dropped
    err = np.abs(orc.matmul(planted, b) - exact64)
    caught = np.mean(err > bound)
    assert caught >= 0.5, caught
