"""The in-place attention path: ehip_gemm_ex_f32 (two-level head strides, the
scale / mask / beta epilogue), ehip_softmax_backward_scaled_f32, and the engine's
attention_heads node.

Each fused product is checked bit for bit against the composition it replaces --
the heads copied out with a plain permute, the same ehip_gemm_f32 product, then
the scale and the mask as separate IEEE element-wise steps (torch fp32 on the
device) -- and against an fp64 product within the K-term tolerance. The engine
node is checked bit for bit against MultiHeadAttention's composed path (split,
scaled_dot_product_attention, merge: src/transformer.cpp:279-349) and against
the oracle composition at the reference's parity metric.
"""
import math

import numpy as np
import pytest

import _compose as K
from _hip import backend, dev, exact, host, k_tol, print_case, ref_close, ref_err
from _oracle import oracle_or_skip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    return backend()


@pytest.fixture(scope="module")
def orc():
    return oracle_or_skip()


@pytest.fixture(scope="module")
def eng():
    # torch's HIP runtime first, as the other GPU fixtures do: initialised after
    # the engine library in a fresh process, torch reports no device.
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test ran without a visible GPU")
    from engine_capi import Engine
    return Engine()


def randn(r, *shape):
    return r.standard_normal(shape, dtype=np.float32)


def heads_of(t, b, s, h, hd):
    """(b, s, h*hd) device tensor -> (b*h, s, hd) contiguous copy (a plain move)."""
    return t.reshape(b, s, h, hd).permute(0, 2, 1, 3).contiguous().reshape(b * h, s, hd)


def merged_of(t, b, s, h, hd):
    """(b*h, s, hd) -> (b, s, h*hd) contiguous copy."""
    return t.reshape(b, h, s, hd).permute(0, 2, 1, 3).contiguous().reshape(b, s, h * hd)


def desc(hip, ta, tb, batch, inner, m, n, k, a, lda, sa, sa2, b, ldb, sb, sb2, c, ldc, sc, sc2,
         alpha=1.0, addend=None, ld_add=0, stride_add=0, period=1, beta=0.0, relu=False,
         residual=None, ld_res=0):
    from ehip import GemmEx
    return GemmEx(int(ta), int(tb), batch, inner, m, n, k, hip.p(a), lda, sa, sa2, hip.p(b), ldb,
                  sb, sb2, hip.p(c), ldc, sc, sc2, alpha,
                  None if addend is None else hip.p(addend), ld_add, stride_add, period, beta,
                  int(relu), None, 0, None if residual is None else hip.p(residual), ld_res)


# (batch, seq, heads, head_dim): the char model's heads (cfg3), a head_dim that
# is not a multiple of 4 (checked loads), tiles that the small kernels take,
# and the 512-token heads of the scaled model.
SHAPES = [(2, 64, 4, 24), (2, 37, 3, 6), (2, 16, 2, 8), (1, 512, 4, 64), (3, 130, 2, 32)]
MASKS = ["none", "causal", "per_head", "per_product", "row"]


def mask_for(kind, r, b, s, h):
    """(mask array or None, ld, stride, period) for the suffix-broadcast kinds."""
    if kind == "none":
        return None, 0, 0, 1
    if kind == "causal":
        m = np.triu(np.full((s, s), -1e9, np.float32), 1)
        return m, s, 0, 1
    if kind == "per_head":
        return randn(r, h, s, s), s, s * s, h
    if kind == "per_product":
        return randn(r, b, h, s, s), s, s * s, b * h
    return randn(r, s), 0, 0, 1  # one row repeated over every row


@pytest.mark.parametrize("b,s,h,hd", SHAPES)
@pytest.mark.parametrize("kind", MASKS)
def test_scores_epilogue_bitexact(hip, b, s, h, hd, kind):
    import torch
    print_case("gemm_ex scores", b, s, h, hd, kind)
    r = np.random.default_rng(b * 1000 + s * 10 + h + hd + MASKS.index(kind))
    d = h * hd
    q, k = dev(randn(r, b, s, d)), dev(randn(r, b, s, d))
    mask, ld, st, period = mask_for(kind, r, b, s, h)
    mk = None if mask is None else dev(mask)
    scale = float(np.float32(1.0) / np.float32(math.sqrt(hd)))
    c = hip.f32((b, h, s, s))
    hip.gemm_ex(desc(hip, False, True, b * h, h, s, s, hd, q, d, s * d, hd, k, d, s * d, hd, c, s,
                     h * s * s, s * s, alpha=scale, addend=mk, ld_add=ld, stride_add=st,
                     period=period))
    raw = hip.gemm(heads_of(q, b, s, h, hd), heads_of(k, b, s, h, hd), trans_b=True)
    want = raw.reshape(b, h, s, s) * torch.tensor(scale, dtype=torch.float32, device="cuda")
    if mk is not None:
        want = want + mk
    exact(host(c), host(want), f"scores {kind}")
    # The product itself against fp64.
    qh = host(q).reshape(b, s, h, hd).transpose(0, 2, 1, 3).astype(np.float64)
    kh = host(k).reshape(b, s, h, hd).transpose(0, 2, 1, 3).astype(np.float64)
    exp = (qh @ kh.transpose(0, 1, 3, 2)) * scale
    if mask is not None:
        exp = exp + mask
    ref_close(host(c), exp, k_tol(hd) * 4, "scores vs fp64")


@pytest.mark.parametrize("b,s,h,hd", SHAPES)
def test_head_products_bitexact(hip, b, s, h, hd):
    """The four other products of the node, each writing or reading heads in place."""
    print_case("gemm_ex head products", b, s, h, hd)
    r = np.random.default_rng(7 + b + s + h + hd)
    d = h * hd
    w = dev(randn(r, b * h, s, s))
    v, g, q, kk = (dev(randn(r, b, s, d)) for _ in range(4))
    hs = lambda t: heads_of(t, b, s, h, hd)  # noqa: E731
    hss, ss, sd = h * s * s, s * s, s * d
    # out = W V -> merged layout
    out = hip.f32((b, s, d))
    hip.gemm_ex(desc(hip, False, False, b * h, h, s, hd, s, w, s, hss, ss, v, d, sd, hd, out, d,
                     sd, hd))
    exact(host(out), host(merged_of(hip.gemm(w, hs(v)), b, s, h, hd)), "W V")
    # dW = g V^T -> heads-major
    dw = hip.f32((b * h, s, s))
    hip.gemm_ex(desc(hip, False, True, b * h, h, s, s, hd, g, d, sd, hd, v, d, sd, hd, dw, s, hss,
                     ss))
    exact(host(dw), host(hip.gemm(hs(g), hs(v), trans_b=True)), "g V^T")
    # dV = W^T g -> merged
    dv = hip.f32((b, s, d))
    hip.gemm_ex(desc(hip, True, False, b * h, h, s, hd, s, w, s, hss, ss, g, d, sd, hd, dv, d, sd,
                     hd))
    exact(host(dv), host(merged_of(hip.gemm(w, hs(g), trans_a=True), b, s, h, hd)), "W^T g")
    # dQ = dS K, dK = dS^T Q -> merged
    dq = hip.f32((b, s, d))
    hip.gemm_ex(desc(hip, False, False, b * h, h, s, hd, s, w, s, hss, ss, kk, d, sd, hd, dq, d,
                     sd, hd))
    exact(host(dq), host(merged_of(hip.gemm(w, hs(kk)), b, s, h, hd)), "dS K")
    dk = hip.f32((b, s, d))
    hip.gemm_ex(desc(hip, True, False, b * h, h, s, hd, s, w, s, hss, ss, q, d, sd, hd, dk, d, sd,
                     hd))
    exact(host(dk), host(merged_of(hip.gemm(w, hs(q), trans_a=True), b, s, h, hd)), "dS^T Q")


def test_epilogue_through_split_k(hip):
    """Few tiles and a long K split the product; the reduction applies the epilogue."""
    import torch
    print_case("gemm_ex split-K epilogue")
    r = np.random.default_rng(11)
    a, bm = dev(randn(r, 2, 2, 64, 8192)), dev(randn(r, 2, 2, 8192, 64))
    add = dev(randn(r, 64, 64))
    c0 = randn(r, 4, 64, 64)
    c = dev(c0)
    hip.gemm_ex(desc(hip, False, False, 4, 2, 64, 64, 8192, a, 8192, 2 * 64 * 8192, 64 * 8192,
                     bm, 64, 2 * 8192 * 64, 8192 * 64, c, 64, 2 * 64 * 64, 64 * 64, alpha=0.375,
                     addend=add, ld_add=64, stride_add=0, period=1, beta=0.5))
    acc = hip.gemm(a.reshape(4, 64, 8192), bm.reshape(4, 8192, 64))
    f = lambda x: torch.tensor(x, dtype=torch.float32, device="cuda")  # noqa: E731
    want = ((acc * f(0.375)) + add) + f(0.5) * dev(c0)
    exact(host(c), host(want), "split-K epilogue")


def test_epilogue_k_zero(hip):
    print_case("gemm_ex k=0")
    r = np.random.default_rng(12)
    add, c0 = randn(r, 5, 7), randn(r, 3, 5, 7)
    c = dev(c0)
    a = dev(np.zeros(1, np.float32))
    hip.gemm_ex(desc(hip, False, False, 3, 1, 5, 7, 0, a, 1, 0, 0, a, 7, 0, 0, c, 7, 35, 0,
                     alpha=2.0, addend=dev(add), ld_add=7, stride_add=0, beta=0.5))
    want = (np.float32(0.0) + add) + np.float32(0.5) * c0
    exact(host(c), want.astype(np.float32), "k=0 epilogue")


def test_gemm_ex_refusals(hip):
    print_case("gemm_ex refusals")
    x = dev(np.zeros(64, np.float32))
    bad = [dict(inner=0), dict(period=0), dict(ld_add=-1)]
    for kw in bad:
        inner = kw.get("inner", 1)
        dsc = desc(hip, False, False, 1, inner, 4, 4, 4, x, 4, 0, 0, x, 4, 0, 0, x, 4, 0, 0,
                   addend=x, ld_add=kw.get("ld_add", 4), period=kw.get("period", 1))
        with pytest.raises(RuntimeError):
            hip.gemm_ex(dsc)


@pytest.mark.parametrize("rows,cols", [(64, 64), (4096, 37), (256, 512), (3, 5000)])
def test_softmax_backward_scaled(hip, rows, cols):
    import torch
    print_case("softmax_backward_scaled", rows, cols)
    r = np.random.default_rng(rows + cols)
    y = hip.softmax(dev(randn(r, rows, cols)))
    g = dev(randn(r, rows, cols))
    scale = float(np.float32(1.0) / np.float32(math.sqrt(24.0)))
    want = hip.softmax_backward(y, g) * torch.tensor(scale, dtype=torch.float32, device="cuda")
    exact(host(hip.softmax_backward(y, g, scale=scale)), host(want), "scaled")
    hip.softmax_backward(y, g, scale=scale, out=g)  # in place over g
    exact(host(g), host(want), "scaled in place")


def mha_params(r, d):
    parts = []
    for _ in range(4):
        parts.append((randn(r, d, d) / np.float32(math.sqrt(d))).ravel())
        parts.append((randn(r, 1, d) * np.float32(0.1)).ravel())
    return np.concatenate(parts)


@pytest.mark.parametrize("b,s,d,heads", [(2, 16, 24, 4), (32, 64, 96, 4), (2, 33, 30, 5),
                                         (1, 128, 256, 4)])
@pytest.mark.parametrize("causal", [False, True])
def test_mha_fused_equals_composed(eng, orc, b, s, d, heads, causal):
    print_case("mha fused vs composed", b, s, d, heads, causal)
    r = np.random.default_rng(b * 100 + s + d + heads + causal)
    x, dy = randn(r, b, s, d), randn(r, b, s, d)
    params = mha_params(r, d)
    mask = np.triu(np.full((s, s), -1e9, np.float32), 1) if causal else None
    # Bias gradients from the separate column sums on both sides (see both_graphs); the
    # batched-product attention (the short path has its own test below).
    prev_db = eng.set_fused_bias_grad(False)
    prev_short = eng.set_short_attention(False)
    try:
        fused = eng.mha_fwd_bwd(x, heads, params, dy, mask=mask, fuse=True, weights=True)
        comp = eng.mha_fwd_bwd(x, heads, params, dy, mask=mask, fuse=False, weights=True)
    finally:
        eng.set_fused_bias_grad(prev_db)
        eng.set_short_attention(prev_short)
    for got, want, what in zip(fused, comp, ("y", "dx", "dparams", "weights")):
        exact(got, want, f"fused {what}")
    # And against the oracle composition (the reference's CPU arithmetic).
    names = ("wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo")
    shapes = [(d, d), (1, d)] * 4
    p, off = {}, 0
    for name, shp in zip(names, shapes):
        n = int(np.prod(shp))
        p[name] = params[off:off + n].reshape(shp)
        off += n
    y, cache = K.mha_fwd(orc, x, p, heads, mask)
    dx, grads = K.mha_bwd(orc, dy, cache)
    # Each output at the K-term tolerance of its own sums: y and dx reduce over d and s;
    # the parameter gradients over the b * s rows.
    tol = 4 * k_tol(max(s, d))
    ref_close(fused[0], y, tol, "y vs oracle")
    ref_close(fused[1], dx, tol, "dx vs oracle")
    off = 0
    for name, shp in zip(names, shapes):
        n = int(np.prod(shp))
        ref_close(fused[2][off:off + n].reshape(shp), grads[name], 4 * k_tol(max(s, d, b * s)),
                  f"{name} vs oracle")
        off += n


# ------------------------------------------------------- bias / ReLU epilogue

@pytest.mark.parametrize("m,k,n", [(8192, 96, 384), (300, 1024, 257), (64, 8, 10),
                                   (2048, 4096, 1024), (4096, 1024, 4096)])
def test_bias_relu_epilogue(hip, m, k, n):
    """Linear's broadcast bias (ld_addend 0), then ReLU: equal bit for bit to
    the separate kernels."""
    print_case("gemm_ex bias/relu", m, k, n)
    r = np.random.default_rng(m + k + n)
    a, b = dev(randn(r, m, k)), dev(randn(r, k, n))
    bias = dev(randn(r, 1, n))
    pre = hip.gemm(a, b) + bias
    y = hip.f32((m, n))
    hip.gemm_ex(desc(hip, False, False, 1, 1, m, n, k, a, k, 0, 0, b, n, 0, 0, y, n, 0, 0,
                     addend=bias, ld_add=0))
    exact(host(y), host(pre), "bias")
    hip.gemm_ex(desc(hip, False, False, 1, 1, m, n, k, a, k, 0, 0, b, n, 0, 0, y, n, 0, 0,
                     addend=bias, ld_add=0, relu=True))
    exact(host(y), host(hip.relu(pre)), "bias + relu")


@pytest.mark.parametrize("m,k,n", [(2048, 384, 96), (2048, 96, 96), (300, 1024, 257),
                                   (64, 8, 10), (2048, 4096, 1024), (8192, 4096, 1024)])
def test_residual_epilogue(hip, m, k, n):
    """The residual add of a Transformer block's branch in the product's epilogue: after
    the bias and beta C, before ReLU, each rounded on its own, so equal bit for bit to the
    separate adds; a residual with its own row stride is read through it."""
    print_case("gemm_ex residual", m, k, n)
    r = np.random.default_rng(m + k + n + 1)
    a, b = dev(randn(r, m, k)), dev(randn(r, k, n))
    bias = dev(randn(r, 1, n))
    wide = dev(randn(r, m, n + 3))
    res = wide[:, 1:n + 1].contiguous()
    c0 = dev(randn(r, m, n))
    pre = hip.gemm(a, b) + bias
    y = hip.f32((m, n))
    hip.gemm_ex(desc(hip, False, False, 1, 1, m, n, k, a, k, 0, 0, b, n, 0, 0, y, n, 0, 0,
                     addend=bias, ld_add=0, residual=res, ld_res=n))
    exact(host(y), host(res + pre), "bias + residual")
    y.copy_(c0)
    hip.gemm_ex(desc(hip, False, False, 1, 1, m, n, k, a, k, 0, 0, b, n, 0, 0, y, n, 0, 0,
                     addend=bias, ld_add=0, beta=1.0, relu=True, residual=wide.view(-1)[1:],
                     ld_res=n + 3))
    exact(host(y), host(hip.relu(pre + c0 + res)), "bias + beta C + strided residual, ReLU")


@pytest.mark.parametrize("ta,m,k,n", [(False, 256, 8192, 256), (True, 96, 2048, 96),
                                      (True, 384, 2048, 96)])
def test_residual_epilogue_split_and_panel(hip, ta, m, k, n):
    """The residual on the other output paths: a product split along K (the reduction
    applies the epilogue) and the A^T B panel products of narrow weight gradients."""
    print_case("gemm_ex residual split/panel", ta, m, k, n)
    r = np.random.default_rng(m + k + n + 7)
    a = dev(randn(r, k, m)) if ta else dev(randn(r, m, k))
    b = dev(randn(r, k, n))
    res = dev(randn(r, m, n))
    pre = hip.gemm(a, b, trans_a=ta)
    y = hip.f32((m, n))
    hip.gemm_ex(desc(hip, ta, False, 1, 1, m, n, k, a, m if ta else k, 0, 0, b, n, 0, 0, y, n, 0,
                     0, residual=res, ld_res=n))
    exact(host(y), host(res + pre), "residual")


def test_residual_refusals(hip):
    """A residual row stride shorter than a row, or a residual on a batched product, is
    refused before any launch."""
    print_case("gemm_ex residual refusals")
    x = dev(np.zeros(64, np.float32))
    for batch, ld in ((1, 3), (2, 4)):
        dsc = desc(hip, False, False, batch, 1, 4, 4, 4, x, 4, 0, 0, x, 4, 0, 0, x, 4, 16, 0,
                   residual=x, ld_res=ld)
        with pytest.raises(RuntimeError):
            hip.gemm_ex(dsc)


def test_relu_epilogue_signs(hip):
    """-0, NaN and +-inf through the ReLU epilogue match the ReLU kernel."""
    print_case("gemm_ex relu signs")
    a = dev(np.array([[1.0], [-1.0], [0.0], [-0.0], [np.nan], [np.inf], [-np.inf], [1e-30]],
                     np.float32))
    b = dev(np.ones((1, 3), np.float32))
    y = hip.f32((8, 3))
    hip.gemm_ex(desc(hip, False, False, 1, 1, 8, 3, 1, a, 1, 0, 0, b, 3, 0, 0, y, 3, 0, 0,
                     relu=True))
    exact(host(y), host(hip.relu(hip.gemm(a, b))), "relu signs")


# ------------------------------------------------------- fused vs composed engine graph

def both_graphs(eng, fn):
    """fn() with fused nodes, then with the reference's node-by-node graph. Both take every
    bias gradient from the separate column sum (the composed graph's bias-add node always
    does): node fusion itself is what must not move a bit; the mid-sized layers' bias sums
    from the dW products, another order, are tested against the separate sums elsewhere."""
    prev = eng.set_fused_nodes(True)
    prev_db = eng.set_fused_bias_grad(False)
    prev_short = eng.set_short_attention(False)  # its own test: test_short_attention_node
    try:
        fused = fn()
        eng.set_fused_nodes(False)
        comp = fn()
    finally:
        eng.set_fused_nodes(prev)
        eng.set_fused_bias_grad(prev_db)
        eng.set_short_attention(prev_short)
    return fused, comp


@pytest.mark.parametrize("rows,inp,out", [(64, 8, 10), (8192, 96, 384), (300, 1024, 257)])
def test_linear_fused_equals_composed(eng, rows, inp, out):
    print_case("linear fused vs composed", rows, inp, out)
    r = np.random.default_rng(rows + inp + out)
    x, w, bias, dy = randn(r, rows, inp), randn(r, inp, out), randn(r, 1, out), randn(r, rows, out)
    fused, comp = both_graphs(eng, lambda: eng.linear_fwd_bwd(x, w, bias, dy))
    for got, want, what in zip(fused, comp, ("y", "dx", "dw", "db")):
        exact(got, want, f"linear {what}")


@pytest.mark.parametrize("b,s,d,heads,ff,causal", [(2, 16, 24, 4, 32, True),
                                                    (32, 64, 96, 4, 384, True),
                                                    (2, 33, 30, 5, 70, False)])
def test_block_fused_equals_composed(eng, b, s, d, heads, ff, causal):
    print_case("block fused vs composed", b, s, d, heads, ff, causal)
    r = np.random.default_rng(b + s + d + heads + ff)
    x, dy = randn(r, b, s, d), randn(r, b, s, d)
    n = eng.block_num_params(d, heads, ff)
    params = randn(r, n) * np.float32(0.1)
    fused, comp = both_graphs(eng, lambda: eng.block_fwd_bwd(x, heads, ff, causal, params, dy))
    for got, want, what in zip(fused, comp, ("y", "dx", "dparams")):
        exact(got, want, f"block {what}")


def test_charlm_training_fused_equals_composed(eng):
    """Five Adam steps of the cfg3 character model: losses and final weights
    are identical under both graphs."""
    import _compose as KC
    print_case("charlm fused vs composed")
    vocab, s, d, heads, ff, layers, b = 121, 64, 96, 4, 384, 2, 32
    r = np.random.default_rng(5)
    ids = r.integers(0, vocab, (b, s)).astype(np.int64)
    targets = r.integers(0, vocab, (b, s)).astype(np.int64)
    shapes = KC.charlm_param_shapes(vocab, d, ff, layers)
    params = np.concatenate([(randn(r, *shp) * np.float32(0.05)).ravel() for shp in shapes])
    fused, comp = both_graphs(eng, lambda: eng.charlm_train(ids, targets, vocab, d, heads, ff,
                                                            layers, params, 5, 1e-3))
    exact(fused[0], comp[0], "losses")
    exact(fused[1], comp[1], "weights")


def test_deferred_weight_grads_equal_immediate(eng):
    """The cfg3 character model with its narrow layers' weight-gradient products queued
    during backward and run in grouped launches before Adam (ehip_gemm_batch_f32): step-1
    gradients, losses and final weights equal, bit for bit, those of the same training
    with every product launched by its node."""
    import _compose as KC
    from workloads import CHARLM_CFG3
    b, s, vocab, d, heads, ff, layers = CHARLM_CFG3
    print_case("charlm deferred weight gradients", CHARLM_CFG3)
    r = np.random.default_rng(9)
    ids = r.integers(0, vocab, (b, s)).astype(np.int64)
    targets = r.integers(0, vocab, (b, s)).astype(np.int64)
    shapes = KC.charlm_param_shapes(vocab, d, ff, layers)
    params = np.concatenate([(randn(r, *shp) * np.float32(0.05)).ravel() for shp in shapes])
    runs = []
    prev = eng.set_deferred_weight_grads(True)
    try:
        for on in (True, False):
            eng.set_deferred_weight_grads(on)
            runs.append(eng.charlm_train(ids, targets, vocab, d, heads, ff, layers, params, 4,
                                         1e-3, grads0=True))
    finally:
        eng.set_deferred_weight_grads(prev)
    for got, want, what in zip(runs[0], runs[1], ("losses", "weights", "step-1 gradients")):
        exact(got, want, f"deferred {what}")


def _cfg3_case(seed):
    import _compose as KC
    from workloads import CHARLM_CFG3
    b, s, vocab, d, heads, ff, layers = CHARLM_CFG3
    r = np.random.default_rng(seed)
    ids = r.integers(0, vocab, (b, s)).astype(np.int64)
    targets = r.integers(0, vocab, (b, s)).astype(np.int64)
    shapes = KC.charlm_param_shapes(vocab, d, ff, layers)
    params = np.concatenate([(randn(r, *shp) * np.float32(0.05)).ravel() for shp in shapes])
    return ids, targets, (vocab, d, heads, ff, layers), params


def test_deferred_weight_grads_accumulate(eng):
    """Gradient accumulation: a second forward and backward adds into gradients the first
    left queued (the queue runs before the add reads them); the sums equal, bit for bit,
    those of the same two passes with every product launched by its node, and twice one
    pass's gradients within the rounding of one add."""
    ids, targets, dims, params = _cfg3_case(13)
    print_case("charlm deferred gradients accumulated over two passes")
    got = {}
    prev = eng.set_deferred_weight_grads(True)
    try:
        for on in (True, False):
            eng.set_deferred_weight_grads(on)
            got[on] = eng.charlm_accumulated_grads(ids, targets, *dims, params, 2)
        once = eng.charlm_accumulated_grads(ids, targets, *dims, params, 1)
    finally:
        eng.set_deferred_weight_grads(prev)
    exact(got[True], got[False], "accumulated gradients")
    assert np.all(np.isfinite(got[True]))
    np.testing.assert_allclose(got[True], 2 * once, rtol=1e-6, atol=1e-12)


def test_orphaned_weight_grad_products_touch_no_reused_memory(eng):
    """A character model whose backward queued its weight-gradient products is destroyed
    before anything reads its gradients; the queue runs at the next engine work, writing
    into buffers it owns and reading operands it keeps. Training a second model right after
    gives the same bits as the same training in a clean state."""
    ids, targets, dims, params = _cfg3_case(17)
    print_case("orphaned weight-gradient products")
    want_losses, want_p = eng.charlm_train(ids, targets, *dims, params, 3, 1e-3)
    eng.charlm_backward_orphan(ids, targets, *dims, params * np.float32(0.5))
    losses, out = eng.charlm_train(ids, targets, *dims, params, 3, 1e-3)
    exact(losses, want_losses, "losses")
    exact(out, want_p, "parameters")


def test_cnn_gradients_fused_vs_composed(eng):
    """cfg2 CNN, one backward: with fused nodes the conv weight sums are queued and run when
    Tensor::grad() reads them. Loss and Linear gradients are the bits of the node-by-node
    graph; the conv weight and bias gradients (another summation order) agree within the
    fp32 bound of their 64 x 28 x 28-term sums."""
    print_case("cnn grads fused vs composed")
    r = np.random.default_rng(2)
    x = r.uniform(0.0, 1.0, (64, 1, 28, 28)).astype(np.float32)
    labels = r.integers(0, 10, 64)
    parts = []
    for shp in K.cnn_param_shapes():  # Kaiming-uniform weights, small random biases
        if len(shp) == 1 or shp[0] == 1:
            parts.append(r.uniform(-0.1, 0.1, int(np.prod(shp))).astype(np.float32))
        else:
            fan_in = int(np.prod(shp[1:])) if len(shp) == 4 else shp[0]
            lim = np.sqrt(6.0 / fan_in)
            parts.append(r.uniform(-lim, lim, int(np.prod(shp))).astype(np.float32))
    params = np.concatenate(parts)
    fused, comp = both_graphs(eng, lambda: eng.cnn_grads(x, labels, params))
    exact(np.float32(fused[0]), np.float32(comp[0]), "loss")
    conv = 8 * 9 + 8 + 16 * 72 + 16
    exact(fused[1][conv:], comp[1][conv:], "linear gradients")
    ref_close(fused[1][:conv], comp[1][:conv], k_tol(64 * 28 * 28), "conv gradients")
    assert np.abs(fused[1][:conv]).max() > 0


@pytest.mark.parametrize("n,c", [(64, 10), (1024, 128), (2048, 121)])
def test_cross_entropy_fused_equals_composed(eng, n, c):
    """The loss as the root of backward: with fused nodes the forward launch also writes the
    logits' gradient and backward hands it over (small heads); the loss and gradient are the
    bits of the separate forward and backward kernels."""
    print_case("cross entropy fused vs composed", n, c)
    r = np.random.default_rng(n + c)
    logits = randn(r, n, c) * 2
    t = r.integers(0, c, n)
    fused, comp = both_graphs(eng, lambda: eng.cross_entropy(logits, t))
    exact(np.float32(fused[0]), np.float32(comp[0]), "loss")
    exact(fused[1], comp[1], "dlogits")


# ------------------------------------------------------- bias gradient from the dW product

@pytest.mark.parametrize("m,n,k", [(96, 96, 2048), (1024, 1024, 8192), (1024, 4096, 8192),
                                   (100, 257, 3000), (784, 10, 64), (384, 96, 2048),
                                   (4096, 1024, 8192)])
def test_colsum_from_dw_product(hip, m, n, k):
    """dW = X^T dY with colsum_b: the product is unchanged bit for bit, the
    column sums of dY match fp64 within the K-term tolerance and repeat
    exactly (split-K, unsplit, edge tiles, and the vector-kernel fallback)."""
    print_case("gemm_ex colsum", m, n, k)
    r = np.random.default_rng(m + n + k)
    x, g = dev(randn(r, k, m)), dev(randn(r, k, n))
    plain = hip.gemm(x, g, trans_a=True)
    c, cs = hip.f32((m, n)), hip.f32((n,))
    d = desc(hip, True, False, 1, 1, m, n, k, x, m, 0, 0, g, n, 0, 0, c, n, 0, 0)
    d.colsum_b = hip.p(cs)
    hip.gemm_ex(d)
    exact(host(c), host(plain), "product with column sums")
    want = host(g).astype(np.float64).sum(axis=0)
    ref_close(host(cs), want, 4 * k_tol(k), "column sums")
    first = host(cs).copy()
    hip.gemm_ex(d)
    exact(host(cs), first, "column sums repeat")


def test_panel_epilogue_and_repeat(hip):
    """A^T B over a long K into few 16 x 16 tiles (gemm_tn_panel, the weight gradients of
    narrow layers): alpha and beta applied after the waves' sums (C = alpha A^T B + beta C0,
    within the statistical fp32 bound of the fp64 product); the same call twice gives the
    same bits, and so does the first product again after products of other shapes."""
    import torch
    from _hip import gemm_stat_bound
    print_case("gemm panel epilogue")
    cases = [(96, 2048, 96), (100, 1500, 37), (384, 2048, 96), (96, 2048, 96)]
    first = None
    for i, (m, k, n) in enumerate(cases):
        g = torch.Generator(device="cuda").manual_seed(m + k + n)
        a = torch.randn(k, m, device="cuda", generator=g)
        b = torch.randn(k, n, device="cuda", generator=g)
        c0 = torch.randn(m, n, device="cuda", generator=g)
        outs = []
        for _ in range(2):
            c = c0.clone()
            hip.gemm_ex(desc(hip, True, False, 1, 1, m, n, k, a, m, 0, 0, b, n, 0, 0, c, n, 0, 0,
                             alpha=0.5, beta=1.0))
            outs.append(host(c))
        exact(outs[1], outs[0], f"panel {m}x{k}x{n} repeat")
        want = 0.5 * (a.double().t() @ b.double()) + c0.double()
        bound = 0.5 * gemm_stat_bound(a.double().norm(dim=0), b.double().norm(dim=0), k) + \
            2.0 ** -22 * want.abs()
        err = (torch.from_numpy(outs[0]).double().to(want.device) - want).abs()
        assert bool((err <= bound).all()), (m, k, n, float((err / bound).max()))
        if i == 0:
            first = outs[0]
        elif (m, k, n) == cases[0]:
            exact(outs[0], first, "panel after products of other shapes")


# (m, k, n, kind): narrow weight gradients with column sums (cfg3's layers), a ragged
# panel (checked tiles), alpha/beta and plain panels, ten of one kind (two launches of at
# most eight), and products that do not take the panel kernel (staged tiles, the
# thread-per-output kernel's column sum) mixed in.
BATCH_CASES = ([(96, 2048, 96, "colsum"), (96, 2048, 384, "colsum"), (384, 2048, 96, "colsum"),
                (96, 2048, 121, "colsum"), (100, 1500, 37, "plain"), (96, 4096, 96, "beta"),
                (1024, 1024, 1024, "plain"), (37, 50, 20, "colsum"), (100, 1500, 37, "beta")] +
               [(64 + 16 * i, 1024, 48, "colsum") for i in range(10)])


def test_gemm_batch_matches_single_calls(hip):
    """ehip_gemm_batch_f32 equals each product run on its own by ehip_gemm_ex_f32 bit for
    bit, outputs and column sums, whatever launches it groups them into;
    ehip_gemm_groupable says which descriptors take the panel kernel."""
    import ctypes as C
    from ehip import GemmEx
    import torch
    print_case("gemm_batch", len(BATCH_CASES), "products")
    gen = torch.Generator(device="cuda").manual_seed(23)
    singles, batch, outs = [], [], []
    for m, k, n, kind in BATCH_CASES:
        a = torch.randn(k, m, device="cuda", generator=gen)
        b = torch.randn(k, n, device="cuda", generator=gen)
        c0 = torch.randn(m, n, device="cuda", generator=gen)
        pair = []
        for _ in range(2):
            c, cs = c0.clone(), torch.full((n,), 7.0, device="cuda")
            beta = 1.0 if kind == "beta" else 0.0
            d = desc(hip, True, False, 1, 1, m, n, k, a, m, 0, 0, b, n, 0, 0, c, n, 0, 0,
                     alpha=0.5 if kind == "beta" else 1.0, beta=beta)
            if kind == "colsum":
                d.colsum_b = hip.p(cs)
            pair.append((d, c, cs))
        singles.append(pair[0][0])
        batch.append(pair[1][0])
        outs.append((pair[0][1:], pair[1][1:], (a, b), kind))
    groupable = [hip.lib.ehip_gemm_groupable(C.byref(d)) for d in batch]
    assert groupable == [1, 1, 1, 1, 1, 1, 0, 0, 1] + [1] * 10, groupable
    for d in singles:
        hip.gemm_ex(d)
    arr = (GemmEx * len(batch))(*batch)
    hip.ok(hip.lib.ehip_gemm_batch_f32(arr, len(batch), hip.stream()), "gemm_batch")
    for (m, k, n, kind), (one, together, _, _) in zip(BATCH_CASES, outs):
        exact(host(together[0]), host(one[0]), f"batched product {m}x{k}x{n} {kind}")
        if kind == "colsum":
            exact(host(together[1]), host(one[1]), f"batched column sums {m}x{k}x{n}")
    # Refusals come before anything runs: a bad descriptor anywhere in the list.
    bad = (GemmEx * 2)(batch[0], batch[1])
    bad[1].m = -1
    with pytest.raises(RuntimeError):
        hip.ok(hip.lib.ehip_gemm_batch_f32(bad, 2, hip.stream()), "gemm_batch")
    with pytest.raises(RuntimeError):
        hip.ok(hip.lib.ehip_gemm_batch_f32(arr, -1, hip.stream()), "gemm_batch")
    hip.ok(hip.lib.ehip_gemm_batch_f32(arr, 0, hip.stream()), "gemm_batch empty")


def test_gemm_batch_groups_k_sliced_products(hip):
    """Untransposed products small enough for the K-sliced tiles (the char model's
    projections: one input, several weights, a bias addend) run grouped by kernel form in
    ehip_gemm_batch_f32 with the bits of their own ehip_gemm_ex_f32 calls: whole and
    checked tiles, with and without the epilogue, slicing K over 2, 4 or 8 waves."""
    import ctypes as C
    from ehip import GemmEx
    import torch
    print_case("gemm_batch K-sliced")
    gen = torch.Generator(device="cuda").manual_seed(29)
    x = torch.randn(2048, 96, device="cuda", generator=gen)
    x2 = torch.randn(100, 384, device="cuda", generator=gen)
    x3 = torch.randn(2048, 192, device="cuda", generator=gen)  # four waves per tile
    cases = [(x, 96, True), (x, 96, True), (x, 96, True), (x, 384, True), (x, 96, False),
             (x2, 96, True), (x2, 37, False), (x2, 96, True), (x3, 96, True), (x3, 96, False)]
    keep, singles, batch = [], [], []
    for a, n, with_bias in cases:
        m, k = a.shape
        b = torch.randn(k, n, device="cuda", generator=gen)
        bias = torch.randn(n, device="cuda", generator=gen) if with_bias else None
        pair = []
        for _ in range(2):
            c = torch.full((m, n), 3.0, device="cuda")
            pair.append((desc(hip, False, False, 1, 1, m, n, k, a, k, 0, 0, b, n, 0, 0, c, n, 0, 0,
                              addend=bias, ld_add=0, period=1), c))
        keep.append((b, bias))
        singles.append(pair[0])
        batch.append(pair[1])
    for d, _ in singles:
        hip.gemm_ex(d)
    arr = (GemmEx * len(batch))(*[d for d, _ in batch])
    hip.ok(hip.lib.ehip_gemm_batch_f32(arr, len(batch), hip.stream()), "gemm_batch")
    for i, ((_, one), (_, together)) in enumerate(zip(singles, batch)):
        exact(host(together), host(one), f"K-sliced product {i} {cases[i][0].shape}x{cases[i][1]}")
    assert [hip.lib.ehip_gemm_groupable(C.byref(d)) for d, _ in batch] == [0] * len(batch)


def test_linear_backward_plan(hip):
    """ehip_linear_backward_plan: 1 for the mid-sized layers whose db the library takes from
    the dW product (cfg3's, more than 64 rows and dY of at most 2^21 elements), 0 for small,
    empty and wide ones (cfg5's), and 0 with the switch off."""
    print_case("linear_backward_plan")
    plan = hip.lib.ehip_linear_backward_plan
    assert plan(2048, 96, 96) == 1 and plan(2048, 96, 384) == 1 and plan(2048, 384, 96) == 1
    assert plan(64, 784, 10) == 0 and plan(0, 96, 96) == 0 and plan(2048, 0, 96) == 0
    assert plan(8192, 1024, 1024) == 0 and plan(8192, 1024, 4096) == 0
    prev = hip.lib.ehip_linear_bias_from_dw(0)
    try:
        assert plan(2048, 96, 96) == 0
    finally:
        hip.lib.ehip_linear_bias_from_dw(prev)


def test_colsum_refusals_and_k_zero(hip):
    print_case("gemm_ex colsum refusals")
    x = dev(np.ones((4, 4), np.float32))
    cs = dev(np.full(4, 7.0, np.float32))
    d = desc(hip, False, True, 1, 1, 4, 4, 4, x, 4, 0, 0, x, 4, 0, 0, hip.f32((4, 4)), 4, 0, 0)
    d.colsum_b = hip.p(cs)
    with pytest.raises(RuntimeError):  # B stored N x K
        hip.gemm_ex(d)
    d = desc(hip, False, False, 2, 1, 4, 4, 4, x, 4, 0, 0, x, 4, 0, 0, hip.f32((2, 4, 4)), 4, 16, 0)
    d.colsum_b = hip.p(cs)
    with pytest.raises(RuntimeError):  # batched
        hip.gemm_ex(d)
    c = hip.f32((4, 4))
    d = desc(hip, False, False, 1, 1, 4, 4, 0, x, 1, 0, 0, x, 4, 0, 0, c, 4, 0, 0)
    d.colsum_b = hip.p(cs)
    hip.gemm_ex(d)
    exact(host(cs), np.zeros(4, np.float32), "k = 0 column sums")


# ------------------------------------------------------- Linear backward in one call

@pytest.mark.parametrize("rows,inp,out", [(64, 784, 10), (64, 8, 10), (33, 100, 7),
                                          (2048, 96, 384), (300, 1024, 257), (100, 3, 20000)])
@pytest.mark.parametrize("want", [("dx", "dw", "db"), ("dw", "db"), ("dx",)])
def test_linear_backward_matches_separate_calls(hip, rows, inp, out, want):
    """ehip_linear_backward_f32 (one launch for small layers) equals the separate
    products and column sum bit for bit; a mid-sized layer's db (more than 64 rows, dy of
    at most 2^21 elements) is the column sum the dw product forms from its staged tiles
    (ehip_gemm_ex_f32's colsum_b) while ehip_linear_bias_from_dw is on (the default), and
    the separate column sum with it off."""
    print_case("linear_backward", rows, inp, out, want)
    r = np.random.default_rng(rows + inp + out + len(want))
    x = randn(r, rows, inp)
    x[x < -1.0] = 0.0  # zero-skip terms
    x, w, dy = dev(x), dev(randn(r, inp, out)), dev(randn(r, rows, out))
    from_dw = None  # asked from the library: the rule also depends on the dw product's plan
    for on in (1, 0):
        prev = hip.lib.ehip_linear_bias_from_dw(on)
        try:
            dx, dw, db = hip.linear_backward(x, w, dy, want)
        finally:
            hip.lib.ehip_linear_bias_from_dw(prev)
        if "dx" in want:
            exact(host(dx), host(hip.gemm(dy, w, trans_b=True)), "dx")
        if "dw" in want:
            exact(host(dw), host(hip.gemm(x, dy, trans_a=True)), "dw")
        if "db" not in want:
            continue
        if on and "dw" in want:
            # Where the column sums came from: equal to the separate sum, or to the dw
            # product's staged sums (which must then differ somewhere for these inputs).
            sep = host(hip.sum_axis(dy, 1, rows, out))
            from_dw = not np.array_equal(host(db), sep)
            if "db" in want and (rows, inp, out) == (2048, 96, 384):
                assert from_dw, "cfg3's feed-forward layer takes db from its dw product"
            if rows <= 64:
                assert not from_dw, "up to 64 rows db is the serial column sum"
            # The plan query an engine asks before queueing the product says the same
            # (where the sums differ; equal sums cannot tell the two paths apart).
            plan = hip.lib.ehip_linear_backward_plan(rows, inp, out)
            assert plan in (0, 1)
            if from_dw:
                assert plan == 1, "db came from the dw product, the plan said otherwise"
        if on and from_dw:
            cw, cs = hip.f32((inp, out)), hip.f32((out,))
            d = desc(hip, True, False, 1, 1, inp, out, rows, x, inp, 0, 0, dy, out, 0, 0, cw, out,
                     0, 0)
            d.colsum_b = hip.p(cs)
            hip.gemm_ex(d)
            exact(host(db), host(cs), "db from the dw product")
            exact(host(dw), host(cw), "dw of the column-sum product")
            ref_close(host(db), host(hip.sum_axis(dy, 1, rows, out)).astype(np.float64),
                      k_tol(rows), "db against the separate sum")
        else:
            exact(host(db), host(hip.sum_axis(dy, 1, rows, out)), "db")


# ------------------------------------------------------- causal skipping

@pytest.mark.parametrize("S,hd,bt", [(512, 64, 32), (256, 32, 64), (300, 64, 48)])
def test_causal_skipping_modes(hip, S, hd, bt):
    """ehip_gemm_ex_t::causal on batched head products: with P zero above the diagonal,
    P V (mode 2) and P^T G (mode 3) give the bits of the full products; Q K^T with the mask
    (mode 1, scale and mask in the epilogue) and G V^T (mode 1, no epilogue) give the full
    products' bits on and below the diagonal, and above it either those or the epilogue of
    zero (the mask value, or 0). 300 is not a multiple of the tiles (edge checks); the
    batch counts are large enough for every product to take the staged tiles."""
    print_case("causal modes", S, hd, bt)
    r = np.random.default_rng(S + hd)
    q, k, v, g = (randn(r, bt, S, hd) for _ in range(4))
    p = np.tril(np.abs(randn(r, bt, S, S)) / S).astype(np.float32)
    mask = np.triu(np.full((S, S), -1e9, np.float32), 1)
    Q, Kd, V, G, P, M = dev(q), dev(k), dev(v), dev(g), dev(p), dev(mask)
    ss, sh = S * S, S * hd
    below = np.tril(np.ones((S, S), bool))

    def run(ta, tb, m, n, kk, a, lda, sa, b, ldb, sb, sc, ldc, causal, **kw):
        c = hip.f32((bt, m, n))
        d = desc(hip, ta, tb, bt, 1, m, n, kk, a, lda, sa, 0, b, ldb, sb, 0, c, ldc, sc, 0, **kw)
        d.causal = causal
        hip.gemm_ex(d)
        return host(c)

    scale = 1.0 / math.sqrt(hd)
    s_full = run(False, True, S, S, hd, Q, hd, sh, Kd, hd, sh, ss, S, 0, alpha=scale,
                 addend=M, ld_add=S, stride_add=0, period=1)
    s_skip = run(False, True, S, S, hd, Q, hd, sh, Kd, hd, sh, ss, S, 1, alpha=scale,
                 addend=M, ld_add=S, stride_add=0, period=1)
    exact(s_skip[:, below], s_full[:, below], "scores on and below the diagonal")
    above = s_skip[:, ~below]
    assert np.all((above == s_full[:, ~below]) | (above == np.float32(-1e9))), "scores above"
    exact(run(False, False, S, hd, S, P, S, ss, V, hd, sh, sh, hd, 2),
          run(False, False, S, hd, S, P, S, ss, V, hd, sh, sh, hd, 0), "P V")
    exact(run(True, False, S, hd, S, P, S, ss, G, hd, sh, sh, hd, 3),
          run(True, False, S, hd, S, P, S, ss, G, hd, sh, sh, hd, 0), "P^T G")
    dp_full = run(False, True, S, S, hd, G, hd, sh, V, hd, sh, ss, S, 0)
    dp_skip = run(False, True, S, S, hd, G, hd, sh, V, hd, sh, ss, S, 1)
    exact(dp_skip[:, below], dp_full[:, below], "dP on and below the diagonal")
    above = dp_skip[:, ~below]
    assert np.all((above == dp_full[:, ~below]) | (above == 0)), "dP above"
    if S == 512:  # the staged tiles did skip: whole tiles above the diagonal hold the epilogue of 0
        assert np.all(s_skip[:, :128, 384:] == np.float32(-1e9))
        assert np.all(dp_skip[:, :128, 384:] == 0)
    # Mode 4: mode 1's values on and below the diagonal; above it, tiles the staged
    # kernels skip keep what C held (a sentinel here), the others mode 1's values.
    sentinel = np.float32(12345.0)

    def run4(a, b, **kw):
        c = dev(np.full((bt, S, S), sentinel, np.float32))
        d = desc(hip, False, True, bt, 1, S, S, hd, a, hd, sh, 0, b, hd, sh, 0, c, S, ss, 0, **kw)
        d.causal = 4
        hip.gemm_ex(d)
        return host(c)

    for got, want, what in ((run4(Q, Kd, alpha=scale, addend=M, ld_add=S, stride_add=0,
                                  period=1), s_skip, "scores"),
                            (run4(G, V), dp_skip, "dP")):
        exact(got[:, below], want[:, below], f"{what} (mode 4) on and below the diagonal")
        assert np.all((got[:, ~below] == want[:, ~below]) | (got[:, ~below] == sentinel)), what
        if S == 512:
            assert np.all(got[:, :128, 384:] == sentinel), f"{what}: whole tiles not stored"
    with pytest.raises(RuntimeError, match="causal"):
        run(False, False, S, hd, S, P, S, ss, V, hd, sh, sh, hd, 5)


@pytest.mark.parametrize("S,mats", [(512, 8), (64, 40), (300, 3), (1, 5), (2048, 2), (2050, 2)])
def test_causal_softmax_matches_full(hip, S, mats):
    """The causal softmax pair reads each row only up to the diagonal: on scores whose
    masked entries are -1e9 + q.k (as the score product writes them), the forward equals
    ehip_softmax_f32 bit for bit, and the scaled backward with y from it equals
    ehip_softmax_backward_scaled_f32 by value (a masked output's zero may differ in sign);
    a row count that is not a whole number of matrices is refused."""
    print_case("causal softmax", S, mats)
    r = np.random.default_rng(S + mats)
    x = randn(r, mats, S, S) * 3
    x = np.where(np.triu(np.ones((S, S), bool), 1), x + np.float32(-1e9), x).astype(np.float32)
    X = dev(x)
    rows = mats * S
    full = hip.softmax(X)
    y = hip.f32(X.shape)
    hip.ok(hip.lib.ehip_softmax_causal_f32(hip.p(X), hip.p(y), rows, S, hip.stream()), "causal")
    exact(host(y), host(full), "forward")
    g = dev(randn(r, mats, S, S))
    want = hip.softmax_backward(full, g, scale=0.125)
    got = hip.f32(X.shape)
    hip.ok(hip.lib.ehip_softmax_backward_scaled_causal_f32(hip.p(y), hip.p(g), hip.p(got), rows,
                                                           S, 0.125, hip.stream()), "causal bwd")
    assert np.array_equal(host(got), host(want)), "backward values"
    if S > 1:
        with pytest.raises(RuntimeError, match="whole"):
            hip.ok(hip.lib.ehip_softmax_causal_f32(hip.p(X), hip.p(y), rows - 1, S,
                                                   hip.stream()), "causal")


@pytest.mark.parametrize("S,mats", [(64, 3), (300, 2), (2050, 2)])
def test_causal_softmax_reads_only_the_triangle(hip, S, mats):
    """Masked entries (right of the diagonal) are not read by the causal pair, on the
    register path (S <= 2048) and on the looped one (2050: more than 2048 columns, not a
    multiple of 4): with NaN planted there in x and g, both outputs equal those computed
    from the -1e9 scores, and the masked outputs are zeros."""
    print_case("causal softmax unread", S, mats)
    r = np.random.default_rng(S * 3 + mats)
    upper = np.triu(np.ones((S, S), bool), 1)
    x = randn(r, mats, S, S) * 3
    g = randn(r, mats, S, S)
    rows = mats * S

    def run(xv, gv):
        X, G = dev(xv), dev(gv)
        y, dx = hip.f32(X.shape), hip.f32(X.shape)
        hip.ok(hip.lib.ehip_softmax_causal_f32(hip.p(X), hip.p(y), rows, S, hip.stream()),
               "causal")
        hip.ok(hip.lib.ehip_softmax_backward_scaled_causal_f32(
            hip.p(y), hip.p(G), hip.p(dx), rows, S, 0.25, hip.stream()), "causal bwd")
        return host(y), host(dx)

    y_mask, dx_mask = run(np.where(upper, x + np.float32(-1e9), x).astype(np.float32), g)
    y_nan, dx_nan = run(np.where(upper, np.float32(np.nan), x).astype(np.float32),
                        np.where(upper, np.float32(np.nan), g).astype(np.float32))
    exact(y_nan, y_mask, "forward with NaN in the masked entries")
    assert np.array_equal(dx_nan, dx_mask), "backward with NaN in the masked entries"
    assert np.all(y_nan[:, upper] == 0) and np.all(dx_nan[:, upper] == 0), "masked outputs"
    assert np.all(np.isfinite(y_nan)) and np.all(np.isfinite(dx_nan))


@pytest.mark.parametrize("b,s,d,heads", [(8, 512, 512, 8), (2, 64, 96, 4), (16, 300, 128, 2),
                                         (1, 2050, 64, 2)])
def test_mha_causal_mask_skipping_keeps_values(eng, b, s, d, heads):
    """The fused attention node under nn::causal_mask (whose score tiles above the diagonal,
    the products with the weights past it and the matching backward products are skipped)
    against the same mask values in a plain tensor (every product computed): outputs,
    input and parameter gradients and attention weights hold the same values (the sign of
    an exactly zero sum aside, which compares equal)."""
    print_case("mha causal skipping", b, s, d, heads)
    r = np.random.default_rng(b * 7 + s + d + heads)
    x, dy = randn(r, b, s, d), randn(r, b, s, d)
    params = mha_params(r, d)
    prev = eng.set_short_attention(False)  # the product path's skipping (short: its own test)
    try:
        tagged = eng.mha_causal_fwd_bwd(x, heads, params, dy, tagged=True)
        plain = eng.mha_causal_fwd_bwd(x, heads, params, dy, tagged=False)
    finally:
        eng.set_short_attention(prev)
    for got, want, what in zip(tagged, plain, ("y", "dx", "dparams", "weights")):
        assert np.array_equal(got, want), f"{what}: {np.sum(got != want)} values differ"


def unflatten_mha(params, d):
    names = ("wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo")
    shapes = [(d, d), (1, d)] * 4
    p, off = {}, 0
    for name, shp in zip(names, shapes):
        n = int(np.prod(shp))
        p[name] = params[off:off + n].reshape(shp)
        off += n
    return p, names, shapes


@pytest.mark.parametrize("b,s,d,heads,causal", [(32, 64, 96, 4, True), (2, 64, 96, 4, False),
                                                (3, 37, 48, 2, True), (4, 64, 256, 4, True)])
def test_short_attention_node(eng, orc, b, s, d, heads, causal):
    """The attention node with sequences and heads of at most 64 values takes one launch per
    direction (nn::set_short_attention, the default; with nn::causal_mask's tagged mask or
    none); the same node through the batched products is the bit-tested path above. Both
    against the reference composition run by the oracle: the short path sums in the
    reference's order, so it meets the reference's metric at 1e-5 where the products are
    held to 4 k_tol; every parameter gradient too."""
    print_case("short attention node", b, s, d, heads, causal)
    r = np.random.default_rng(b * 11 + s + d + heads + causal)
    x, dy = randn(r, b, s, d), randn(r, b, s, d)
    params = mha_params(r, d)
    mask = np.triu(np.full((s, s), -1e9, np.float32), 1) if causal else None

    def run(short):
        prev = eng.set_short_attention(short)
        prev_db = eng.set_fused_bias_grad(False)
        try:
            if causal:
                return eng.mha_causal_fwd_bwd(x, heads, params, dy, tagged=True)
            return eng.mha_fwd_bwd(x, heads, params, dy, mask=None, fuse=True, weights=True)
        finally:
            eng.set_short_attention(prev)
            eng.set_fused_bias_grad(prev_db)

    short, prod = run(True), run(False)
    p, names, shapes = unflatten_mha(params, d)
    y, cache = K.mha_fwd(orc, x, p, heads, mask)
    dx, grads = K.mha_bwd(orc, dy, cache)
    for name, got_s, got_p, w in (("y", short[0], prod[0], y), ("dx", short[1], prod[1], dx)):
        es, ep = ref_err(got_s, w), ref_err(got_p, w)
        print(f"{name}: short {es:.2e}, products {ep:.2e}")
        assert es <= k_tol(max(s, d)), (name, es)
    off = 0
    for name, shp in zip(names, shapes):
        n = int(np.prod(shp))
        es = ref_err(short[2][off:off + n].reshape(shp), grads[name])
        assert es <= k_tol(b * s), (name, es)
        off += n
    w_ref = cache[3][3]
    assert ref_err(short[3], w_ref) <= 1e-5
