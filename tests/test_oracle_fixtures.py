"""Pins the CPU restatement against the reference's PyTorch-replay fixtures.

Each case mirrors one test of the reference's tests/test_reference.cpp (the line ranges are
given per test) and uses its tolerances: 1e-4 absolute, 2e-4 for the optimiser trajectories.
Fixtures for ops off the training path (sigmoid, tanh, GELU, SGD) are replayed where the
oracle has the op, and listed as out of scope otherwise.
"""
import math

import numpy as np
import pytest

import _compose as K
from _fixtures import ALL, load
from _oracle import oracle_or_skip

TOL = 1e-4


@pytest.fixture(scope="module")
def orc():
    return oracle_or_skip()


def close(got, want, tol=TOL):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, (got.shape, want.shape)
    dev = float(np.max(np.abs(got - want))) if got.size else 0.0
    assert dev <= tol, f"largest deviation {dev:.3e} > {tol}"


def test_all_fixtures_parse():
    assert len(ALL) == 23
    for name in ALL:
        assert load(name), name


# tests/test_reference.cpp:97-114
@pytest.mark.parametrize("name", ["matmul", "matmul_batched", "matmul_shared"])
def test_matmul(orc, name):
    f = load(name)
    c, da, db = K.matmul_fwd_bwd(orc, f["a"], f["b"], f["grad_output"])
    close(c, f["output"])
    close(da, f["grad.a"])
    close(db, f["grad.b"])


# tests/test_reference.cpp:116-130
@pytest.mark.parametrize("name", ["softmax", "softmax_3d"])
def test_softmax(orc, name):
    f = load(name)
    y = orc.softmax(f["input"])
    close(y, f["output"])
    close(orc.softmax_backward(y, f["grad_output"]), f["grad.input"])


# tests/test_reference.cpp:132-158 (ReLU only: sigmoid/tanh/GELU are off the path)
def test_relu(orc):
    f = load("act_relu")
    close(orc.relu(f["input"]), f["output"])
    close(orc.relu_backward(f["input"], f["grad_output"]), f["grad.input"])


# tests/test_reference.cpp:160-188 (sum and mean along an axis)
@pytest.mark.parametrize("tag,axis,op", [("sum0", 0, "sum"), ("sum1", 1, "sum"),
                                         ("mean1", 1, "mean")])
def test_reductions(orc, tag, axis, op):
    f = load("reductions")
    x = f["input"]
    y = orc.sum_axis(x, axis)
    g = f["grad_output." + tag]
    if op == "mean":
        scale = np.float32(1.0) / np.float32(x.shape[axis])
        y = orc.scalar_mul(y, scale)
        g = orc.scalar_mul(g, scale)
    close(y, f["output." + tag])
    dx = np.broadcast_to(np.expand_dims(g, axis), x.shape)
    close(dx, f["grad." + tag])


# tests/test_reference.cpp:194-214
@pytest.mark.parametrize("name", ["linear", "linear_3d"])
def test_linear(orc, name):
    f = load(name)
    y, cache = K.linear_fwd(orc, f["input"], f["weight"], f["bias"])
    close(y, f["output"])
    dx, dw, db = K.linear_bwd(orc, f["grad_output"], cache)
    close(dx, f["grad.input"])
    close(dw, f["grad.weight"])
    close(db, f["grad.bias"])


# tests/test_reference.cpp:216-242
@pytest.mark.parametrize("name,stride,pad", [("conv2d_pad1", 1, 1), ("conv2d_stride2", 2, 0)])
def test_conv2d(orc, name, stride, pad):
    f = load(name)
    y, cache = K.conv2d_fwd(orc, f["input"], f["weight"], f["bias"], stride, pad)
    close(y, f["output"])
    dx, dw, db = K.conv2d_bwd(orc, f["grad_output"], cache)
    close(dx, f["grad.input"])
    close(dw, f["grad.weight"])
    close(db, f["grad.bias"])


# tests/test_reference.cpp:244-250
def test_maxpool(orc):
    f = load("maxpool2d")
    y, cache = K.maxpool_fwd(orc, f["input"], 2, 2)
    close(y, f["output"], 0.0)
    close(K.maxpool_bwd(orc, f["grad_output"], cache), f["grad.input"], 0.0)


# tests/test_reference.cpp:253-268
def test_layernorm(orc):
    f = load("layernorm")
    y, cache = K.layernorm_fwd(orc, f["input"], f["gamma"], f["beta"])
    close(y, f["output"])
    dx, dg, db = K.layernorm_bwd(orc, f["grad_output"], cache)
    close(dx, f["grad.input"])
    close(dg, f["grad.gamma"])
    close(db, f["grad.beta"])


# tests/test_reference.cpp:270-289
def test_cross_entropy(orc):
    f = load("cross_entropy")
    t = f["targets"].astype(np.int64)
    loss, probs = orc.cross_entropy(f["logits"], t)
    close(np.float32(loss).reshape(f["output"].shape), f["output"])
    close(orc.cross_entropy_backward(probs, t, 1.0), f["grad.logits"])


# tests/test_reference.cpp:295-319
@pytest.mark.parametrize("name", ["attention", "attention_causal"])
def test_attention(orc, name):
    f = load(name)
    mask = f["mask"] if name == "attention_causal" else None
    y, cache = K.attention_fwd(orc, f["q"], f["k"], f["v"], mask)
    close(y, f["output"])
    close(cache[3], f["weights"])
    dq, dk, dv = K.attention_bwd(orc, f["grad_output"], cache)
    close(dq, f["grad.q"])
    close(dk, f["grad.k"])
    close(dv, f["grad.v"])


# tests/test_reference.cpp:321-348
def test_multihead_attention(orc):
    f = load("multihead_attention")
    p = {}
    for tag, k in (("query", "q"), ("key", "k"), ("value", "v"), ("out", "o")):
        p["w" + k] = f[f"w.{tag}.weight"]
        p["b" + k] = f[f"w.{tag}.bias"]
    y, cache = K.mha_fwd(orc, f["input"], p, 2, None)
    close(y, f["output"])
    dx, g = K.mha_bwd(orc, f["grad_output"], cache)
    close(dx, f["grad.input"])
    for tag, k in (("query", "q"), ("key", "k"), ("value", "v"), ("out", "o")):
        close(g["w" + k], f[f"grad.{tag}.weight"])
        close(g["b" + k], f[f"grad.{tag}.bias"])


BLOCK_NAMES = ["norm1.gamma", "norm1.beta", "norm2.gamma", "norm2.beta", "query.weight",
               "query.bias", "key.weight", "key.bias", "value.weight", "value.bias",
               "out.weight", "out.bias", "ff1.weight", "ff1.bias", "ff2.weight", "ff2.bias"]


# tests/test_reference.cpp:350-377
def test_transformer_block(orc):
    f = load("transformer_block")
    p = {k: f["w." + n] for k, n in zip(K.BLOCK_KEYS, BLOCK_NAMES)}
    y, cache = K.block_fwd(orc, f["input"], p, 2, None)
    close(y, f["output"])
    dx, g = K.block_bwd(orc, f["grad_output"], cache)
    close(dx, f["grad.input"])
    for k, n in zip(K.BLOCK_KEYS, BLOCK_NAMES):
        close(g[k], f["grad." + n])


def _mse_grad(orc, w, target):
    """d/dw of mean((w - target)^2) through the reference graph: sub, mul, sum, scalar mul."""
    diff = orc.binary("sub", w, target)
    n = diff.size
    gs = np.full(diff.shape, np.float32(1.0) * (np.float32(1.0) / np.float32(n)), np.float32)
    half = orc.binary("mul", gs, diff)
    return orc.binary("add", half, half)


# tests/test_reference.cpp:387-406
def test_adam_trajectory(orc):
    f = load("adam")
    w = f["initial"].copy()
    opt = K.AdamState([w], 0.1)
    for step in range(10):
        g = _mse_grad(orc, w, f["target"])
        opt.step(orc, [w], [g])
        close(w, f[f"step.{step}"], 2e-4)


# tests/test_reference.cpp:407-422 (SGD is off the path; kept because the oracle has it)
def test_sgd_momentum_trajectory(orc):
    f = load("sgd_momentum")
    w = f["initial"].copy()
    vel = np.zeros_like(w)
    for step in range(10):
        g = _mse_grad(orc, w, f["target"])
        orc.sgd(w, g, vel, 0.05, 0.9, 0.0)
        close(w, f[f"step.{step}"], 2e-4)


def test_positional_encoding_closed_form(orc):
    pe = orc.positional_encoding(16, 8)
    pos = np.arange(16)[:, None].astype(np.float64)
    i = np.arange(8)[None, :]
    ang = pos / np.power(10000.0, 2.0 * (i // 2) / 8.0)
    want = np.where(i % 2 == 0, np.sin(ang), np.cos(ang))
    assert np.max(np.abs(pe - want)) < 1e-5


def test_causal_mask_closed_form(orc):
    m = orc.causal_mask(5)
    assert np.array_equal(m, np.triu(np.full((5, 5), -1e9, np.float32), 1))


# Random123's published known-answer vectors for Philox4x32-10 (counter, key, output).
PHILOX_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff, 0xffffffff), (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_known_answers(orc, ctr, key, want):
    assert tuple(int(v) for v in orc.philox(ctr, key)) == want


def test_dropout_oracle_properties(orc):
    """The dropout restatement: the keep rate is binomial around 1 - p (5 sigma), kept
    values are x / keep exactly, dropped ones 0, and the mask depends only on the counter
    (a call at offset k equals the tail of a call at 0)."""
    r = np.random.default_rng(5)
    n, p = 1 << 20, 0.3
    x = r.standard_normal(n).astype(np.float32)
    y, m = orc.dropout(x, p, seed=1234, offset=0)
    keep = np.float32(1.0) - np.float32(p)
    scale = np.float32(1.0) / keep
    kept = m != 0
    sigma = np.sqrt(n * keep * (1 - keep))
    assert abs(kept.sum() - n * keep) < 5 * sigma
    assert np.all(m[kept] == scale)
    np.testing.assert_array_equal(y, (x * m).astype(np.float32))
    y2, m2 = orc.dropout(x[37:], p, seed=1234, offset=37)
    np.testing.assert_array_equal(m2, m[37:])
    _, m3 = orc.dropout(x, p, seed=1235, offset=0)
    assert (m3 != m).mean() > 0.3  # another seed, another mask
