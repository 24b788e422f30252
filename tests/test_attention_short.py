"""Attention of short sequences in one launch per direction (csrc/attention.hip,
ehip_attention_short_f32 / _backward_f32) against the reference composition run by the oracle
(tests/_compose.py: scores = Q K^T * scale + mask, softmax, weights V, and the backward of
each node, src/transformer.cpp:279-304): weights, output and dq, dk, dv within the reference's
metric at 1e-5 (the kernels sum in the reference's order, so only the device exp differs);
masked weights exactly 0; heads addressed in place in (batch, seq, width) activations; zero
entries (the reference's zero skip) and the refusal of sequences beyond 64."""
import math

import numpy as np
import pytest

import _compose as K
from _hip import backend, dev, host, print_case, ref_err
from _oracle import oracle_or_skip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    return backend()


@pytest.fixture(scope="module")
def orc():
    return oracle_or_skip()


def split(t, heads):
    b, s, w = t.shape
    return np.ascontiguousarray(t.reshape(b, s, heads, w // heads).transpose(0, 2, 1, 3))


def merge(t):
    b, h, s, hd = t.shape
    return np.ascontiguousarray(t.transpose(0, 2, 1, 3).reshape(b, s, h * hd))


@pytest.mark.parametrize("b,s,heads,hd,causal", [(32, 64, 4, 24, True), (32, 64, 4, 24, False),
                                                 (3, 37, 2, 8, True), (2, 17, 1, 64, False),
                                                 (4, 1, 3, 5, True), (2, 64, 2, 64, True),
                                                 (5, 9, 3, 3, False)])
def test_attention_short_vs_reference(hip, orc, b, s, heads, hd, causal):
    print_case("attention short", b, s, heads, hd, causal)
    r = np.random.default_rng(b * 1000 + s * 10 + hd + causal)
    w = heads * hd
    q, k, v, g = (r.standard_normal((b, s, w), dtype=np.float32) for _ in range(4))
    q[:, ::3, ::5] = 0.0  # the reference skips zero A operands
    g[:, 1::4, ::3] = 0.0
    scale = 1.0 / math.sqrt(hd)
    mask = np.triu(np.full((s, s), -1e9, np.float32), 1) if causal else None
    out_ref, cache = K.attention_fwd(orc, split(q, heads), split(k, heads), split(v, heads), mask)
    dq_ref, dk_ref, dv_ref = K.attention_bwd(orc, split(g, heads), cache)
    Q, Kd, V, G = dev(q), dev(k), dev(v), dev(g)
    weights, out = hip.attention_short(Q, Kd, V, heads, np.float32(scale), causal)
    dq, dk, dv = hip.attention_short_backward(Q, Kd, V, weights, G, heads, np.float32(scale), causal)
    wts = host(weights)
    errs = {"weights": ref_err(wts, cache[3]), "out": ref_err(host(out), merge(out_ref)),
            "dq": ref_err(host(dq), merge(dq_ref)), "dk": ref_err(host(dk), merge(dk_ref)),
            "dv": ref_err(host(dv), merge(dv_ref))}
    print("worst reference-metric errors:", {k_: f"{e:.1e}" for k_, e in errs.items()})
    for name, e in errs.items():
        assert e <= 1e-5, (name, e)
    if causal:
        assert np.all(wts[..., np.triu(np.ones((s, s), bool), 1)] == 0.0)
    # Skipping outputs leaves the others as they were.
    only_v = hip.attention_short_backward(Q, Kd, V, weights, G, heads, np.float32(scale), causal,
                                          want=(False, False, True))
    assert only_v[0] is None and np.array_equal(host(only_v[2]), host(dv))


def test_attention_short_refusals(hip):
    print_case("attention short refusals")
    x = dev(np.zeros((1, 65, 8), np.float32))
    assert hip.lib.ehip_attention_short_supported(64, 64) == 1
    assert hip.lib.ehip_attention_short_supported(65, 8) == 0
    assert hip.lib.ehip_attention_short_supported(8, 65) == 0
    before = hip.launched()
    with pytest.raises(RuntimeError, match="exceed"):
        hip.attention_short(x, x, x, 1, 1.0, True)
    assert hip.launched() == before


def test_attention_short_nonfinite_operands(hip, orc):
    """The reference skips zero A terms (src/tensor_ops.cpp:553-560), which matters only
    when the other operand is not finite: a key whose score underflows exp (weight exactly
    0) facing a V row of +inf leaves the output finite in the reference, where a plain
    multiply-add would make it NaN. The kernels take the exact path when an operand of a
    product is not finite; the backward, whose dP row meets inf * 0, is NaN where the
    reference's is and equal elsewhere."""
    print_case("attention short non-finite")
    r = np.random.default_rng(77)
    b, s, heads, hd = 2, 16, 2, 8
    w = heads * hd
    q, k, v, g = (r.standard_normal((b, s, w), dtype=np.float32) for _ in range(4))
    q[:, :, :hd] = 1.0 + np.abs(q[:, :, :hd])   # head 0: every query positive ...
    k[:, 3, :hd] = -50.0                        # ... so key 3's scores underflow exp
    v[:, 3, :hd] = np.inf
    scale = 1.0 / math.sqrt(hd)
    out_ref, cache = K.attention_fwd(orc, split(q, heads), split(k, heads), split(v, heads), None)
    dq_ref, dk_ref, dv_ref = K.attention_bwd(orc, split(g, heads), cache)
    assert np.all(cache[3][:, 0, :, 3] == 0.0) and np.all(np.isfinite(out_ref))
    Q, Kd, V, G = dev(q), dev(k), dev(v), dev(g)
    weights, out = hip.attention_short(Q, Kd, V, heads, np.float32(scale), False)
    dq, dk, dv = hip.attention_short_backward(Q, Kd, V, weights, G, heads, np.float32(scale),
                                              False)
    assert ref_err(host(weights), cache[3]) <= 1e-5
    assert np.all(np.isfinite(host(out))) and ref_err(host(out), merge(out_ref)) <= 1e-5
    for name, got, want in (("dq", host(dq), merge(dq_ref)), ("dk", host(dk), merge(dk_ref)),
                            ("dv", host(dv), merge(dv_ref))):
        assert np.array_equal(np.isnan(got), np.isnan(want)), name
        assert np.array_equal(np.isinf(got), np.isinf(want)), name
        fin = np.isfinite(want)
        assert ref_err(got[fin], want[fin]) <= 1e-5, name
