"""The kernels behind Tensor::max(axis), slice / concat / stack and nn::Sigmoid / Tanh /
GELU (ehip_max_axis_f32, ehip_copy_rows_f32, ehip_activation_f32 and their backward
entry points), against the reference's definitions (src/tensor.cpp:383-552,
src/nn.cpp:154-198).

The moves and the maximum are bit-exact: the copy against numpy slicing, the maximum and
its index against a scan in axis order with the reference's strict > (a leading NaN stays
the maximum, a later NaN is never taken, ties keep the first). The activations use the
device's expf / tanhf, which may differ from the host's by a few ulp: the forward and
backward are checked against the same expressions in float64, within 2e-6 relative plus
the fp32 rounding of the terms that cancel (1 + tanh near -1 in GELU, 1 - y^2 and 1 - y
in the derivatives: 4 ulp of the term's size), far below the 1e-4 at which the
reference's PyTorch fixtures hold these layers (checked by its own suite,
tests/test_dropin.py). A wrong branch of the stable sigmoid, a dropped cube term in
GELU or a transposed derivative moves values by orders of magnitude more."""
import ctypes

import numpy as np
import pytest

from _hip import backend, dev, exact, host, print_case

pytestmark = pytest.mark.gpu

ALPHA = np.float64(np.float32(0.7978845608028654))
BETA = np.float64(np.float32(0.044715))


@pytest.fixture(scope="module")
def hip():
    return backend()


def act64(kind, x):
    x = x.astype(np.float64)
    if kind == 0:
        return np.where(x >= 0, 1.0 / (1.0 + np.exp(-x)), np.exp(x) / (1.0 + np.exp(x)))
    if kind == 1:
        return np.tanh(x)
    return 0.5 * x * (1.0 + np.tanh(ALPHA * (x + BETA * x ** 3)))


def dact64(kind, x, y):
    x, y = x.astype(np.float64), y.astype(np.float64)
    if kind == 0:
        return y * (1.0 - y)
    if kind == 1:
        return 1.0 - y * y
    t = np.tanh(ALPHA * (x + BETA * x ** 3))
    return 0.5 * (1.0 + t) + 0.5 * x * (1.0 - t * t) * ALPHA * (1.0 + 3.0 * BETA * x * x)


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("n", [1, 7, 4096, 100003])
def test_activation_forward_backward(hip, kind, n):
    print_case("activation", kind, n)
    r = np.random.default_rng(kind * 10 + n)
    x = (r.standard_normal(n) * 4).astype(np.float32)
    x[: min(n, 6)] = np.array([0.0, -0.0, 30.0, -30.0, 100.0, -100.0], np.float32)[: min(n, 6)]
    g = r.standard_normal(n).astype(np.float32)
    X, G = dev(x), dev(g)
    Y, DX = hip.f32((n,)), hip.f32((n,))
    hip.ok(hip.lib.ehip_activation_f32(kind, hip.p(X), hip.p(Y), n, None), "activation")
    y = host(Y)
    want = act64(kind, x)
    ulp4 = 4 * 2.0 ** -24
    x64 = np.abs(x.astype(np.float64))
    cancel = x64 if kind == 2 else 0.0  # 0.5 x (1 + tanh): the sum's rounding, times |x|
    assert np.all(np.abs(y - want) <= 2e-6 * np.abs(want) + ulp4 * cancel + 1e-30), kind
    hip.ok(hip.lib.ehip_activation_backward_f32(kind, hip.p(X), hip.p(Y), hip.p(G), hip.p(DX), n,
                                                None), "activation backward")
    dx = host(DX)
    dwant = g.astype(np.float64) * dact64(kind, x, y)  # the derivative at the stored y
    ga = np.abs(g.astype(np.float64))
    if kind == 0:
        cancel = ga * np.abs(y)  # y (1 - y)
    elif kind == 1:
        cancel = ga  # 1 - y^2
    else:
        cancel = ga * (1.0 + x64 * ALPHA * (1.0 + 3.0 * BETA * x64 * x64))
    assert np.all(np.abs(dx - dwant) <= 2e-6 * np.abs(dwant) + ulp4 * cancel + 1e-30), kind
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(dx))


def test_activation_refusals(hip):
    X = dev(np.zeros(4, np.float32))
    with pytest.raises(RuntimeError):
        hip.ok(hip.lib.ehip_activation_f32(3, hip.p(X), hip.p(X), 4, None), "kind")
    with pytest.raises(RuntimeError):
        hip.ok(hip.lib.ehip_activation_backward_f32(0, hip.p(X), None, hip.p(X), hip.p(X), 4,
                                                    None), "null")


@pytest.mark.parametrize("shape,axis,start,count", [((6, 5, 7), 1, 1, 3), ((4, 1024), 1, 256, 512),
                                                    ((3, 9), 0, 2, 1), ((2, 3, 4, 5), 3, 4, 1),
                                                    ((5, 333), 1, 3, 301)])
def test_copy_rows_slices_exactly(hip, shape, axis, start, count):
    """A slice and its scatter back (the forward and backward of Tensor::slice) as the
    engine issues them: per outer index, count x inner floats."""
    print_case("copy_rows", shape, axis, start, count)
    r = np.random.default_rng(len(shape) + start)
    x = r.standard_normal(shape).astype(np.float32)
    outer = int(np.prod(shape[:axis])) if axis else 1
    inner = int(np.prod(shape[axis + 1:])) if axis + 1 < len(shape) else 1
    L = shape[axis]
    X = dev(x)
    Y = hip.f32((outer * count * inner,))
    hip.ok(hip.lib.ehip_copy_rows_f32(ctypes.c_void_p(X.data_ptr() + 4 * start * inner), L * inner,
                                      hip.p(Y), count * inner, outer, count * inner, None), "slice")
    want = np.take(x, range(start, start + count), axis=axis)
    exact(host(Y).reshape(want.shape), want, "slice")
    D = dev(np.zeros(shape, np.float32))
    hip.ok(hip.lib.ehip_copy_rows_f32(hip.p(Y), count * inner,
                                      ctypes.c_void_p(D.data_ptr() + 4 * start * inner), L * inner,
                                      outer, count * inner, None), "scatter")
    back = np.zeros(shape, np.float32)
    idx = [slice(None)] * len(shape)
    idx[axis] = slice(start, start + count)
    back[tuple(idx)] = want
    exact(host(D), back, "slice backward")
    with pytest.raises(RuntimeError):
        hip.ok(hip.lib.ehip_copy_rows_f32(hip.p(X), 1, hip.p(Y), 8, 2, 4, None), "pitch < len")


def max_scan(x3):
    """The reference's scan: first element, then strictly greater ones, in axis order."""
    outer, A, inner = x3.shape
    y = np.empty((outer, inner), np.float32)
    arg = np.empty((outer, inner), np.int32)
    for o in range(outer):
        for i in range(inner):
            best, ba = x3[o, 0, i], 0
            for a in range(1, A):
                if x3[o, a, i] > best:
                    best, ba = x3[o, a, i], a
            y[o, i], arg[o, i] = best, ba
    return y, arg


@pytest.mark.parametrize("outer,A,inner", [(3, 5, 4), (1, 300, 1), (7, 1, 9), (2, 64, 33)])
def test_max_axis_exact(hip, outer, A, inner):
    print_case("max_axis", outer, A, inner)
    r = np.random.default_rng(outer * A + inner)
    x = r.integers(-3, 4, (outer, A, inner)).astype(np.float32)  # many ties
    x[0, 0, 0] = np.nan  # a leading NaN stays the maximum
    if A > 2:
        x[-1, 1, -1] = np.nan  # a later NaN is never taken
    y, arg = max_scan(x)
    X = dev(x)
    Y = hip.f32((outer, inner))
    import torch
    ARG = torch.empty((outer, inner), dtype=torch.int32, device="cuda")
    hip.ok(hip.lib.ehip_max_axis_f32(hip.p(X), hip.p(Y), ARG.data_ptr(), outer, A, inner, None),
           "max_axis")
    exact(host(Y), y, "maximum")
    np.testing.assert_array_equal(ARG.cpu().numpy(), arg)
    g = r.standard_normal((outer, inner)).astype(np.float32)
    g[0, 0] = -0.0
    DX = hip.f32((outer, A, inner))
    hip.ok(hip.lib.ehip_max_axis_backward_f32(hip.p(dev(g)), ARG.data_ptr(), hip.p(DX), outer, A,
                                              inner, None), "max_axis backward")
    want = np.zeros((outer, A, inner), np.float32)
    for o in range(outer):
        for i in range(inner):
            want[o, arg[o, i], i] = np.float32(0.0) + g[o, i]
    exact(host(DX), want, "max backward")
    assert not np.signbit(host(DX)[0, arg[0, 0], 0]), "0 + g turns -0 into +0"
