"""The implicit-GEMM convolution (ehip_conv2d_igemm_f32 / _backward_f32) against the
reference's wide composition, replayed on the oracle: im2col, the product with the
transposed weight, the bias add and the permute, and its autograd backward (dcols =
g W, col2im; dW = g^T cols; db = column sums) (src/conv.cpp:280-338 of the reference).

The device sums in another order than the reference's serial loops, so each output is
checked twice: against the oracle's composition with the reference's metric at the
K-term tolerance, and against the exact (float64) product with the worst-case fp32
bound (K + 2) u sum |a| |b| per element -- a dropped term, a wrong window offset or a
transposed operand moves an element by about one product magnitude, far beyond it.
"""
import numpy as np
import pytest

from _hip import backend, dev, exact, host, k_tol, print_case, ref_close
from _oracle import oracle_or_skip

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


@pytest.fixture(scope="module")
def hip():
    return backend()


@pytest.fixture(scope="module")
def orc():
    return oracle_or_skip()


def randn(r, *shape):
    return r.standard_normal(shape, dtype=np.float32)


def im2col64(x, kh, kw, stride, pad):
    """(N, C, H, W) -> (N, oH oW, C kH kW) in float64, k ordered (c, i, j)."""
    n, c, h, w = x.shape
    oh = (h + 2 * pad - kh) // stride + 1
    ow = (w + 2 * pad - kw) // stride + 1
    xp = np.zeros((n, c, h + 2 * pad, w + 2 * pad))
    xp[:, :, pad:pad + h, pad:pad + w] = x
    cols = np.empty((n, oh, ow, c, kh, kw))
    for i in range(kh):
        for j in range(kw):
            cols[:, :, :, :, i, j] = xp[:, :, i:i + stride * oh:stride,
                                        j:j + stride * ow:stride].transpose(0, 2, 3, 1)
    return cols.reshape(n, oh * ow, c * kh * kw)


def col2im64(dcols, shape, kh, kw, stride, pad):
    """The adjoint of im2col64: (N, oH oW, C kH kW) -> (N, C, H, W) in float64."""
    n, c, h, w = shape
    oh = (h + 2 * pad - kh) // stride + 1
    ow = (w + 2 * pad - kw) // stride + 1
    d = dcols.reshape(n, oh, ow, c, kh, kw)
    xp = np.zeros((n, c, h + 2 * pad, w + 2 * pad))
    for i in range(kh):
        for j in range(kw):
            xp[:, :, i:i + stride * oh:stride, j:j + stride * ow:stride] += \
                d[:, :, :, :, i, j].transpose(0, 3, 1, 2)
    return xp[:, :, pad:pad + h, pad:pad + w]


def exact_products(x, w, b, g, stride, pad):
    """Exact y, dx, dw, db and their worst-case fp32 bounds."""
    n, c, h, wd = x.shape
    oc, _, kh, kw = w.shape
    cols = im2col64(x.astype(np.float64), kh, kw, stride, pad)  # n, P, K
    acols = np.abs(cols)
    W = w.reshape(oc, -1).astype(np.float64)
    K = W.shape[1]
    P = cols.shape[1]
    g2 = g.reshape(n, oc, P).astype(np.float64)  # n, oc, P
    aW, ag2 = np.abs(W), np.abs(g2)
    y = np.matmul(cols, W.T).transpose(0, 2, 1)
    yb = (K + 2) * U * np.matmul(acols, aW.T).transpose(0, 2, 1)
    if b is not None:
        y = y + b.astype(np.float64)[None, :, None]
        yb = yb + U * np.abs(y)
    dcols = np.matmul(g2.transpose(0, 2, 1), W)
    adcols = np.matmul(ag2.transpose(0, 2, 1), aW)
    dx = col2im64(dcols, x.shape, kh, kw, stride, pad)
    dxb = (oc * kh * kw + 2) * U * col2im64(adcols, x.shape, kh, kw, stride, pad)
    dw = np.tensordot(g2, cols, axes=([0, 2], [0, 1])).reshape(w.shape)
    dwb = (n * P + 2) * U * np.tensordot(ag2, acols, axes=([0, 2], [0, 1])).reshape(w.shape)
    db = g2.sum(axis=(0, 2))
    dbb = (n * P + 2) * U * np.abs(g2).sum(axis=(0, 2))
    oh = (h + 2 * pad - kh) // stride + 1
    return ((y.reshape(n, oc, oh, -1), yb.reshape(n, oc, oh, -1)), (dx, dxb), (dw, dwb),
            (db, dbb))


def within(got, exact_and_bound, what):
    want, bound = exact_and_bound
    err = np.abs(got.astype(np.float64) - want)
    worst = float(np.max(err - bound)) if err.size else 0.0
    assert np.all(err <= bound + 1e-30), f"{what}: beyond the fp32 bound by {worst:.3e}"


# (x shape, out_channels, kernel, stride, padding): wide layers of the reference's kind,
# ragged sizes off every tile edge, stride above the kernel (pixels no window covers),
# 1x1, a kernel as large as the padded input, split-K on either product, both tile sizes;
# the input gradient by stride phase (strides 2-4) and by per-tap gather (stride 5, and
# more than 65535 image phases).
CASES = [((4, 64, 16, 16), 128, 3, 1, 1),
         ((2, 32, 15, 15), 96, 5, 2, 2),
         ((8, 16, 32, 32), 64, 3, 1, 1),
         ((3, 5, 13, 7), 7, 3, 2, 1),
         ((2, 3, 11, 10), 5, 2, 3, 0),
         ((2, 96, 9, 9), 80, 1, 1, 0),
         ((1, 4, 5, 6), 3, 7, 1, 1),
         ((5, 20, 12, 12), 33, 4, 2, 3),
         ((64, 8, 28, 28), 16, 3, 1, 1),
         ((2, 6, 17, 19), 10, 3, 4, 2),
         ((2, 4, 12, 12), 6, 3, 5, 1),
         ((2, 136, 10, 10), 130, 3, 2, 1),
         ((16400, 2, 3, 3), 3, 2, 2, 0)]


@pytest.mark.parametrize("shape,co,k,stride,pad", CASES)
@pytest.mark.parametrize("bias", [True, False])
def test_conv_igemm_vs_oracle(hip, orc, shape, co, k, stride, pad, bias):
    import _compose as K
    print_case("conv-igemm", shape, co, k, stride, pad, bias)
    r = np.random.default_rng(sum(shape) * 17 + co * 5 + k * 3 + stride + pad + bias)
    x = randn(r, *shape)
    x[..., ::5] = 0.0
    w = randn(r, co, shape[1], k, k) * np.float32(np.sqrt(2.0 / (shape[1] * k * k)))
    b = randn(r, co) if bias else None
    y, cache = K.conv2d_fwd(orc, x, w, b, stride, pad)
    g = randn(r, *y.shape)
    dx, dw, db = K.conv2d_bwd(orc, g, cache)
    ex = exact_products(x, w, b, g, stride, pad)
    X, Wd, G = dev(x), dev(w), dev(g)
    Y = host(hip.conv2d_igemm(X, Wd, dev(b) if bias else None, stride, pad))
    kk = shape[1] * k * k
    ref_close(Y, y, k_tol(kk), "forward")
    within(Y, ex[0], "forward")
    DX, DW, DB = hip.conv2d_igemm_backward(X, Wd, G, stride, pad, (True, True, bias))
    DX, DW = host(DX), host(DW)
    terms = y.shape[0] * y.shape[2] * y.shape[3]
    ref_close(DX, dx, k_tol(co * k * k), "dx")
    within(DX, ex[1], "dx")
    ref_close(DW, dw, k_tol(terms), "dweight")
    within(DW, ex[2], "dweight")
    if bias:
        DB = host(DB)
        ref_close(DB, db, k_tol(terms), "dbias")
        within(DB, ex[3], "dbias")
    # deterministic, and each output independent of which others are asked for
    DX2, _, _ = hip.conv2d_igemm_backward(X, Wd, G, stride, pad, (True, False, False))
    _, DW2, DB2 = hip.conv2d_igemm_backward(X, Wd, G, stride, pad, (False, True, bias))
    exact(host(DX2), DX, "dx alone")
    exact(host(DW2), DW, "dweight alone")
    if bias:
        exact(host(DB2), DB, "dbias alone")


@pytest.mark.parametrize("shape,co,k,stride,pad", [((32, 128, 28, 28), 128, 3, 1, 1),
                                                   ((16, 64, 56, 56), 128, 3, 2, 1),
                                                   ((8, 128, 32, 32), 128, 3, 2, 1)])
def test_conv_igemm_large_vs_exact(hip, shape, co, k, stride, pad):
    """Layers of a ResNet stage (K = 1152 / 576, up to 25088 output pixels; the 128 x 128
    tiles of every product): too large for the oracle's serial loops in a test, checked
    against the exact float64 products with the worst-case fp32 bound."""
    print_case("conv-igemm-large", shape, co, k, stride, pad)
    r = np.random.default_rng(shape[0] + co)
    x = randn(r, *shape)
    w = randn(r, co, shape[1], k, k) * np.float32(np.sqrt(2.0 / (shape[1] * k * k)))
    b = randn(r, co)
    oh = (shape[2] + 2 * pad - k) // stride + 1
    g = randn(r, shape[0], co, oh, oh)
    ex = exact_products(x, w, b, g, stride, pad)
    X, Wd, G = dev(x), dev(w), dev(g)
    within(host(hip.conv2d_igemm(X, Wd, dev(b), stride, pad)), ex[0], "forward")
    DX, DW, DB = hip.conv2d_igemm_backward(X, Wd, G, stride, pad)
    within(host(DX), ex[1], "dx")
    within(host(DW), ex[2], "dweight")
    within(host(DB), ex[3], "dbias")


def test_conv_igemm_empty_batch_and_errors(hip):
    import ctypes
    import ehip as E
    print_case("conv-igemm-errors")
    x = dev(np.zeros(16, np.float32))
    w0 = E.window(0, 4, 5, 5, 3, 3, 1, 1)
    before = hip.launched()
    hip.ok(hip.lib.ehip_conv2d_igemm_f32(hip.p(x), hip.p(x), None, hip.p(x), ctypes.byref(w0),
                                         8, hip.stream()), "empty forward")
    hip.ok(hip.lib.ehip_conv2d_igemm_backward_f32(hip.p(x), hip.p(x), hip.p(x), hip.p(x),
                                                  hip.p(x), hip.p(x), ctypes.byref(w0), 8,
                                                  hip.stream()), "empty backward")
    assert hip.launched() == before
    w1 = E.window(1, 4, 5, 5, 3, 3, 1, 1)
    with pytest.raises(RuntimeError):
        hip.ok(hip.lib.ehip_conv2d_igemm_f32(hip.p(x), hip.p(x), None, hip.p(x),
                                             ctypes.byref(w1), 0, hip.stream()), "no channels")
    with pytest.raises(RuntimeError):
        hip.ok(hip.lib.ehip_conv2d_igemm_backward_f32(hip.p(x), None, hip.p(x), hip.p(x), None,
                                                      None, ctypes.byref(w1), 8, hip.stream()),
               "dx without weight")
    assert hip.launched() == before
