"""Shapes beyond one launch's grid extents run, as the reference runs them (its ops seam
takes any shape; include/engine/detail/cuda_ops.hpp:14-23): batched products and
transposes of more than 65535 matrices (the grid's z and y extents; the host launches
consecutive ranges), sums over an axis with more than 65535 outer slabs, and LayerNorm rows
wider than the 8192 columns held in registers (test_hip_kernels.py: test_layernorm). Integer
operands make every product exact in fp32, so the batched results are compared bit for bit
with numpy's."""
import numpy as np
import pytest

from _hip import backend, dev, exact, host, print_case
from _oracle import oracle_or_skip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    return backend()


@pytest.fixture(scope="module")
def orc():
    return oracle_or_skip()


def ints(r, *shape, lo=-4, hi=5):
    return r.integers(lo, hi, shape).astype(np.float32)


@pytest.mark.parametrize("batch,m,n,k", [(65536, 32, 32, 32), (65537, 32, 32, 32),
                                         (65537, 128, 128, 32), (70000, 5, 7, 300)])
def test_gemm_batch_beyond_grid(hip, batch, m, n, k):
    """32 x 32 products take the K-sliced tiles, 128 x 128 the staged 128-tile kernel, and
    5 x 7 x 300 the K-sliced tiles with edge checks; every product, those on both sides of
    the 65535 boundary included, equals numpy's exactly."""
    print_case("gemm batch", batch, m, n, k)
    r = np.random.default_rng(batch + m + k)
    a, b = ints(r, batch, m, k), ints(r, batch, k, n)
    got = host(hip.gemm(dev(a), dev(b)))
    exact(got, np.matmul(a, b), "batched product")


def test_gemm_ex_two_level_batch_beyond_grid(hip):
    """The extended product with two-level strides (2 heads per sample) and a per-head addend
    and scale in the epilogue over 65538 products: product z reads sample z / 2, head z % 2,
    and adds addend[z % 2]."""
    from ehip import GemmEx
    samples, heads, s, hd = 32769, 2, 32, 32
    batch = samples * heads
    print_case("gemm_ex two-level batch", batch)
    r = np.random.default_rng(5)
    q = ints(r, samples, s, heads, hd)      # (sample, seq, head, dim) activations
    kk = ints(r, samples, s, heads, hd)
    add = ints(r, heads, s, s)
    Q, K, A = dev(q), dev(kk), dev(add)
    c = hip.f32((samples, heads, s, s))
    d = GemmEx(0, 1, batch, heads, s, s, hd, hip.p(Q), heads * hd, s * heads * hd, hd,
               hip.p(K), heads * hd, s * heads * hd, hd, hip.p(c), s, heads * s * s, s * s,
               0.5, hip.p(A), s, s * s, heads, 0.0, 0)
    hip.gemm_ex(d)
    qh = q.transpose(0, 2, 1, 3)
    kh = kk.transpose(0, 2, 3, 1)
    want = (np.matmul(qh, kh) * np.float32(0.5) + add[None]).astype(np.float32)
    exact(host(c), want, "scores")


@pytest.mark.parametrize("batch,rows,cols", [(65536, 3, 5), (65537, 3, 5), (70001, 33, 2)])
def test_transpose_batch_beyond_grid(hip, batch, rows, cols):
    print_case("transpose batch", batch, rows, cols)
    x = np.random.default_rng(batch).standard_normal((batch, rows, cols), dtype=np.float32)
    exact(host(hip.transpose(dev(x))), np.ascontiguousarray(x.transpose(0, 2, 1)), "transpose")


@pytest.mark.parametrize("outer,axis_len,inner", [(65536, 100, 1), (65537, 70, 1),
                                                  (70000, 3, 2)])
def test_sum_axis_outer_beyond_grid(hip, orc, outer, axis_len, inner):
    """More than 65535 outer slabs: the serial kernel (the reference's a-ascending order),
    bit for bit."""
    print_case("sum_axis outer", outer, axis_len, inner)
    x = np.random.default_rng(outer).standard_normal((outer, axis_len, inner), dtype=np.float32)
    got = host(hip.sum_axis(dev(x), outer, axis_len, inner)).reshape(outer, inner)
    exact(got, orc.sum_axis(x, 1).reshape(outer, inner), "sum_axis")
