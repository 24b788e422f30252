"""Shared helpers of the GPU parity tests: the device backend, host<->device
conversion, and the comparison rules.

Comparison rules (each test states which one it applies):
  exact      bit-for-bit equality (integer and index work, moves, ordered sums,
             element-wise arithmetic and the optimiser updates);
  ref_close  the reference's own parity metric, |got - want| / max(1, |want|) <= tol
             (tests/test_cuda_parity.cpp:101-112 of the reference), with tol = 1e-5
             for row kernels and max(1e-5, 2 K 2^-24) for K-long sums
             (tests/test_cuda_parity.cpp:313-315).
"""
import numpy as np
import pytest

from conftest import print_case  # noqa: F401  (re-exported for the tests)


def backend():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test ran without a visible GPU")
    from ehip import Backend
    return Backend()


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def exact(got, want, what=""):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if got.dtype == np.float32:
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    else:
        bad = np.flatnonzero(got != want)
    assert bad.size == 0, (f"{what}: {bad.size} of {got.size} elements differ, first at "
                           f"{bad[:4]}: got {got.ravel()[bad[:4]]} want {want.ravel()[bad[:4]]}")


def ref_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    if got.size == 0:
        return 0.0
    return float(np.max(np.abs(got - want) / np.maximum(1.0, np.abs(want))))


def ref_close(got, want, tol=1e-5, what=""):
    assert np.all(np.isfinite(got)), f"{what}: non-finite values"
    e = ref_err(got, want)
    assert e <= tol, f"{what}: parity error {e:.3e} > {tol:.1e}"
    return e


def k_tol(k):
    return max(1e-5, 2.0 * k / 2.0 ** 24)


def gemm_stat_bound(row_norms, col_norms, k, c=2.0):
    """Per-element bound on the fp32 rounding error of a K-term dot product:
    c sqrt(K) u ||a_i|| ||b_j|| (u = 2^-24), batched over a leading axis when given.

    Rounding errors of a sum accumulate like a random walk: a serial fp32 sum of N(0,1)
    products has an error of standard deviation about u K / 5 ~ u ||a_i|| ||b_j|| / 5, and
    blocked or tree orders less, so c sqrt(K) leaves a wide margin for any correct order
    while staying far below the worst case (K + 2) u sum_k |a_ik| |b_kj|, which grows like
    K^2 u. At K = 12544 the bound is about 0.17 for unit-variance operands, so dropping a
    single product a_ik b_kj (mean magnitude 2 / pi) fails it in most draws, and a wrong
    index or a systematically dropped term fails it surely."""
    scale = c * np.sqrt(k) * 2.0 ** -24
    if isinstance(row_norms, np.ndarray):
        return scale * np.multiply.outer(row_norms, col_norms)
    return scale * row_norms.unsqueeze(-1) * col_norms.unsqueeze(-2)  # torch tensors
