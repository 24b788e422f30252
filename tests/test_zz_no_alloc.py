"""ehip_gemm_f32_noalloc against ehip_gemm_f32, through the C ABI: the same arguments give the
same bits (same kernels and tile plan; only the split-K partials live in the fixed device
array), on two calls in a row with the second smaller, and a product whose partials would
exceed the fixed 32 MiB is refused before anything runs.
"""
import ctypes as C

import pytest

from _hip import exact, print_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test ran without a visible GPU")
    from ehip import Backend
    return Backend()


def call(hip, fn, ta, tb, a, b, c, m, n, k, beta=0.0):
    lda, ldb = a.shape[1], b.shape[1]
    return fn(int(ta), int(tb), 1, m, n, k, C.c_void_p(a.data_ptr()), lda, 0,
              C.c_void_p(b.data_ptr()), ldb, 0, beta, C.c_void_p(c.data_ptr()), n, 0,
              hip.stream())


def product(hip, ta, tb, m, n, k, seed, beta=0.0):
    """(no-allocation result, allocating result) of op(A) op(B) + beta C0."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    a = torch.randn((k, m) if ta else (m, k), device="cuda", generator=g)
    b = torch.randn((n, k) if tb else (k, n), device="cuda", generator=g)
    c0 = torch.randn(m, n, device="cuda", generator=g)
    got, want = c0.clone(), c0.clone()
    before = hip.arena_stats().allocations
    hip.ok(call(hip, hip.lib.ehip_gemm_f32_noalloc, ta, tb, a, b, got, m, n, k, beta),
           "gemm_noalloc")
    assert hip.arena_stats().allocations == before, "the no-allocation entry point allocated"
    hip.ok(call(hip, hip.lib.ehip_gemm_f32, ta, tb, a, b, want, m, n, k, beta), "gemm")
    torch.cuda.synchronize()
    return got.cpu().numpy(), want.cpu().numpy()


def test_noalloc_matches_gemm_twice_smaller_second(hip):
    # 1024 x 1024 x 8192 with A transposed: a weight-gradient product, 8 K-splits whose
    # partials fill 32 MiB of the array; then a smaller split product on the same array.
    for case in [(True, False, 1024, 1024, 8192, 1, 0.0), (False, True, 256, 128, 4096, 2, 1.0)]:
        print_case("gemm noalloc", *case)
        got, want = product(hip, *case)
        exact(got, want, f"noalloc vs gemm {case}")


def test_noalloc_unsplit_and_small(hip):
    for case in [(False, False, 512, 512, 512, 3, 0.0), (False, False, 64, 784, 10, 4, 0.0)]:
        print_case("gemm noalloc", *case)
        got, want = product(hip, *case)
        exact(got, want, f"noalloc vs gemm {case}")


def test_noalloc_refuses_beyond_its_array(hip):
    """65408 x 128 x 4096: 511 tiles of 128 x 128 split twice along K, 67 MB of partials,
    more than the array holds: EHIP_EINVAL, C untouched, nothing launched."""
    import torch
    print_case("gemm noalloc refusal")
    m, n, k = 65408, 128, 4096
    a = torch.zeros(m, k, device="cuda")
    b = torch.zeros(k, n, device="cuda")
    c = torch.full((m, n), 7.0, device="cuda")
    torch.cuda.synchronize()
    launched = hip.launched()
    rc = call(hip, hip.lib.ehip_gemm_f32_noalloc, False, False, a, b, c, m, n, k)
    assert rc == 1, rc
    assert "no allocation" in hip.error()
    assert hip.launched() == launched
    torch.cuda.synchronize()
    assert bool((c == 7.0).all())
