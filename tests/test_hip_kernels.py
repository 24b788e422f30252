"""Kernel-level parity of the HIP backend against the CPU oracle, through the C ABI.

Each test feeds the same seeded inputs to the device kernel (libehip.so via ctypes) and
to the oracle's restatement of the reference loop it replaces, and compares with the rule
named in tests/_hip.py: `exact` where the reference's result is reproducible bit for bit,
`ref_close` (the reference's |d|/max(1,|want|) metric) where the device sums in another
order or uses the device exp/log.
"""
import numpy as np
import pytest

from _hip import (backend, dev, exact, gemm_stat_bound, host, k_tol, print_case, ref_close,
                  ref_err)
from _oracle import oracle_or_skip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    return backend()


@pytest.fixture(scope="module")
def orc():
    return oracle_or_skip()


def rng(seed):
    return np.random.default_rng(seed)


def randn(r, *shape):
    return r.standard_normal(shape, dtype=np.float32)


# ------------------------------------------------------------------ GEMM

GEMM_SHAPES = [(1, 1, 1), (7, 5, 3), (33, 17, 65), (64, 64, 64), (128, 9, 8), (5, 300, 2),
               (130, 257, 129), (256, 256, 256), (512, 512, 512), (2048, 96, 96),
               (64, 784, 10), (9, 4096, 8), (72, 3000, 16)]


@pytest.mark.parametrize("m,k,n", GEMM_SHAPES)
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_modes_vs_oracle(hip, orc, m, k, n, ta, tb):
    print_case("gemm", m, k, n, ta, tb)
    r = rng(m * 7919 + k * 31 + n + 2 * ta + tb)
    a = randn(r, m, k)
    b = randn(r, k, n)
    a_st = np.ascontiguousarray(a.T) if ta else a
    b_st = np.ascontiguousarray(b.T) if tb else b
    got = host(hip.gemm(dev(a_st), dev(b_st), trans_a=ta, trans_b=tb))
    want = orc.matmul(a, b)
    exact64 = a.astype(np.float64) @ b.astype(np.float64)
    # The reference's metric at the K-term bound; where the device misses it, fp64
    # arbitrates: the device value must be at least as close to the exact product as the
    # reference's own serial sum is (the two rounding errors can add up past the bound).
    err = np.abs(got - want) / np.maximum(1.0, np.abs(want))
    miss = err > k_tol(k)
    assert np.all(np.abs(got - exact64)[miss] <= np.abs(want - exact64)[miss]), \
        f"gemm {m}x{k}x{n} ta={ta} tb={tb}: {int(miss.sum())} elements beyond {k_tol(k):.2e} " \
        f"and farther from the exact product than the reference"
    # The device error against the exact product stays within a small multiple
    # of the CPU's own serial-sum error, and within the statistical bound everywhere.
    e_gpu = np.sqrt(np.mean((got - exact64) ** 2))
    e_cpu = np.sqrt(np.mean((want - exact64) ** 2))
    assert e_gpu <= 4.0 * e_cpu + 1e-7, (e_gpu, e_cpu)
    bound = gemm_stat_bound(np.linalg.norm(a.astype(np.float64), axis=1),
                            np.linalg.norm(b.astype(np.float64), axis=0), k)
    assert np.all(np.abs(got - exact64) <= bound)


# Shapes that select each tile configuration of the dispatcher (gemm.hip): the 256 x 256
# tiles (grid >= 256 tiles), 128 x 128 x 32, 128 x 64 x 32 (thin, batched), each also with
# ragged edges (the checked kernels) and split-K. The CPU oracle is too slow at these sizes,
# so float64 is the arbiter, with the reference's K-scaled tolerance.
TILE_CASES = [
    ("L 256x256", 1, 4096, 256, 4096), ("L ragged", 1, 4100, 300, 4096),
    ("M 128x128x32", 1, 2048, 512, 1024), ("M ragged", 1, 2050, 515, 1030),
    ("M split-K", 1, 1024, 8192, 1024), ("S 128x64 batched", 32, 512, 512, 64),
    ("S ragged batched", 16, 500, 77, 60), ("M batched K=64", 256, 512, 64, 512),
    # 32 x 32 tiles with K sliced over the waves (gemm_kslice): 8, 2 and 1 waves per
    # workgroup, whole and ragged tiles, a batch of attention-sized products.
    ("K-sliced 512^3 W=8", 1, 512, 512, 512), ("K-sliced W=2", 1, 2048, 96, 96),
    ("K-sliced ragged", 1, 1000, 300, 200), ("K-sliced batched K=24", 128, 64, 24, 64),
    # A^T B over a long K into few 16 x 16 tiles, one workgroup of 16 waves per tile
    # (gemm_tn_panel; the TA mode takes it, the others the tiles above): whole, ragged
    # (checked loads, K not a multiple of 128), and a K long enough for 32 chunks a wave.
    ("P 96x96 K=2048", 1, 96, 2048, 96), ("P 96x384", 1, 96, 2048, 384),
    ("P ragged", 1, 100, 1500, 37), ("P K=65536", 1, 64, 65536, 64),
]


@pytest.mark.parametrize("name,batch,m,k,n", TILE_CASES)
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False)])
def test_gemm_tile_configs_vs_fp64(hip, name, batch, m, k, n, ta, tb):
    import torch
    print_case("gemm-tiles", name, batch, m, k, n, ta, tb)
    g = torch.Generator(device="cuda").manual_seed(m + n + k + batch)
    a = torch.randn(batch, m, k, device="cuda", generator=g)
    b = torch.randn(batch, k, n, device="cuda", generator=g)
    a_st = a.transpose(1, 2).contiguous() if ta else a
    b_st = b.transpose(1, 2).contiguous() if tb else b
    got = hip.gemm(a_st if batch > 1 else a_st[0], b_st if batch > 1 else b_st[0], trans_a=ta,
                   trans_b=tb)
    want = torch.matmul(a.double(), b.double()).reshape(got.shape)
    bound = gemm_stat_bound(a.double().norm(dim=2), b.double().norm(dim=1), k).reshape(got.shape)
    ratio = ((got.double() - want).abs() / bound.clamp(min=1e-30)).max().item()
    assert ratio <= 1.0, f"{name}: error reaches {ratio:.3f} of the statistical fp32 bound"


@pytest.mark.parametrize("m,k,n", [(37, 53, 29), (256, 512, 128), (9, 50176, 8),
                                   (4096, 64, 4096), (4096, 256, 4096)])
def test_gemm_integer_inputs_exact(hip, m, k, n):
    """Small-integer operands: every partial sum is exact in fp32, so any summation order
    must give the exact product (tests/test_cuda_parity.cpp:344-363 of the reference)."""
    print_case("gemm-int", m, k, n)
    r = rng(11)
    a = r.integers(-3, 4, (m, k)).astype(np.float32)
    b = r.integers(-3, 4, (k, n)).astype(np.float32)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)  # exact: |sums| < 2^53
    exact(host(hip.gemm(dev(a), dev(b))), want, "integer gemm")


SMALL_EXACT = [(7, 5, 3), (64, 10, 784), (784, 64, 10), (200, 96, 96), (33, 128, 65),
               (1, 1, 1), (3, 100, 2)]


@pytest.mark.parametrize("m,k,n", SMALL_EXACT)
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_small_k_bitexact(hip, orc, m, k, n, ta, tb):
    """Products with K <= 128 take the thread-per-output kernel: k order from zero with the
    zero skip of the reference's i-k-j loop, so they equal the CPU bit for bit."""
    print_case("gemm-small-exact", m, k, n, ta, tb)
    r = rng(m * 31 + k * 7 + n + 2 * ta + tb)
    a = randn(r, m, k)
    a[:, ::3] = 0.0  # zero A entries take the skip
    b = randn(r, k, n)
    a_st = np.ascontiguousarray(a.T) if ta else a
    b_st = np.ascontiguousarray(b.T) if tb else b
    got = host(hip.gemm(dev(a_st), dev(b_st), trans_a=ta, trans_b=tb))
    exact(got, orc.matmul(a, b), f"small gemm {m}x{k}x{n} ta={ta} tb={tb}")


def test_gemm_small_batched_bitexact(hip, orc):
    """Attention-shaped batched products (cfg3's head shapes, 8 heads' worth)."""
    print_case("gemm-small-batched")
    r = rng(77)
    q, kt = randn(r, 8, 64, 24), randn(r, 8, 24, 64)
    exact(host(hip.gemm(dev(q), dev(kt))), orc.matmul(q, kt), "scores")
    p, v = randn(r, 8, 64, 64), randn(r, 8, 64, 24)
    exact(host(hip.gemm(dev(p), dev(v))), orc.matmul(p, v), "probs x V")


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("m,k,n", [(64, 784, 10), (10, 2048, 9), (96, 512, 20)])
def test_gemm_small_wave(hip, orc, m, k, n, ta, tb):
    """Few outputs, long K: the wave-per-output kernel, within the fp32 summation bound and
    deterministic."""
    print_case("gemm-small-wave", m, k, n, ta, tb)
    r = rng(m + k + n + ta * 2 + tb)
    a, b = randn(r, m, k), randn(r, k, n)
    a_st = np.ascontiguousarray(a.T) if ta else a
    b_st = np.ascontiguousarray(b.T) if tb else b
    got = host(hip.gemm(dev(a_st), dev(b_st), trans_a=ta, trans_b=tb))
    ref_close(got, orc.matmul(a, b), k_tol(k), "wave gemm")
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    bound = gemm_stat_bound(np.linalg.norm(a64, axis=1), np.linalg.norm(b64, axis=0), k)
    assert np.all(np.abs(got - a64 @ b64) <= bound), "beyond the statistical fp32 bound"
    again = host(hip.gemm(dev(a_st), dev(b_st), trans_a=ta, trans_b=tb))
    exact(again, got, "repeat")


@pytest.mark.parametrize("ab,bb", [(True, True), (True, False), (False, True)])
def test_gemm_batched_shared(hip, orc, ab, bb):
    print_case("gemm-batched", ab, bb)
    r = rng(5)
    a = randn(r, 6, 40, 24) if ab else randn(r, 40, 24)
    b = randn(r, 6, 24, 33) if bb else randn(r, 24, 33)
    got = host(hip.gemm(dev(a), dev(b)))
    ref_close(got, orc.matmul(a, b), k_tol(24), "batched gemm")


@pytest.mark.parametrize("m,k,n", [(70, 45, 90), (512, 128, 256), (500, 100, 130)])
def test_gemm_beta_accumulates(hip, orc, m, k, n):
    """beta = 1 onto a nonzero destination (tests/test_cuda_parity.cpp:263-290): the
    thread-per-output kernel, and the K-sliced tiles whole and ragged."""
    print_case("gemm-beta", m, k, n)
    r = rng(9 + m)
    a, b, c0 = randn(r, m, k), randn(r, k, n), randn(r, m, n)
    c = dev(c0)
    hip.gemm(dev(a), dev(b), c=c, beta=1.0)
    want = orc.binary("add", orc.matmul(a, b), c0)
    ref_close(host(c), want, k_tol(k) + 1e-6, "beta=1")


def test_gemm_splitk_beta(hip, orc):
    print_case("gemm-splitk-beta")
    r = rng(10)
    a, b, c0 = randn(r, 16, 8192), randn(r, 8192, 8), randn(r, 16, 8)
    c = dev(c0)
    hip.gemm(dev(a), dev(b), c=c, beta=1.0)
    ref_close(host(c), orc.binary("add", orc.matmul(a, b), c0), k_tol(8192), "split-K beta")


def test_gemm_deterministic(hip):
    print_case("gemm-determinism")
    r = rng(12)
    a, b = dev(randn(r, 300, 700)), dev(randn(r, 700, 200))
    exact(host(hip.gemm(a, b)), host(hip.gemm(a, b)), "repeat")


@pytest.mark.parametrize("m,k,n", [(512, 512, 512), (1000, 300, 200), (2048, 96, 96), (64, 784, 10),
                                   (96, 2048, 96)])
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_matmul_backward_pair_bits(hip, m, k, n, beta):
    """ehip_matmul_backward_f32 gives the bits of the two ehip_gemm_f32 calls it replaces
    (dA = dC B^T, dB = A^T dC), whether the two products share one launch (both on the
    K-sliced tiles: 512^3, the ragged 1000 x 300 x 200) or not (the others); also with only
    one of the outputs requested."""
    import ctypes as C
    import torch
    print_case("matmul-backward", m, k, n, beta)
    g = torch.Generator(device="cuda").manual_seed(m + k + n)
    a = torch.randn(m, k, device="cuda", generator=g)
    b = torch.randn(k, n, device="cuda", generator=g)
    dc = torch.randn(m, n, device="cuda", generator=g)
    da0 = torch.randn(m, k, device="cuda", generator=g)
    db0 = torch.randn(k, n, device="cuda", generator=g)
    p = lambda t: C.c_void_p(t.data_ptr()) if t is not None else None

    def pair(da, db):
        hip.ok(hip.lib.ehip_matmul_backward_f32(m, k, n, p(a), k, p(b), n, p(dc), n, p(da), k,
                                                beta, p(db), n, beta, hip.stream()), "pair")

    da, db = da0.clone(), db0.clone()
    pair(da, db)
    want_a = hip.gemm(dc, b, c=da0.clone(), trans_b=True, beta=beta)
    want_b = hip.gemm(a, dc, c=db0.clone(), trans_a=True, beta=beta)
    exact(host(da), host(want_a), "dA")
    exact(host(db), host(want_b), "dB")
    only_a, only_b = da0.clone(), db0.clone()
    pair(only_a, None)
    pair(None, only_b)
    exact(host(only_a), host(want_a), "dA alone")
    exact(host(only_b), host(want_b), "dB alone")


def test_gemm_backward_products(hip, orc):
    """cfg 1: C = A B and both backward products at 512^3, N(0,1) from one seed, against
    the reference's graph (materialised transposes, src/tensor_ops.cpp:570-585)."""
    print_case("gemm-cfg1")
    r = rng(1)
    a, b, dc = randn(r, 512, 512), randn(r, 512, 512), randn(r, 512, 512)
    A, B, dC = dev(a), dev(b), dev(dc)
    ref_close(host(hip.gemm(A, B)), orc.matmul(a, b), k_tol(512), "C")
    ref_close(host(hip.gemm(dC, B, trans_b=True)), orc.matmul(dc, orc.transpose(b)), k_tol(512),
              "dA")
    ref_close(host(hip.gemm(A, dC, trans_a=True)), orc.matmul(orc.transpose(a), dc), k_tol(512),
              "dB")
    a64, b64, dc64 = (x.astype(np.float64) for x in (a, b, dc))
    for what, got, x, y in (("C", hip.gemm(A, B), a64, b64),
                            ("dA", hip.gemm(dC, B, trans_b=True), dc64, b64.T),
                            ("dB", hip.gemm(A, dC, trans_a=True), a64.T, dc64)):
        bound = gemm_stat_bound(np.linalg.norm(x, axis=1), np.linalg.norm(y, axis=0), 512)
        assert np.all(np.abs(host(got) - x @ y) <= bound), f"{what}: beyond the statistical bound"


# ------------------------------------------------------------------ element-wise

@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
@pytest.mark.parametrize("shape,inner", [((1000,), 1000), ((50176, 8), 8), ((33, 7), 7),
                                         ((64, 96), 96), ((4, 3, 5), 15), ((1 << 22, 4), 4)])
def test_binary_exact(hip, orc, op, shape, inner):
    print_case("binary", op, shape, inner)
    r = rng(len(shape) * 100 + inner)
    a = randn(r, *shape)
    b = randn(r, inner) + (3.0 if op == "div" else 0.0)
    code = {"add": 0, "sub": 1, "mul": 2, "div": 3}[op]
    exact(host(hip.binary(code, dev(a), dev(b))), orc.binary(op, a, b).reshape(shape), op)


@pytest.mark.parametrize("n", [1, 3, 4, 1023, 4096 * 4 + 5, 1 << 20, (1 << 24) + 6])
def test_unary_exact(hip, orc, n):
    print_case("unary", n)
    r = rng(n)
    x, g = randn(r, n), randn(r, n)
    x[::7] = 0.0
    x[1::11] = -0.0
    X, G = dev(x), dev(g)
    exact(host(hip.relu(X)), orc.relu(x), "relu")
    exact(host(hip.relu_backward(X, G)), orc.relu_backward(x, g), "relu_backward")
    exact(host(hip.scalar(X, 0.125, 0.0)), orc.scalar_mul(x, 0.125), "t*k")
    exact(host(hip.scalar(X, 1.0, 2.5)), orc.scalar_add(x, 2.5), "t+k")


@pytest.mark.parametrize("n", [5, 4096, 100003, (1 << 24) + 2])
def test_accumulate_and_add_backward_exact(hip, orc, n):
    print_case("accumulate", n)
    r = rng(n + 1)
    g, base = randn(r, n), randn(r, n)
    g[::5] = -0.0
    zero = np.zeros(n, np.float32)
    want_init = orc.accumulate(zero.copy(), g)
    want_acc = orc.accumulate(base.copy(), g)
    exact(host(hip.accumulate_grad(dev(zero), dev(g), True)), want_init, "init")
    exact(host(hip.accumulate_grad(dev(base), dev(g), False)), want_acc, "accumulate")
    for acc_a in (False, True):
        for acc_b in (False, True):
            da, db = dev(base), dev(base * 2)
            hip.add_backward(dev(g), da, db, acc_a, acc_b)
            exact(host(da), want_acc if acc_a else want_init, f"da {acc_a}{acc_b}")
            exact(host(db), orc.accumulate((base * 2).copy(), g) if acc_b else want_init,
                  f"db {acc_a}{acc_b}")


@pytest.mark.parametrize("n", [5, 4096, 100003, (1 << 22) + 3])
@pytest.mark.parametrize("mode_a,mode_b", [(1, 1), (2, 2), (1, 2), (2, 1), (1, 0), (0, 2)])
def test_mul_backward_exact(hip, orc, n, mode_a, mode_b):
    """The fused multiply backward equals the composed node bit for bit: the oracle's
    product g * b (g * a), added to the existing gradient when accumulating (mode 2),
    written otherwise (mode 1), skipped (mode 0); with zeros, -0 and unaligned lengths."""
    print_case("mul-backward", n, mode_a, mode_b)
    r = rng(n + 10 * mode_a + mode_b)
    g, a, b = randn(r, n), randn(r, n), randn(r, n)
    a[::5] = 0.0
    b[1::7] = -0.0
    base_a, base_b = randn(r, n), randn(r, n)
    da = dev(base_a) if mode_a else None
    db = dev(base_b) if mode_b else None
    hip.mul_backward(dev(g), dev(a), dev(b), da, db, mode_a == 2, mode_b == 2)
    if mode_a:
        p = orc.binary("mul", g, b)
        exact(host(da), orc.accumulate(base_a.copy(), p) if mode_a == 2 else p, "da")
    if mode_b:
        p = orc.binary("mul", g, a)
        exact(host(db), orc.accumulate(base_b.copy(), p) if mode_b == 2 else p, "db")


@pytest.mark.parametrize("n", [7, 4096, 65537, (1 << 24) + 3])
def test_adam_trajectory_exact(hip, orc, n):
    """Ten Adam steps, bias corrections from the host as in src/optim.cpp:119-120."""
    print_case("adam", n)
    r = rng(n + 2)
    p = randn(r, n)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    P, M, V = dev(p), dev(m), dev(v)
    for t in range(1, 11):
        g = randn(r, n)
        c1, c2 = orc.adam_bias(0.9, 0.999, t)
        orc.adam(p, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.01 if t % 2 else 0.0, c1, c2)
        hip.adam(P, dev(g), M, V, 1e-3, 0.9, 0.999, 1e-8, 0.01 if t % 2 else 0.0, c1, c2)
    exact(host(P), p, "p")
    exact(host(M), m, "m")
    exact(host(V), v, "v")


def test_adam_multi_exact(hip, orc):
    """One launch over tensors of ragged sizes (tails, chunk boundaries, an unaligned view)
    equals the per-tensor update bit for bit."""
    print_case("adam-multi")
    import torch
    r = rng(44)
    sizes = [1, 3, 4, 4096, 4097, 12289, 100003]
    host = [[randn(r, n), randn(r, n), np.zeros(n, np.float32), np.zeros(n, np.float32)]
            for n in sizes]
    devs = [[dev(a) for a in t] for t in host]
    # an unaligned view: element 1 of a larger buffer
    big = [dev(randn(r, 1001)), dev(randn(r, 1001)), dev(np.zeros(1001, np.float32)),
           dev(np.zeros(1001, np.float32))]
    views = [b[1:] for b in big]
    vhost = [host_of(b)[1:].copy() for b in big]
    for t in range(1, 4):
        c1, c2 = orc.adam_bias(0.9, 0.999, t)
        for h in host + [vhost]:
            orc.adam(h[0], h[1], h[2], h[3], 1e-3, 0.9, 0.999, 1e-8, 0.0, c1, c2)
        hip.adam_multi([tuple(d) for d in devs] + [tuple(views)], 1e-3, 0.9, 0.999, 1e-8, 0.0,
                       c1, c2)
    for h, d in zip(host, devs):
        exact(host_of(d[0]), h[0], "p")
        exact(host_of(d[2]), h[2], "m")
        exact(host_of(d[3]), h[3], "v")
    exact(host_of(views[0]), vhost[0], "unaligned p")


def host_of(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_sgd_exact(hip, orc):
    print_case("sgd")
    r = rng(3)
    p = randn(r, 1001)
    vel = np.zeros_like(p)
    P, VEL = dev(p), dev(vel)
    for _ in range(5):
        g = randn(r, 1001)
        orc.sgd(p, g, vel, 0.05, 0.9, 1e-4)
        hip.sgd(P, dev(g), VEL, 0.05, 0.9, 1e-4)
    exact(host(P), p, "p")
    exact(host(VEL), vel, "velocity")


def test_fill_scale(hip):
    print_case("fill-scale")
    x = dev(np.zeros(1027, np.float32))
    hip.fill(x, 1.5)
    hip.scale(x, 3.0)
    exact(host(x), np.full(1027, 4.5, np.float32), "fill*scale")


# ------------------------------------------------------------------ layout

@pytest.mark.parametrize("shape,order", [((32, 64, 4, 24), (0, 2, 1, 3)),
                                         ((3, 5, 7), (2, 0, 1)), ((64, 784, 8), (0, 2, 1)),
                                         ((2, 3, 4, 5, 6), (4, 2, 0, 3, 1)),
                                         ((16, 32, 8, 64), (0, 2, 1, 3))])
def test_permute_exact(hip, orc, shape, order):
    print_case("permute", shape, order)
    x = randn(rng(4), *shape)
    exact(host(hip.permute(dev(x), order)), orc.permute(x, order), "permute")


@pytest.mark.parametrize("shape", [(1, 1), (5, 3), (65, 130), (3, 96, 121), (128, 24, 64)])
def test_transpose_exact(hip, orc, shape):
    print_case("transpose", shape)
    x = randn(rng(6), *shape)
    exact(host(hip.transpose(dev(x))), orc.transpose(x), "transpose")


WINDOWS = [((64, 1, 28, 28), 3, 1, 1), ((64, 8, 14, 14), 3, 1, 1), ((2, 3, 9, 7), 3, 2, 0),
           ((2, 2, 8, 8), 2, 2, 0), ((1, 4, 11, 13), 5, 3, 2), ((3, 2, 6, 6), 3, 1, 0)]


@pytest.mark.parametrize("shape,k,stride,pad", WINDOWS)
def test_im2col_col2im_exact(hip, orc, shape, k, stride, pad):
    print_case("im2col", shape, k, stride, pad)
    r = rng(sum(shape) + k)
    x = randn(r, *shape)
    cols = orc.im2col(x, k, k, stride, pad)
    exact(host(hip.im2col(dev(x), k, k, stride, pad)), cols, "im2col")
    g = randn(r, *cols.shape)
    exact(host(hip.col2im(dev(g), shape, k, k, stride, pad)),
          orc.col2im(g, shape, k, k, stride, pad), "col2im")


CONV_CASES = [((64, 1, 28, 28), 8, 3, 1, 1), ((64, 8, 14, 14), 16, 3, 1, 1),
              ((2, 3, 9, 7), 5, 3, 2, 0), ((3, 2, 11, 13), 4, 5, 3, 2), ((1, 4, 6, 6), 7, 2, 2, 0),
              ((2, 5, 8, 8), 3, 1, 1, 0),
              ((1, 2, 3, 2100), 4, 3, 1, 1)]  # rows too wide for an LDS tile: per-pixel kernels


@pytest.mark.parametrize("shape,co,k,stride,pad", CONV_CASES)
@pytest.mark.parametrize("bias", [True, False])
def test_conv2d_direct(hip, orc, shape, co, k, stride, pad, bias):
    """The direct kernels against the reference's composition (im2col, product with the
    transposed weight, bias add, permute; autograd backward), replayed on the oracle:
    forward and input gradient bit for bit, weight and bias gradients within the bound of
    any fp32 summation order of their N oH oW terms."""
    import _compose as K
    print_case("conv2d-direct", shape, co, k, stride, pad, bias)
    r = rng(sum(shape) * 13 + co * 7 + k + stride + pad)
    x = randn(r, *shape)
    x[..., ::5] = 0.0  # zero inputs take the reference's skip
    w = randn(r, co, shape[1], k, k) * 0.5
    b = randn(r, co) if bias else None
    y, cache = K.conv2d_fwd(orc, x, w, b, stride, pad)
    Y = hip.conv2d(dev(x), dev(w), dev(b) if bias else None, stride, pad)
    exact(host(Y), y, "forward")
    g = randn(r, *y.shape)
    g[:, :, ::3] = 0.0  # zero gradients take the skip of the dcols product
    dx, dw, db = K.conv2d_bwd(orc, g, cache)
    exact(host(hip.conv2d_backward_input(dev(g), dev(w), shape, stride, pad)), dx, "dx")
    DW, DB = hip.conv2d_backward_weight(dev(x), dev(g), w.shape, stride, pad, bias)
    terms = y.shape[0] * y.shape[2] * y.shape[3]
    ref_close(host(DW), dw, k_tol(terms), "dweight")
    # rigorous per-element bound against fp64: (terms + 2) u sum |g| |x_col|
    cols = orc.im2col(x, k, k, stride, pad).astype(np.float64)
    g2 = g.reshape(shape[0], co, -1).transpose(0, 2, 1).reshape(-1, co).astype(np.float64)
    exact_dw = (g2.T @ cols).reshape(w.shape)
    bound = (terms + 2) * 2.0 ** -24 * (np.abs(g2).T @ np.abs(cols)).reshape(w.shape)
    assert np.all(np.abs(host(DW) - exact_dw) <= bound + 1e-30), "dweight beyond the fp32 bound"
    if bias:
        ref_close(host(DB), db, k_tol(terms), "dbias")
        bound_b = (terms + 2) * 2.0 ** -24 * np.abs(g2).sum(axis=0)
        assert np.all(np.abs(host(DB) - g2.sum(axis=0)) <= bound_b + 1e-30), "dbias bound"
    # deterministic: a second call gives the same bits
    DW2, _ = hip.conv2d_backward_weight(dev(x), dev(g), w.shape, stride, pad, bias)
    exact(host(DW2), host(DW), "dweight repeat")


POOL_CASES = [((64, 1, 28, 28), 8, 3, 1, 1, 2), ((64, 8, 14, 14), 16, 3, 1, 1, 2),
              ((2, 3, 9, 7), 5, 3, 1, 1, 2), ((2, 2, 12, 12), 4, 3, 1, 1, 3),
              ((3, 2, 11, 10), 3, 2, 2, 0, 2), ((1, 1, 5, 5), 2, 3, 1, 1, 2),
              ((4, 16, 10, 10), 32, 3, 1, 1, 2), ((3, 5, 13, 6), 7, 3, 1, 1, 2),
              ((2, 3, 8, 9), 6, 3, 1, 1, 4)]


@pytest.mark.parametrize("shape,co,k,stride,pad,pk", POOL_CASES)
@pytest.mark.parametrize("bias_shift", [0.0, -2.0])
def test_conv2d_relu_maxpool_fused(hip, orc, shape, co, k, stride, pad, pk, bias_shift):
    """Fused Conv2d -> ReLU -> MaxPool2d against the reference's three nodes replayed on the
    oracle: pooled values, argmax and the input gradient bit for bit, weight and bias
    gradients within the fp32 summation bound. A negative bias makes whole windows ReLU to
    zero, where the first element wins and the gradient is masked."""
    import _compose as K
    print_case("conv-relu-pool", shape, co, k, stride, pad, pk, bias_shift)
    r = rng(sum(shape) + co * 3 + k + pk + int(bias_shift))
    x = randn(r, *shape)
    x[..., ::7] = 0.0
    w = randn(r, co, shape[1], k, k) * 0.5
    b = randn(r, co) + bias_shift
    y, cache = K.conv2d_fwd(orc, x, w, b, stride, pad)
    ry = orc.relu(y)
    pooled, am = orc.maxpool(ry, pk, pk)
    P, AM = hip.conv2d_relu_maxpool(dev(x), dev(w), dev(b), stride, pad, pk)
    exact(host(P), pooled, "pooled")
    exact(host(AM), am, "argmax")
    g = randn(r, *pooled.shape)
    dry = orc.maxpool_backward(am, g, ry.shape)
    dy = orc.relu_backward(y, dry)
    dx, dw, db = K.conv2d_bwd(orc, dy, cache)
    DX, DW, DB = hip.conv2d_relu_maxpool_backward(dev(x), dev(w), dev(g), P, AM, stride, pad, pk)
    exact(host(DX), dx, "dx")
    terms = y.shape[0] * y.shape[2] * y.shape[3]
    ref_close(host(DW), dw, k_tol(terms), "dweight")
    ref_close(host(DB), db, k_tol(terms), "dbias")
    cols = orc.im2col(x, k, k, stride, pad).astype(np.float64)
    g2 = dy.reshape(shape[0], co, -1).transpose(0, 2, 1).reshape(-1, co).astype(np.float64)
    bound = (terms + 2) * 2.0 ** -24 * (np.abs(g2).T @ np.abs(cols)).reshape(w.shape)
    assert np.all(np.abs(host(DW) - (g2.T @ cols).reshape(w.shape)) <= bound + 1e-30)


@pytest.mark.parametrize("need", ["dx", "dw", "both"])
def test_conv2d_relu_maxpool_partial_outputs(hip, need):
    """The fused backward with only the input gradient or only the weight gradients: dx the
    same bits as the call that computes both, the weight gradients (whose pixel split follows
    the threads left to them) within the fp32 summation tolerance, and each repeatable."""
    print_case("conv-relu-pool partial outputs", need)
    r = rng(91)
    x = randn(r, 4, 6, 10, 10)
    w = randn(r, 12, 6, 3, 3) * 0.5
    b = randn(r, 12)
    P, AM = hip.conv2d_relu_maxpool(dev(x), dev(w), dev(b), 1, 1, 2)
    g = randn(r, *host(P).shape)
    DX, DW, DB = hip.conv2d_relu_maxpool_backward(dev(x), dev(w), dev(g), P, AM, 1, 1, 2)
    dx2, dw2, db2 = hip.conv2d_relu_maxpool_backward(dev(x), dev(w), dev(g), P, AM, 1, 1, 2,
                                                     need_dx=need != "dw", need_dw=need != "dx")
    if need != "dw":
        exact(host(dx2), host(DX), "dx")
    if need != "dx":
        terms = 4 * 10 * 10
        ref_close(host(dw2), host(DW), k_tol(terms), "dweight")
        ref_close(host(db2), host(DB), k_tol(terms), "dbias")
        _, dw3, db3 = hip.conv2d_relu_maxpool_backward(dev(x), dev(w), dev(g), P, AM, 1, 1, 2,
                                                       need_dx=need != "dw")
        exact(host(dw3), host(dw2), "dweight repeat")
        exact(host(db3), host(db2), "dbias repeat")


def test_conv2d_relu_maxpool_partials_batched(hip):
    """The two-part backward (tile partials, then one reduction launch for several layers)
    gives the bits of the one-call backward, for the cfg2 layers and an odd one, with and
    without dx and the bias."""
    print_case("conv-relu-pool partials batched")
    r = rng(33)
    layers = [((64, 1, 28, 28), 8, True, False), ((64, 8, 14, 14), 16, True, True),
              ((3, 5, 13, 6), 7, False, True)]
    jobs, want = [], []
    for shape, co, bias, need_dx in layers:
        x = dev(randn(r, *shape))
        w = dev(randn(r, co, shape[1], 3, 3) * 0.5)
        b = dev(randn(r, co))
        P, AM = hip.conv2d_relu_maxpool(x, w, b, 1, 1, 2)
        g = dev(randn(r, *host(P).shape))
        DX, DW, DB = hip.conv2d_relu_maxpool_backward(x, w, g, P, AM, 1, 1, 2,
                                                      need_dx=need_dx, bias=bias)
        got = hip.conv2d_relu_maxpool_partials(x, w, g, P, AM, 1, 1, 2, need_dx=need_dx)
        assert got is not None
        dx, part, chunks = got
        if need_dx:
            exact(host(dx), host(DX), "dx")
        jobs.append((part, chunks, tuple(w.shape), bias))
        want.append((DW, DB))
    for (dw, db), (DW, DB) in zip(hip.conv_weight_reduce(jobs), want):
        exact(host(dw), host(DW), "dweight")
        if db is not None:
            exact(host(db), host(DB), "dbias")
    # a layer without the tile path reports no partials
    cw, pw = hip.conv_relu_pool_windows((3, 2, 11, 10), (3, 2, 2, 2), 2, 0, 2)
    import ctypes
    assert hip.lib.ehip_conv2d_relu_maxpool_partials(ctypes.byref(cw), 3, ctypes.byref(pw), 1,
                                                     None) == 0


def test_adam_multi_reduce_matches_two_calls(hip):
    """The weight sums and the Adam step in one launch: gradients, parameters and moments
    equal the separate reduction followed by the multi-tensor step, bit for bit (a tensor
    whose gradient no job fills, and a job whose gradient is no parameter, included)."""
    print_case("adam multi reduce")
    r = rng(71)
    layers = [((64, 1, 28, 28), 8), ((64, 8, 14, 14), 16)]
    jobs, params = [], []
    for shape, co in layers:
        x = dev(randn(r, *shape))
        w = dev(randn(r, co, shape[1], 3, 3) * 0.5)
        b = dev(randn(r, co))
        P, AM = hip.conv2d_relu_maxpool(x, w, b, 1, 1, 2)
        g = dev(randn(r, *host(P).shape))
        _, part, chunks = hip.conv2d_relu_maxpool_partials(x, w, g, P, AM, 1, 1, 2,
                                                           need_dx=shape[1] > 1)
        jobs.append((part, chunks, w.shape, b.shape))
        params += [w, b]
    lin = dev(randn(r, 10, 784))
    lin_g = dev(randn(r, 10, 784))
    hp = dict(lr=1e-3, b1=0.9, b2=0.999, eps=1e-8, wd=0.0, c1=0.1, c2=0.001)

    def run(fused):
        ps = [t.clone() for t in params] + [lin.clone()]
        ms = [dev(randn(rng(5 + i), *t.shape) * 0.1) for i, t in enumerate(ps)]
        vs = [dev(np.abs(randn(rng(9 + i), *t.shape)) * 0.01) for i, t in enumerate(ps)]
        grads = [hip.f32(t.shape) for t in params] + [lin_g.clone()]
        js = [(part, chunks, grads[2 * i], grads[2 * i + 1])
              for i, (part, chunks, _, _) in enumerate(jobs)]
        # the first layer's bias is left out of the step: its sum is only stored
        groups = [(ps[i], grads[i], ms[i], vs[i]) for i in range(len(ps)) if i != 1]
        if fused:
            hip.adam_multi_reduce(groups, js, **hp)
        else:
            outs = hip.conv_weight_reduce([(part, chunks, tuple(g.shape), True)
                                           for part, chunks, g, _ in js])
            for (dw, db), (_, _, g, gb) in zip(outs, js):
                g.copy_(dw)
                gb.copy_(db)
            hip.adam_multi(groups, **hp)
        return [host(t) for t in ps + ms + vs + grads]

    for got, want in zip(run(True), run(False)):
        exact(got, want, "adam multi reduce")


def test_conv2d_relu_maxpool_nonfinite_weight(hip, orc):
    """An infinite weight: the input gradient still skips zero output gradients as the
    reference's product does (no inf * 0), bit for bit against the oracle."""
    import _compose as K
    print_case("conv-relu-pool inf weight")
    r = rng(57)
    shape, co = (2, 3, 9, 7), 5
    x = randn(r, *shape)
    w = randn(r, co, shape[1], 3, 3) * 0.5
    b = randn(r, co)
    y, cache = K.conv2d_fwd(orc, x, w, b, 1, 1)
    ry = orc.relu(y)
    pooled, am = orc.maxpool(ry, 2, 2)
    g = randn(r, *pooled.shape)
    w_inf = w.copy()
    w_inf[1, 2, 0, 1] = np.inf
    w_inf[3, 0, 2, 2] = -np.inf
    cache_inf = (cache[0], cache[1], cache[2], orc.transpose(w_inf.reshape(co, -1)), 1, 1, True)
    dry = orc.maxpool_backward(am, g, ry.shape)
    dy = orc.relu_backward(y, dry)
    dx, _, _ = K.conv2d_bwd(orc, dy, cache_inf)
    assert np.isinf(dx).any() and not np.isnan(dx).any()
    DX, _, _ = hip.conv2d_relu_maxpool_backward(dev(x), dev(w_inf), dev(g), dev(pooled),
                                                dev(am), 1, 1, 2)
    exact(host(DX), dx, "dx")


def test_conv2d_relu_maxpool_nonfinite_input(hip, orc):
    """An infinite input: the weight gradients keep the full sum over positions (inf times a
    zero gradient is NaN, as in the reference's product), so the NaN and inf entries of dW
    and db fall where the oracle's do, and the finite ones agree within the fp32 bound."""
    import _compose as K
    print_case("conv-relu-pool inf input")
    r = rng(58)
    shape, co = (2, 3, 9, 8), 5
    x = randn(r, *shape)
    w = randn(r, co, shape[1], 3, 3) * 0.5
    b = randn(r, co)
    y, cache = K.conv2d_fwd(orc, x, w, b, 1, 1)
    ry = orc.relu(y)
    pooled, am = orc.maxpool(ry, 2, 2)
    g = randn(r, *pooled.shape)
    x_inf = x.copy()
    x_inf[1, 2, 4, 5] = np.inf
    cols = orc.im2col(x_inf, 3, 3, 1, 1)
    cache_inf = (cache[0], cache[1], cols, cache[3], 1, 1, True)
    dry = orc.maxpool_backward(am, g, ry.shape)
    dy = orc.relu_backward(y, dry)
    _, dw, db = K.conv2d_bwd(orc, dy, cache_inf)
    _, DW, DB = hip.conv2d_relu_maxpool_backward(dev(x_inf), dev(w), dev(g), dev(pooled),
                                                 dev(am), 1, 1, 2)
    DW, DB = host(DW), host(DB)
    assert np.isnan(dw).any()
    assert np.array_equal(np.isnan(DW), np.isnan(dw)) and np.array_equal(np.isinf(DW), np.isinf(dw))
    fin = np.isfinite(dw)
    ref_close(DW[fin], dw[fin], k_tol(2 * 9 * 8), "dweight finite entries")
    exact(np.isnan(DB), np.isnan(db), "dbias NaN pattern")


def test_conv2d_relu_maxpool_refusals(hip):
    import ctypes
    import ehip as E
    print_case("conv-relu-pool-refusals")
    cw = E.window(2, 3, 8, 8, 3, 3, 1, 1)
    overlapping = E.window(2, 4, 8, 8, 3, 3, 2, 0)   # kernel 3, stride 2
    assert hip.lib.ehip_conv2d_relu_maxpool_supported(ctypes.byref(cw), 4,
                                                      ctypes.byref(overlapping)) == 0
    good = E.window(2, 4, 8, 8, 2, 2, 2, 0)
    assert hip.lib.ehip_conv2d_relu_maxpool_supported(ctypes.byref(cw), 4, ctypes.byref(good)) == 1
    x = dev(np.zeros(16, np.float32))
    before = hip.launched()
    with pytest.raises(RuntimeError, match="kernel == stride"):
        hip.ok(hip.lib.ehip_conv2d_relu_maxpool_f32(hip.p(x), hip.p(x), None, hip.p(x), hip.p(x),
                                                    ctypes.byref(cw), 4, ctypes.byref(overlapping),
                                                    hip.stream()), "fused")
    assert hip.launched() == before


def test_conv2d_direct_refuses_wide_layers(hip):
    import ctypes
    import ehip as E
    print_case("conv2d-wide")
    w = E.window(1, 64, 8, 8, 3, 3, 1, 1)
    assert hip.lib.ehip_conv2d_direct_supported(ctypes.byref(w), 256) == 0
    assert hip.lib.ehip_conv2d_direct_supported(ctypes.byref(w), 8) == 1
    x = dev(np.zeros(16, np.float32))
    before = hip.launched()
    with pytest.raises(RuntimeError, match="direct path"):
        hip.ok(hip.lib.ehip_conv2d_forward_f32(hip.p(x), hip.p(x), None, hip.p(x),
                                               ctypes.byref(w), 256, hip.stream()), "conv")
    assert hip.launched() == before


@pytest.mark.parametrize("shape,k,stride", [((64, 8, 28, 28), 2, 2), ((64, 16, 14, 14), 2, 2),
                                            ((2, 3, 9, 9), 3, 2), ((2, 2, 7, 7), 3, 1),
                                            ((2, 3, 9, 7), 2, 2), ((1, 2, 10, 11), 3, 3),
                                            ((3, 1, 5, 5), 5, 5), ((4, 4, 13, 6), 2, 2),
                                            ((8, 64, 112, 112), 2, 2)])
@pytest.mark.parametrize("float_index", [False, True])
def test_maxpool_exact(hip, orc, shape, k, stride, float_index):
    """Overlapping windows and ties included: the first strict maximum wins. The
    float-index variant stores the argmax as float, as the reference's device path does."""
    print_case("maxpool", shape, k, stride, float_index)
    r = rng(sum(shape))
    x = np.round(randn(r, *shape) * 2) / 2  # many ties
    y, am = orc.maxpool(x, k, stride)
    Y, AM = hip.maxpool(dev(x), k, stride, float_index=float_index)
    exact(host(Y), y, "max")
    exact(host(AM), am.astype(np.float32) if float_index else am, "argmax")
    g = randn(r, *y.shape)
    exact(host(hip.maxpool_backward(AM, dev(g), shape, k, stride)),
          orc.maxpool_backward(am, g, shape), "maxpool backward")


@pytest.mark.parametrize("shape,k,stride", [((2, 3, 9, 7), 2, 2), ((2, 2, 7, 7), 3, 1)])
def test_maxpool_nan_and_signed_zero(hip, orc, shape, k, stride):
    """NaN inputs and -0 gradients on both kernel paths (non-overlapping tiles and
    general windows) against the reference's comparisons."""
    print_case("maxpool nan", shape, k, stride)
    r = rng(7 + sum(shape))
    x = np.round(randn(r, *shape) * 2) / 2
    x.ravel()[::5] = np.nan
    x.ravel()[1::7] = -0.0
    y, am = orc.maxpool(x, k, stride)
    Y, AM = hip.maxpool(dev(x), k, stride)
    exact(host(Y), y, "max")
    exact(host(AM), am, "argmax")
    g = randn(r, *y.shape)
    g.ravel()[::3] = -0.0
    exact(host(hip.maxpool_backward(AM, dev(g), shape, k, stride)),
          orc.maxpool_backward(am, g, shape), "maxpool backward")


@pytest.mark.parametrize("n,p,seed,offset", [(1, 0.5, 7, 0), (1000, 0.1, 2 ** 40 + 3, 0),
                                           (4097, 0.5, 99, 3), ((1 << 20) + 5, 0.9, 5, 2 ** 33 + 1),
                                           (777, 0.0, 1, 8)])
def test_dropout_matches_oracle(hip, orc, n, p, seed, offset):
    """The device mask, output and kept scale equal the Philox restatement bit for bit."""
    print_case("dropout", n, p, seed, offset)
    x = randn(rng(n), n)
    want_y, want_m = orc.dropout(x, p, seed, offset)
    y, m = hip.dropout(dev(x), p, seed, offset)
    exact(host(m), want_m, "mask")
    exact(host(y), want_y, "y")


def test_select_and_scatter_rows_exact(hip, orc):
    print_case("select-scatter")
    r = rng(8)
    table = randn(r, 121, 96)
    idx = r.integers(0, 121, 2048)
    out = host(hip.select_rows(dev(table), dev(idx.astype(np.int32))))
    exact(out, orc.select_rows(table, idx), "select_rows")
    g = randn(r, 2048, 96)
    order = np.argsort(idx, kind="stable")
    counts = np.bincount(idx, minlength=121)
    row_ptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    dx = dev(np.zeros((121, 96), np.float32))
    hip.scatter_add_rows(dev(g), dev(row_ptr), dev(order.astype(np.int32)), dx)
    exact(host(dx), orc.scatter_add_rows(g, idx, (121, 96)), "scatter_add_rows")


# ------------------------------------------------------------------ reductions

@pytest.mark.parametrize("outer,axis_len,inner", [(1, 50, 8), (4, 10, 4096), (1, 50176, 8),
                                                  (1, 2048, 96), (1, 8192, 1024), (3, 1000, 7)])
def test_sum_axis(hip, orc, outer, axis_len, inner):
    print_case("sum_axis", outer, axis_len, inner)
    x = randn(rng(axis_len), outer, axis_len, inner)
    got = host(hip.sum_axis(dev(x), outer, axis_len, inner)).reshape(outer, inner)
    want = orc.sum_axis(x, 1).reshape(outer, inner)
    if axis_len <= 64 or outer * inner >= 16384:
        exact(got, want, "serial sum_axis")
    else:
        ref_close(got, want, k_tol(axis_len), "chunked sum_axis")


@pytest.mark.parametrize("outer,axis_len,inner", [(1, 8192, 4096), (1, 1000, 256), (3, 500, 1024),
                                                  (1, 777, 260), (2, 4000, 512)])
def test_sum_axis_vector_path_bitexact(hip, orc, outer, axis_len, inner):
    """The float4 column-sum kernel adds every column in the same order as the
    scalar one: an aligned input (vector path) and the same values at a
    misaligned address (scalar path) give the same bits."""
    print_case("sum_axis vector", outer, axis_len, inner)
    x = randn(rng(axis_len + inner), outer, axis_len, inner)
    flat = np.concatenate([np.zeros(1, np.float32), x.ravel()])
    buf = dev(flat)
    mis = buf[1:]  # 4 bytes past a 16-byte boundary
    al = dev(x.ravel())
    got_vec = host(hip.sum_axis(al, outer, axis_len, inner))
    got_sca = host(hip.sum_axis(mis, outer, axis_len, inner))
    exact(got_vec, got_sca, "vector vs scalar column sums")
    want = orc.sum_axis(x, 1).reshape(-1)
    ref_close(got_vec, want, k_tol(axis_len), "sum_axis vs oracle")


def column_sums_emulated(x3):
    """The fixed summation order of the device column sums (reduce.hip), restated
    in float32 numpy for x3 (slabs, rows, cols): row blocks of rpb rows, row lanes
    l, l + RL, ... within a block, lanes added in order, then the block partials
    the same way."""
    slabs, rows, cols = x3.shape
    cw = 1
    while cw < cols and cw < 64:
        cw *= 2
    tiles = -(-cols // cw)
    rl = 256 // cw
    blocks = -(-1024 // (tiles * slabs))
    blocks = max(1, min(blocks, -(-rows // (2 * rl)), 64 * rl))
    rpb = -(-rows // blocks)
    blocks = -(-rows // rpb)

    def block_sum(m, r0, r1):
        s = np.zeros(m.shape[1:], np.float32)
        for lane in range(rl):
            acc = np.zeros(m.shape[1:], np.float32)
            for r in range(r0 + lane, r1, rl):
                acc = acc + m[r]
            s = s + acc
        return s

    out = np.empty((slabs, cols), np.float32)
    for z in range(slabs):
        if blocks == 1:
            out[z] = block_sum(x3[z], 0, rows)
            continue
        part = np.stack([block_sum(x3[z], b * rpb, min(rows, (b + 1) * rpb)) for b in range(blocks)])
        out[z] = block_sum(part, 0, blocks)
    return out


@pytest.mark.parametrize("outer,axis_len,inner", [(1, 2048, 96), (1, 8192, 1024), (1, 8192, 4096),
                                                  (1, 777, 260), (1, 3000, 121), (1, 100, 5),
                                                  (3, 500, 1024), (5000, 100, 1)])
def test_column_sums_order_exact(hip, outer, axis_len, inner):
    """The device column sums (scalar and float4 kernels, one slab or many) give
    exactly the blocked order restated above."""
    print_case("column sums order", outer, axis_len, inner)
    x = randn(rng(axis_len * 3 + inner), outer, axis_len, inner)
    got = host(hip.sum_axis(dev(x), outer, axis_len, inner)).reshape(outer, inner)
    exact(got, column_sums_emulated(x), "column sums")
    again = host(hip.sum_axis(dev(x), outer, axis_len, inner)).reshape(outer, inner)
    exact(again, got, "column sums repeat")


@pytest.mark.parametrize("n", [1, 1000, 1 << 20])
def test_reduce_sum(hip, orc, n):
    print_case("reduce_sum", n)
    x = randn(rng(n), n)
    d, f = hip.reduce_sum(dev(x))
    assert abs(float(host(d)[0]) - orc.sum(x)) <= 1e-9 * max(1.0, np.abs(x).sum())
    d2, _ = hip.reduce_sum(dev(x), squares=True)
    assert abs(float(host(d2)[0]) - orc.sum_squares(x)) <= 1e-9 * orc.sum_squares(x)
    assert host(f)[0] == np.float32(host(d)[0])


# ------------------------------------------------------------------ rows

@pytest.mark.parametrize("rows,cols", [(8192, 64), (64, 512), (3, 5), (17, 2048), (4, 4000),
                                       (2, 8192), (3, 30000), (2, 40000), (5, 1000), (9, 130),
                                       (4096, 4096), (32768, 512)])
def test_softmax(hip, orc, rows, cols):
    print_case("softmax", rows, cols)
    r = rng(rows * cols)
    x, g = randn(r, rows, cols) * 3, randn(r, rows, cols)
    y = hip.softmax(dev(x))
    want = orc.softmax(x)
    # The row sum is `cols` long: the reference's K-scaled tolerance applies.
    ref_close(host(y), want, k_tol(cols), "softmax")
    # fp64 arbiter: the device is at least as close to the exact softmax as the CPU is.
    x64 = x.astype(np.float64)
    e64 = np.exp(x64 - x64.max(axis=1, keepdims=True))
    exact64 = e64 / e64.sum(axis=1, keepdims=True)
    assert np.abs(host(y) - exact64).max() <= 2 * np.abs(want - exact64).max() + 1e-7
    yh = host(y)
    ref_close(host(hip.softmax_backward(y, dev(g))), orc.softmax_backward(yh, g), k_tol(cols),
              "softmax backward")


@pytest.mark.parametrize("rows,d", [(2048, 96), (512, 64), (7, 1024), (33, 100), (4, 3000),
                                   (8192, 1024), (300, 260), (64, 4096), (16, 8192),
                                   (2048, 512), (9000, 256), (5000, 257), (700, 2048),
                                   (600, 2000), (20000, 100), (2048, 256), (160, 200),
                                   (1, 8), (8191, 128), (64, 8193), (3, 20000),
                                   (600, 10000)])
def test_layernorm(hip, orc, rows, d):
    print_case("layernorm", rows, d)
    r = rng(rows + d)
    x = randn(r, rows, d) * 2 + 0.5
    gamma, beta, dy = randn(r, d), randn(r, d), randn(r, rows, d)
    out, xhat, inv = hip.layernorm(dev(x), dev(gamma), dev(beta))
    o, xh, iv = orc.layernorm(x, gamma, beta)
    ref_close(host(out), o, k_tol(d), "out")
    ref_close(host(xhat), xh, k_tol(d), "xhat")
    ref_close(host(inv), iv, k_tol(d), "inv_std")
    dx, dg, db = hip.layernorm_backward(dev(dy), dev(xh), dev(gamma), dev(iv))
    wdx, wdg, wdb = orc.layernorm_backward(dy, xh, gamma, iv)
    ref_close(host(dx), wdx, k_tol(d), "dx")
    ref_close(host(dg), wdg, k_tol(rows), "dgamma")
    ref_close(host(db), wdb, k_tol(rows), "dbeta")
    # dgamma is bit-identical across runs (tests/test_cuda_parity.cpp:644-740).
    dx2, dg2, db2 = hip.layernorm_backward(dev(dy), dev(xh), dev(gamma), dev(iv))
    exact(host(dg2), host(dg), "dgamma repeat")


@pytest.mark.parametrize("d", [64, 96, 121])
def test_layernorm_backward_split_rows_match_serial(hip, orc, d):
    """dx is row-local: 2048 rows (groups of 16, four waves per group) and the
    same rows inside 8200 (groups of 17, one wave walking each group; under
    2^20 elements, so still the small-problem kernels) give the same bits;
    the split kernel's dgamma/dbeta stay within the K-term tolerance."""
    print_case("layernorm split vs serial", d)
    r = rng(d + 7)
    big = 8200
    xh = randn(r, big, d)
    dy = randn(r, big, d)
    gamma = randn(r, d)
    inv = (np.abs(randn(r, big)) + 0.5).astype(np.float32)
    dx_s, dg_s, db_s = hip.layernorm_backward(dev(dy[:2048]), dev(xh[:2048]), dev(gamma),
                                              dev(inv[:2048]))
    dx_b, _, _ = hip.layernorm_backward(dev(dy), dev(xh), dev(gamma), dev(inv))
    exact(host(dx_s), host(dx_b)[:2048], "dx split vs serial")
    wdx, wdg, wdb = orc.layernorm_backward(dy[:2048], xh[:2048], gamma, inv[:2048])
    ref_close(host(dg_s), wdg, k_tol(2048), "dgamma")
    ref_close(host(db_s), wdb, k_tol(2048), "dbeta")


@pytest.mark.parametrize("rows,d", [(1024, 1024), (8192, 1024), (700, 2048), (1100, 999),
                                    (4097, 256)])
def test_layernorm_backward_partials_match_one_call(hip, orc, rows, d):
    """The deferred LayerNorm backward (dx and per-group partials now, the dgamma / dbeta
    sums later as a weight-reduce job with one weight per column) gives the bits of the
    one-call backward, which takes the same row kernel and reduction; the shapes cover
    four rows in flight (8192 x 1024), one (700 x 2048, 32 columns a lane), an unaligned
    width (999) and a row count that leaves the last group short. The reduction is also
    checked against the oracle, and a wrong group count is refused."""
    print_case("layernorm partials", rows, d)
    r = rng(rows + 3 * d)
    xh, dy = randn(r, rows, d), randn(r, rows, d)
    gamma = randn(r, d)
    inv = (np.abs(randn(r, rows)) + 0.5).astype(np.float32)
    one = hip.layernorm_backward(dev(dy), dev(xh), dev(gamma), dev(inv))
    got = hip.layernorm_backward_partials(dev(dy), dev(xh), dev(gamma), dev(inv))
    assert got is not None, "a shape of at least 2^20 elements takes the deferred form"
    dx, part, groups = got
    [(dg, db)] = hip.conv_weight_reduce([(part, groups, (d, 1), True)])
    exact(host(dx), host(one[0]), "dx")
    exact(host(dg).reshape(d), host(one[1]), "dgamma")
    exact(host(db), host(one[2]), "dbeta")
    wdx, wdg, wdb = orc.layernorm_backward(dy, xh, gamma, inv)
    ref_close(host(dx), wdx, k_tol(d), "dx")
    ref_close(host(dg).reshape(d), wdg, k_tol(rows), "dgamma")
    ref_close(host(db), wdb, k_tol(rows), "dbeta")
    # Accumulating into a gradient already held: old + dx in one add per element (the
    # bits of the separate accumulate pass), and the same partials; rows wider than 1024
    # columns are refused.
    old = randn(r, rows, d)
    acc = dev(old)
    if d > 1024:
        with pytest.raises(RuntimeError, match="at most 1024"):
            hip.layernorm_backward_partials(dev(dy), dev(xh), dev(gamma), dev(inv), dx=acc)
        exact(host(acc), old, "refused call leaves dx")
    else:
        _, part2, _ = hip.layernorm_backward_partials(dev(dy), dev(xh), dev(gamma), dev(inv),
                                                      dx=acc)
        exact(host(acc), old + host(dx), "dx accumulated")
        exact(host(part2), host(part), "partials while accumulating")
    with pytest.raises(RuntimeError, match="groups"):
        hip.layernorm_backward_partials(dev(dy), dev(xh), dev(gamma), dev(inv), groups=groups + 1)


def test_layernorm_backward_partials_small_shapes_refused(hip):
    """Shapes under 2^17 elements or wider than 2048 columns are summed in one call only:
    the size query returns 0 and the entry point refuses them."""
    print_case("layernorm partials small")
    for rows, d in [(1024, 96), (600, 4096)]:
        x = dev(np.ones((rows, d), np.float32))
        g = dev(np.ones(d, np.float32))
        inv = dev(np.ones(rows, np.float32))
        assert hip.layernorm_backward_partials(x, x, g, inv) is None
        with pytest.raises(RuntimeError, match="groups"):
            hip.layernorm_backward_partials(x, x, g, inv, groups=1)


@pytest.mark.parametrize("rows,cols", [(64, 10), (2048, 121), (8, 5), (16, 32000), (3, 40000),
                                       (100, 256), (600, 32000), (9, 1002), (1024, 128),
                                       (1000, 100), (1025, 10), (1, 1)])
def test_cross_entropy(hip, orc, rows, cols):
    print_case("xent", rows, cols)
    r = rng(rows * 3 + cols)
    logits = randn(r, rows, cols) * 2
    t = r.integers(0, cols, rows)
    T = dev(t.astype(np.int32))
    loss, probs = hip.cross_entropy(dev(logits), T)
    want_loss, want_probs = orc.cross_entropy(logits, t)
    ref_close(host(probs), want_probs, k_tol(cols), "probs")
    assert abs(float(host(loss)[0]) - want_loss) <= k_tol(max(rows, cols)) * max(1.0, abs(want_loss))
    one = dev(np.ones(1, np.float32))
    dx = host(hip.cross_entropy_backward(probs, T, one))
    exact(dx, orc.cross_entropy_backward(host(probs), t, 1.0), "backward from device probs")
    fused = host(hip.softmax_xent_backward(dev(logits), T, one))
    exact(fused, dx, "fused == two-kernel")
    ref_close(fused, orc.cross_entropy_backward(want_probs, t, 1.0), k_tol(cols), "vs oracle")


@pytest.mark.parametrize("rows,cols", [(64, 10), (1024, 128), (1000, 100), (7, 65), (1, 1)])
def test_cross_entropy_fused_gradient(hip, rows, cols):
    """The one-launch forward with the logits' gradient for an upstream gradient of 1: loss
    and probabilities as ehip_cross_entropy_f32 gives them, the gradient as the backward
    kernel gives it from those probabilities with grad 1, bit for bit; an out-of-range label
    still makes the loss NaN and subtracts nothing."""
    print_case("xent-fused", rows, cols)
    r = rng(rows * 5 + cols)
    logits = dev(randn(r, rows, cols) * 2)
    t = r.integers(0, cols, rows).astype(np.int32)
    if rows > 2:
        t[1] = cols + 3
    T = dev(t)
    loss, probs = hip.cross_entropy(logits, T)
    loss2, probs2, dl = hip.cross_entropy_fused(logits, T)
    exact(host(probs2), host(probs), "probs")
    exact(host(loss2), host(loss), "loss")
    one = dev(np.ones(1, np.float32))
    exact(host(dl), host(hip.cross_entropy_backward(probs, T, one)), "dlogits")
    assert hip.lib.ehip_cross_entropy_fused_supported(1025, 10) == 0
    assert hip.lib.ehip_cross_entropy_fused_supported(64, 129) == 0


def test_cross_entropy_bad_label_is_nan(hip):
    print_case("xent-bad-label")
    logits = dev(np.zeros((2, 4), np.float32))
    loss, _ = hip.cross_entropy(logits, dev(np.array([1, 9], np.int32)))
    assert np.isnan(host(loss)[0])


def test_refusals_are_errors(hip):
    """Refused geometry comes back as an error status, never a launch."""
    print_case("refusals")
    x = dev(np.zeros(16, np.float32))
    before = hip.launched()
    with pytest.raises(RuntimeError, match="do not match the window"):
        import ehip as E
        w = E.window(1, 1, 4, 4, 3, 3, 1, 0)
        w.out_h = 7
        import ctypes
        hip.ok(hip.lib.ehip_im2col_f32(hip.p(x), hip.p(x), ctypes.byref(w), hip.stream()),
               "im2col")
    with pytest.raises(RuntimeError, match="layernorm: bad shape"):
        hip.ok(hip.lib.ehip_layernorm_f32(hip.p(x), hip.p(x), hip.p(x), hip.p(x), hip.p(x),
                                          hip.p(x), -1, 16, 1e-5, hip.stream()), "layernorm")
    with pytest.raises(RuntimeError, match="beyond exact indices"):
        import ehip as E
        import ctypes
        w = E.window(1, 1, 4097, 4097, 2, 2, 2, 0)  # 2^24 + 8193 inputs: float index inexact
        hip.ok(hip.lib.ehip_maxpool_fidx_f32(hip.p(x), hip.p(x), hip.p(x), ctypes.byref(w),
                                             hip.stream()), "maxpool_fidx")
    assert hip.launched() == before


def test_gemm_probe(hip):
    """ehip_gemm_probe_arm / _read: only batch-1 products of the armed transposes and shapes
    are timed (the tile kernel and its split-K reduction between two events), their count and
    2mnk FLOPs are reported, the results are the unprobed products' bits, and reading
    disarms (a second read and a second arm while armed are refused)."""
    import torch
    print_case("gemm probe")
    g = torch.Generator(device="cuda").manual_seed(3)
    a = torch.randn(8192, 1024, device="cuda", generator=g)
    b = torch.randn(8192, 256, device="cuda", generator=g)
    want = hip.gemm(a, b, trans_a=True)  # 1024 x 256 x 8192: split along K
    hip.gemm_probe_arm(True, False, [(1024, 256, 8192), (64, 64, 64)], 8)
    with pytest.raises(RuntimeError, match="already armed"):
        hip.gemm_probe_arm(True, False, [(1024, 256, 8192)], 8)
    got = [hip.gemm(a, b, trans_a=True) for _ in range(2)]
    hip.gemm(a[:, :256].contiguous(), b, trans_a=True)  # another shape: not probed
    hip.gemm(b, a[:256, :256].contiguous())             # another mode: not probed
    ms, n, flop = hip.gemm_probe_read()
    assert n == 2 and flop == 2 * 2.0 * 1024 * 256 * 8192, (n, flop)
    assert ms > 0.0
    for x in got:
        exact(host(x), host(want), "probed product")
    with pytest.raises(RuntimeError, match="not armed"):
        hip.gemm_probe_read()


@pytest.mark.parametrize("m,n,k,epi", [(8192, 1024, 1024, "plain"), (4096, 1024, 384, "beta"),
                                       (4096, 2048, 256, "residual")])
def test_nt_pipeline_matches_staged_tiles(hip, m, n, k, epi):
    """A B^T of batch 1 in whole 128 x 128 tiles runs gemm_nt_pipe; the same product as
    both entries of a batch of two (operand strides 0) runs the staged tiles, which the
    pipeline's MFMA chain repeats: the outputs agree bit for bit, plain, with beta = 1 and
    with a residual in the epilogue (shapes that neither batch splits along K)."""
    import torch
    from ehip import GemmEx
    print_case("nt pipeline vs staged", m, n, k, epi)
    g = torch.Generator(device="cuda").manual_seed(m + n + k)
    a = torch.randn(m, k, device="cuda", generator=g)
    b = torch.randn(n, k, device="cuda", generator=g)
    c0 = torch.randn(m, n, device="cuda", generator=g)
    res = torch.randn(m, n, device="cuda", generator=g)
    outs = []
    for batch in (1, 2):
        c = c0.repeat(batch, 1).contiguous()
        d = GemmEx()
        d.trans_a, d.trans_b, d.batch, d.inner = 0, 1, batch, 1
        d.m, d.n, d.k = m, n, k
        d.a, d.lda, d.stride_a = hip.p(a), k, 0
        d.b, d.ldb, d.stride_b = hip.p(b), k, 0
        d.c, d.ldc, d.stride_c = hip.p(c), n, m * n
        d.alpha, d.addend_period = 1.0, 1
        d.beta = 1.0 if epi == "beta" else 0.0
        if epi == "residual" and batch == 1:
            d.residual, d.ld_residual = hip.p(res), n
        hip.gemm_ex(d)
        if epi == "residual" and batch == 2:
            c[:m] += res  # the separate add the epilogue replaces
        outs.append(host(c[:m]))
    exact(outs[0], outs[1], f"pipeline vs staged ({epi})")
