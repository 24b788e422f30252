"""cfg 4 at its configured size, against the oracle: the inputs bench.py
times, checked by value. Softmax-cross-entropy backward on 8192 x 32000 logits drawn
N(0, 2) with uniform labels; ReLU backward and the fused add backward (both modes) on 2^28
elements drawn N(0, 1); ten fused Adam steps over a 2^28-parameter flat buffer.

Element-wise work is bit-exact (the oracle restates src/tensor_ops.cpp:605-618,
src/tensor.cpp:168-203 and src/optim.cpp:147-160 per element); the cross-entropy gradient
is within k_tol(32000) of the oracle's softmax (src/nn.cpp:386-405: the device sums each row
in a tree where the reference sums serially) and bit-identical to the two-kernel path
(forward probabilities, then their backward). These are the same kernel instantiations as
the 2^24-element cases of test_hip_kernels.py (non-temporal from 2^24 elements); here each
1 GiB array is compared in full. Inputs are drawn on the device from a seeded generator
(fast at this size) and copied to the host for the oracle.
"""
import numpy as np
import pytest

from _hip import backend, exact, host, k_tol, print_case
from _oracle import oracle_or_skip

pytestmark = pytest.mark.gpu

N28 = 1 << 28


@pytest.fixture(scope="module")
def hip():
    return backend()


@pytest.fixture(scope="module")
def orc():
    return oracle_or_skip()


def randn(seed, n, std=1.0):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(n, device="cuda", generator=g)
    return x.mul_(std) if std != 1.0 else x


def ref_close_chunked(got, want, tol, what, chunk=1 << 24):
    """The reference's metric |got - want| / max(1, |want|) <= tol, in chunks (a 2^28-element
    float64 temporary per operand would be 2 GiB)."""
    worst = 0.0
    for i in range(0, got.size, chunk):
        g = got.ravel()[i:i + chunk].astype(np.float64)
        w = want.ravel()[i:i + chunk].astype(np.float64)
        assert np.all(np.isfinite(g)), f"{what}: non-finite values"
        worst = max(worst, float(np.max(np.abs(g - w) / np.maximum(1.0, np.abs(w)))))
    assert worst <= tol, f"{what}: parity error {worst:.3e} > {tol:.1e}"
    return worst


def test_softmax_xent_backward_8192x32000(hip, orc):
    import torch
    rows, cols = 8192, 32000
    print_case("cfg4 softmax-xent backward", rows, cols)
    logits = randn(41, rows * cols, std=2.0).view(rows, cols)
    g = torch.Generator(device="cuda").manual_seed(42)
    tg = torch.randint(0, cols, (rows,), device="cuda", dtype=torch.int32, generator=g)
    one = torch.ones(1, device="cuda")
    fused = host(hip.softmax_xent_backward(logits, tg, one))
    _, probs = hip.cross_entropy(logits, tg)
    two = host(hip.cross_entropy_backward(probs, tg, one))
    del probs
    exact(fused, two, "fused == forward + backward kernels")
    del two
    print("device done; oracle", flush=True)
    x, t = host(logits), host(tg).astype(np.int64)
    del logits
    _, want_probs = orc.cross_entropy(x, t)
    want = orc.cross_entropy_backward(want_probs, t, 1.0)
    del want_probs
    e = ref_close_chunked(fused, want, k_tol(cols), "dlogits vs oracle")
    print(f"softmax-xent backward 8192x32000: worst reference metric {e:.2e}", flush=True)


def test_relu_backward_2p28(hip, orc):
    print_case("cfg4 relu backward", N28)
    x, g = randn(51, N28), randn(52, N28)
    dx = host(hip.relu_backward(x, g))
    exact(dx, orc.relu_backward(host(x), host(g)), "relu_backward")


@pytest.mark.parametrize("accumulate", [False, True])
def test_add_backward_2p28(hip, orc, accumulate):
    """The fused add backward hands g to both operands: initialising fresh gradients (the
    reference's first write, 0 + g) or adding into existing ones (grad + g)."""
    print_case("cfg4 add backward", N28, accumulate)
    g = randn(61, N28)
    if accumulate:
        base_a, base_b = randn(62, N28), randn(63, N28)
    else:
        import torch
        base_a, base_b = torch.empty(N28, device="cuda"), torch.empty(N28, device="cuda")
    ha = host(base_a) if accumulate else np.zeros(N28, np.float32)
    hb = host(base_b) if accumulate else np.zeros(N28, np.float32)
    hip.add_backward(g, base_a, base_b, accumulate, accumulate)
    gh = host(g)
    exact(host(base_a), orc.accumulate(ha, gh), "dA")
    del ha
    exact(host(base_b), orc.accumulate(hb, gh), "dB")


def test_adam_ten_steps_2p28(hip, orc):
    """Ten Adam steps (lr 1e-3, betas 0.9 / 0.999, eps 1e-8; weight decay on odd steps) with
    fresh N(0, 1) gradients each step, bias corrections from the host as in
    src/optim.cpp:119-120; p, m and v bit-exact after the tenth."""
    import torch
    print_case("cfg4 adam", N28, "10 steps")
    P = randn(71, N28)
    M, V = torch.zeros(N28, device="cuda"), torch.zeros(N28, device="cuda")
    p = host(P)
    m, v = np.zeros(N28, np.float32), np.zeros(N28, np.float32)
    for t in range(1, 11):
        G = randn(100 + t, N28)
        c1, c2 = orc.adam_bias(0.9, 0.999, t)
        wd = 0.01 if t % 2 else 0.0
        hip.adam(P, G, M, V, 1e-3, 0.9, 0.999, 1e-8, wd, c1, c2)
        orc.adam(p, host(G), m, v, 1e-3, 0.9, 0.999, 1e-8, wd, c1, c2)
        print(f"adam step {t} done", flush=True)
    exact(host(P), p, "p")
    exact(host(M), m, "m")
    exact(host(V), v, "v")
