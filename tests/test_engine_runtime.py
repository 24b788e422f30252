"""The engine's runtime contract on the GPU: residency, the arena, failure handling, the
queued convolution weight sums, and the wide-convolution paths (implicit GEMM, im2col + GEMM).

Residency follows the reference's transfer-accounting tests
(tests/test_cuda_parity.cpp:786-818 and 988-1036 of the reference): values computed on the
device stay there until read, a chain of resident work uploads nothing, and gradients stay
resident. Here a whole resident training step is the chain: after its first steps it moves
no bytes between host and device, and reading the loss is one download.

Failure handling: the reference's device ops report a failed launch and fall back to the CPU
(src/cuda/kernels.cu:81-157, src/storage.cpp:334-342); this engine has no CPU path, so a
refused launch raises instead, and the contract tested is that it raises cleanly and leaves
the model and optimiser as they were: the following steps give the bits of a run in which
the failed step never happened. Launches are refused through ehip_fail_launch_after (the
run-time form of ENGINE_HIP_FAIL_LAUNCH): at every launch position of the CNN step, and at
every ninth (and the last) of the char-Transformer step's.
"""
import numpy as np
import pytest

import workloads as W
from _hip import exact, k_tol, print_case, ref_close
from _oracle import ref_or_skip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test ran without a visible GPU")
    from engine_capi import Engine
    return Engine()


@pytest.fixture(scope="module")
def hip(eng):
    from ehip import Backend
    return Backend()


def transfers(hip):
    from ehip import TransferStats
    import ctypes as C
    s = TransferStats()
    hip.lib.ehip_transfer_stats(C.byref(s))
    return s


def cnn_trainer(eng, lr=1e-3):
    from engine_capi import Trainer
    x, labels, params = W.cnn_inputs()
    return Trainer.cnn(eng, x, labels, params, lr=lr)


def charlm_trainer(eng):
    from engine_capi import Trainer
    b, s, vocab, d, h, ff, layers = W.CHARLM_CFG3
    ids, targets = W.lm_inputs(3, b, s, vocab)
    params = W.lm_init_params(11, vocab, d, ff, layers)
    return Trainer.charlm(eng, ids, targets, vocab, d, h, ff, layers, params, lr=1e-3)


# ------------------------------------------------------------------ residency and the arena

@pytest.mark.parametrize("which", ["cnn_cfg2", "charlm_cfg3"])
def test_resident_step_moves_nothing(eng, hip, which):
    """After two steps, three more training steps (forward, backward, Adam) copy nothing
    between host and device; reading the loss is then exactly one 4-byte download."""
    print_case("resident step", which)
    tr = cnn_trainer(eng) if which == "cnn_cfg2" else charlm_trainer(eng)
    tr.step()
    tr.step()
    eng.synchronize()
    hip.lib.ehip_reset_transfer_stats()
    for _ in range(3):
        tr.step()
    eng.synchronize()
    s = transfers(hip)
    assert (s.to_device_count, s.to_host_count) == (0, 0), \
        (s.to_device_count, s.to_device_bytes, s.to_host_count, s.to_host_bytes)
    loss = tr.loss()
    s = transfers(hip)
    assert np.isfinite(loss)
    assert (s.to_device_count, s.to_host_count, s.to_host_bytes) == (0, 1, 4)
    tr.close()


def test_arena_flat_after_warmup_and_trim(eng, hip):
    """The arena reaches hipMalloc only while the first steps size their buffers: from the
    third step on, steps are served from the cache; ehip_arena_trim returns every cached
    block to the driver."""
    print_case("arena")
    tr = charlm_trainer(eng)
    tr.step()
    tr.step()
    eng.synchronize()
    before = hip.arena_stats().driver_allocations
    allocs = hip.arena_stats().allocations
    for _ in range(8):
        tr.step()
    eng.synchronize()
    after = hip.arena_stats()
    assert after.driver_allocations == before, (before, after.driver_allocations)
    assert after.allocations > allocs  # the steps did allocate, from the cache
    tr.close()
    eng.synchronize()
    hip.ok(hip.lib.ehip_arena_trim(), "trim")
    s = hip.arena_stats()
    assert s.bytes_cached == 0
    assert s.bytes_reserved == s.bytes_in_use


# ------------------------------------------------------------------ failure injection

def launches_per_step(eng, hip, tr):
    eng.synchronize()
    n0 = hip.launched()
    tr.step()
    eng.synchronize()
    return hip.launched() - n0


def run_with_failure(eng, hip, make, fail_at, steps_before=2, steps_after=3):
    """steps_before steps, then a step whose fail_at-th launch is refused (it must raise),
    then steps_after steps: (losses of the later steps, final parameters)."""
    tr = make(eng)
    for _ in range(steps_before):
        tr.step()
    failed = hip.lib.ehip_kernels_failed()
    hip.lib.ehip_fail_launch_after(fail_at)
    try:
        with pytest.raises(RuntimeError, match="ENGINE_HIP_FAIL_LAUNCH"):
            tr.step()
    finally:
        hip.lib.ehip_fail_launch_after(0)
    assert hip.lib.ehip_kernels_failed() == failed + 1
    losses = []
    for _ in range(steps_after):
        tr.step()
        losses.append(tr.loss())
    out = tr.params()
    tr.close()
    return np.array(losses, np.float32), out


@pytest.mark.parametrize("which", ["cnn_cfg2", "charlm_cfg3"])
def test_refused_launch_raises_and_leaves_state(eng, hip, which):
    """A refused launch at any position of a training step (forward, backward, the queued
    weight sums, the Adam update) raises, and the steps after it give the same bits as a
    run in which that step never happened (2 + 3 steps)."""
    make = cnn_trainer if which == "cnn_cfg2" else charlm_trainer
    tr = make(eng)
    tr.step()
    tr.step()  # the first steps also materialise the optimiser state and fills
    n = launches_per_step(eng, hip, tr)
    tr.close()
    ref = make(eng)
    for _ in range(2):
        ref.step()
    want = []
    for _ in range(3):
        ref.step()
        want.append(ref.loss())
    want_p = ref.params()
    ref.close()
    want = np.array(want, np.float32)
    positions = range(1, n + 1) if n <= 16 else sorted(set(range(1, n + 1, 9)) | {n})
    for k in positions:
        print_case("refused launch", which, k, "of", n)
        losses, params = run_with_failure(eng, hip, make, k)
        exact(losses, want, f"losses after a failure at launch {k}")
        exact(params, want_p, f"parameters after a failure at launch {k}")


def test_orphaned_weight_sums_touch_no_reused_memory(eng):
    """A CNN whose fused convolution blocks queued their weight sums is destroyed before
    anything reads its gradients; the queue then runs at the start of the next backward,
    writing into buffers it owns. A second model trained right after gives the same bits as
    the same training in a clean state (its buffers may reuse the first model's blocks)."""
    print_case("orphaned weight sums")
    x, labels, params = W.cnn_inputs()
    want_losses, want_p = eng.cnn_train(x, labels, params, 3, 1e-3)
    eng.cnn_backward_orphan(x, labels, params * np.float32(0.5))
    losses, out = eng.cnn_train(x, labels, params, 3, 1e-3)
    exact(losses, want_losses, "losses")
    exact(out, want_p, "parameters")


# ------------------------------------------------------------------ wide convolution

@pytest.mark.parametrize("n,c,hw,oc,k,stride,pad", [(4, 64, 16, 128, 3, 1, 1),
                                                    (2, 32, 15, 96, 5, 2, 2)])
@pytest.mark.parametrize("igemm", [True, False])
def test_wide_conv2d_paths(eng, n, c, hw, oc, k, stride, pad, igemm):
    """Convolutions too wide for the direct kernels (out_channels * C_in * kH * kW above
    8192) run as implicit GEMMs, or, with that switched off, through im2col, the MFMA
    product, the bias and the permute (src/conv.cpp:280-338 of the reference); forward
    and all three gradients against the compiled reference with its metric at the
    K-term bound."""
    print_case("wide conv", n, c, hw, oc, k, stride, pad, igemm)
    ref = ref_or_skip()
    was = eng.set_conv_implicit_gemm(igemm)
    ref.set_threads(8)
    assert oc * c * k * k > 8192
    r = np.random.default_rng(n * 1000 + c + oc)
    x = r.standard_normal((n, c, hw, hw), dtype=np.float32)
    w = (r.standard_normal((oc, c, k, k)) * np.sqrt(2.0 / (c * k * k))).astype(np.float32)
    b = r.standard_normal(oc, dtype=np.float32)
    oh = (hw + 2 * pad - k) // stride + 1
    dy = r.standard_normal((n, oc, oh, oh), dtype=np.float32)
    try:
        y, dx, dw, db = eng.conv2d_fwd_bwd(x, w, b, stride, pad, dy)
    finally:
        eng.set_conv_implicit_gemm(was)
    wy, wdx, wdw, wdb = ref.conv2d_fwd_bwd(x, w, b, stride, pad, dy)
    ref_close(y, wy, k_tol(c * k * k), "y")
    ref_close(dx, wdx, k_tol(oc * k * k), "dx")
    ref_close(dw, wdw, k_tol(n * oh * oh), "dw")
    ref_close(db, wdb, k_tol(n * oh * oh), "db")


# ------------------------------------------------------------------ queued LayerNorm sums

@pytest.mark.parametrize("rows,d", [(1024, 1024), (2048, 1000), (2048, 96), (1024, 128),
                                    (1366, 96)])
def test_layernorm_queued_sums_match_one_call(eng, hip, rows, d):
    """A LayerNorm of at least 2^17 elements queues its dgamma / dbeta sums during backward
    (only dx and the group partials are computed there); reading the gradients runs the
    queue. The values are the one-call backward's, bit for bit: cfg5's and cfg3's shapes
    (1024 and 96 wide), exactly 2^17 elements and just above it."""
    print_case("engine layernorm queued", rows, d)
    import torch
    r = np.random.default_rng(rows + d)
    x = (r.standard_normal((rows, d)) * 2 + 0.5).astype(np.float32)
    gamma = r.standard_normal(d).astype(np.float32)
    beta = r.standard_normal(d).astype(np.float32)
    dy = r.standard_normal((rows, d)).astype(np.float32)
    assert hip.lib.ehip_layernorm_backward_partials(rows, d, None) > 0
    y, dx, dg, db = eng.layernorm_fwd_bwd(x, gamma, beta, dy)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out, xhat, inv = hip.layernorm(dev(x), dev(gamma), dev(beta))
    wdx, wdg, wdb = hip.layernorm_backward(dev(dy), xhat, dev(gamma), inv)
    exact(y, out.cpu().numpy(), "y")
    exact(dx, wdx.cpu().numpy(), "dx")
    exact(dg, wdg.cpu().numpy(), "dgamma")
    exact(db, wdb.cpu().numpy(), "dbeta")
