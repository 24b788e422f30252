"""Captured steps (ehip_graph_*, the engine's Trainer graph mode): a step recorded once into a
HIP graph and replayed with one launch must leave exactly the bits the eager step leaves.

No counterpart in the reference, whose training step is a host loop of launches
(src/optim.cpp:113-162 after src/autograd.cpp's backward): the eager engine step, itself
checked against the reference elsewhere, is the oracle here, and every comparison is exact.
Each replay is followed by eager work (a second trainer's step) and a synchronising read, so
a graph that only matches on its first replay, or that a later eager allocation can corrupt,
fails.
"""
import ctypes

import numpy as np
import pytest

from _hip import backend, print_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    return backend()


@pytest.fixture(scope="module")
def eng():
    from engine_capi import Engine
    return Engine()


def read(hip, ptr, n):
    out = np.empty(n, np.float32)
    hip.ok(hip.lib.ehip_memcpy_d2h(out.ctypes.data, ptr, n * 4, None), "read back")
    return out


def test_graph_replays_ops_on_new_inputs(hip):
    """A captured add + ReLU reads its inputs at each replay, not at capture."""
    import torch
    print_case("graph-ops")
    n = 12345
    a = torch.zeros(n, device="cuda")
    b = torch.zeros(n, device="cuda")
    t = torch.empty(n, device="cuda")
    y = torch.empty(n, device="cuda")
    torch.cuda.synchronize()
    lib = hip.lib
    hip.ok(lib.ehip_graph_begin(), "begin")
    assert lib.ehip_capturing() == 1
    before = hip.launched()
    hip.ok(lib.ehip_binary_f32(0, hip.p(a), hip.p(b), hip.p(t), n, 1, None), "add")
    hip.ok(lib.ehip_relu_f32(hip.p(t), hip.p(y), n, None), "relu")
    g = ctypes.c_void_p()
    hip.ok(lib.ehip_graph_end(ctypes.byref(g)), "end")
    assert lib.ehip_capturing() == 0
    r = np.random.default_rng(5)
    for rep in range(4):
        av = r.standard_normal(n).astype(np.float32)
        bv = r.standard_normal(n).astype(np.float32)
        a.copy_(torch.from_numpy(av))
        b.copy_(torch.from_numpy(bv))
        torch.cuda.synchronize()
        hip.ok(lib.ehip_graph_launch(g, None), "launch")
        got = read(hip, hip.p(y), n)
        want = np.maximum(av + bv, np.float32(0))
        np.testing.assert_array_equal(got, want, err_msg=f"replay {rep}")
    hip.ok(lib.ehip_graph_destroy(g), "destroy")
    assert hip.launched() - before == 6  # two recorded kernels, four graph launches


def test_graph_holds_its_blocks(hip):
    """A block handed out during the capture and freed there is held for the graph: eager
    allocations do not receive it while the graph lives, so a replay cannot overwrite them."""
    print_case("graph-arena")
    lib = hip.lib
    n = 4096
    hip.ok(lib.ehip_synchronize(), "sync")
    hip.ok(lib.ehip_graph_begin(), "begin")
    p = ctypes.c_void_p()
    hip.ok(lib.ehip_arena_alloc(n * 4, ctypes.byref(p)), "alloc in capture")
    hip.ok(lib.ehip_fill_f32(p, n, 1.0, None), "fill in capture")
    lib.ehip_arena_free(p)
    g = ctypes.c_void_p()
    hip.ok(lib.ehip_graph_end(ctypes.byref(g)), "end")
    st = hip.arena_stats()
    assert st.bytes_graph_held >= n * 4
    mine = []
    for _ in range(8):  # every cached block of the class, had p gone back to the cache
        q = ctypes.c_void_p()
        hip.ok(lib.ehip_arena_alloc(n * 4, ctypes.byref(q)), "eager alloc")
        assert q.value != p.value
        hip.ok(lib.ehip_fill_f32(q, n, 2.0, None), "eager fill")
        mine.append(q)
    hip.ok(lib.ehip_graph_launch(g, None), "launch")
    np.testing.assert_array_equal(read(hip, p.value, n), np.ones(n, np.float32))
    for q in mine:
        np.testing.assert_array_equal(read(hip, q.value, n), np.full(n, 2.0, np.float32))
        lib.ehip_arena_free(q)
    hip.ok(lib.ehip_graph_destroy(g), "destroy")
    assert hip.arena_stats().bytes_graph_held == 0


def test_store_values(hip):
    """ehip_store_f32 writes up to 16 host values through the kernel arguments, exactly,
    also into a graph (each replay stores the values of the capture)."""
    print_case("store")
    lib = hip.lib
    buf = ctypes.c_void_p()
    hip.ok(lib.ehip_arena_alloc(64 * 4, ctypes.byref(buf)), "alloc")
    hip.ok(lib.ehip_fill_f32(buf, 64, -1.0, None), "fill")
    vals = np.array([1.5, -0.0, np.float32(1e-45), 3e38, np.inf, -7.25, 0.1] + [2.0] * 9,
                    np.float32)
    hip.ok(lib.ehip_store_f32(buf, vals.ctypes.data, 7, None), "store 7")
    got = read(hip, buf.value, 64)
    np.testing.assert_array_equal(got[:7].view(np.uint32), vals[:7].view(np.uint32))
    np.testing.assert_array_equal(got[7:], np.full(57, -1.0, np.float32))
    hip.ok(lib.ehip_graph_begin(), "begin")
    hip.ok(lib.ehip_store_f32(buf, vals.ctypes.data, 16, None), "store 16 in capture")
    g = ctypes.c_void_p()
    hip.ok(lib.ehip_graph_end(ctypes.byref(g)), "end")
    vals[:] = 9.0  # the capture keeps the values it saw
    for _ in range(2):
        hip.ok(lib.ehip_fill_f32(buf, 64, -1.0, None), "fill")
        hip.ok(lib.ehip_graph_launch(g, None), "launch")
        got = read(hip, buf.value, 64)
        assert got[0] == 1.5 and np.all(got[7:16] == 2.0) and np.all(got[16:] == -1.0)
    hip.ok(lib.ehip_graph_destroy(g), "destroy")
    assert lib.ehip_store_f32(buf, vals.ctypes.data, 17, None) != 0
    assert lib.ehip_store_f32(None, vals.ctypes.data, 3, None) != 0
    hip.ok(lib.ehip_store_f32(None, None, 0, None), "store nothing")
    lib.ehip_arena_free(buf)


def test_graph_refuses_host_work(hip):
    """Host transfers, synchronisation, trimming and nested captures are refused during a
    capture, which goes on; an aborted capture leaves nothing behind."""
    print_case("graph-refusals")
    lib = hip.lib
    buf = ctypes.c_void_p()
    hip.ok(lib.ehip_arena_alloc(1024, ctypes.byref(buf)), "alloc")
    host = np.zeros(256, np.float32)
    hip.ok(lib.ehip_graph_begin(), "begin")
    try:
        assert lib.ehip_memcpy_h2d(buf, host.ctypes.data, 1024, None) != 0
        assert "graph" in hip.error()
        assert lib.ehip_memcpy_d2h(host.ctypes.data, buf, 1024, None) != 0
        assert lib.ehip_synchronize() != 0
        assert lib.ehip_arena_trim() != 0
        assert lib.ehip_graph_begin() != 0
        assert lib.ehip_capturing() == 1
    finally:
        hip.ok(lib.ehip_graph_abort(), "abort")
    assert lib.ehip_capturing() == 0
    lib.ehip_arena_free(buf)
    assert hip.arena_stats().bytes_graph_held == 0
    g = ctypes.c_void_p()
    assert lib.ehip_graph_end(ctypes.byref(g)) != 0 and not g.value
    assert lib.ehip_graph_launch(None, None) != 0


def test_graph_noalloc_split_gemm(hip):
    """The allocation-free GEMM recorded into a graph (a caller it exists for): a split-K
    product whose partials live in the library's fixed device array replays on new inputs
    with the bits of the allocating call, also with eager allocation-free products using
    the same array between the replays."""
    import torch
    print_case("graph-noalloc")
    lib = hip.lib
    m = n = 256
    k = 4096  # four 128 x 128 tiles: K split sixteen ways
    r = np.random.default_rng(9)
    a = torch.from_numpy(r.standard_normal((k, m), dtype=np.float32)).cuda()
    b = torch.from_numpy(r.standard_normal((k, n), dtype=np.float32)).cuda()
    c, other = hip.f32((m, n)), hip.f32((m, n))
    torch.cuda.synchronize()

    def noalloc(out, x):
        return lib.ehip_gemm_f32_noalloc(1, 0, 1, m, n, k, hip.p(x), m, 0, hip.p(b), n, 0, 0.0,
                                         hip.p(out), n, 0, None)

    hip.ok(lib.ehip_graph_begin(), "begin")
    hip.ok(noalloc(c, a), "noalloc in capture")
    g = ctypes.c_void_p()
    hip.ok(lib.ehip_graph_end(ctypes.byref(g)), "end")
    for rep in range(3):
        a.copy_(torch.from_numpy(r.standard_normal((k, m), dtype=np.float32)))
        torch.cuda.synchronize()
        hip.ok(lib.ehip_graph_launch(g, None), "launch")
        hip.ok(noalloc(other, b), "eager noalloc between replays")
        want = hip.gemm(a, b, trans_a=True)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(c.cpu().numpy().view(np.uint32),
                                      want.cpu().numpy().view(np.uint32), err_msg=f"replay {rep}")
    hip.ok(lib.ehip_graph_destroy(g), "destroy")


def _pair(eng, kind):
    from engine_capi import Trainer
    import workloads as W
    if kind == "cnn":
        x, labels, params = W.cnn_inputs()
        return [Trainer.cnn(eng, x, labels, params, lr=1e-3) for _ in range(2)]
    b, s, vocab, d, h, ff, layers = W.CHARLM_CFG3
    ids, targets = W.lm_inputs(3, b, s, vocab)
    params = W.lm_init_params(11, vocab, d, ff, layers)
    return [Trainer.charlm(eng, ids, targets, vocab, d, h, ff, layers, params, lr=1e-3)
            for _ in range(2)]


@pytest.mark.parametrize("kind", ["cnn", "charlm"])
def test_trainer_graph_steps_match_eager(eng, hip, kind):
    """cfg 2's CNN and cfg 3's character Transformer: eight graph-mode steps (one eager, one
    capture + replay, six replays) against eight eager steps of a twin trainer, loss by loss
    and parameter by parameter, exactly; then graph mode off and two more eager steps."""
    print_case("trainer-graph", kind)
    graphed, eager = _pair(eng, kind)
    graphed.set_graph(True)
    try:
        for step in range(8):
            before = hip.launched()
            graphed.step()
            launches = hip.launched() - before
            if step >= 2:  # Adam's three device scalars stored, then the replay
                assert launches == 2, f"step {step}: {launches} launches"
            eager.step()  # eager work between replays
            lg, le = graphed.loss(), eager.loss()
            assert lg == le, f"{kind} step {step}: loss {lg!r} != {le!r}"
            if step in (1, 2, 7):
                np.testing.assert_array_equal(graphed.params(), eager.params(),
                                              err_msg=f"{kind} step {step}")
        graphed.set_graph(False)
        for step in range(2):
            graphed.step()
            eager.step()
        assert graphed.loss() == eager.loss()
        np.testing.assert_array_equal(graphed.params(), eager.params())
    finally:
        graphed.close()
        eager.close()
    assert hip.arena_stats().bytes_graph_held == 0
