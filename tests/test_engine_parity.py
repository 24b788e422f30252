"""Layer- and model-level parity of the C++ engine on the GPU.

Two anchors, as in the reference's own suite:
  - the 23 PyTorch-replay fixtures (tests/test_reference.cpp of the reference), at the
    reference's tolerance: 1e-4 absolute, 2e-4 for the optimiser trajectory;
  - the reference CPU path on seeded inputs: the oracle restatement composed in
    tests/_compose.py (bit-identical to the compiled reference, see
    test_oracle_vs_ref.py), or the compiled reference itself where it is built, compared
    with the reference's parity metric |d| / max(1, |want|) (tests/_hip.py).
"""
import json
import os

import numpy as np
import pytest

import _compose as K
import _trajectory as TR
from _fixtures import load
from _hip import k_tol, print_case, ref_close, ref_err
from _oracle import Ref, oracle_or_skip, ref_or_skip

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def eng():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test ran without a visible GPU")
    from engine_capi import Engine
    return Engine()


@pytest.fixture(scope="module")
def orc():
    return oracle_or_skip()


@pytest.fixture(scope="module")
def cpu(orc):
    """The fastest bit-exact CPU reference available: the compiled reference if it is
    built, else the restatement through _compose."""
    try:
        r = Ref()
        r.set_threads(8)
        return r
    except (FileNotFoundError, OSError):
        return None


def close(got, want, tol=TOL, what=""):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    dev = float(np.max(np.abs(got - want))) if got.size else 0.0
    assert dev <= tol, f"{what}: largest deviation {dev:.3e} > {tol}"


# ------------------------------------------------------------------ fixtures

def test_fixture_matmul(eng):
    print_case("fixture matmul")
    f = load("matmul")
    c, da, db = eng.matmul_fwd_bwd(f["a"], f["b"], f["grad_output"])
    close(c, f["output"], what="C")
    close(da, f["grad.a"], what="dA")
    close(db, f["grad.b"], what="dB")
    for name in ("matmul_batched", "matmul_shared"):
        f = load(name)
        close(eng.matmul(f["a"], f["b"]), f["output"], what=name)


@pytest.mark.parametrize("name", ["softmax", "softmax_3d"])
def test_fixture_softmax(eng, name):
    print_case("fixture", name)
    f = load(name)
    x = f["input"]
    y, dx = eng.unary_fwd_bwd("softmax", x.reshape(-1, x.shape[-1]),
                              f["grad_output"].reshape(-1, x.shape[-1]))
    close(y.reshape(x.shape), f["output"], what="y")
    close(dx.reshape(x.shape), f["grad.input"], what="dx")


def test_fixture_relu(eng):
    print_case("fixture relu")
    f = load("act_relu")
    x = f["input"]
    y, dx = eng.unary_fwd_bwd("relu", x.reshape(-1, x.shape[-1]),
                              f["grad_output"].reshape(-1, x.shape[-1]))
    close(y.reshape(x.shape), f["output"])
    close(dx.reshape(x.shape), f["grad.input"])


@pytest.mark.parametrize("tag,axis", [("sum0", 0), ("sum1", 1)])
def test_fixture_reductions(eng, tag, axis):
    print_case("fixture reductions", tag)
    f = load("reductions")
    y, dx = eng.sum_axis_fwd_bwd(f["input"], axis, f["grad_output." + tag])
    close(y, f["output." + tag])
    close(dx, f["grad." + tag])


@pytest.mark.parametrize("name", ["linear", "linear_3d"])
def test_fixture_linear(eng, name):
    print_case("fixture", name)
    f = load(name)
    y, dx, dw, db = eng.linear_fwd_bwd(f["input"], f["weight"], f["bias"], f["grad_output"])
    close(y, f["output"], what="y")
    close(dx, f["grad.input"], what="dx")
    close(dw, f["grad.weight"], what="dw")
    close(db.reshape(f["grad.bias"].shape), f["grad.bias"], what="db")


@pytest.mark.parametrize("name,stride,pad", [("conv2d_pad1", 1, 1), ("conv2d_stride2", 2, 0)])
def test_fixture_conv2d(eng, name, stride, pad):
    print_case("fixture", name)
    f = load(name)
    y, dx, dw, db = eng.conv2d_fwd_bwd(f["input"], f["weight"], f["bias"], stride, pad,
                                       f["grad_output"])
    close(y, f["output"], what="y")
    close(dx, f["grad.input"], what="dx")
    close(dw, f["grad.weight"], what="dw")
    close(db, f["grad.bias"], what="db")


def test_fixture_maxpool(eng):
    print_case("fixture maxpool")
    f = load("maxpool2d")
    y, dx = eng.maxpool_fwd_bwd(f["input"], 2, 2, f["grad_output"])
    close(y, f["output"], 0.0)
    close(dx, f["grad.input"], 0.0)


def test_fixture_layernorm(eng):
    print_case("fixture layernorm")
    f = load("layernorm")
    y, dx, dg, db = eng.layernorm_fwd_bwd(f["input"], f["gamma"], f["beta"], f["grad_output"])
    close(y, f["output"])
    close(dx, f["grad.input"])
    close(dg, f["grad.gamma"])
    close(db, f["grad.beta"])


def test_fixture_cross_entropy(eng):
    print_case("fixture cross_entropy")
    f = load("cross_entropy")
    loss, dl = eng.cross_entropy(f["logits"], f["targets"].astype(np.int64))
    close(np.float32(loss).reshape(f["output"].shape), f["output"])
    close(dl, f["grad.logits"])


@pytest.mark.parametrize("name", ["attention", "attention_causal"])
def test_fixture_attention(eng, name):
    print_case("fixture", name)
    f = load(name)
    mask = f["mask"] if name == "attention_causal" else None
    y, w, dq, dk, dv = eng.attention_fwd_bwd(f["q"], f["k"], f["v"], mask, f["grad_output"])
    close(y, f["output"], what="y")
    close(w, f["weights"], what="weights")
    close(dq, f["grad.q"], what="dq")
    close(dk, f["grad.k"], what="dk")
    close(dv, f["grad.v"], what="dv")


def test_fixture_multihead_attention(eng):
    print_case("fixture multihead_attention")
    f = load("multihead_attention")
    tags = ("query", "key", "value", "out")
    params = np.concatenate([np.concatenate([f[f"w.{t}.weight"].ravel(), f[f"w.{t}.bias"].ravel()])
                             for t in tags])
    y, dx, dp = eng.mha_fwd_bwd(f["input"], 2, params, f["grad_output"])
    close(y, f["output"], what="y")
    close(dx, f["grad.input"], what="dx")
    off = 0
    for t in tags:
        for part in ("weight", "bias"):
            want = f[f"grad.{t}.{part}"]
            close(dp[off:off + want.size].reshape(want.shape), want, what=f"{t}.{part}")
            off += want.size


BLOCK_NAMES = ["norm1.gamma", "norm1.beta", "norm2.gamma", "norm2.beta", "query.weight",
               "query.bias", "key.weight", "key.bias", "value.weight", "value.bias",
               "out.weight", "out.bias", "ff1.weight", "ff1.bias", "ff2.weight", "ff2.bias"]


def test_fixture_transformer_block(eng):
    print_case("fixture transformer_block")
    f = load("transformer_block")
    params = np.concatenate([f["w." + n].ravel() for n in BLOCK_NAMES])
    x = f["input"]
    ff = f["w.ff1.weight"].shape[1]
    y, dx, dp = eng.block_fwd_bwd(x, 2, ff, False, params, f["grad_output"])
    close(y, f["output"], what="y")
    close(dx, f["grad.input"], what="dx")
    off = 0
    for n in BLOCK_NAMES:
        want = f["grad." + n]
        close(dp[off:off + want.size].reshape(want.shape), want, what=n)
        off += want.size


@pytest.mark.parametrize("max_norm", [0.5, 1e6])
def test_clip_grad_norm_vs_reference(eng, max_norm):
    """optim::clip_grad_norm (src/optim.cpp:168-208) against the compiled reference: one
    global norm over every gradient (a parameter without one is skipped), scaled by
    max_norm / (norm + 1e-6) only when the norm exceeds max_norm."""
    from _oracle import ref_or_skip
    ref = ref_or_skip()
    print_case("clip-grad-norm", max_norm)
    r = np.random.default_rng(12)
    sizes = [1000, -37, 4096, 3, 70001]
    n = sum(s for s in sizes if s > 0)
    g = r.standard_normal(n).astype(np.float32)
    norm, clipped = eng.clip_grad_norm(g, sizes, max_norm)
    want_norm, want = ref.clip_grad_norm(g, sizes, max_norm)
    exact64 = float(np.sqrt((g.astype(np.float64) ** 2).sum()))
    assert abs(norm - want_norm) <= 1e-6 * want_norm, (norm, want_norm)
    assert abs(norm - exact64) <= 1e-6 * exact64
    ref_close(clipped, want, 1e-6, "clipped gradients")
    if max_norm >= exact64:
        np.testing.assert_array_equal(clipped, g)  # no clipping: untouched


def test_fixture_adam_trajectory(eng):
    print_case("fixture adam")
    f = load("adam")
    traj = eng.mse_adam(f["initial"], f["target"], 10, 0.1)
    for step in range(10):
        close(traj[step].reshape(f["initial"].shape), f[f"step.{step}"], 2e-4, f"step {step}")


# ------------------------------------------------------------------ seeded, vs the CPU path

def rng(seed):
    return np.random.default_rng(seed)


def test_conv2d_cfg2_shapes(eng, orc):
    """cfg 2's second convolution (8 -> 16, 14x14, pad 1) at batch 64."""
    print_case("conv cfg2")
    r = rng(21)
    x = r.standard_normal((64, 8, 14, 14), dtype=np.float32)
    w = r.standard_normal((16, 8, 3, 3), dtype=np.float32) * 0.2
    b = r.standard_normal(16, dtype=np.float32)
    dy = r.standard_normal((64, 16, 14, 14), dtype=np.float32)
    y, dx, dw, db = eng.conv2d_fwd_bwd(x, w, b, 1, 1, dy)
    wy, cache = K.conv2d_fwd(orc, x, w, b, 1, 1)
    wdx, wdw, wdb = K.conv2d_bwd(orc, dy, cache)
    ref_close(y, wy, k_tol(72), "y")
    ref_close(dx, wdx, k_tol(16 * 9), "dx")
    ref_close(dw, wdw, k_tol(64 * 14 * 14), "dw")
    ref_close(db, wdb, k_tol(64 * 14 * 14), "db")


def test_block_cfg3_shapes(eng, orc):
    """One pre-LN block at cfg 3's width (d 96, 4 heads, FFN 384), causal, batch 4."""
    print_case("block cfg3")
    r = rng(22)
    d, heads, ff, b, s = 96, 4, 384, 4, 64
    n = eng.block_num_params(d, heads, ff)
    params = r.standard_normal(n, dtype=np.float32) * 0.1
    params[:4 * d] = np.tile(np.concatenate([np.ones(d), np.zeros(d)]), 2)  # LN gamma/beta
    x = r.standard_normal((b, s, d), dtype=np.float32)
    dy = r.standard_normal((b, s, d), dtype=np.float32)
    y, dx, dp = eng.block_fwd_bwd(x, heads, ff, True, params, dy)
    p, _ = K.block_params(params, d, ff)
    wy, cache = K.block_fwd(orc, x, p, heads, orc.causal_mask(s))
    wdx, g = K.block_bwd(orc, dy, cache)
    wdp = np.concatenate([g[k].ravel() for k in K.BLOCK_KEYS])
    ref_close(y, wy, k_tol(ff), "y")
    ref_close(dx, wdx, k_tol(b * s), "dx")
    ref_close(dp, wdp, k_tol(b * s), "dparams")


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
@pytest.mark.parametrize("shape_a,shape_b", [((64, 96), (64, 96)), ((33, 7), (7,)),
                                             ((4, 3, 5), (3, 5)), ((1 << 16,), (1 << 16,))])
def test_binary_nodes_vs_reference(eng, op, shape_a, shape_b):
    """The four element-wise nodes forward and backward through the engine (the multiply
    node's backward one fused launch for same shapes) against the compiled reference:
    equal values (a -0.0 that the engine's adopted gradient keeps compares equal to the
    reference's +0.0); the broadcast operand's gradient is a sum over rows, at the K-term
    bound."""
    ref = ref_or_skip()
    print_case("binary node", op, shape_a, shape_b)
    r = rng(len(shape_a) * 10 + len(shape_b))
    a = r.standard_normal(shape_a, dtype=np.float32)
    b = r.standard_normal(shape_b, dtype=np.float32) + (3.0 if op == "div" else 0.0)
    a.ravel()[::9] = 0.0
    dy = r.standard_normal(shape_a, dtype=np.float32)
    y, da, db = eng.binary_fwd_bwd(op, a, b, dy)
    wy, wda, wdb = ref.binary_fwd_bwd(op, a, b, dy)
    assert np.array_equal(y, wy) and np.array_equal(da, wda)
    if shape_a == shape_b:
        assert np.array_equal(db, wdb)
    else:
        ref_close(db, wdb, k_tol(a.size // b.size), "db")


def test_embedding_exact(eng, orc):
    """Gather and its ordered scatter-add are bit-exact with the reference."""
    print_case("embedding")
    r = rng(23)
    table = r.standard_normal((121, 96), dtype=np.float32)
    ids = r.integers(0, 121, (8, 64)).astype(np.float32)
    dy = r.standard_normal((8, 64, 96), dtype=np.float32)
    y, dt = eng.embedding_fwd_bwd(table, ids, dy)
    idx = ids.ravel().astype(np.int64)
    assert np.array_equal(y.reshape(-1, 96).view(np.uint32),
                          orc.select_rows(table, idx).view(np.uint32))
    assert np.array_equal(dt.view(np.uint32),
                          orc.scatter_add_rows(dy.reshape(-1, 96), idx, (121, 96)).view(np.uint32))


def cnn_inputs(seed=2, batch=64):
    r = rng(seed)
    x = r.uniform(0.0, 1.0, (batch, 1, 28, 28)).astype(np.float32)
    labels = r.integers(0, 10, batch)
    params = []
    for shp in K.cnn_param_shapes():  # Kaiming-uniform weights, zero biases
        if len(shp) == 1 or shp[0] == 1:
            params.append(np.zeros(int(np.prod(shp)), np.float32))
        else:
            fan_in = int(np.prod(shp[1:])) if len(shp) == 4 else shp[0]
            lim = np.sqrt(6.0 / fan_in)
            params.append(r.uniform(-lim, lim, int(np.prod(shp))).astype(np.float32))
    return x, labels, np.concatenate(params)


def test_cnn_training_trajectory(eng, orc, cpu):
    """cfg 2: ten Adam steps (lr 1e-3) of the small CNN on one seeded batch. Every step's
    loss within 1e-5 relative of the reference CPU path; with the compiled reference, the
    step-1 gradients of every tensor and the ten steps' updates as tests/_trajectory.py
    states."""
    print_case("cnn train cfg2")
    x, labels, params = cnn_inputs()
    losses, out = eng.cnn_train(x, labels, params, 10, 1e-3)
    if cpu is not None:
        want_losses, want_out = cpu.cnn_train(x, labels, params, 10, 1e-3)
    else:
        want_losses, want_out = K.cnn_train(orc, x, labels, params, 10, 1e-3)
    rel = np.abs(losses - want_losses) / np.abs(want_losses)
    print("cnn loss rel err per step:", rel)
    assert np.all(rel <= 1e-5), rel
    if cpu is not None:
        loss, g = eng.cnn_grads(x, labels, params)
        want_loss, want_g = cpu.cnn_grads(x, labels, params)
        assert abs(loss - want_loss) <= 1e-5 * abs(want_loss)
        layout = TR.cnn_layout()
        TR.check_gradients(g, want_g, layout, 64 * 28 * 28, "cnn")
        TR.check_updates(params, out, want_out, want_g, layout, 1e-3, 10, "cnn")


def lm_trajectory(eng, orc, cpu, dims, seed, steps, xavier, what, golden=None):
    """Ten (or STEPS) Adam steps of the character model through the engine against the
    compiled reference (or the restatement, fewer steps, when that is not built). Per-step
    losses within 1e-5 relative, or, with GOLDEN (a tests/golden JSON holding the reference's
    Release and FMA-contracted loss curves of this workload), within twice the distance
    between those two curves where that is larger; the live reference must reproduce the
    golden's Release curve bit for bit, so the bound belongs to these inputs."""
    vocab, d, heads, ff, layers, b, s = dims
    shapes = K.charlm_param_shapes(vocab, d, ff, layers)
    assert sum(int(np.prod(p)) for p in shapes) == eng.charlm_num_params(vocab, s, d, heads, ff,
                                                                         layers)
    params, ids, targets = TR.lm_case(dims, seed, xavier, shapes)
    if cpu is None:  # the restatement is slow: fewer steps, losses only
        steps = min(steps, 3 if d < 128 else 1)
    losses, out, g0 = eng.charlm_train(ids, targets, vocab, d, heads, ff, layers, params, steps,
                                       1e-3, grads0=True)
    if cpu is not None:
        want, want_out, want_g0 = cpu.charlm_train(ids, targets, vocab, d, heads, ff, layers,
                                                   params, steps, 1e-3, grads0=True)
    else:
        want, want_out = K.charlm_train(orc, ids, targets, params, vocab, d, heads, ff, layers,
                                        steps, 1e-3)
    rel = np.abs(losses - want) / np.abs(want)
    bound = np.full(len(want), 1e-5)
    if golden is not None:
        with open(os.path.join(os.path.dirname(__file__), "golden", golden)) as f:
            g = json.load(f)
        assert tuple(g["dims"]) == tuple(dims) and g["seed"] == seed and g["steps"] >= steps
        if cpu is not None:
            assert np.array_equal(np.asarray(want, np.float32),
                                  np.asarray(g["losses"][:steps], np.float32)), (want, g["losses"])
        bound = TR.loss_bounds(g["losses"][:len(want)], g["losses_fma"][:len(want)])
    print(f"{what} loss rel err per step:", rel)
    print(f"{what} bound per step:        ", bound)
    assert np.all(rel <= bound), (rel, bound)
    if cpu is not None:
        layout = TR.lm_layout(vocab, d, ff, layers)
        TR.check_gradients(g0, want_g0, layout, b * s, what)
        TR.check_updates(params, out, want_out, want_g0, layout, 1e-3, steps, what)


def test_charlm_training_trajectory(eng, orc, cpu):
    """cfg 3: the character Transformer (2 blocks, d 96, 4 heads, FFN 384, context 64,
    vocab 121, batch 32), ten Adam steps; per-step loss within 1e-5 relative, step-1
    gradients and the updates as tests/_trajectory.py states."""
    print_case("charlm train cfg3")
    lm_trajectory(eng, orc, cpu, (121, 96, 4, 384, 2, 32, 64), 3, 10, False, "charlm",
                  golden="cfg3_reference.json")


def test_charlm_trajectory_separate_bias_sums(eng, orc, cpu):
    """The cfg 3 trajectory with every bias gradient from the separate column sum
    (nn::set_fused_bias_grad(false)) instead of the default, where the mid-sized layers take
    theirs from the weight-gradient products' column sums: both orders hold the per-step
    losses within 1e-5 relative and pass the gradient and update checks."""
    print_case("charlm train cfg3, separate bias sums")
    prev = eng.set_fused_bias_grad(False)
    try:
        lm_trajectory(eng, orc, cpu, (121, 96, 4, 384, 2, 32, 64), 3, 10, False,
                      "charlm separate-db", golden="cfg3_reference.json")
    finally:
        eng.set_fused_bias_grad(prev)


def test_transformer_medium_trajectory(eng, orc, cpu):
    """A deeper, wider stack than cfg 3 (4 pre-LN blocks, d 256, 8 heads, FFN 1024, context
    128, vocab 256, batch 8), so the larger GEMM tiles and longer reductions run inside a
    training step; three Adam steps, checked as the cfg 3 trajectory."""
    print_case("transformer medium")
    lm_trajectory(eng, orc, cpu, (256, 256, 8, 1024, 4, 8, 128), 5, 3, True, "medium")


# ------------------------------------------------------------------ checkpoints

def test_checkpoint_interop_with_reference(eng, tmp_path):
    """Parameters saved by the engine load in the compiled reference (strict names and
    shapes, the reference's weight format) with the same bits, and the other way round."""
    from engine_capi import Trainer
    from _oracle import ref_or_skip
    ref = ref_or_skip()
    print_case("checkpoint interop")
    x, labels, params = cnn_inputs()
    tr = Trainer.cnn(eng, x, labels, params, lr=1e-3)
    for _ in range(3):
        tr.step()
    p3 = tr.params()
    path = str(tmp_path / "engine.cppaieng")
    tr.save(path)
    np.testing.assert_array_equal(ref.cnn_load(path, p3.size), p3)
    q = (rng(41).standard_normal(p3.size) * 0.1).astype(np.float32)
    path2 = str(tmp_path / "reference.cppaieng")
    ref.cnn_save(q, path2)
    tr2 = Trainer.cnn(eng, x, labels, None, lr=1e-3)
    tr2.load(path2)
    np.testing.assert_array_equal(tr2.params(), q)
    tr.close()
    tr2.close()


def test_checkpoint_exact_resume(eng, tmp_path):
    """Six Adam steps in one run equal three steps, a save of the parameters and the Adam
    state, a load into a freshly initialised trainer and three more steps -- bit for bit."""
    from engine_capi import Trainer
    print_case("checkpoint resume")
    x, labels, params = cnn_inputs()
    whole = Trainer.cnn(eng, x, labels, params, lr=1e-3)
    for _ in range(6):
        whole.step()
    want = whole.params()
    first = Trainer.cnn(eng, x, labels, params, lr=1e-3)
    for _ in range(3):
        first.step()
    pp, op = str(tmp_path / "p.cppaieng"), str(tmp_path / "adam.cppaieng")
    first.save(pp, op)
    second = Trainer.cnn(eng, x, labels, None, lr=1e-3)
    second.load(pp, op)
    for _ in range(3):
        second.step()
    np.testing.assert_array_equal(second.params(), want)
    for t in (whole, first, second):
        t.close()


def test_checkpoint_refuses_bad_files(eng, tmp_path):
    """A truncated file, another format and a shape mismatch are errors, not crashes."""
    from engine_capi import Trainer
    print_case("checkpoint refusals")
    x, labels, params = cnn_inputs()
    tr = Trainer.cnn(eng, x, labels, params, lr=1e-3)
    good = tmp_path / "good.cppaieng"
    tr.save(str(good))
    data = good.read_bytes()
    bad = tmp_path / "truncated.cppaieng"
    bad.write_bytes(data[: len(data) // 2])
    with pytest.raises(RuntimeError, match="ends inside"):
        tr.load(str(bad))
    other = tmp_path / "other.bin"
    other.write_bytes(b"NOTAFILE" + data[8:])
    with pytest.raises(RuntimeError, match="not a CPPAIENG"):
        tr.load(str(other))
    small = Trainer.cnn(eng, x, labels, None, lr=1e-3, c1=4)
    with pytest.raises(RuntimeError, match="has no tensor"):  # names carry the layer shapes
        small.load(str(good))
    # Same names, same value count, another shape: the first tensor's (8, 1, 3, 3) -> (8, 1, 9, 1).
    import struct
    name_len = struct.unpack_from("<I", data, 16)[0]
    dims_at = 16 + 4 + name_len + 4
    assert struct.unpack_from("<4Q", data, dims_at) == (8, 1, 3, 3)
    reshaped = bytearray(data)
    struct.pack_into("<4Q", reshaped, dims_at, 8, 1, 9, 1)
    odd = tmp_path / "reshaped.cppaieng"
    odd.write_bytes(bytes(reshaped))
    with pytest.raises(RuntimeError, match="in the model and"):
        tr.load(str(odd))
    tr.close()
    small.close()


# ------------------------------------------------------------------ dropout

@pytest.mark.parametrize("p", [0.1, 0.5])
def test_dropout_module(eng, orc, p):
    """nn::Dropout after manual_seed(s): the first draw is the generator's mask at offset
    0 (the Philox restatement), y = x * mask and dx = dy * mask bit for bit; in evaluation
    mode the layer is the identity and passes the gradient through."""
    print_case("dropout module", p)
    r = rng(8)
    n = 10007
    x, dy = r.standard_normal(n).astype(np.float32), r.standard_normal(n).astype(np.float32)
    y, dx = eng.dropout_fwd_bwd(x, p, 2024, dy)
    want_y, m = orc.dropout(x, p, 2024, 0)
    np.testing.assert_array_equal(y, want_y)
    np.testing.assert_array_equal(dx, (dy * m).astype(np.float32))
    y2, dx2 = eng.dropout_fwd_bwd(x, p, 2024, dy, eval_mode=True)
    np.testing.assert_array_equal(y2, x)
    np.testing.assert_array_equal(dx2, dy)
