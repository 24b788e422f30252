"""The trajectory checks the GPU tests apply (tests/_trajectory.py) can fail: they accept the
oracle's training run, which equals the compiled reference bit for bit, and reject the same
run with one mistake planted in the oracle, on the CPU -- the LayerNorm beta gradient missing
its last row's term (a dropped term in one reduction, src/transformer.cpp:123-150).
"""
import numpy as np
import pytest

import _compose as K
import _trajectory as TR
from _oracle import oracle_or_skip, ref_or_skip

DIMS = (11, 16, 2, 32, 2, 4, 8)  # vocab, d, heads, ff, layers, batch, seq
STEPS, LR = 3, 1e-3


class DroppedRow:
    """The oracle, except that LayerNorm's dbeta leaves out the last row."""

    def __init__(self, orc):
        self.orc = orc

    def __getattr__(self, name):
        return getattr(self.orc, name)

    def layernorm_backward(self, dy, xhat, gamma, inv):
        dx, dg, db = self.orc.layernorm_backward(dy, xhat, gamma, inv)
        last = np.asarray(dy, np.float32).reshape(-1, dy.shape[-1])[-1]
        return dx, dg, (db - last).astype(np.float32)


def run(ops, ids, targets, params):
    vocab, d, heads, ff, layers, b, s = DIMS
    shapes = K.charlm_param_shapes(vocab, d, ff, layers)
    _, g0 = K.charlm_loss_and_grads(ops, ids, targets, K.split_flat(params, shapes), vocab, d,
                                    heads, ff, layers, ops.positional_encoding(s, d),
                                    ops.causal_mask(s))
    losses, out = K.charlm_train(ops, ids, targets, params, vocab, d, heads, ff, layers, STEPS,
                                 LR)
    return losses, out, np.concatenate([g.ravel() for g in g0])


@pytest.fixture(scope="module")
def case():
    orc, ref = oracle_or_skip(), ref_or_skip()
    ref.set_threads(4)
    vocab, d, heads, ff, layers, b, s = DIMS
    r = np.random.default_rng(41)
    import workloads as W
    params = W.lm_init_params(41, vocab, d, ff, layers)
    ids = r.integers(0, vocab, (b, s)).astype(np.float32)
    targets = r.integers(0, vocab, b * s)
    want = ref.charlm_train(ids, targets, vocab, d, heads, ff, layers, params, STEPS, LR,
                            grads0=True)
    return orc, ids, targets, params, want


def test_checks_accept_the_oracle(case):
    orc, ids, targets, params, (want_l, want_p, want_g) = case
    losses, out, g0 = run(orc, ids, targets, params)
    layout = TR.lm_layout(*(DIMS[i] for i in (0, 1, 3, 4)))
    TR.check_gradients(g0, want_g, layout, DIMS[5] * DIMS[6], "oracle")
    TR.check_updates(params, out, want_p, want_g, layout, LR, STEPS, "oracle")


def test_checks_reject_a_dropped_term(case):
    orc, ids, targets, params, (want_l, want_p, want_g) = case
    losses, out, g0 = run(DroppedRow(orc), ids, targets, params)
    layout = TR.lm_layout(*(DIMS[i] for i in (0, 1, 3, 4)))
    with pytest.raises(AssertionError, match="norm1.beta|norm2.beta"):
        TR.check_gradients(g0, want_g, layout, DIMS[5] * DIMS[6], "planted")
    with pytest.raises(AssertionError):
        TR.check_updates(params, out, want_p, want_g, layout, LR, STEPS, "planted")
