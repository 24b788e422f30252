"""Checks of a training trajectory against the compiled reference: step-1 gradients of every
parameter tensor, then the Adam updates the trajectory made.

Why updates and not parameters element by element: Adam's step lr m / (sqrt(v) + eps)
normalises each gradient element, so rounding-level differences between two summation orders
(GPU tiles against the reference's serial loops) reach every parameter at about their relative
size (1e-7 .. 1e-4), and a parameter that moved by a large fraction of its own value (embedding
rows, LayerNorm betas and biases starting at 0) then differs by more than 1e-5 of its value
although the update agrees to 1e-4. The update vector, final minus initial, is what the
gradients determine, so it is what is compared.

Gradients that vanish in exact arithmetic: the attention key projection's bias. Adding a
vector c to every key of a sequence adds q.c to every score of a query row, which the row
softmax removes, so dL/db_key = 0 identically (src/transformer.cpp:279-304, 332-358). Both
engines produce rounding noise there (about 1e-9 against gradients of order 1e-2), and Adam
turns noise of either sign into steps of +-lr, so those updates are not comparable; the check
is instead that both sides' gradients are at that noise floor.
"""
import numpy as np

from _hip import k_tol, ref_close

GRAD_REL = 1e-3      # per tensor: |g - g_ref| / |g_ref| (L2); measured <= 1e-4
GRAD_ELEM = 1e-2     # per element: |g - g_ref| <= GRAD_ELEM * rms(g_ref) of its tensor
UPDATE_REL = 1e-2    # per tensor: |u - u_ref| / |u_ref| (L2) over well-conditioned elements
ELEMENT_UPD = 1e-2   # well-conditioned element: |u - u_ref| <= ELEMENT_UPD * lr * steps ...
OUTLIERS = 1e-3      # ... for all but this fraction of a tensor's (at least one element)
WELL = 1e-3          # well-conditioned element: |g_ref| >= WELL * rms(g_ref) of its tensor
ZERO_FLOOR = 1e-5    # vanishing gradient: max |g| <= ZERO_FLOOR * max |g| of the key weight


def cnn_layout(c1=8, c2=16, classes=10, flat=784):
    return [("conv1.weight", (c1, 1, 3, 3)), ("conv1.bias", (c1,)),
            ("conv2.weight", (c2, c1, 3, 3)), ("conv2.bias", (c2,)),
            ("linear.weight", (flat, classes)), ("linear.bias", (1, classes))]


def lm_layout(vocab, d, ff, layers):
    import workloads as W
    return [(n, s) for n, s, _ in W.lm_param_layout(vocab, d, ff, layers)]


def lm_case(dims, seed, xavier, param_shapes):
    """The seeded inputs of a language-model trajectory: parameters (LayerNorm gamma 1 and
    beta 0, biases 0, weights Xavier-uniform or normal with std 0.02 for the vocabulary
    rows and sqrt(2 / fan_in) otherwise), then tokens and targets, all from one generator."""
    vocab, d, heads, ff, layers, b, s = dims
    r = np.random.default_rng(seed)
    params = []
    for shp in param_shapes:
        size = int(np.prod(shp))
        if len(shp) == 1:  # LayerNorm: gamma 1, beta 0, in that order per norm
            params.append(np.ones(size, np.float32) if len(params) % 2 == 1 else
                          np.zeros(size, np.float32))
        elif shp[0] == 1:
            params.append(np.zeros(size, np.float32))
        elif xavier:
            lim = np.sqrt(6.0 / (shp[0] + shp[1]))
            params.append(r.uniform(-lim, lim, size).astype(np.float32))
        else:
            params.append((r.standard_normal(size) * (0.02 if shp[0] == vocab else
                                                      np.sqrt(2.0 / shp[0]))).astype(np.float32))
    ids = r.integers(0, vocab, (b, s)).astype(np.float32)
    targets = r.integers(0, vocab, b * s)
    return np.concatenate(params), ids, targets


def loss_bounds(ref, ref_fma, floor=1e-5, factor=2.0):
    """Per-step relative bound on a trajectory's losses: the floor, or FACTOR times how far
    the reference's own FMA-contracted build (another valid fp32 rounding of the same
    source) moved that step's loss, whichever is larger. Past a few Adam steps a training
    trajectory amplifies rounding, so two correct engines drift apart by that much."""
    ref, ref_fma = np.asarray(ref, np.float64), np.asarray(ref_fma, np.float64)
    return np.maximum(floor, factor * np.abs(ref_fma - ref) / np.abs(ref))


def vanishing(name):
    return name.endswith("attn.key.bias")


def split(flat, layout):
    out, off = {}, 0
    for name, shape in layout:
        n = int(np.prod(shape))
        out[name] = np.asarray(flat[off:off + n], np.float64)
        off += n
    assert off == len(flat), (off, len(flat))
    return out


def check_gradients(got, want, layout, reduce_len, what):
    """Step-1 gradients, every tensor: the reference's metric |d| / max(1, |want|) at the
    K-term bound k_tol(reduce_len), and, because gradients are mostly far below 1 where that
    metric is an absolute one, |d| / |want| <= GRAD_REL in the L2 norm and every element
    within GRAD_ELEM of the tensor's rms gradient (both engines start from the same
    parameters here, so no element may stray); vanishing gradients at the noise floor on
    both sides."""
    g, w = split(got, layout), split(want, layout)
    worst = worst_elem = 0.0
    for name, _ in layout:
        if vanishing(name):
            key_w = name.replace("bias", "weight")
            floor = ZERO_FLOOR * np.abs(w[key_w]).max()
            assert np.abs(g[name]).max() <= floor and np.abs(w[name]).max() <= floor, \
                f"{what} {name}: a gradient that vanishes identically is above the noise floor"
            continue
        ref_close(g[name], w[name], k_tol(reduce_len), f"{what} gradient {name}")
        nw = np.linalg.norm(w[name])
        ratio = np.linalg.norm(g[name] - w[name]) / nw if nw > 0 else np.linalg.norm(g[name])
        worst = max(worst, ratio)
        assert ratio <= GRAD_REL, f"{what} gradient {name}: |d| / |g| = {ratio:.3e}"
        rms = np.sqrt(np.mean(w[name] ** 2))
        elem = np.abs(g[name] - w[name]).max() / rms if rms > 0 else np.abs(g[name]).max()
        worst_elem = max(worst_elem, elem)
        assert elem <= GRAD_ELEM, f"{what} gradient {name}: an element is {elem:.3e} rms off"
    print(f"{what}: step-1 gradients, worst |d| / |g| per tensor {worst:.2e}, worst element "
          f"{worst_elem:.2e} rms")
    return worst


def check_updates(p0, got, want, grads0, layout, lr, steps, what):
    """Final parameters after `steps` Adam steps from p0, as updates u = p - p0 against the
    reference's. Per tensor (vanishing-gradient tensors excepted), over its well-conditioned
    elements (|g0| >= WELL rms(g0), where rounding noise is under 0.1 % of the gradient):
    |u - u_ref| / |u_ref| <= UPDATE_REL in the L2 norm, and all but a fraction OUTLIERS of
    them within ELEMENT_UPD lr steps. A few elements may legitimately go further: a ReLU
    whose pre-activation lies within rounding of zero can take the other branch in one
    engine once the parameters differ by rounding, which changes that position's
    contribution to later gradients. Every element of every tensor within 2 lr steps
    (Adam's reach)."""
    P0, G, W, G0 = split(p0, layout), split(got, layout), split(want, layout), split(grads0, layout)
    worst_norm, worst_elem, cond, outliers = 0.0, 0.0, 0, 0
    total = 0
    for name, _ in layout:
        d = np.abs(G[name] - W[name])
        assert d.max() <= 2 * lr * steps, f"{what} {name}: beyond Adam's reach"
        total += d.size
        if vanishing(name):
            continue
        g0 = G0[name]
        rms = np.sqrt(np.mean(g0 ** 2))
        well = np.abs(g0) >= WELL * rms if rms > 0 else np.zeros(g0.shape, bool)
        cond += int(well.sum())
        if not well.any():
            continue
        u, uw = G[name][well] - P0[name][well], W[name][well] - P0[name][well]
        ratio = np.linalg.norm(u - uw) / max(np.linalg.norm(uw), 1e-30)
        off = np.abs(u - uw) / (lr * steps)
        far = int(np.sum(off > ELEMENT_UPD))
        worst_norm, worst_elem = max(worst_norm, ratio), max(worst_elem, off.max())
        outliers += far
        assert ratio <= UPDATE_REL, f"{what} {name}: |u - u_ref| / |u_ref| = {ratio:.3e}"
        assert far <= max(1, int(OUTLIERS * off.size)), \
            f"{what} {name}: {far} of {off.size} updates beyond {ELEMENT_UPD} lr steps"
    print(f"{what}: updates after {steps} steps, worst |du| / |u| per tensor {worst_norm:.2e}, "
          f"{outliers} of {cond} well-conditioned elements beyond {ELEMENT_UPD} lr steps "
          f"(worst {worst_elem:.2e}; {total} elements in all)")
    return worst_norm, worst_elem
