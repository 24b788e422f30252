"""Forward/backward compositions of the reference's layers, over a pluggable `ops` backend.

Each function restates what the reference's autograd graph computes for one layer or model,
in the reference's own operation sequence and gradient-accumulation order, so that with the
oracle as `ops` the results are bit-identical to the compiled reference (where the order of
three or more accumulated contributions matters, the comment gives it). `ops` is either
tests._oracle.Oracle (the CPU restatement) or a device backend with the same method names.

Reference graph sources:
  matmul fwd/bwd       src/tensor_ops.cpp:475-586
  Linear               src/nn.cpp:101-130
  Conv2d               src/conv.cpp:234-253, 280-338
  MaxPool2d            src/conv.cpp:367-473
  LayerNorm            src/transformer.cpp:82-179
  cross_entropy_loss   src/nn.cpp:324-408
  attention / MHA      src/transformer.cpp:279-358
  TransformerBlock     src/transformer.cpp:392-414
  Embedding            src/transformer.cpp:206-231, src/tensor.cpp:556-604
  Adam                 src/optim.cpp:113-162
"""
import math

import numpy as np


def fold_if(ops, d, shape):
    return d if d.shape == tuple(shape) else ops.fold_leading(d, tuple(shape))


# ---------------------------------------------------------------- dense
def matmul_fwd_bwd(ops, a, b, g):
    c = ops.matmul(a, b)
    da = fold_if(ops, ops.matmul(g, ops.transpose(b)), a.shape)
    db = fold_if(ops, ops.matmul(ops.transpose(a), g), b.shape)
    return c, da, db


def linear_fwd(ops, x, w, bias):
    """Returns (out, cache). x may be (..., in): it is viewed as 2-D rows."""
    flat = x.reshape(-1, w.shape[0])
    mm = ops.matmul(flat, w)
    out = ops.binary("add", mm, bias) if bias is not None else mm
    return out.reshape(x.shape[:-1] + (w.shape[1],)), (flat, w, bias is not None, x.shape)


def linear_bwd(ops, g, cache):
    flat, w, has_bias, xshape = cache
    g2 = g.reshape(-1, w.shape[1])
    db = ops.fold_leading(g2, (1, w.shape[1])) if has_bias else None
    dflat = ops.matmul(g2, ops.transpose(w))
    dw = ops.matmul(ops.transpose(flat), g2)
    return dflat.reshape(xshape), dw, db


# ---------------------------------------------------------------- conv
def conv2d_fwd(ops, x, w, bias, stride, pad):
    n, c, h, wd = x.shape
    oc, _, kh, kw = w.shape
    oh = (h + 2 * pad - kh) // stride + 1
    ow = (wd + 2 * pad - kw) // stride + 1
    cols = ops.im2col(x, kh, kw, stride, pad)
    wt = ops.transpose(w.reshape(oc, c * kh * kw))
    out = ops.matmul(cols, wt)
    if bias is not None:
        out = ops.binary("add", out, bias)
    y = ops.permute(out.reshape(n, oh * ow, oc), (0, 2, 1)).reshape(n, oc, oh, ow)
    return y, (x.shape, w.shape, cols, wt, stride, pad, bias is not None)


def conv2d_bwd(ops, g, cache, need_dx=True):
    xshape, wshape, cols, wt, stride, pad, has_bias = cache
    n = xshape[0]
    oc, c, kh, kw = wshape
    g2 = ops.permute(g.reshape(n, oc, -1), (0, 2, 1)).reshape(-1, oc)
    db = ops.fold_leading(g2, (oc,)) if has_bias else None
    dcols = ops.matmul(g2, ops.transpose(wt)) if need_dx else None
    dwt = ops.matmul(ops.transpose(cols), g2)
    dw = ops.transpose(dwt).reshape(wshape)
    dx = ops.col2im(dcols, xshape, kh, kw, stride, pad) if need_dx else None
    return dx, dw, db


def maxpool_fwd(ops, x, k, stride):
    y, am = ops.maxpool(x, k, stride)
    return y, (am, x.shape)


def maxpool_bwd(ops, g, cache):
    am, xshape = cache
    return ops.maxpool_backward(am, g, xshape)


# ---------------------------------------------------------------- rows
def layernorm_fwd(ops, x, gamma, beta):
    out, xhat, inv = ops.layernorm(x, gamma, beta)
    return out, (xhat, inv, gamma)


def layernorm_bwd(ops, g, cache):
    xhat, inv, gamma = cache
    dx, dg, db = ops.layernorm_backward(g, xhat, gamma, inv)
    return dx, dg, db


def attention_fwd(ops, q, k, v, mask):
    scale = np.float32(1.0) / np.float32(math.sqrt(np.float32(q.shape[-1])))
    kt = ops.transpose(k)
    scores = ops.scalar_mul(ops.matmul(q, kt), scale)
    if mask is not None:
        scores = ops.binary("add", scores, mask)
    w = ops.softmax(scores)
    return ops.matmul(w, v), (q, kt, v, w, scale)


def attention_bwd(ops, g, cache):
    q, kt, v, w, scale = cache
    dw = ops.matmul(g, ops.transpose(v))
    dv = ops.matmul(ops.transpose(w), g)
    ds = ops.scalar_mul(ops.softmax_backward(w, dw), scale)
    dq = ops.matmul(ds, ops.transpose(kt))
    dkt = ops.matmul(ops.transpose(q), ds)
    return dq, ops.transpose(dkt), dv


def mha_fwd(ops, x, p, heads, mask):
    """p: dict with wq,bq,wk,bk,wv,bv,wo,bo (Linear layout: W (in,out), b (1,out))."""
    b, s, d = x.shape
    hd = d // heads

    def split(t):
        return ops.permute(t.reshape(b, s, heads, hd), (0, 2, 1, 3))

    qy, cq = linear_fwd(ops, x, p["wq"], p["bq"])
    ky, ck = linear_fwd(ops, x, p["wk"], p["bk"])
    vy, cv = linear_fwd(ops, x, p["wv"], p["bv"])
    att, ca = attention_fwd(ops, split(qy), split(ky), split(vy), mask)
    merged = ops.permute(att, (0, 2, 1, 3)).reshape(b, s, d)
    out, co = linear_fwd(ops, merged, p["wo"], p["bo"])
    return out, (cq, ck, cv, ca, co, b, s, heads, hd)


def mha_bwd(ops, g, cache):
    cq, ck, cv, ca, co, b, s, heads, hd = cache
    d = heads * hd
    dmerged, dwo, dbo = linear_bwd(ops, g, co)
    datt = ops.permute(dmerged.reshape(b, s, heads, hd), (0, 2, 1, 3))
    dq, dk, dv = attention_bwd(ops, datt, ca)

    def merge(t):
        return ops.permute(t, (0, 2, 1, 3)).reshape(b, s, d)

    # Reverse topological order reaches the value branch first, then key, then
    # query, so the shared input accumulates ((dv + dk) + dq).
    dxv, dwv, dbv = linear_bwd(ops, merge(dv), cv)
    dxk, dwk, dbk = linear_bwd(ops, merge(dk), ck)
    dxq, dwq, dbq = linear_bwd(ops, merge(dq), cq)
    dx = dxv.copy()
    ops.accumulate(dx, dxk)
    ops.accumulate(dx, dxq)
    grads = {"wq": dwq, "bq": dbq, "wk": dwk, "bk": dbk, "wv": dwv, "bv": dbv, "wo": dwo,
             "bo": dbo}
    return dx, grads


BLOCK_KEYS = ("ln1_g", "ln1_b", "ln2_g", "ln2_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
              "w1", "b1", "w2", "b2")


def block_params(flat, d, ff):
    """Splits a TransformerBlock's flat parameters() vector (src/transformer.cpp:416-426)."""
    shapes = [(d,), (d,), (d,), (d,)] + [(d, d), (1, d)] * 4 + [(d, ff), (1, ff), (ff, d), (1, d)]
    out, off = {}, 0
    for key, shp in zip(BLOCK_KEYS, shapes):
        n = int(np.prod(shp))
        out[key] = np.ascontiguousarray(flat[off:off + n].reshape(shp))
        off += n
    return out, off


def block_fwd(ops, x, p, heads, mask):
    n1, c1 = layernorm_fwd(ops, x, p["ln1_g"], p["ln1_b"])
    a, ca = mha_fwd(ops, n1, p, heads, mask)
    h = ops.binary("add", x, a)
    n2, c2 = layernorm_fwd(ops, h, p["ln2_g"], p["ln2_b"])
    f1, cf1 = linear_fwd(ops, n2, p["w1"], p["b1"])
    r = ops.relu(f1)
    f2, cf2 = linear_fwd(ops, r, p["w2"], p["b2"])
    out = ops.binary("add", h, f2)
    return out, (c1, ca, c2, cf1, f1, cf2)


def block_bwd(ops, g, cache):
    c1, ca, c2, cf1, f1, cf2 = cache
    dr, dw2, db2 = linear_bwd(ops, g, cf2)
    df1 = ops.relu_backward(f1, dr)
    dn2, dw1, db1 = linear_bwd(ops, df1, cf1)
    dh2, dg2, dbt2 = layernorm_bwd(ops, dn2, c2)
    dh = g.copy()
    ops.accumulate(dh, dh2)
    dn1, ga = mha_bwd(ops, dh, ca)
    dx1, dg1, dbt1 = layernorm_bwd(ops, dn1, c1)
    dx = dh.copy()
    ops.accumulate(dx, dx1)
    grads = dict(ga)
    grads.update({"ln1_g": dg1, "ln1_b": dbt1, "ln2_g": dg2, "ln2_b": dbt2, "w1": dw1, "b1": db1,
                  "w2": dw2, "b2": db2})
    return dx, grads


# ---------------------------------------------------------------- models
def cnn_param_shapes(c1=8, c2=16, hw=28, classes=10, in_c=1):
    flat = c2 * (hw // 4) * (hw // 4)
    return [(c1, in_c, 3, 3), (c1,), (c2, c1, 3, 3), (c2,), (flat, classes), (1, classes)]


def split_flat(flat, shapes):
    """Copies of the tensors of a flat parameter vector (the training loops update them in
    place, so views would train the caller's vector)."""
    out, off = [], 0
    for s in shapes:
        n = int(np.prod(s))
        out.append(np.array(flat[off:off + n], np.float32).reshape(s))
        off += n
    return out


def cnn_loss_and_grads(ops, x, labels, params):
    w1, b1, w2, b2, wl, bl = params
    y1, cc1 = conv2d_fwd(ops, x, w1, b1, 1, 1)
    r1 = ops.relu(y1)
    p1, cp1 = maxpool_fwd(ops, r1, 2, 2)
    y2, cc2 = conv2d_fwd(ops, p1, w2, b2, 1, 1)
    r2 = ops.relu(y2)
    p2, cp2 = maxpool_fwd(ops, r2, 2, 2)
    flat = p2.reshape(p2.shape[0], -1)
    logits, cl = linear_fwd(ops, flat, wl, bl)
    loss, probs = ops.cross_entropy(logits, labels)
    dlogits = ops.cross_entropy_backward(probs, labels, 1.0)
    dflat, dwl, dbl = linear_bwd(ops, dlogits, cl)
    dr2 = maxpool_bwd(ops, dflat.reshape(p2.shape), cp2)
    dy2 = ops.relu_backward(y2, dr2)
    dp1, dw2, db2 = conv2d_bwd(ops, dy2, cc2)
    dr1 = maxpool_bwd(ops, dp1, cp1)
    dy1 = ops.relu_backward(y1, dr1)
    _, dw1, db1 = conv2d_bwd(ops, dy1, cc1, need_dx=False)
    return loss, [dw1, db1, dw2, db2, dwl, dbl]


class AdamState:
    def __init__(self, params, lr, b1=0.9, b2=0.999, eps=1e-8, wd=0.0):
        self.lr, self.b1, self.b2, self.eps, self.wd = lr, b1, b2, eps, wd
        self.m = [np.zeros_like(p) for p in params]
        self.v = [np.zeros_like(p) for p in params]
        self.t = 0

    def step(self, ops, params, grads):
        self.t += 1
        c1, c2 = ops.adam_bias(self.b1, self.b2, self.t)
        for p, g, m, v in zip(params, grads, self.m, self.v):
            ops.adam(p, np.ascontiguousarray(g, np.float32), m, v, self.lr, self.b1, self.b2,
                     self.eps, self.wd, c1, c2)


def cnn_train(ops, x, labels, flat_params, steps, lr):
    params = split_flat(np.asarray(flat_params, np.float32), cnn_param_shapes(hw=x.shape[2]))
    opt = AdamState(params, lr)
    losses = []
    for _ in range(steps):
        loss, grads = cnn_loss_and_grads(ops, x, labels, params)
        opt.step(ops, params, grads)
        losses.append(loss)
    return np.array(losses, np.float32), np.concatenate([p.ravel() for p in params])


def charlm_param_shapes(vocab, d, ff, layers):
    blk = [(d,), (d,), (d,), (d,)] + [(d, d), (1, d)] * 4 + [(d, ff), (1, ff), (ff, d), (1, d)]
    return [(vocab, d)] + blk * layers + [(d, vocab), (1, vocab)]


def charlm_loss_and_grads(ops, ids, targets, params, vocab, d, heads, ff, layers, pe, mask):
    table = params[0]
    b, s = ids.shape
    idx = np.rint(ids.ravel()).astype(np.int64)
    emb = ops.select_rows(table, idx).reshape(b, s, d)
    h = ops.binary("add", emb, pe)
    caches = []
    for li in range(layers):
        p = dict(zip(BLOCK_KEYS, params[1 + 16 * li:1 + 16 * (li + 1)]))
        h, c = block_fwd(ops, h, p, heads, mask)
        caches.append(c)
    wh, bh = params[-2], params[-1]
    logits, ch = linear_fwd(ops, h, wh, bh)
    loss, probs = ops.cross_entropy(logits.reshape(b * s, vocab), targets)
    dl = ops.cross_entropy_backward(probs, targets, 1.0).reshape(b, s, vocab)
    dh, dwh, dbh = linear_bwd(ops, dl, ch)
    block_grads = []
    for li in reversed(range(layers)):
        dh, g = block_bwd(ops, dh, caches[li])
        block_grads.append([g[k] for k in BLOCK_KEYS])
    dtable = ops.scatter_add_rows(dh.reshape(b * s, d), idx, table.shape)
    grads = [dtable]
    for g in reversed(block_grads):
        grads.extend(g)
    grads.extend([dwh, dbh])
    return loss, grads


def charlm_train(ops, ids, targets, flat_params, vocab, d, heads, ff, layers, steps, lr):
    params = split_flat(np.asarray(flat_params, np.float32),
                        charlm_param_shapes(vocab, d, ff, layers))
    s = ids.shape[1]
    pe = ops.positional_encoding(s, d)
    mask = ops.causal_mask(s)
    opt = AdamState(params, lr)
    losses = []
    for _ in range(steps):
        loss, grads = charlm_loss_and_grads(ops, ids, targets, params, vocab, d, heads, ff,
                                            layers, pe, mask)
        opt.step(ops, params, grads)
        losses.append(loss)
    return np.array(losses, np.float32), np.concatenate([p.ravel() for p in params])
