"""ctypes binding of libengine_hip.so, the C ABI of the C++ engine (engine/src/capi.cpp).

`Engine` has the method names and argument conventions of the reference engine's C shim,
so one test can run the same inputs through the reference's CPU path and through this
engine on the GPU. Arrays are numpy; the engine copies them to the device and back.
`Trainer` keeps a model, its Adam state and a batch resident for timing training steps.
Loading fails loudly when the library is missing: there is no fallback.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ROOT, "lib", "libengine_hip.so")

_f32p = C.POINTER(C.c_float)
_i64p = C.POINTER(C.c_int64)
_i64 = C.c_int64


def _fp(a):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f32p)


def _ip(a):
    assert a.dtype == np.int64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_i64p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def load_library(path=LIB_PATH):
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run __graft_entry__.build()")
    lib = C.CDLL(path)
    lib.eng_last_error.restype = C.c_char_p
    lib.eng_block_num_params.restype = _i64
    lib.eng_charlm_num_params.restype = _i64
    lib.eng_adam_steps.argtypes = [_f32p, _f32p, _i64, _i64] + [C.c_float] * 5
    lib.eng_cnn_grads.argtypes = [_f32p, _i64p] + [_i64] * 6 + [_f32p, _f32p, _f32p]
    lib.eng_cnn_train.argtypes = [_f32p, _i64p] + [_i64] * 6 + [_f32p, _i64, C.c_float, _f32p,
                                                                 _f32p]
    lib.eng_charlm_train.argtypes = [_f32p, _i64p] + [_i64] * 7 + [_f32p, _i64, C.c_float, _f32p,
                                                                    _f32p]
    lib.eng_charlm_train_grads.argtypes = [_f32p, _i64p] + [_i64] * 7 + [
        _f32p, _i64, C.c_float, _f32p, _f32p, _f32p]
    lib.eng_trainer_cnn.restype = C.c_void_p
    lib.eng_trainer_cnn.argtypes = [_f32p, _i64p] + [_i64] * 6 + [_f32p, C.c_float]
    lib.eng_trainer_charlm.restype = C.c_void_p
    lib.eng_trainer_charlm.argtypes = [_f32p, _i64p] + [_i64] * 7 + [_f32p, C.c_float]
    for name in ("eng_trainer_step", "eng_trainer_loss", "eng_trainer_params",
                 "eng_trainer_num_params", "eng_trainer_destroy"):
        getattr(lib, name).argtypes = [C.c_void_p] + (
            [_f32p] if name in ("eng_trainer_loss", "eng_trainer_params") else [])
    lib.eng_trainer_set_graph.argtypes = [C.c_void_p, C.c_int]
    lib.eng_trainer_num_params.restype = _i64
    lib.eng_trainer_destroy.restype = None
    return lib


class Engine:
    """The C++ engine on the GPU, one method per eng_* entry point."""

    def __init__(self, path=LIB_PATH):
        self.lib = load_library(path)
        if not self.lib.eng_available():
            raise RuntimeError("libengine_hip: no usable gfx950 device")

    def _ok(self, rc):
        if rc != 0:
            raise RuntimeError(self.lib.eng_last_error().decode())

    def synchronize(self):
        self._ok(self.lib.eng_synchronize())

    def repeat_gemm(self, reps, a, b, c, trans_a=False, trans_b=False, beta=0.0):
        """Enqueues `reps` ehip_gemm_f32 calls from C++ on torch's current stream: a, b, c
        are 2-D contiguous CUDA tensors, c = op(a) op(b) + beta c."""
        import torch
        am, ak = a.shape
        m, k = (ak, am) if trans_a else (am, ak)
        bk, bn = b.shape
        n = bk if trans_b else bn
        f = self.lib.eng_repeat_gemm
        f.argtypes = [C.c_int, C.c_int] + [_i64] * 4 + [C.c_void_p, _i64, _i64] * 2 + [
            C.c_float, C.c_void_p, _i64, _i64, C.c_void_p, C.c_int]
        self._ok(f(int(trans_a), int(trans_b), 1, m, n, k, a.data_ptr(), a.shape[1], 0,
                   b.data_ptr(), b.shape[1], 0, beta, c.data_ptr(), n, 0,
                   torch.cuda.current_stream().cuda_stream, reps))

    BANDWIDTH_OPS = {"layernorm": 0, "layernorm_backward": 1, "sum_axis": 2, "softmax": 3,
                     "softmax_backward": 4, "maxpool": 5, "maxpool_backward": 6,
                     "layernorm_backward_rows": 7, "layernorm_backward_rows_acc": 8}

    def repeat_bandwidth(self, reps, op, tensors, extents=(), f=0.0, window=None):
        """Enqueues `reps` calls of a bandwidth-bound ehip entry point from C++ on torch's
        current stream (see eng_repeat_bandwidth): tensors are CUDA tensors in the entry
        point's pointer order, extents its integer sizes, window an ehip window struct."""
        import torch
        ptrs = (C.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])
        ext = (_i64 * max(1, len(extents)))(*extents)
        fn = self.lib.eng_repeat_bandwidth
        fn.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_float, C.c_void_p, C.c_void_p,
                       C.c_int]
        self._ok(fn(self.BANDWIDTH_OPS[op], ptrs, ext, f,
                    C.byref(window) if window is not None else None,
                    torch.cuda.current_stream().cuda_stream, reps))

    def repeat_matmul_backward(self, reps, a, b, dc, da, db):
        """Enqueues `reps` ehip_matmul_backward_f32 calls (dA = dC B^T, dB = A^T dC) from C++
        on torch's current stream; 2-D contiguous CUDA tensors."""
        import torch
        m, k = a.shape
        n = b.shape[1]
        f = self.lib.eng_repeat_matmul_backward
        f.argtypes = [_i64] * 3 + [C.c_void_p] * 6 + [C.c_int]
        self._ok(f(m, k, n, a.data_ptr(), b.data_ptr(), dc.data_ptr(), da.data_ptr(),
                   db.data_ptr(), torch.cuda.current_stream().cuda_stream, reps))

    def repeat_conv_relu_pool_backward(self, reps, x, weight, g, out, argmax, dweight, dbias,
                                       conv_window, pool_window, dx=None):
        """Enqueues `reps` fused conv-block backward calls from C++ on torch's current stream
        (torch CUDA tensors; windows are ehip.Window structures)."""
        import torch
        f = self.lib.eng_repeat_conv_relu_pool_backward
        f.argtypes = [C.c_void_p] * 8 + [C.c_void_p, _i64, C.c_void_p, C.c_void_p, C.c_int]
        ptr = lambda t: t.data_ptr() if t is not None else None
        self._ok(f(ptr(x), ptr(weight), ptr(g), ptr(out), ptr(argmax), ptr(dx), ptr(dweight),
                   ptr(dbias), C.addressof(conv_window), weight.shape[0],
                   C.addressof(pool_window), torch.cuda.current_stream().cuda_stream, reps))

    def matmul(self, a, b):
        a, b = _f32(a), _f32(b)
        ab, bb = a.ndim > 2, b.ndim > 2
        batch_shape = a.shape[:-2] if ab else b.shape[:-2]
        batch = int(np.prod(batch_shape)) if (ab or bb) else 1
        m, k = a.shape[-2:]
        n = b.shape[-1]
        c = np.empty(tuple(batch_shape) + (m, n), np.float32)
        self._ok(self.lib.eng_matmul(_fp(a), _fp(b), _fp(c), _i64(batch), _i64(m), _i64(k),
                                     _i64(n), int(ab), int(bb)))
        return c

    def matmul_fwd_bwd(self, a, b, dc):
        a, b, dc = _f32(a), _f32(b), _f32(dc)
        m, k = a.shape
        n = b.shape[1]
        c = np.empty((m, n), np.float32)
        da, db = np.empty_like(a), np.empty_like(b)
        self._ok(self.lib.eng_matmul_fwd_bwd(_fp(a), _fp(b), _fp(dc), _i64(m), _i64(k), _i64(n),
                                             _fp(c), _fp(da), _fp(db)))
        return c, da, db

    def binary_fwd_bwd(self, op, a, b, dy):
        a, b, dy = _f32(a), _f32(b), _f32(dy)
        ops = {"add": 0, "sub": 1, "mul": 2, "div": 3}
        sa, sb = np.array(a.shape, np.int64), np.array(b.shape, np.int64)
        y, da, db = np.empty_like(a), np.empty_like(a), np.empty_like(b)
        self._ok(self.lib.eng_binary_fwd_bwd(ops[op], _fp(a), _ip(sa), a.ndim, _fp(b), _ip(sb),
                                             b.ndim, _fp(dy), _fp(y), _fp(da), _fp(db)))
        return y, da, db

    def permute_fwd_bwd(self, x, order, dy):
        x, dy = _f32(x), _f32(dy)
        s, o = np.array(x.shape, np.int64), np.array(order, np.int64)
        y = np.empty(tuple(x.shape[i] for i in order), np.float32)
        dx = np.empty_like(x)
        self._ok(self.lib.eng_permute_fwd_bwd(_fp(x), _ip(s), x.ndim, _ip(o), _fp(dy), _fp(y),
                                              _fp(dx)))
        return y, dx

    def sum_axis_fwd_bwd(self, x, axis, dy):
        x, dy = _f32(x), _f32(dy)
        s = np.array(x.shape, np.int64)
        y = np.empty(dy.shape, np.float32)
        dx = np.empty_like(x)
        self._ok(self.lib.eng_sum_axis_fwd_bwd(_fp(x), _ip(s), x.ndim, axis, _fp(dy), _fp(y),
                                               _fp(dx)))
        return y, dx

    def unary_fwd_bwd(self, which, x, dy):
        x, dy = _f32(x), _f32(dy)
        y, dx = np.empty_like(x), np.empty_like(x)
        rows, cols = x.shape
        self._ok(self.lib.eng_unary_fwd_bwd({"relu": 0, "softmax": 1}[which], _fp(x), _i64(rows),
                                            _i64(cols), _fp(dy), _fp(y), _fp(dx)))
        return y, dx

    def sum(self, x):
        x = _f32(x)
        out = np.empty(1, np.float32)
        self._ok(self.lib.eng_sum(_fp(x), _i64(x.size), _fp(out)))
        return out

    def im2col(self, x, kh, kw, stride, pad):
        x = _f32(x)
        n, c, h, w = x.shape
        oh = (h + 2 * pad - kh) // stride + 1
        ow = (w + 2 * pad - kw) // stride + 1
        cols = np.empty((n * oh * ow, c * kh * kw), np.float32)
        self._ok(self.lib.eng_im2col(_fp(x), *[_i64(v) for v in x.shape], _i64(kh), _i64(kw),
                                     _i64(stride), _i64(pad), _fp(cols)))
        return cols

    def col2im(self, cols, shape, kh, kw, stride, pad):
        cols = _f32(cols)
        x = np.empty(shape, np.float32)
        self._ok(self.lib.eng_col2im(_fp(cols), *[_i64(v) for v in shape], _i64(kh), _i64(kw),
                                     _i64(stride), _i64(pad), _fp(x)))
        return x

    def conv2d_fwd_bwd(self, x, w, bias, stride, pad, dy):
        x, w, bias, dy = _f32(x), _f32(w), _f32(bias), _f32(dy)
        n, c, h, ww = x.shape
        oc, _, k, _ = w.shape
        y = np.empty(dy.shape, np.float32)
        dx, dw, db = np.empty_like(x), np.empty_like(w), np.empty_like(bias)
        self._ok(self.lib.eng_conv2d_fwd_bwd(_fp(x), _fp(w), _fp(bias), _i64(n), _i64(c),
                                             _i64(h), _i64(ww), _i64(oc), _i64(k), _i64(stride),
                                             _i64(pad), _fp(dy), _fp(y), _fp(dx), _fp(dw),
                                             _fp(db)))
        return y, dx, dw, db

    def maxpool_fwd_bwd(self, x, k, stride, dy):
        x, dy = _f32(x), _f32(dy)
        y = np.empty(dy.shape, np.float32)
        dx = np.empty_like(x)
        self._ok(self.lib.eng_maxpool_fwd_bwd(_fp(x), *[_i64(v) for v in x.shape], _i64(k),
                                              _i64(stride), _fp(dy), _fp(y), _fp(dx)))
        return y, dx

    def layernorm_fwd_bwd(self, x, gamma, beta, dy):
        x, gamma, beta, dy = _f32(x), _f32(gamma), _f32(beta), _f32(dy)
        d = x.shape[-1]
        rows = x.size // d
        y, dx = np.empty_like(x), np.empty_like(x)
        dg, db = np.empty(d, np.float32), np.empty(d, np.float32)
        self._ok(self.lib.eng_layernorm_fwd_bwd(_fp(x), _fp(gamma), _fp(beta), _i64(rows),
                                                _i64(d), _fp(dy), _fp(y), _fp(dx), _fp(dg),
                                                _fp(db)))
        return y, dx, dg, db

    def cross_entropy(self, logits, targets):
        logits = _f32(logits)
        t = np.ascontiguousarray(targets, np.int64)
        n, c = logits.shape
        loss = np.empty(1, np.float32)
        dl = np.empty_like(logits)
        self._ok(self.lib.eng_cross_entropy(_fp(logits), _ip(t), _i64(n), _i64(c), _fp(loss),
                                            _fp(dl)))
        return float(loss[0]), dl

    def embedding_fwd_bwd(self, table, ids, dy):
        table, ids, dy = _f32(table), _f32(ids), _f32(dy)
        v, d = table.shape
        b, s = ids.shape
        y = np.empty((b, s, d), np.float32)
        dt = np.empty_like(table)
        self._ok(self.lib.eng_embedding_fwd_bwd(_fp(table), _i64(v), _i64(d), _fp(ids), _i64(b),
                                                _i64(s), _fp(dy), _fp(y), _fp(dt)))
        return y, dt

    def adam_steps(self, p, grads, lr, b1=0.9, b2=0.999, eps=1e-8, wd=0.0):
        p = _f32(p).copy()
        grads = _f32(grads)
        self._ok(self.lib.eng_adam_steps(_fp(p), _fp(grads), p.size, grads.size // p.size, lr,
                                         b1, b2, eps, wd))
        return p

    def dropout_fwd_bwd(self, x, p, seed, dy, eval_mode=False):
        x, dy = _f32(x), _f32(dy)
        y, dx = np.empty_like(x), np.empty_like(x)
        f = self.lib.eng_dropout_fwd_bwd
        f.argtypes = [_f32p, _i64, C.c_float, C.c_uint64, C.c_int, _f32p, _f32p, _f32p]
        self._ok(f(_fp(x), x.size, p, seed, int(eval_mode), _fp(dy), _fp(y), _fp(dx)))
        return y, dx

    def clip_grad_norm(self, grads, sizes, max_norm):
        """grads: concatenated gradients of the parameters whose size is positive; a
        negative size is a parameter without a gradient. Returns (norm, clipped)."""
        g = _f32(grads).copy()
        sz = np.ascontiguousarray(sizes, np.int64)
        norm = C.c_float()
        self._ok(self.lib.eng_clip_grad_norm(_fp(g), _ip(sz), len(sz), C.c_float(max_norm),
                                             C.byref(norm)))
        return norm.value, g

    def attention_fwd_bwd(self, q, k, v, mask, dy):
        q, k, v, dy = _f32(q), _f32(k), _f32(v), _f32(dy)
        b, h, s, dk = q.shape
        y = np.empty_like(q)
        w = np.empty((b, h, s, s), np.float32)
        dq, dkk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
        mp = _fp(_f32(mask)) if mask is not None else None
        self._ok(self.lib.eng_attention_fwd_bwd(_fp(q), _fp(k), _fp(v), mp, _i64(b), _i64(h),
                                                _i64(s), _i64(dk), _fp(dy), _fp(y), _fp(w),
                                                _fp(dq), _fp(dkk), _fp(dv)))
        return y, w, dq, dkk, dv

    def linear_fwd_bwd(self, x, w, bias, dy):
        x, w, bias, dy = _f32(x), _f32(w), _f32(bias), _f32(dy)
        fin, fout = w.shape
        rows = x.size // fin
        y = np.empty(x.shape[:-1] + (fout,), np.float32)
        dx, dw, db = np.empty_like(x), np.empty_like(w), np.empty(bias.shape, np.float32)
        self._ok(self.lib.eng_linear_fwd_bwd(_fp(x), _i64(rows), _i64(fin), _i64(fout), _fp(w),
                                             _fp(bias), _fp(dy), _fp(y), _fp(dx), _fp(dw),
                                             _fp(db)))
        return y, dx, dw, db

    def mha_fwd_bwd(self, x, heads, params, dy, mask=None, fuse=True, weights=False):
        """MultiHeadAttention forward + backward; mask (seq, seq) or None. fuse
        picks the in-place attention node or the composed split/attend/merge
        path. weights=True also returns the (b, heads, s, s) attention."""
        x, params, dy = _f32(x), _f32(params), _f32(dy)
        b, s, d = x.shape
        y, dx, dp = np.empty_like(x), np.empty_like(x), np.empty_like(params)
        mp = None if mask is None else _f32(mask)
        w = np.empty((b, heads, s, s), np.float32) if weights else None
        self._ok(self.lib.eng_mha_fwd_bwd(_fp(x), _i64(b), _i64(s), _i64(d), _i64(heads),
                                          _fp(params), _fp(dy), _fp(y), _fp(dx), _fp(dp),
                                          None if mp is None else _fp(mp), int(fuse),
                                          None if w is None else _fp(w)))
        return (y, dx, dp, w) if weights else (y, dx, dp)

    def mha_causal_fwd_bwd(self, x, heads, params, dy, tagged=True):
        """Fused MultiHeadAttention forward + backward under the causal mask of
        nn::causal_mask (tagged: its products may skip the masked blocks) or under a
        plain copy of its values (every product in full). Returns y, dx, dparams and
        the attention weights."""
        x, params, dy = _f32(x), _f32(params), _f32(dy)
        b, s, d = x.shape
        y, dx, dp = np.empty_like(x), np.empty_like(x), np.empty_like(params)
        w = np.empty((b, heads, s, s), np.float32)
        self._ok(self.lib.eng_mha_causal_fwd_bwd(_fp(x), _i64(b), _i64(s), _i64(d), _i64(heads),
                                                 _fp(params), _fp(dy), _fp(y), _fp(dx), _fp(dp),
                                                 _fp(w), int(bool(tagged))))
        return y, dx, dp, w

    def mse_adam(self, w0, target, steps, lr):
        w0, target = _f32(w0).ravel().copy(), _f32(target).ravel().copy()
        traj = np.empty((steps, w0.size), np.float32)
        self.lib.eng_mse_adam.argtypes = [_f32p, _f32p, _i64, _i64, C.c_float, _f32p]
        self._ok(self.lib.eng_mse_adam(_fp(w0), _fp(target), w0.size, steps, lr, _fp(traj)))
        return traj

    def set_fused_nodes(self, on):
        """Fused graph nodes on (default) or the reference's node-by-node graph;
        returns the previous setting."""
        return bool(self.lib.eng_set_fused_nodes(int(bool(on))))

    def set_short_attention(self, on):
        """Attention of sequences and heads of at most 64 values in one launch per direction
        (default on) or through the batched products; returns the previous setting."""
        return bool(self.lib.eng_set_short_attention(int(bool(on))))

    def set_deferred_weight_grads(self, on):
        """Narrow layers' weight-gradient products queued and run together (default on) or
        launched by each node; returns the previous setting."""
        return bool(self.lib.eng_set_deferred_weight_grads(int(bool(on))))

    def set_conv_implicit_gemm(self, on):
        """Wide convolutions as implicit GEMMs (default on) or the reference's im2col
        composition; returns the previous setting."""
        return bool(self.lib.eng_set_conv_implicit_gemm(int(bool(on))))

    def set_fused_bias_grad(self, on):
        """Bias gradients of mid-sized layers from the weight-gradient products' column sums
        (default on) or the separate column sum; returns the previous setting."""
        return bool(self.lib.eng_set_fused_bias_grad(int(bool(on))))

    def block_num_params(self, d, heads, ff):
        return self.lib.eng_block_num_params(_i64(d), _i64(heads), _i64(ff))

    def block_fwd_bwd(self, x, heads, ff, causal, params, dy):
        x, params, dy = _f32(x), _f32(params), _f32(dy)
        b, s, d = x.shape
        y, dx = np.empty_like(x), np.empty_like(x)
        dp = np.empty_like(params)
        self._ok(self.lib.eng_block_fwd_bwd(_fp(x), _i64(b), _i64(s), _i64(d), _i64(heads),
                                            _i64(ff), int(causal), _fp(params), _fp(dy), _fp(y),
                                            _fp(dx), _fp(dp)))
        return y, dx, dp

    def cnn_grads(self, x, labels, params, c1=8, c2=16, classes=10):
        """One forward and backward of the small CNN: (loss, flat gradients in parameter
        order)."""
        x, params = _f32(x), _f32(params)
        labels = np.ascontiguousarray(labels, np.int64)
        b, cin, hw, _ = x.shape
        loss = np.empty(1, np.float32)
        grads = np.empty_like(params)
        self._ok(self.lib.eng_cnn_grads(_fp(x), _ip(labels), b, cin, c1, c2, hw, classes,
                                        _fp(params), _fp(loss), _fp(grads)))
        return float(loss[0]), grads

    def cnn_backward_orphan(self, x, labels, params, c1=8, c2=16, classes=10):
        """Forward + backward of a CNN destroyed before its queued weight sums ran."""
        x, params = _f32(x), _f32(params)
        labels = np.ascontiguousarray(labels, np.int64)
        b, cin, hw, _ = x.shape
        f = self.lib.eng_cnn_backward_orphan
        f.argtypes = [_f32p, _i64p] + [_i64] * 6 + [_f32p]
        self._ok(f(_fp(x), _ip(labels), b, cin, c1, c2, hw, classes, _fp(params)))

    def charlm_accumulated_grads(self, ids, targets, vocab, d, heads, ff, layers, params,
                                 passes):
        """The character model's gradients summed over `passes` forward + backward passes."""
        ids, params = _f32(ids), _f32(params)
        targets = np.ascontiguousarray(targets, np.int64)
        b, s = ids.shape
        out = np.empty_like(params)
        f = self.lib.eng_charlm_accumulated_grads
        f.argtypes = [_f32p, _i64p] + [_i64] * 7 + [_f32p, _i64, _f32p]
        self._ok(f(_fp(ids), _ip(targets), b, s, vocab, d, heads, ff, layers, _fp(params),
                   passes, _fp(out)))
        return out

    def charlm_backward_orphan(self, ids, targets, vocab, d, heads, ff, layers, params):
        """Forward + backward of a character model destroyed before its queued work ran."""
        ids, params = _f32(ids), _f32(params)
        targets = np.ascontiguousarray(targets, np.int64)
        b, s = ids.shape
        f = self.lib.eng_charlm_backward_orphan
        f.argtypes = [_f32p, _i64p] + [_i64] * 7 + [_f32p]
        self._ok(f(_fp(ids), _ip(targets), b, s, vocab, d, heads, ff, layers, _fp(params)))

    def cnn_train(self, x, labels, params, steps, lr, c1=8, c2=16, classes=10):
        x, params = _f32(x), _f32(params)
        labels = np.ascontiguousarray(labels, np.int64)
        b, cin, hw, _ = x.shape
        losses = np.empty(steps, np.float32)
        out = np.empty_like(params)
        self._ok(self.lib.eng_cnn_train(_fp(x), _ip(labels), b, cin, c1, c2, hw, classes,
                                        _fp(params), steps, lr, _fp(losses), _fp(out)))
        return losses, out

    def charlm_num_params(self, vocab, seq, d, heads, ff, layers):
        return self.lib.eng_charlm_num_params(_i64(vocab), _i64(seq), _i64(d), _i64(heads),
                                              _i64(ff), _i64(layers))

    def charlm_train(self, ids, targets, vocab, d, heads, ff, layers, params, steps, lr,
                     grads0=False):
        """`steps` Adam steps on one batch: per-step losses and the final parameters, and
        with grads0 the first step's gradients (flat, parameter order) as a third value."""
        ids, params = _f32(ids), _f32(params)
        targets = np.ascontiguousarray(targets, np.int64)
        b, s = ids.shape
        losses = np.empty(steps, np.float32)
        out = np.empty_like(params)
        g0 = np.empty_like(params) if grads0 else None
        self._ok(self.lib.eng_charlm_train_grads(_fp(ids), _ip(targets), b, s, vocab, d, heads,
                                                 ff, layers, _fp(params), steps, lr, _fp(losses),
                                                 _fp(g0) if grads0 else None, _fp(out)))
        return (losses, out, g0) if grads0 else (losses, out)


class Trainer:
    """A resident model + Adam + batch; step() enqueues one training step without waiting."""

    def __init__(self, engine, handle):
        if not handle:
            raise RuntimeError(engine.lib.eng_last_error().decode())
        self.engine, self.lib, self.h = engine, engine.lib, handle

    @classmethod
    def cnn(cls, engine, x, labels, params=None, lr=1e-3, c1=8, c2=16, classes=10):
        x = _f32(x)
        labels = np.ascontiguousarray(labels, np.int64)
        b, cin, hw, _ = x.shape
        p = _fp(_f32(params)) if params is not None else None
        return cls(engine, engine.lib.eng_trainer_cnn(_fp(x), _ip(labels), b, cin, c1, c2, hw,
                                                      classes, p, lr))

    @classmethod
    def charlm(cls, engine, ids, targets, vocab, d, heads, ff, layers, params=None, lr=1e-3):
        ids = _f32(ids)
        targets = np.ascontiguousarray(targets, np.int64)
        b, s = ids.shape
        p = _fp(_f32(params)) if params is not None else None
        return cls(engine, engine.lib.eng_trainer_charlm(_fp(ids), _ip(targets), b, s, vocab, d,
                                                         heads, ff, layers, p, lr))

    def save(self, params_path, opt_path=None):
        """Parameters in the reference's weight format; Adam state too when opt_path."""
        f = self.lib.eng_trainer_save
        f.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p]
        if f(self.h, params_path.encode(), opt_path.encode() if opt_path else None) != 0:
            raise RuntimeError(self.lib.eng_last_error().decode())

    def load(self, params_path, opt_path=None):
        f = self.lib.eng_trainer_load
        f.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p]
        if f(self.h, params_path.encode(), opt_path.encode() if opt_path else None) != 0:
            raise RuntimeError(self.lib.eng_last_error().decode())

    def step(self):
        if self.lib.eng_trainer_step(self.h) != 0:
            raise RuntimeError(self.lib.eng_last_error().decode())

    def set_graph(self, on=True):
        """Graph mode: the second step is captured into one HIP graph (the first runs eagerly
        and creates the Adam state); every later step refreshes Adam's step size and bias
        corrections in device memory and replays the graph with one launch."""
        if self.lib.eng_trainer_set_graph(self.h, int(bool(on))) != 0:
            raise RuntimeError(self.lib.eng_last_error().decode())

    def loss(self):
        out = C.c_float()
        if self.lib.eng_trainer_loss(self.h, C.byref(out)) != 0:
            raise RuntimeError(self.lib.eng_last_error().decode())
        return out.value

    def num_params(self):
        return self.lib.eng_trainer_num_params(self.h)

    def params(self):
        out = np.empty(self.num_params(), np.float32)
        if self.lib.eng_trainer_params(self.h, _fp(out)) != 0:
            raise RuntimeError(self.lib.eng_last_error().decode())
        return out

    def close(self):
        if self.h:
            self.lib.eng_trainer_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
