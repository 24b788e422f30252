"""ctypes bindings for the test-only checkers under oracle/.

`Oracle` wraps oracle/liboracle.so (the CPU restatement). `Ref` wraps
oracle/_ref/libref_engine.so (the reference engine compiled from its own
sources). Both take and return numpy arrays. This module lives under tests/
because only tests, smoke() and bench.py's cpu_baseline may load the oracle.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref_engine.so")

_f32p = C.POINTER(C.c_float)
_i64p = C.POINTER(C.c_int64)
_i32p = C.POINTER(C.c_int32)
_i64 = C.c_int64


def fp(a):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


def ip(a):
    assert a.dtype == np.int64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_i64p)


def i32p(a):
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_i32p)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class OrcWindow(C.Structure):
    _fields_ = [(n, C.c_int64) for n in (
        "batch", "channels", "height", "width", "kernel_h", "kernel_w", "stride", "padding",
        "out_h", "out_w")]


def window(n, c, h, w, kh, kw, stride, pad):
    oh = (h + 2 * pad - kh) // stride + 1
    ow = (w + 2 * pad - kw) // stride + 1
    return OrcWindow(n, c, h, w, kh, kw, stride, pad, oh, ow)


class Oracle:
    """The CPU restatement, one method per oracle.h entry point."""

    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run make -C oracle)")
        self.lib = L = C.CDLL(path)
        L.orc_sum.restype = C.c_double
        L.orc_sum_squares.restype = C.c_double
        L.orc_cross_entropy.restype = C.c_float
        for name in ("orc_scalar_add", "orc_scalar_mul"):
            getattr(L, name).argtypes = [_f32p, _f32p, _i64, C.c_float]
        L.orc_adam.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64] + [C.c_float] * 7
        L.orc_sgd.argtypes = [_f32p, _f32p, _f32p, _i64] + [C.c_float] * 3
        L.orc_adam_bias.argtypes = [C.c_float, C.c_float, _i64, _f32p, _f32p]
        L.orc_layernorm.argtypes = [_f32p] * 6 + [_i64, _i64, C.c_float]
        L.orc_cross_entropy_backward.argtypes = [_f32p, _i64p, _f32p, _i64, _i64, C.c_float]
        L.orc_causal_mask.argtypes = [_f32p, _i64, C.c_float]

    # --- dense -----------------------------------------------------------
    def matmul(self, a, b):
        a, b = f32(a), f32(b)
        ab, bb = a.ndim > 2, b.ndim > 2
        batch_shape = a.shape[:-2] if ab else b.shape[:-2]
        batch = int(np.prod(batch_shape)) if (ab or bb) else 1
        m, k = a.shape[-2:]
        n = b.shape[-1]
        assert b.shape[-2] == k
        c = np.empty(tuple(batch_shape) + (m, n), np.float32)
        self.lib.orc_matmul(fp(a), fp(b), fp(c), _i64(batch), _i64(m), _i64(k), _i64(n),
                            int(ab), int(bb))
        return c

    def transpose(self, x):
        x = f32(x)
        rows, cols = x.shape[-2:]
        batch = x.size // max(1, rows * cols)
        y = np.empty(x.shape[:-2] + (cols, rows), np.float32)
        self.lib.orc_transpose(fp(x), fp(y), _i64(batch), _i64(rows), _i64(cols))
        return y

    def permute(self, x, order):
        x = f32(x)
        shape = np.array(x.shape, np.int64)
        o = np.array(order, np.int64)
        y = np.empty(tuple(x.shape[i] for i in order), np.float32)
        self.lib.orc_permute(fp(x), fp(y), C.c_int(x.ndim), ip(shape), ip(o))
        return y

    # --- element-wise ----------------------------------------------------
    def binary(self, op, a, b):
        a, b = f32(a), f32(b)
        ops = {"add": 0, "sub": 1, "mul": 2, "div": 3}
        inner = b.size
        assert a.size % inner == 0
        out = np.empty_like(a)
        self.lib.orc_binary(ops[op], fp(a), fp(b), fp(out), _i64(inner), _i64(a.size // inner))
        return out

    def scalar_add(self, x, k):
        x = f32(x)
        y = np.empty_like(x)
        self.lib.orc_scalar_add(fp(x), fp(y), x.size, k)
        return y

    def scalar_mul(self, x, k):
        x = f32(x)
        y = np.empty_like(x)
        self.lib.orc_scalar_mul(fp(x), fp(y), x.size, k)
        return y

    def relu(self, x):
        x = f32(x)
        y = np.empty_like(x)
        self.lib.orc_relu(fp(x), fp(y), _i64(x.size))
        return y

    def relu_backward(self, x, g):
        x, g = f32(x), f32(g)
        dx = np.empty_like(x)
        self.lib.orc_relu_backward(fp(x), fp(g), fp(dx), _i64(x.size))
        return dx

    def accumulate(self, grad, g):
        self.lib.orc_accumulate(fp(grad), fp(f32(g)), _i64(grad.size))
        return grad

    # --- reductions --------------------------------------------------------
    def sum_axis(self, x, axis):
        x = f32(x)
        outer = int(np.prod(x.shape[:axis]))
        inner = int(np.prod(x.shape[axis + 1:]))
        out_shape = x.shape[:axis] + x.shape[axis + 1:]
        if not out_shape:
            out_shape = (1,)
        y = np.empty(out_shape, np.float32)
        self.lib.orc_sum_axis(fp(x), fp(y), _i64(outer), _i64(x.shape[axis]), _i64(inner))
        return y

    def fold_leading(self, x, target_shape):
        x = f32(x)
        inner = int(np.prod(target_shape))
        y = np.empty(target_shape, np.float32)
        self.lib.orc_sum_axis(fp(x), fp(y), _i64(1), _i64(x.size // inner), _i64(inner))
        return y

    def sum(self, x):
        x = f32(x)
        return self.lib.orc_sum(fp(x), _i64(x.size))

    def sum_squares(self, x):
        x = f32(x)
        return self.lib.orc_sum_squares(fp(x), _i64(x.size))

    # --- convolution and pooling ----------------------------------------
    def im2col(self, x, kh, kw, stride, pad):
        x = f32(x)
        w = window(*x.shape, kh, kw, stride, pad)
        cols = np.empty((w.batch * w.out_h * w.out_w, w.channels * kh * kw), np.float32)
        self.lib.orc_im2col(fp(x), fp(cols), C.byref(w))
        return cols

    def col2im(self, cols, shape, kh, kw, stride, pad):
        cols = f32(cols)
        w = window(*shape, kh, kw, stride, pad)
        x = np.empty(shape, np.float32)
        self.lib.orc_col2im(fp(cols), fp(x), C.byref(w))
        return x

    def maxpool(self, x, k, stride, pad=0):
        x = f32(x)
        w = window(*x.shape, k, k, stride, pad)
        y = np.empty((w.batch, w.channels, w.out_h, w.out_w), np.float32)
        am = np.empty(y.shape, np.int32)
        self.lib.orc_maxpool(fp(x), fp(y), i32p(am), C.byref(w))
        return y, am

    def maxpool_backward(self, argmax, g, in_shape):
        dx = np.empty(in_shape, np.float32)
        g = f32(g)
        self.lib.orc_maxpool_backward(i32p(np.ascontiguousarray(argmax, np.int32)), fp(g), fp(dx),
                                      _i64(g.size), _i64(dx.size))
        return dx

    # --- row kernels ------------------------------------------------------
    def softmax(self, x):
        x = f32(x)
        y = np.empty_like(x)
        cols = x.shape[-1]
        self.lib.orc_softmax(fp(x), fp(y), _i64(x.size // cols), _i64(cols))
        return y

    def softmax_backward(self, y, g):
        y, g = f32(y), f32(g)
        dx = np.empty_like(y)
        cols = y.shape[-1]
        self.lib.orc_softmax_backward(fp(y), fp(g), fp(dx), _i64(y.size // cols), _i64(cols))
        return dx

    def layernorm(self, x, gamma, beta, eps=1e-5):
        x, gamma, beta = f32(x), f32(gamma), f32(beta)
        d = x.shape[-1]
        rows = x.size // d
        out, xhat = np.empty_like(x), np.empty_like(x)
        inv = np.empty(rows, np.float32)
        self.lib.orc_layernorm(fp(x), fp(gamma), fp(beta), fp(out), fp(xhat), fp(inv),
                               _i64(rows), _i64(d), eps)
        return out, xhat, inv

    def layernorm_backward(self, dy, xhat, gamma, inv):
        dy, xhat, gamma, inv = f32(dy), f32(xhat), f32(gamma), f32(inv)
        d = dy.shape[-1]
        dx = np.empty_like(dy)
        dg, db = np.empty(d, np.float32), np.empty(d, np.float32)
        self.lib.orc_layernorm_backward(fp(dy), fp(xhat), fp(gamma), fp(inv), fp(dx), fp(dg),
                                        fp(db), _i64(dy.size // d), _i64(d))
        return dx, dg, db

    def cross_entropy(self, logits, targets):
        logits = f32(logits)
        t = np.ascontiguousarray(targets, np.int64)
        probs = np.empty_like(logits)
        n, c = logits.shape
        loss = self.lib.orc_cross_entropy(fp(logits), ip(t), fp(probs), _i64(n), _i64(c))
        return float(np.float32(loss)), probs

    def cross_entropy_backward(self, probs, targets, grad=1.0):
        probs = f32(probs)
        t = np.ascontiguousarray(targets, np.int64)
        dx = np.empty_like(probs)
        n, c = probs.shape
        self.lib.orc_cross_entropy_backward(fp(probs), ip(t), fp(dx), n, c, grad)
        return dx

    # --- optimisers ---------------------------------------------------------
    def adam_bias(self, b1, b2, t):
        c1, c2 = C.c_float(), C.c_float()
        self.lib.orc_adam_bias(b1, b2, t, C.byref(c1), C.byref(c2))
        return c1.value, c2.value

    def adam(self, p, g, m, v, lr, b1, b2, eps, wd, c1, c2):
        self.lib.orc_adam(fp(p), fp(f32(g)), fp(m), fp(v), p.size, lr, b1, b2, eps, wd, c1, c2)

    def sgd(self, p, g, vel, lr, momentum, wd):
        self.lib.orc_sgd(fp(p), fp(f32(g)), fp(vel) if vel is not None else None, p.size, lr,
                         momentum, wd)

    # --- gathers ------------------------------------------------------------
    def select_rows(self, x, idx):
        x = f32(x)
        idx = np.ascontiguousarray(idx, np.int64)
        rs = x.size // x.shape[0]
        out = np.empty((len(idx),) + x.shape[1:], np.float32)
        self.lib.orc_select_rows(fp(x), ip(idx), fp(out), _i64(len(idx)), _i64(rs))
        return out

    def scatter_add_rows(self, g, idx, shape):
        g = f32(g)
        idx = np.ascontiguousarray(idx, np.int64)
        dx = np.zeros(shape, np.float32)
        rs = dx.size // shape[0]
        self.lib.orc_scatter_add_rows(fp(g), ip(idx), fp(dx), _i64(len(idx)), _i64(rs))
        return dx

    def philox(self, ctr, key):
        c = np.ascontiguousarray(ctr, np.uint32)
        k = np.ascontiguousarray(key, np.uint32)
        out = np.empty(4, np.uint32)
        u32p = C.POINTER(C.c_uint32)
        self.lib.orc_philox4x32_10(c.ctypes.data_as(u32p), k.ctypes.data_as(u32p),
                                   out.ctypes.data_as(u32p))
        return out

    def dropout(self, x, p, seed, offset=0):
        x = f32(x)
        y, m = np.empty_like(x), np.empty_like(x)
        self.lib.orc_dropout.argtypes = [_f32p, _f32p, _f32p, _i64, C.c_float, C.c_uint64,
                                         C.c_uint64]
        self.lib.orc_dropout(fp(x), fp(y), fp(m), x.size, p, seed, offset)
        return y, m

    def positional_encoding(self, s, d):
        out = np.empty((s, d), np.float32)
        self.lib.orc_positional_encoding(fp(out), _i64(s), _i64(d))
        return out

    def causal_mask(self, s, value=-1e9):
        out = np.empty((s, s), np.float32)
        self.lib.orc_causal_mask(fp(out), s, value)
        return out


class Ref:
    """The compiled reference engine, through oracle/ref_shim.cpp."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (needs the reference checkout)")
        self.lib = L = C.CDLL(path)
        L.ref_last_error.restype = C.c_char_p
        L.ref_block_num_params.restype = _i64
        L.ref_charlm_num_params.restype = _i64
        L.ref_adam_steps.argtypes = [_f32p, _f32p, _i64, _i64] + [C.c_float] * 5
        L.ref_cnn_train.argtypes = [_f32p, _i64p] + [_i64] * 6 + [_f32p, _i64, C.c_float,
                                                                    _f32p, _f32p]
        L.ref_charlm_train.argtypes = [_f32p, _i64p] + [_i64] * 7 + [_f32p, _i64, C.c_float,
                                                                      _f32p, _f32p]
        L.ref_charlm_train_grads.argtypes = [_f32p, _i64p] + [_i64] * 7 + [
            _f32p, _i64, C.c_float, _f32p, _f32p, _f32p]

    def _ok(self, rc):
        if rc != 0:
            raise RuntimeError(self.lib.ref_last_error().decode())

    def set_threads(self, n):
        self.lib.ref_set_threads(int(n))

    def num_threads(self):
        return self.lib.ref_num_threads()

    def matmul(self, a, b):
        a, b = f32(a), f32(b)
        ab, bb = a.ndim > 2, b.ndim > 2
        batch_shape = a.shape[:-2] if ab else b.shape[:-2]
        batch = int(np.prod(batch_shape)) if (ab or bb) else 1
        m, k = a.shape[-2:]
        n = b.shape[-1]
        c = np.empty(tuple(batch_shape) + (m, n), np.float32)
        self._ok(self.lib.ref_matmul(fp(a), fp(b), fp(c), _i64(batch), _i64(m), _i64(k), _i64(n),
                                     int(ab), int(bb)))
        return c

    def matmul_fwd_bwd(self, a, b, dc):
        a, b, dc = f32(a), f32(b), f32(dc)
        m, k = a.shape
        n = b.shape[1]
        c = np.empty((m, n), np.float32)
        da, db = np.empty_like(a), np.empty_like(b)
        self._ok(self.lib.ref_matmul_fwd_bwd(fp(a), fp(b), fp(dc), _i64(m), _i64(k), _i64(n),
                                             fp(c), fp(da), fp(db)))
        return c, da, db

    def binary_fwd_bwd(self, op, a, b, dy):
        a, b, dy = f32(a), f32(b), f32(dy)
        ops = {"add": 0, "sub": 1, "mul": 2, "div": 3}
        sa, sb = np.array(a.shape, np.int64), np.array(b.shape, np.int64)
        y, da, db = np.empty_like(a), np.empty_like(a), np.empty_like(b)
        self._ok(self.lib.ref_binary_fwd_bwd(ops[op], fp(a), ip(sa), a.ndim, fp(b), ip(sb), b.ndim,
                                             fp(dy), fp(y), fp(da), fp(db)))
        return y, da, db

    def permute_fwd_bwd(self, x, order, dy):
        x, dy = f32(x), f32(dy)
        s, o = np.array(x.shape, np.int64), np.array(order, np.int64)
        y = np.empty(tuple(x.shape[i] for i in order), np.float32)
        dx = np.empty_like(x)
        self._ok(self.lib.ref_permute_fwd_bwd(fp(x), ip(s), x.ndim, ip(o), fp(dy), fp(y), fp(dx)))
        return y, dx

    def sum_axis_fwd_bwd(self, x, axis, dy):
        x, dy = f32(x), f32(dy)
        s = np.array(x.shape, np.int64)
        y = np.empty(dy.shape, np.float32)
        dx = np.empty_like(x)
        self._ok(self.lib.ref_sum_axis_fwd_bwd(fp(x), ip(s), x.ndim, axis, fp(dy), fp(y), fp(dx)))
        return y, dx

    def unary_fwd_bwd(self, which, x, dy):
        x, dy = f32(x), f32(dy)
        y, dx = np.empty_like(x), np.empty_like(x)
        rows, cols = x.shape
        self._ok(self.lib.ref_unary_fwd_bwd({"relu": 0, "softmax": 1}[which], fp(x), _i64(rows),
                                            _i64(cols), fp(dy), fp(y), fp(dx)))
        return y, dx

    def im2col(self, x, kh, kw, stride, pad):
        x = f32(x)
        w = window(*x.shape, kh, kw, stride, pad)
        cols = np.empty((w.batch * w.out_h * w.out_w, w.channels * kh * kw), np.float32)
        self._ok(self.lib.ref_im2col(fp(x), *[_i64(v) for v in x.shape], _i64(kh), _i64(kw),
                                     _i64(stride), _i64(pad), fp(cols)))
        return cols

    def col2im(self, cols, shape, kh, kw, stride, pad):
        cols = f32(cols)
        x = np.empty(shape, np.float32)
        self._ok(self.lib.ref_col2im(fp(cols), *[_i64(v) for v in shape], _i64(kh), _i64(kw),
                                     _i64(stride), _i64(pad), fp(x)))
        return x

    def conv2d_fwd_bwd(self, x, w, bias, stride, pad, dy):
        x, w, bias, dy = f32(x), f32(w), f32(bias), f32(dy)
        n, c, h, ww = x.shape
        oc, _, k, _ = w.shape
        y = np.empty(dy.shape, np.float32)
        dx, dw, db = np.empty_like(x), np.empty_like(w), np.empty_like(bias)
        self._ok(self.lib.ref_conv2d_fwd_bwd(fp(x), fp(w), fp(bias), _i64(n), _i64(c), _i64(h),
                                             _i64(ww), _i64(oc), _i64(k), _i64(stride), _i64(pad),
                                             fp(dy), fp(y), fp(dx), fp(dw), fp(db)))
        return y, dx, dw, db

    def maxpool_fwd_bwd(self, x, k, stride, dy):
        x, dy = f32(x), f32(dy)
        y = np.empty(dy.shape, np.float32)
        dx = np.empty_like(x)
        self._ok(self.lib.ref_maxpool_fwd_bwd(fp(x), *[_i64(v) for v in x.shape], _i64(k),
                                              _i64(stride), fp(dy), fp(y), fp(dx)))
        return y, dx

    def layernorm_fwd_bwd(self, x, gamma, beta, dy):
        x, gamma, beta, dy = f32(x), f32(gamma), f32(beta), f32(dy)
        d = x.shape[-1]
        rows = x.size // d
        y, dx = np.empty_like(x), np.empty_like(x)
        dg, db = np.empty(d, np.float32), np.empty(d, np.float32)
        self._ok(self.lib.ref_layernorm_fwd_bwd(fp(x), fp(gamma), fp(beta), _i64(rows), _i64(d),
                                                fp(dy), fp(y), fp(dx), fp(dg), fp(db)))
        return y, dx, dg, db

    def cross_entropy(self, logits, targets):
        logits = f32(logits)
        t = np.ascontiguousarray(targets, np.int64)
        n, c = logits.shape
        loss = np.empty(1, np.float32)
        dl = np.empty_like(logits)
        self._ok(self.lib.ref_cross_entropy(fp(logits), ip(t), _i64(n), _i64(c), fp(loss), fp(dl)))
        return float(loss[0]), dl

    def embedding_fwd_bwd(self, table, ids, dy):
        table, ids, dy = f32(table), f32(ids), f32(dy)
        v, d = table.shape
        b, s = ids.shape
        y = np.empty((b, s, d), np.float32)
        dt = np.empty_like(table)
        self._ok(self.lib.ref_embedding_fwd_bwd(fp(table), _i64(v), _i64(d), fp(ids), _i64(b),
                                                _i64(s), fp(dy), fp(y), fp(dt)))
        return y, dt

    def adam_steps(self, p, grads, lr, b1=0.9, b2=0.999, eps=1e-8, wd=0.0):
        p = f32(p).copy()
        grads = f32(grads)
        self._ok(self.lib.ref_adam_steps(fp(p), fp(grads), p.size, grads.size // p.size, lr, b1,
                                         b2, eps, wd))
        return p

    def cnn_save(self, params, path, in_c=1, c1=8, c2=16, hw=28, classes=10):
        """The reference's save_parameters of its CNN holding `params`."""
        p = f32(params)
        self.lib.ref_cnn_save.argtypes = [_f32p] + [_i64] * 5 + [C.c_char_p]
        self._ok(self.lib.ref_cnn_save(fp(p), in_c, c1, c2, hw, classes, path.encode()))

    def cnn_load(self, path, n_params, in_c=1, c1=8, c2=16, hw=28, classes=10):
        """The reference's strict load_parameters into its CNN; the flat parameters."""
        out = np.empty(n_params, np.float32)
        self.lib.ref_cnn_load.argtypes = [C.c_char_p] + [_i64] * 5 + [_f32p]
        self._ok(self.lib.ref_cnn_load(path.encode(), in_c, c1, c2, hw, classes, fp(out)))
        return out

    def sum(self, x):
        """Tensor::sum(): the double accumulation cast to float."""
        x = f32(x)
        out = np.empty(1, np.float32)
        self._ok(self.lib.ref_sum(fp(x), _i64(x.size), fp(out)))
        return out[0]

    def mean(self, x):
        x = f32(x)
        out = np.empty(1, np.float32)
        self._ok(self.lib.ref_mean(fp(x), _i64(x.size), fp(out)))
        return out[0]

    def scalar(self, x, k, mul=False):
        """x + k, or x * k when mul."""
        x = f32(x)
        out = np.empty_like(x)
        self._ok(self.lib.ref_scalar(fp(x), _i64(x.size), C.c_float(k), int(mul), fp(out)))
        return out

    def clip_grad_norm(self, grads, sizes, max_norm):
        """grads: concatenated gradients of the parameters whose size is positive; a
        negative size is a parameter without a gradient. Returns (norm, clipped)."""
        g = f32(grads).copy()
        sz = np.ascontiguousarray(sizes, np.int64)
        norm = C.c_float()
        self._ok(self.lib.ref_clip_grad_norm(fp(g), ip(sz), len(sz), C.c_float(max_norm),
                                             C.byref(norm)))
        return norm.value, g

    def attention_fwd_bwd(self, q, k, v, mask, dy):
        q, k, v, dy = f32(q), f32(k), f32(v), f32(dy)
        b, h, s, dk = q.shape
        y = np.empty_like(q)
        w = np.empty((b, h, s, s), np.float32)
        dq, dkk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
        mp = fp(f32(mask)) if mask is not None else None
        self._ok(self.lib.ref_attention_fwd_bwd(fp(q), fp(k), fp(v), mp, _i64(b), _i64(h),
                                                _i64(s), _i64(dk), fp(dy), fp(y), fp(w), fp(dq),
                                                fp(dkk), fp(dv)))
        return y, w, dq, dkk, dv

    def block_num_params(self, d, heads, ff):
        return self.lib.ref_block_num_params(_i64(d), _i64(heads), _i64(ff))

    def block_fwd_bwd(self, x, heads, ff, causal, params, dy):
        x, params, dy = f32(x), f32(params), f32(dy)
        b, s, d = x.shape
        y, dx = np.empty_like(x), np.empty_like(x)
        dp = np.empty_like(params)
        self._ok(self.lib.ref_block_fwd_bwd(fp(x), _i64(b), _i64(s), _i64(d), _i64(heads),
                                            _i64(ff), int(causal), fp(params), fp(dy), fp(y),
                                            fp(dx), fp(dp)))
        return y, dx, dp

    def cnn_grads(self, x, labels, params, c1=8, c2=16, classes=10):
        """One forward and backward: (loss, flat gradients in parameter order)."""
        x, params = f32(x), f32(params)
        labels = np.ascontiguousarray(labels, np.int64)
        b, cin, hw, _ = x.shape
        loss = np.empty(1, np.float32)
        grads = np.empty_like(params)
        f = self.lib.ref_cnn_grads
        f.argtypes = [_f32p, _i64p] + [_i64] * 6 + [_f32p, _f32p, _f32p]
        self._ok(f(fp(x), ip(labels), b, cin, c1, c2, hw, classes, fp(params), fp(loss),
                   fp(grads)))
        return float(loss[0]), grads

    def cnn_train(self, x, labels, params, steps, lr, c1=8, c2=16, classes=10):
        x, params = f32(x), f32(params)
        labels = np.ascontiguousarray(labels, np.int64)
        b, cin, hw, _ = x.shape
        losses = np.empty(steps, np.float32)
        out = np.empty_like(params)
        self._ok(self.lib.ref_cnn_train(fp(x), ip(labels), b, cin, c1, c2, hw, classes,
                                        fp(params), steps, lr, fp(losses), fp(out)))
        return losses, out

    def charlm_num_params(self, vocab, seq, d, heads, ff, layers):
        return self.lib.ref_charlm_num_params(_i64(vocab), _i64(seq), _i64(d), _i64(heads),
                                              _i64(ff), _i64(layers))

    def charlm_train(self, ids, targets, vocab, d, heads, ff, layers, params, steps, lr,
                     grads0=False):
        """`steps` Adam steps on one batch: per-step losses and the final parameters, and
        with grads0 the first step's gradients (flat, parameter order) as a third value."""
        ids, params = f32(ids), f32(params)
        targets = np.ascontiguousarray(targets, np.int64)
        b, s = ids.shape
        losses = np.empty(steps, np.float32)
        out = np.empty_like(params)
        if not grads0:
            self._ok(self.lib.ref_charlm_train(fp(ids), ip(targets), b, s, vocab, d, heads, ff,
                                               layers, fp(params), steps, lr, fp(losses), fp(out)))
            return losses, out
        g0 = np.empty_like(params)
        self._ok(self.lib.ref_charlm_train_grads(fp(ids), ip(targets), b, s, vocab, d, heads, ff,
                                                 layers, fp(params), steps, lr, fp(losses),
                                                 fp(g0), fp(out)))
        return losses, out, g0


def oracle_or_skip():
    import pytest
    try:
        return Oracle()
    except (FileNotFoundError, OSError) as e:
        pytest.skip(str(e))


def ref_or_skip():
    import pytest
    try:
        return Ref()
    except (FileNotFoundError, OSError) as e:
        pytest.skip(str(e))
