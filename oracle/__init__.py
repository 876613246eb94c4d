"""CPU oracle -- TEST INFRASTRUCTURE ONLY.

ctypes wrapper over liboracle_cpu.so, the C restatement of vearo-backend-cpu's
hot-path functions (oracle/vearo_cpu_ref.c). Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import this package; the product
(vearo_amd, libvearo_hip.so) never does.

Arrays are numpy float32. Strided inputs are passed as (base array, dims,
element strides) so views behave like vearo-core's strided tensors.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_cpu.so")
MAX_RANK = 8


class Layout(ctypes.Structure):
    _fields_ = [
        ("rank", ctypes.c_int32),
        ("dims", c_int64 * MAX_RANK),
        ("strides", c_int64 * MAX_RANK),
    ]


class Panic(RuntimeError):
    """The reference CPU backend would panic with this message."""


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
    lib = ctypes.CDLL(LIB_PATH)
    L = POINTER(Layout)
    f = c_void_p
    err = [c_char_p, c_size_t]
    sig = {
        "vo_binary": [c_int, f, L, f, L, f, L] + err,
        "vo_gelu": [f, L, f],
        "vo_softmax": [f, L, c_int, f] + err,
        "vo_sum": [f, L, c_int, c_int, f] + err,
        "vo_mean": [f, L, c_int, c_int, f] + err,
        "vo_layernorm": [f, L, f, L, f, L, c_float, f] + err,
        "vo_layernorm_backward": [f, L, f, L, L, f, L, c_float, f, f, f] + err,
        "vo_embedding": [f, L, f, L, f] + err,
        "vo_embedding_backward": [f, L, L, f, L, f] + err,
        "vo_cross_entropy": [f, L, f, L, f] + err,
        "vo_cross_entropy_backward": [f, L, f, L, f, c_int64, f] + err,
        "vo_gelu_grad_mask": [f, c_int64, f],
        "vo_reduce_to": [f, L, POINTER(c_int64), c_int, f] + err,
        "vo_softmax_backward_composite": [f, f, L, c_int, f] + err,
        "vo_gelu_bias_forward": [f, f, c_int64, c_int64, f],
        "vo_gelu_bias_backward": [f, f, f, c_int64, c_int64, f, f],
        "vo_format_f32": [c_float, c_char_p, c_size_t],
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = None if name in (
            "vo_gelu", "vo_gelu_grad_mask", "vo_gelu_bias_forward",
            "vo_gelu_bias_backward", "vo_format_f32") else c_int
    return lib


lib = _load()


def layout(dims, strides=None) -> Layout:
    dims = [int(d) for d in dims]
    if strides is None:
        strides, acc = [0] * len(dims), 1
        for i in range(len(dims) - 1, -1, -1):
            strides[i] = acc
            acc *= dims[i]
    l = Layout()
    l.rank = len(dims)
    for i, (d, s) in enumerate(zip(dims, strides)):
        l.dims[i] = d
        l.strides[i] = int(s)
    return l


def _view(a):
    """(contiguous base, Layout) for a numpy float32 array or a strided view."""
    a = np.asarray(a, dtype=np.float32)
    if a.size == 0:
        return np.zeros(1, np.float32), layout(a.shape)
    # Express the view over its own base buffer via element strides.
    if a.flags["C_CONTIGUOUS"]:
        return a, layout(a.shape)
    base = a.base if a.base is not None and isinstance(a.base, np.ndarray) else None
    if base is not None and base.dtype == np.float32 and base.flags["C_CONTIGUOUS"] and \
            a.__array_interface__["data"][0] == base.__array_interface__["data"][0]:
        strides = [s // 4 for s in a.strides]
        return base, layout(a.shape, strides)
    c = np.ascontiguousarray(a)
    return c, layout(c.shape)


def _ptr(a):
    return a.ctypes.data_as(c_void_p)


def _call(fn, *args):
    buf = ctypes.create_string_buffer(512)
    rc = fn(*args, buf, 512)
    if rc != 0:
        raise Panic(buf.value.decode())


def binary(op: int, l, r):
    lb, ll = _view(l)
    rb, rl = _view(r)
    try:
        shape = np.broadcast_shapes(np.shape(l), np.shape(r))
    except ValueError:
        shape = np.shape(l)  # the C oracle reports the reference's panic
    out = np.empty(shape, np.float32)
    ob = out if out.size else np.zeros(1, np.float32)
    _call(lib.vo_binary, op, _ptr(lb), ll, _ptr(rb), rl, _ptr(ob), layout(shape))
    return out


def gelu(x):
    xb, xl = _view(x)
    out = np.empty(np.shape(x), np.float32)
    if out.size:
        lib.vo_gelu(_ptr(xb), xl, _ptr(out))
    return out


def softmax(x, dim):
    xb, xl = _view(x)
    out = np.empty(np.shape(x), np.float32)
    ob = out if out.size else np.zeros(1, np.float32)
    _call(lib.vo_softmax, _ptr(xb), xl, dim, _ptr(ob))
    return out


def reduce(x, dim, keep_dim=False, mean=False):
    xb, xl = _view(x)
    shape = list(np.shape(x))
    if keep_dim:
        shape[dim] = 1
    else:
        shape.pop(dim)
    out = np.zeros(shape, np.float32)
    ob = out if out.size else np.zeros(1, np.float32)
    fn = lib.vo_mean if mean else lib.vo_sum
    _call(fn, _ptr(xb), xl, dim, int(keep_dim), _ptr(ob))
    return out


def layernorm(x, w, b, eps):
    xb, xl = _view(x)
    wb, wl = _view(w)
    bb, bl = _view(b)
    out = np.zeros(np.shape(x), np.float32)
    ob = out if out.size else np.zeros(1, np.float32)
    _call(lib.vo_layernorm, _ptr(xb), xl, _ptr(wb), wl, _ptr(bb), bl, c_float(eps), _ptr(ob))
    return out


def layernorm_backward(x, w, b, go, eps):
    xb, xl = _view(x)
    wb, wl = _view(w)
    _, bl = _view(b)
    gb_, gl = _view(go)
    gx = np.zeros(np.shape(x), np.float32)
    gw = np.zeros(np.shape(w), np.float32)
    gbias = np.zeros(np.shape(b), np.float32)
    gxb = gx if gx.size else np.zeros(1, np.float32)
    _call(lib.vo_layernorm_backward, _ptr(xb), xl, _ptr(wb), wl, bl, _ptr(gb_), gl,
          c_float(eps), _ptr(gxb), _ptr(gw), _ptr(gbias))
    return gx, gw, gbias


def embedding(ids, w):
    ib, il = _view(ids)
    wb, wl = _view(w)
    out = np.zeros(tuple(np.shape(ids)) + (np.shape(w)[1] if np.ndim(w) == 2 else 0,), np.float32)
    ob = out if out.size else np.zeros(1, np.float32)
    _call(lib.vo_embedding, _ptr(ib), il, _ptr(wb), wl, _ptr(ob))
    return out


def embedding_backward(ids, w_shape, go):
    ib, il = _view(ids)
    wl = layout(w_shape)
    gb_, gl = _view(go)
    gw = np.zeros(w_shape, np.float32)
    gwb = gw if gw.size else np.zeros(1, np.float32)
    _call(lib.vo_embedding_backward, _ptr(ib), il, wl, _ptr(gb_), gl, _ptr(gwb))
    return gw


def cross_entropy(logits, targets):
    lb, ll = _view(logits)
    tb, tl = _view(targets)
    out = np.zeros(1, np.float32)
    _call(lib.vo_cross_entropy, _ptr(lb), ll, _ptr(tb), tl, _ptr(out))
    return out


def cross_entropy_backward(logits, targets, grad_out):
    lb, ll = _view(logits)
    tb, tl = _view(targets)
    go = np.ascontiguousarray(grad_out, np.float32).reshape(-1)
    gl = np.zeros(np.shape(logits), np.float32)
    glb = gl if gl.size else np.zeros(1, np.float32)
    gob = go if go.size else np.zeros(1, np.float32)
    _call(lib.vo_cross_entropy_backward, _ptr(lb), ll, _ptr(tb), tl, _ptr(gob), go.size, _ptr(glb))
    return gl


def gelu_grad_mask(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    if x.size:
        lib.vo_gelu_grad_mask(_ptr(x), x.size, _ptr(out))
    return out


def reduce_to(grad, target_shape):
    g = np.ascontiguousarray(grad, np.float32)
    t = (c_int64 * max(1, len(target_shape)))(*[int(v) for v in target_shape])
    out = np.zeros(target_shape, np.float32)
    ob = out if out.size else np.zeros(1, np.float32)
    gb_ = g if g.size else np.zeros(1, np.float32)
    _call(lib.vo_reduce_to, _ptr(gb_), layout(g.shape), t, len(target_shape), _ptr(ob))
    return out


def softmax_backward_composite(x, dy, dim):
    x = np.ascontiguousarray(x, np.float32)
    dy = np.ascontiguousarray(dy, np.float32)
    dx = np.zeros_like(x)
    _call(lib.vo_softmax_backward_composite, _ptr(x), _ptr(dy), layout(x.shape), dim, _ptr(dx))
    return dx


def gelu_bias_forward(x, bias):
    x = np.ascontiguousarray(x, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    rows, C = x.shape
    y = np.empty_like(x)
    lib.vo_gelu_bias_forward(_ptr(x), _ptr(bias), rows, C, _ptr(y))
    return y


def gelu_bias_backward(x, bias, dy):
    x = np.ascontiguousarray(x, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    dy = np.ascontiguousarray(dy, np.float32)
    rows, C = x.shape
    dx = np.empty_like(x)
    db = np.empty(C, np.float32)
    lib.vo_gelu_bias_backward(_ptr(x), _ptr(bias), _ptr(dy), rows, C, _ptr(dx), _ptr(db))
    return dx, db


def format_f32(v: float) -> str:
    buf = ctypes.create_string_buffer(64)
    lib.vo_format_f32(c_float(v), buf, 64)
    return buf.value.decode()
