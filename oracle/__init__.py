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


class GptConfig(ctypes.Structure):
    """vo_gpt_config: SimpleGPT with one block (B x S ids, width D, H heads,
    MLP width F, vocabulary V, max_seq_len P)."""
    _fields_ = [(n, c_int64) for n in ("B", "S", "D", "H", "F", "V", "P")]


GPT_PARAM_NAMES = ("wte", "wpe", "ln1_w", "ln1_b", "q_w", "q_b", "k_w", "k_b", "v_w", "v_b",
                   "o_w", "o_b", "ln2_w", "ln2_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b",
                   "lnf_w", "lnf_b", "lm_w")


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
        "vo_math": [c_int, f, f, c_int64],
        "vo_reduce_to": [f, L, POINTER(c_int64), c_int, f] + err,
        "vo_softmax_backward_composite": [f, f, L, c_int, f] + err,
        "vo_gelu_bias_forward": [f, f, c_int64, c_int64, f],
        "vo_gelu_bias_backward": [f, f, f, c_int64, c_int64, f, f],
        "vo_format_f32": [c_float, c_char_p, c_size_t],
        "vo_set_threads": [c_int],
        "vo_matmul": [f, L, f, L, f] + err,
        "vo_fused_attention": [f, f, f, c_int64, c_int64, c_int64, c_int64, f, L, f],
        "vo_fused_attention_backward": [f, f, f, c_int64, c_int64, c_int64, c_int64, f, L, f, f,
                                        f, f],
        "vo_adamw_step": [f, f, f, f, c_int64, c_int, c_float, c_float, c_float, c_float,
                          c_float],
        "vo_gpt_param_numel": [POINTER(GptConfig), POINTER(c_int64)],
        "vo_gpt_step": [POINTER(GptConfig), POINTER(c_void_p), f, f, f, POINTER(c_void_p)] + err,
        "vo_gpt_step_ex": [POINTER(GptConfig), POINTER(c_void_p), f, f, c_int, f, POINTER(c_void_p)] + err,
        "vo_attention_unfused": [f, f, f, c_int64, c_int64, c_int64, c_int64, f, L, f] + err,
        "vo_attention_unfused_backward": [f, f, f, c_int64, c_int64, c_int64, c_int64, f, L, f, f, f,
                                          f] + err,
        "vo_checkpoint_save": [c_char_p, c_int, POINTER(c_void_p), L] + err,
        "vo_checkpoint_load": [c_char_p, c_int, POINTER(c_void_p), L] + err,
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = None if name in (
            "vo_gelu", "vo_gelu_grad_mask", "vo_gelu_bias_forward",
            "vo_gelu_bias_backward", "vo_format_f32", "vo_set_threads", "vo_adamw_step",
            "vo_gpt_param_numel") else c_int
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


def set_threads(n: int) -> None:
    lib.vo_set_threads(int(n))


def matmul(a, b):
    """Batched matmul with broadcast batch dims (operands made contiguous first,
    as the reference does)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    batch = np.broadcast_shapes(a.shape[:-2], b.shape[:-2]) if a.ndim >= 2 and b.ndim >= 2 else ()
    shape = tuple(batch) + ((a.shape[-2], b.shape[-1]) if a.ndim >= 2 and b.ndim >= 2 else ())
    out = np.zeros(shape, np.float32)
    ob = out if out.size else np.zeros(1, np.float32)
    ab = a if a.size else np.zeros(1, np.float32)
    bb = b if b.size else np.zeros(1, np.float32)
    _call(lib.vo_matmul, _ptr(ab), layout(a.shape), _ptr(bb), layout(b.shape), _ptr(ob))
    return out


def _att_args(q, k, v, mask):
    q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
    if mask is None:
        return q, k, v, None, None
    m = np.ascontiguousarray(mask, np.float32)
    return q, k, v, m, layout(m.shape)


def fused_attention(q, k, v, mask=None):
    q, k, v, m, ml = _att_args(q, k, v, mask)
    B, H, S, Dk = q.shape
    out = np.zeros_like(q)
    lib.vo_fused_attention(_ptr(q), _ptr(k), _ptr(v), B, H, S, Dk,
                           _ptr(m) if m is not None else None, ml, _ptr(out))
    return out


def fused_attention_backward(q, k, v, mask, go):
    q, k, v, m, ml = _att_args(q, k, v, mask)
    go = np.ascontiguousarray(go, np.float32)
    B, H, S, Dk = q.shape
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    lib.vo_fused_attention_backward(_ptr(q), _ptr(k), _ptr(v), B, H, S, Dk,
                                    _ptr(m) if m is not None else None, ml, _ptr(go),
                                    _ptr(dq), _ptr(dk), _ptr(dv))
    return dq, dk, dv


def attention_unfused(q, k, v, mask=None):
    """MultiHeadAttention's unfused path (VEARO_USE_FUSED_ATTENTION=0,
    nn:603-613): q.matmul(k^T).mul(scale) (+ mask), softmax(3), matmul(v)."""
    q, k, v, m, ml = _att_args(q, k, v, mask)
    B, H, S, Dk = q.shape
    out = np.zeros_like(q)
    _call(lib.vo_attention_unfused, _ptr(q), _ptr(k), _ptr(v), B, H, S, Dk,
          _ptr(m) if m is not None else None, ml, _ptr(out))
    return out


def attention_unfused_backward(q, k, v, mask, go):
    """dq, dk, dv of the unfused path: its tape's arms walked back."""
    q, k, v, m, ml = _att_args(q, k, v, mask)
    go = np.ascontiguousarray(go, np.float32)
    B, H, S, Dk = q.shape
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    _call(lib.vo_attention_unfused_backward, _ptr(q), _ptr(k), _ptr(v), B, H, S, Dk,
          _ptr(m) if m is not None else None, ml, _ptr(go), _ptr(dq), _ptr(dk), _ptr(dv))
    return dq, dk, dv


def adamw_step(p, g, m, v, t, lr, beta1, beta2, eps, wd):
    """In place on float32 contiguous arrays p, m, v."""
    for a in (p, m, v):
        assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    g = np.ascontiguousarray(g, np.float32)
    lib.vo_adamw_step(_ptr(p), _ptr(g), _ptr(m), _ptr(v), p.size, int(t), c_float(lr),
                      c_float(beta1), c_float(beta2), c_float(eps), c_float(wd))


def gpt_param_shapes(cfg: GptConfig):
    D, F, V, P = cfg.D, cfg.F, cfg.V, cfg.P
    return [(V, D), (P, D), (D,), (D,), (D, D), (D,), (D, D), (D,), (D, D), (D,), (D, D), (D,),
            (D,), (D,), (F, D), (F,), (D, F), (D,), (D,), (D,), (V, D)]


def gpt_step(cfg: GptConfig, params, ids, targets, grads: bool = True, fused_attention: bool = True):
    """(loss, [grad per parameter] or None) of one SimpleGPT forward(+backward);
    fused_attention=False takes MultiHeadAttention's unfused path."""
    params = [np.ascontiguousarray(p, np.float32) for p in params]
    shapes = gpt_param_shapes(cfg)
    assert len(params) == len(shapes)
    for p, sh in zip(params, shapes):
        assert p.shape == sh, (p.shape, sh)
    ids = np.ascontiguousarray(ids, np.float32)
    targets = np.ascontiguousarray(targets, np.float32)
    pp = (c_void_p * len(params))(*[p.ctypes.data for p in params])
    loss = np.zeros(1, np.float32)
    gs = gp = None
    if grads:
        gs = [np.zeros(sh, np.float32) for sh in shapes]
        gp = (c_void_p * len(gs))(*[g.ctypes.data for g in gs])
    _call(lib.vo_gpt_step_ex, ctypes.byref(cfg), pp, _ptr(ids), _ptr(targets), 0 if fused_attention else 1,
          _ptr(loss), gp)
    return float(loss[0]), gs


class CheckpointIOError(OSError):
    """The reference's save/load_checkpoint would return this io::Error."""


def _ckpt_args(arrays):
    n = len(arrays)
    ptrs = (c_void_p * max(n, 1))()
    lays = (Layout * max(n, 1))()
    keep = []
    for i, a in enumerate(arrays):
        if a.dtype != np.float32:
            raise TypeError("checkpoint tensors are float32")
        keep.append(a)
        ptrs[i] = a.ctypes.data if a.size else None
        if a.flags["C_CONTIGUOUS"]:
            lays[i] = layout(a.shape)
        else:
            lays[i] = layout(a.shape, [st // 4 for st in a.strides])
    return n, ptrs, lays, keep


def _ckpt_call(fn, path, arrays):
    n, ptrs, lays, keep = _ckpt_args(arrays)
    buf = ctypes.create_string_buffer(512)
    rc = fn(os.fsencode(path), n, ptrs, lays, buf, 512)
    del keep
    if rc == 1:
        raise Panic(buf.value.decode())
    if rc == 2:
        raise CheckpointIOError(buf.value.decode())


def checkpoint_save(path, arrays) -> None:
    """save_checkpoint (crates/vearo/src/checkpoint.rs:9-33) of float32 arrays."""
    _ckpt_call(lib.vo_checkpoint_save, path, [np.asarray(a) for a in arrays])


def checkpoint_load(path, arrays) -> None:
    """load_checkpoint (checkpoint.rs:40-91) into float32 arrays, in place."""
    _ckpt_call(lib.vo_checkpoint_load, path, arrays)


def math_fn(which, x):
    """The C library's expf / logf / tanhf (which = 0 / 1 / 2) on every element."""
    xb = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.empty_like(xb)
    if xb.size:
        lib.vo_math(int(which), _ptr(xb), _ptr(out), xb.size)
    return out.reshape(np.shape(x))
