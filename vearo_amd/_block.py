"""ctypes binding of the config[4] training step (include/vearo_block.h,
vearo_amd/lib/libvearo_backend.so). Plumbing for tests, bench and smoke; the
step itself runs in the C++ driver on the C ABI. No CPU fallback."""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int64, c_void_p

import numpy as np

from . import _abi

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libvearo_backend.so")
NPARAMS = 21
PARAM_NAMES = ("wte", "wpe", "ln1_w", "ln1_b", "q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "o_w", "o_b",
               "ln2_w", "ln2_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b", "lnf_w", "lnf_b", "lm_w")


class GptConfig(ctypes.Structure):
    _fields_ = [(n, c_int64) for n in ("B", "S", "D", "H", "F", "V", "P")]


def param_shapes(c: GptConfig):
    D, F, V, P = c.D, c.F, c.V, c.P
    return [(V, D), (P, D), (D,), (D,), (D, D), (D,), (D, D), (D,), (D, D), (D,), (D, D), (D,),
            (D,), (D,), (F, D), (F,), (D, F), (D,), (D,), (D,), (V, D)]


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build with __graft_entry__.build() (no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    H = c_void_p
    sig = {
        "vb_gpt_create": (c_int, [POINTER(GptConfig), POINTER(c_void_p)]),
        "vb_gpt_destroy": (None, [H]),
        "vb_gpt_param": (c_int, [H, c_int, POINTER(c_void_p), POINTER(c_int64)]),
        "vb_gpt_grad": (c_int, [H, c_int, POINTER(c_void_p), POINTER(c_int64)]),
        "vb_gpt_inputs": (c_int, [H, POINTER(c_void_p), POINTER(c_void_p)]),
        "vb_gpt_forward_backward": (c_int, [H, c_int]),
        "vb_gpt_loss_ptr": (c_void_p, [H]),
        "vb_gpt_adamw": (c_int, [H, c_float, c_float, c_float, c_float, c_float]),
        "vb_gpt_train_step": (c_int, [H, c_float, c_float, c_float, c_float, c_float]),
        "vb_last_error": (ctypes.c_char_p, []),
        "vb_gpt_save": (c_int, [H, ctypes.c_char_p]),
        "vb_gpt_load": (c_int, [H, ctypes.c_char_p]),
        "vb_gpt_set_gemm_engine": (c_int, [H, c_int]),
        "vb_dropin_create": (c_int, [POINTER(GptConfig), POINTER(c_void_p)]),
        "vb_dropin_destroy": (None, [H]),
        "vb_dropin_set_fused_attention": (c_int, [H, c_int]),
        "vb_dropin_fused_attention": (c_int, [H]),
        "vb_dropin_set_fold_weight_grads": (c_int, [H, c_int]),
        "vb_dropin_fold_weight_grads": (c_int, [H]),
        "vb_dropin_set_param": (c_int, [H, c_int, c_void_p, c_int64]),
        "vb_dropin_get_param": (c_int, [H, c_int, c_void_p, c_int64]),
        "vb_dropin_get_grad": (c_int, [H, c_int, c_void_p, c_int64]),
        "vb_dropin_set_inputs": (c_int, [H, c_void_p, c_void_p]),
        "vb_dropin_step": (c_int, [H, c_int, c_int, c_float, c_float, c_float, c_float, c_float, c_int,
                                   POINTER(c_float)]),
        "vb_dropin_phase_ms": (c_int, [H, POINTER(ctypes.c_double), c_int]),
        "vb_dropin_phase_name": (ctypes.c_char_p, [c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


lib = _load()


def check(rc: int) -> None:
    if rc != 0:
        raise _abi.VhError(rc, (lib.vb_last_error() or b"").decode())


class Gpt:
    """One SimpleGPT (one block) on the device."""

    def __init__(self, cfg: GptConfig):
        self.cfg = cfg
        h = c_void_p()
        check(lib.vb_gpt_create(ctypes.byref(cfg), ctypes.byref(h)))
        self.h = h
        self.shapes = param_shapes(cfg)

    def _ptr(self, fn, i):
        p, n = c_void_p(), c_int64()
        check(fn(self.h, i, ctypes.byref(p), ctypes.byref(n)))
        return p.value, n.value

    def set_params(self, params) -> None:
        for i, a in enumerate(params):
            a = np.ascontiguousarray(a, np.float32)
            p, n = self._ptr(lib.vb_gpt_param, i)
            assert a.size == n and a.shape == self.shapes[i], (i, a.shape, self.shapes[i])
            _abi.check(_abi.lib.vh_h2d(p, a.ctypes.data, a.nbytes))

    def _get(self, fn, i):
        p, n = self._ptr(fn, i)
        out = np.empty(self.shapes[i], np.float32)
        _abi.sync()
        _abi.check(_abi.lib.vh_d2h(out.ctypes.data, p, out.nbytes))
        return out

    def params(self):
        return [self._get(lib.vb_gpt_param, i) for i in range(NPARAMS)]

    def grads(self):
        return [self._get(lib.vb_gpt_grad, i) for i in range(NPARAMS)]

    def set_inputs(self, ids, targets) -> None:
        i, t = c_void_p(), c_void_p()
        check(lib.vb_gpt_inputs(self.h, ctypes.byref(i), ctypes.byref(t)))
        ids = np.ascontiguousarray(ids, np.float32).reshape(-1)
        targets = np.ascontiguousarray(targets, np.float32).reshape(-1)
        assert ids.size == self.cfg.B * self.cfg.S and targets.size == ids.size
        _abi.check(_abi.lib.vh_h2d(i.value, ids.ctypes.data, ids.nbytes))
        _abi.check(_abi.lib.vh_h2d(t.value, targets.ctypes.data, targets.nbytes))

    def set_gemm_engine(self, engine: int) -> None:
        """vh_gemm engine of the dense products: 0 (this library's kernels) or
        2 (hipBLASLt, an A/B reference)."""
        check(lib.vb_gpt_set_gemm_engine(self.h, engine))

    def forward_backward(self, backward: bool = True) -> None:
        check(lib.vb_gpt_forward_backward(self.h, 1 if backward else 0))

    def loss(self) -> float:
        out = np.empty(1, np.float32)
        _abi.sync()
        _abi.check(_abi.lib.vh_d2h(out.ctypes.data, lib.vb_gpt_loss_ptr(self.h), 4))
        return float(out[0])

    def adamw(self, lr=0.02, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.01) -> None:
        check(lib.vb_gpt_adamw(self.h, lr, beta1, beta2, eps, wd))

    def train_step(self, lr=0.02, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.01) -> None:
        check(lib.vb_gpt_train_step(self.h, lr, beta1, beta2, eps, wd))

    def save(self, path) -> None:
        """The parameters as a `.ve` checkpoint (checkpoint.rs:9-33)."""
        check(lib.vb_gpt_save(self.h, os.fsencode(path)))

    def load(self, path) -> None:
        """Parameters from a `.ve` checkpoint (checkpoint.rs:40-91)."""
        check(lib.vb_gpt_load(self.h, os.fsencode(path)))

    def close(self) -> None:
        if self.h is not None:
            lib.vb_gpt_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


DROPIN_NPHASES = 23


class DropIn:
    """The same model and step issued op by op through the HIP BackendOps
    table in the reference's own order (SimpleGPT::forward's tape, then
    backward_impl's arms, then AdamW::step): include/vearo_block.h vb_dropin_*."""

    def __init__(self, cfg: GptConfig, fused_attention=None, fold_weight_grads=True):
        """fused_attention: None keeps the reference's switch (the environment
        variable VEARO_USE_FUSED_ATTENTION), True / False force the path.
        fold_weight_grads: the Matmul arm's shared-weight gradient as one
        product over all rows (True) or the reference's per-batch product and
        reduce_to (False)."""
        self.cfg = cfg
        h = c_void_p()
        check(lib.vb_dropin_create(ctypes.byref(cfg), ctypes.byref(h)))
        self.h = h
        self.shapes = param_shapes(cfg)
        if fused_attention is not None:
            check(lib.vb_dropin_set_fused_attention(self.h, int(bool(fused_attention))))
        check(lib.vb_dropin_set_fold_weight_grads(self.h, int(bool(fold_weight_grads))))

    @property
    def fused_attention(self) -> bool:
        return bool(lib.vb_dropin_fused_attention(self.h))

    @property
    def fold_weight_grads(self) -> bool:
        return bool(lib.vb_dropin_fold_weight_grads(self.h))

    def set_params(self, params) -> None:
        for i, a in enumerate(params):
            a = np.ascontiguousarray(a, np.float32)
            assert a.shape == self.shapes[i], (i, a.shape, self.shapes[i])
            check(lib.vb_dropin_set_param(self.h, i, a.ctypes.data, a.size))

    def _get(self, fn, i):
        out = np.empty(self.shapes[i], np.float32)
        check(fn(self.h, i, out.ctypes.data, out.size))
        return out

    def params(self):
        return [self._get(lib.vb_dropin_get_param, i) for i in range(NPARAMS)]

    def grads(self):
        return [self._get(lib.vb_dropin_get_grad, i) for i in range(NPARAMS)]

    def set_inputs(self, ids, targets) -> None:
        ids = np.ascontiguousarray(ids, np.float32).reshape(-1)
        targets = np.ascontiguousarray(targets, np.float32).reshape(-1)
        assert ids.size == self.cfg.B * self.cfg.S and targets.size == ids.size
        check(lib.vb_dropin_set_inputs(self.h, ids.ctypes.data, targets.ctypes.data))

    def step(self, backward=True, adamw=False, lr=0.02, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.01,
             timing=False, want_loss=True):
        """One step; returns the loss (or None with want_loss=False, which
        leaves the step queued)."""
        loss = c_float()
        check(lib.vb_dropin_step(self.h, int(backward), int(adamw), lr, beta1, beta2, eps, wd, int(timing),
                                 ctypes.byref(loss) if want_loss else None))
        return float(loss.value) if want_loss else None

    def phase_ms(self) -> dict:
        """Per-phase milliseconds of the last step run with timing=True."""
        ms = (ctypes.c_double * DROPIN_NPHASES)()
        check(lib.vb_dropin_phase_ms(self.h, ms, DROPIN_NPHASES))
        return {lib.vb_dropin_phase_name(i).decode(): ms[i] for i in range(DROPIN_NPHASES)}

    def close(self) -> None:
        if self.h is not None:
            lib.vb_dropin_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
