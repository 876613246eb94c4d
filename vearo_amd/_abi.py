"""ctypes binding of libvearo_hip.so (declared in include/vearo_hip.h).

This is plumbing for Python callers (tests, bench, smoke): every call goes
straight to the C ABI, which launches the gfx950 kernels. There is no CPU
fallback: if the library has not been built, importing this module raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libvearo_hip.so")

VH_OK = 0
VH_ERR_INVALID = 1
VH_ERR_HIP = 2
VH_ERR_NOT_INIT = 3
VH_ERR_DEVICE_PANIC = 4
VH_ERR_UNSUPPORTED = 5
VH_ERR_OOM = 6
VH_ERR_IO = 7
MAX_RANK = 8

OP_ADD, OP_SUB, OP_MUL, OP_DIV = 0, 1, 2, 3


class VhLayout(ctypes.Structure):
    _fields_ = [
        ("rank", c_int32),
        ("pad_", c_int32),
        ("dims", c_int64 * MAX_RANK),
        ("strides", c_int64 * MAX_RANK),
    ]


class VhMemStats(ctypes.Structure):
    _fields_ = [
        ("live_bytes", c_size_t),
        ("cached_bytes", c_size_t),
        ("peak_bytes", c_size_t),
        ("hip_bytes", c_size_t),
    ]


class VhGemmDesc(ctypes.Structure):
    """vh_gemm_desc (include/vearo_hip.h)."""
    _fields_ = [
        ("M", c_int64), ("N", c_int64), ("K", c_int64),
        ("a", c_void_p), ("a_sm", c_int64), ("a_sk", c_int64),
        ("b", c_void_p), ("b_sk", c_int64), ("b_sn", c_int64),
        ("c", c_void_p), ("c_sm", c_int64),
        ("batch", c_int64 * 2), ("a_sb", c_int64 * 2), ("b_sb", c_int64 * 2), ("c_sb", c_int64 * 2),
        ("e", c_void_p), ("e_sm", c_int64), ("e_sn", c_int64), ("e_sb", c_int64 * 2),
        ("alpha", c_float), ("accumulate", c_int32), ("causal", c_int32), ("engine", c_int32),
    ]


GEMM_DENSE, GEMM_SKIP_UPPER, GEMM_K_LE_M, GEMM_K_GE_M = 0, 1, 2, 3
GEMM_ENGINE_DEFAULT, GEMM_ENGINE_TILED, GEMM_ENGINE_LIBRARY, GEMM_ENGINE_WIDE = 0, 1, 2, 3
MATH_EXP, MATH_LOG, MATH_TANH = 0, 1, 2
GEMM_PATH_NONE, GEMM_PATH_TILED, GEMM_PATH_SPLIT_K, GEMM_PATH_PERSISTENT, GEMM_PATH_LIBRARY, GEMM_PATH_BATCHED = range(6)


class VhError(RuntimeError):
    """A non-zero return from the C ABI; `code` is the VH_ERR_* value."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[vh error {code}] {msg}")
        self.code = code
        self.msg = msg


class DevicePanic(VhError):
    """The device met data the CPU backend panics on; msg is the CPU's text."""


fp = c_void_p  # device pointers travel as void*

# name -> (restype, argtypes)
SIGNATURES = {
    "vh_init": (c_int, [c_int]),
    "vh_shutdown": (c_int, []),
    "vh_last_error": (ctypes.c_char_p, []),
    "vh_stream": (c_void_p, []),
    "vh_gemm_last_path": (c_int, []),
    "vh_device_cu_count": (c_int, []),
    "vh_sync": (c_int, []),
    "vh_check_device_error": (c_int, []),
    "vh_alloc": (c_int, [c_size_t, c_int, POINTER(c_void_p)]),
    "vh_free": (c_int, [c_void_p]),
    "vh_h2d": (c_int, [c_void_p, c_void_p, c_size_t]),
    "vh_d2h": (c_int, [c_void_p, c_void_p, c_size_t]),
    "vh_d2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "vh_fill_f32": (c_int, [fp, c_float, c_int64, c_void_p]),
    "vh_math_probe": (c_int, [c_int32, fp, fp, c_int64, c_void_p]),
    "vh_mem_stats_get": (c_int, [POINTER(VhMemStats)]),
    "vh_empty_cache": (c_int, []),
    "vh_layernorm_fwd": (c_int, [fp, fp, fp, fp, c_int64, c_int64, c_float, c_void_p]),
    "vh_layernorm_bwd": (
        c_int,
        [fp, fp, fp, fp, fp, fp, c_int64, c_int64, c_float, c_void_p, c_size_t, c_void_p],
    ),
    "vh_layernorm_bwd_scratch_bytes": (c_size_t, [c_int64, c_int64]),
    "vh_layernorm_bwd_noalloc": (c_int, [fp, fp, fp, fp, fp, fp, c_int64, c_int64, c_float, c_void_p]),
    "vh_gelu_fwd": (c_int, [fp, fp, c_int64, c_void_p]),
    "vh_gelu_bias_fwd": (c_int, [fp, fp, fp, c_int64, c_int64, c_void_p]),
    "vh_gelu_grad_mul": (c_int, [fp, fp, fp, c_int64, c_void_p]),
    "vh_gelu_bias_bwd": (
        c_int,
        [fp, fp, fp, fp, fp, c_int64, c_int64, c_void_p, c_size_t, c_void_p],
    ),
    "vh_gelu_bias_bwd_scratch_bytes": (c_size_t, [c_int64, c_int64]),
    "vh_softmax_fwd": (c_int, [fp, fp, c_int64, c_int64, c_int, c_void_p]),
    "vh_softmax_bwd": (c_int, [fp, fp, fp, c_int64, c_int64, c_int, c_int, c_void_p]),
    "vh_embedding_fwd": (c_int, [fp, fp, fp, c_int64, c_int64, c_int64, c_void_p]),
    "vh_embedding_bwd": (
        c_int,
        [fp, fp, fp, c_int64, c_int64, c_int64, c_void_p, c_size_t, c_void_p],
    ),
    "vh_embedding_bwd_scratch_bytes": (c_size_t, [c_int64, c_int64, c_int64]),
    "vh_cross_entropy_fwd": (
        c_int,
        [fp, fp, fp, c_int64, c_int64, c_void_p, c_size_t, c_void_p],
    ),
    "vh_cross_entropy_fwd_scratch_bytes": (c_size_t, [c_int64]),
    "vh_cross_entropy_bwd": (c_int, [fp, fp, fp, fp, c_int64, c_int64, c_void_p]),
    "vh_cross_entropy_fwd_ld": (
        c_int,
        [fp, c_int64, fp, fp, c_int64, c_int64, c_void_p, c_size_t, c_void_p],
    ),
    "vh_cross_entropy_bwd_ld": (c_int, [fp, c_int64, fp, fp, fp, c_int64, c_int64, c_void_p]),
    "vh_cross_entropy_fwd_rs_ld": (
        c_int,
        [fp, c_int64, fp, fp, fp, c_int64, c_int64, c_void_p, c_size_t, c_void_p],
    ),
    "vh_cross_entropy_bwd_rs_ld": (c_int, [fp, c_int64, fp, fp, fp, fp, c_int64, c_int64, c_void_p]),
    "vh_cross_entropy_fwd_bwd_ld": (
        c_int,
        [fp, c_int64, fp, fp, fp, fp, c_int64, c_int64, c_void_p, c_size_t, c_void_p],
    ),
    "vh_binary": (c_int, [c_int, fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp, c_void_p]),
    "vh_reduce": (c_int, [c_int, fp, POINTER(VhLayout), c_int, fp, c_void_p]),
    "vh_strided_copy": (c_int, [fp, POINTER(VhLayout), fp, c_void_p]),
    "vh_sum_rows": (c_int, [fp, c_int64, c_int64, fp, c_void_p, c_size_t, c_void_p]),
    "vh_sum_rows_scratch_bytes": (c_size_t, [c_int64, c_int64]),
    "vh_gemm": (c_int, [POINTER(VhGemmDesc), c_void_p]),
    "vh_matmul": (c_int, [fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp, c_void_p]),
    "vh_fused_attention_fwd": (
        c_int,
        [fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp, POINTER(VhLayout),
         c_int, fp, POINTER(VhLayout), c_void_p, c_size_t, c_void_p],
    ),
    "vh_fused_attention_bwd": (
        c_int,
        [fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp, POINTER(VhLayout),
         c_int, fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp,
         POINTER(VhLayout), c_void_p, c_size_t, c_void_p],
    ),
    "vh_fused_attention_scratch_bytes": (c_size_t, [c_int64, c_int64, c_int64, c_int]),
    "vh_attention_mask_is_causal": (
        c_int,
        [fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp,
         POINTER(VhLayout), POINTER(c_int), c_void_p],
    ),
    "vh_fused_attention_bwd_probs": (
        c_int,
        [fp, fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp, POINTER(VhLayout), c_int, fp,
         POINTER(VhLayout), fp, POINTER(VhLayout), fp, POINTER(VhLayout), fp, POINTER(VhLayout),
         c_void_p, c_size_t, c_void_p],
    ),
    "vh_adamw_step": (
        c_int,
        [fp, fp, fp, fp, c_int64, c_int32, c_float, c_float, c_float, c_float, c_float, c_void_p],
    ),
    "vh_adamw_step_multi": (
        c_int,
        [c_int, POINTER(c_void_p), POINTER(c_void_p), POINTER(c_void_p), POINTER(c_void_p), POINTER(c_int64),
         c_int32, c_float, c_float, c_float, c_float, c_float, c_void_p],
    ),
    "vh_checkpoint_save": (c_int, [ctypes.c_char_p, c_int32, POINTER(c_void_p), POINTER(VhLayout), c_void_p]),
    "vh_checkpoint_load": (c_int, [ctypes.c_char_p, c_int32, POINTER(c_void_p), POINTER(VhLayout), c_void_p]),
}


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            " (there is no CPU fallback)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


lib = _load()


def last_error() -> str:
    return (lib.vh_last_error() or b"").decode()


def check(rc: int) -> None:
    """Raise VhError / DevicePanic for a non-zero C ABI return code."""
    if rc != VH_OK:
        msg = last_error()
        if rc == VH_ERR_DEVICE_PANIC:
            raise DevicePanic(rc, msg)
        raise VhError(rc, msg)


def layout(dims, strides=None) -> VhLayout:
    dims = [int(d) for d in dims]
    if strides is None:
        strides, acc = [0] * len(dims), 1
        for i in range(len(dims) - 1, -1, -1):
            strides[i] = acc
            acc *= dims[i]
    l = VhLayout()
    l.rank = len(dims)
    for i, (d, s) in enumerate(zip(dims, strides)):
        l.dims[i] = d
        l.strides[i] = int(s)
    return l


_initialised = False


def init(device: int = 0) -> None:
    global _initialised
    check(lib.vh_init(device))
    _initialised = True


def sync() -> None:
    check(lib.vh_sync())


class DeviceBuffer:
    """An arena allocation of `nbytes` (freed on close / garbage collection)."""

    def __init__(self, nbytes: int, zero: bool = False):
        p = c_void_p()
        check(lib.vh_alloc(int(nbytes), 1 if zero else 0, ctypes.byref(p)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            check(lib.vh_h2d(b.ptr, a.ctypes.data, a.nbytes))
        return b

    def to_array(self, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            check(lib.vh_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib.vh_h2d(self.ptr, a.ctypes.data, a.nbytes))

    def close(self) -> None:
        if self.ptr is not None:
            lib.vh_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def mem_stats() -> VhMemStats:
    s = VhMemStats()
    check(lib.vh_mem_stats_get(ctypes.byref(s)))
    return s
