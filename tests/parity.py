"""Shared helpers for the GPU parity tests: run a C-ABI entry point on numpy
inputs and compare with the CPU oracle under the north-star criterion
|gpu - cpu| <= 1e-5 + 1e-4 * |cpu| (elementwise, as numpy.allclose)."""
import ctypes

import numpy as np

ATOL = 1e-5
RTOL = 1e-4


def dev(vh, a):
    return vh.DeviceBuffer.from_array(np.ascontiguousarray(a, dtype=np.float32))


def out(vh, shape):
    n = int(np.prod(shape)) if len(shape) else 1
    return vh.DeviceBuffer(max(4, 4 * n))


def fetch(vh, buf, shape):
    vh.sync()
    return buf.to_array(shape)


# Every assert_parity call appends its statistics here; tests/conftest.py
# writes the list as JSON at the end of the session when VH_PARITY_REPORT
# names a file.
REPORT = []


def _errs(a, b):
    d = np.abs(a - b)
    fin = np.isfinite(d)
    d = d[fin]
    if d.size == 0:
        return 0.0, 0.0
    return float(d.max()), float((d / np.maximum(np.abs(b[fin]), 1e-30)).max())


def assert_parity(gpu, cpu, ref64=None, name=""):
    """Elementwise allclose(gpu, cpu, rtol=1e-4, atol=1e-5). Where a long f32
    sum makes the CPU oracle itself drift further than that from the exact
    (float64) value, the GPU passes an element if it is no further from the
    float64 value than the oracle is (plus the same tolerance); the number of
    elements that pass only that way is counted ("fallback") and reported.
    Returns (and records in REPORT) max-abs / max-rel of GPU - oracle and, with
    ref64, of both sides against float64."""
    gpu = np.asarray(gpu, np.float64)
    cpu = np.asarray(cpu, np.float64)
    assert gpu.shape == cpu.shape, (name, gpu.shape, cpu.shape)
    assert np.all(np.isfinite(gpu) == np.isfinite(cpu)), f"{name}: non-finite mismatch"
    fin = np.isfinite(cpu)
    ok = np.abs(gpu - cpu) <= ATOL + RTOL * np.abs(cpu)
    ok |= ~fin & (gpu == cpu)
    strict_fail = int((~ok).sum())
    stats = {"name": name, "n": int(ok.size)}
    stats["gpu_vs_cpu_max_abs"], stats["gpu_vs_cpu_max_rel"] = _errs(gpu, cpu)
    if ref64 is not None:
        ref64 = np.asarray(ref64, np.float64)
        stats["gpu_vs_f64_max_abs"], stats["gpu_vs_f64_max_rel"] = _errs(gpu, ref64)
        stats["cpu_vs_f64_max_abs"], stats["cpu_vs_f64_max_rel"] = _errs(cpu, ref64)
        if not ok.all():
            ok |= np.abs(gpu - ref64) <= np.abs(cpu - ref64) + ATOL + RTOL * np.abs(ref64)
    stats["fallback"] = strict_fail - int((~ok).sum())
    REPORT.append(stats)
    if stats["fallback"]:
        print(f"{name}: {stats['fallback']} of {ok.size} elements pass only through the float64 fallback",
              flush=True)
    if not ok.all():
        bad = np.argwhere(~ok)[:5]
        detail = [(tuple(i), gpu[tuple(i)], cpu[tuple(i)]) for i in bad]
        raise AssertionError(f"{name}: {int((~ok).sum())} of {ok.size} elements out of tolerance; "
                             f"first: {detail}")
    return stats


def max_errs(gpu, cpu):
    gpu = np.asarray(gpu, np.float64)
    cpu = np.asarray(cpu, np.float64)
    d = np.abs(gpu - cpu)
    return float(d.max(initial=0.0)), float((d / np.maximum(np.abs(cpu), 1e-30)).max(initial=0.0))


def ptr(buf):
    return ctypes.c_void_p(buf.ptr)


# Float64 statements of the row ops, for the fallback of assert_parity where a
# long f32 sum makes the oracle drift (non-finite inputs give NaN rows).
def ln64(x, w, b, eps, dy):
    x = x.astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        m = x.mean(1, keepdims=True)
        rstd = 1.0 / np.sqrt(((x - m) ** 2).mean(1, keepdims=True) + eps)
        xh = (x - m) * rstd
        g = dy * w
        dx = rstd * (g - g.mean(1, keepdims=True) - xh * (g * xh).mean(1, keepdims=True))
    return xh * w + b, dx


def softmax64(x, dy):
    x = x.astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.exp(x - x.max(1, keepdims=True))
        y = e / e.sum(1, keepdims=True)
        return y, y * (dy - (dy * y).sum(1, keepdims=True))
