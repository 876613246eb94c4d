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


def assert_parity(gpu, cpu, ref64=None, name=""):
    """Elementwise allclose(gpu, cpu, rtol=1e-4, atol=1e-5). Where a long f32
    sum makes the CPU oracle itself drift further than that from the exact
    (float64) value, the GPU passes an element if it is no further from the
    float64 value than the oracle is (plus the same tolerance)."""
    gpu = np.asarray(gpu, np.float64)
    cpu = np.asarray(cpu, np.float64)
    assert gpu.shape == cpu.shape, (name, gpu.shape, cpu.shape)
    assert np.all(np.isfinite(gpu) == np.isfinite(cpu)), f"{name}: non-finite mismatch"
    fin = np.isfinite(cpu)
    ok = np.abs(gpu - cpu) <= ATOL + RTOL * np.abs(cpu)
    ok |= ~fin & (gpu == cpu)
    if ref64 is not None and not ok.all():
        ref64 = np.asarray(ref64, np.float64)
        ok |= np.abs(gpu - ref64) <= np.abs(cpu - ref64) + ATOL + RTOL * np.abs(ref64)
    if not ok.all():
        bad = np.argwhere(~ok)[:5]
        detail = [(tuple(i), gpu[tuple(i)], cpu[tuple(i)]) for i in bad]
        raise AssertionError(f"{name}: {int((~ok).sum())} of {ok.size} elements out of tolerance; "
                             f"first: {detail}")


def max_errs(gpu, cpu):
    gpu = np.asarray(gpu, np.float64)
    cpu = np.asarray(cpu, np.float64)
    d = np.abs(gpu - cpu)
    return float(d.max(initial=0.0)), float((d / np.maximum(np.abs(cpu), 1e-30)).max(initial=0.0))


def ptr(buf):
    return ctypes.c_void_p(buf.ptr)
