"""Arena scratch across streams: entries given scratch = NULL on two caller
streams, back to back, each taking blocks the other just freed (the arena
makes the new stream wait for the old one's event), give the same bits as on
the runtime stream."""
import ctypes

import numpy as np
import pytest

from parity import dev, fetch, out

pytestmark = pytest.mark.gpu


class Streams:
    def __init__(self, n):
        self.h = ctypes.CDLL("libamdhip64.so.7")
        self.h.hipStreamCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.h.hipStreamDestroy.argtypes = [ctypes.c_void_p]
        self.h.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
        self.s = []
        for _ in range(n):
            p = ctypes.c_void_p()
            assert self.h.hipStreamCreateWithFlags(ctypes.byref(p), 1) == 0  # non-blocking, default priority
            self.s.append(p)

    def sync(self):
        for p in self.s:
            assert self.h.hipStreamSynchronize(p) == 0

    def close(self):
        self.sync()
        for p in self.s:
            assert self.h.hipStreamDestroy(p) == 0


def test_layernorm_bwd_arena_scratch_on_two_streams(vh):
    rows, C = 4096, 768
    r = np.random.default_rng(21)
    w = (1 + 0.02 * r.standard_normal(C)).astype(np.float32)
    W = dev(vh, w)
    sets = []
    for _ in range(4):
        x = r.standard_normal((rows, C), dtype=np.float32)
        dy = r.standard_normal((rows, C), dtype=np.float32)
        sets.append((dev(vh, x), dev(vh, dy)))
    ref = []
    for X, DY in sets:  # runtime stream
        DX, DW, DB = out(vh, (rows, C)), out(vh, (C,)), out(vh, (C,))
        vh.check(vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C, 1e-5, None, 0, None))
        ref.append((fetch(vh, DX, (rows, C)), fetch(vh, DW, (C,)), fetch(vh, DB, (C,))))
    st = Streams(2)
    try:
        outs = []
        for rep in range(3):
            for i, (X, DY) in enumerate(sets):
                DX, DW, DB = out(vh, (rows, C)), out(vh, (C,)), out(vh, (C,))
                vh.check(vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C, 1e-5,
                                                 None, 0, st.s[i % 2]))
                outs.append((i, DX, DW, DB))
        st.sync()
        for i, DX, DW, DB in outs:
            np.testing.assert_array_equal(fetch(vh, DX, (rows, C)), ref[i][0])
            np.testing.assert_array_equal(fetch(vh, DW, (C,)), ref[i][1])
            np.testing.assert_array_equal(fetch(vh, DB, (C,)), ref[i][2])
    finally:
        st.close()
