"""vh_layernorm_bwd_noalloc: the LayerNorm backward with its partials in the
device-resident scratch, called through the C ABI and checked bit for bit
against vh_layernorm_bwd (same kernels) on two calls in a row, the second on a
smaller input, plus the oracle on the small one and the size limit."""
import numpy as np
import pytest

import oracle as O
from parity import assert_parity, dev, fetch, out

pytestmark = pytest.mark.gpu


def _inputs(tag, rows, C):
    r = np.random.default_rng(0x5EED0000 + tag)
    x = r.standard_normal((rows, C), dtype=np.float32)
    w = (1 + 0.02 * r.standard_normal(C)).astype(np.float32)
    dy = r.standard_normal((rows, C), dtype=np.float32)
    return x, w, dy


def _run(vh, fn, X, W, DY, rows, C):
    DX, DW, DB = out(vh, (rows, C)), out(vh, (C,)), out(vh, (C,))
    if fn == "noalloc":
        # No arena (or any vh_alloc) traffic inside the call.
        vh.sync()
        before = vh.mem_stats()
        rc = vh.lib.vh_layernorm_bwd_noalloc(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C, 1e-5, None)
        after = vh.mem_stats()
        assert (after.hip_bytes, after.live_bytes, after.cached_bytes) == \
            (before.hip_bytes, before.live_bytes, before.cached_bytes)
    else:
        need = vh.lib.vh_layernorm_bwd_scratch_bytes(rows, C)
        S = vh.DeviceBuffer(need)
        rc = vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C, 1e-5, S.ptr, need,
                                     None)
    vh.check(rc)
    return fetch(vh, DX, (rows, C)), fetch(vh, DW, (C,)), fetch(vh, DB, (C,))


def test_noalloc_matches_scratch_entry_two_calls(vh):
    # A large call then a smaller one: the second finds the first's partials in
    # the shared scratch and must not depend on them.
    for tag, (rows, C) in ((11, (16384, 768)), (12, (300, 96))):
        x, w, dy = _inputs(tag, rows, C)
        X, W, DY = dev(vh, x), dev(vh, w), dev(vh, dy)
        got = _run(vh, "noalloc", X, W, DY, rows, C)
        ref = _run(vh, "scratch", X, W, DY, rows, C)
        for g, r_, name in zip(got, ref, ("dx", "dgamma", "dbeta")):
            np.testing.assert_array_equal(g, r_, err_msg=f"{name} at [{rows},{C}]")
        if rows <= 300:
            cdx, cdw, cdb = O.layernorm_backward(x, w, np.zeros(C, np.float32), dy, 1e-5)
            assert_parity(got[0], cdx, name="dx")
            assert_parity(got[1], cdw, name="dgamma")
            assert_parity(got[2], cdb, name="dbeta")


def test_noalloc_scalar_units_and_zero_rows(vh):
    # Operands off 16-byte alignment take the one-float-unit kernels.
    rows, C = 257, 130
    x, w, dy = _inputs(13, rows, C)
    pad = lambda a: dev(vh, np.concatenate([np.zeros(1, np.float32), a.ravel()]))
    X, W, DY = pad(x), pad(w), pad(dy)
    DX, DW, DB = out(vh, (rows * C + 1,)), out(vh, (C + 1,)), out(vh, (C + 1,))
    vh.check(vh.lib.vh_layernorm_bwd_noalloc(X.ptr + 4, W.ptr + 4, DY.ptr + 4, DX.ptr + 4, DW.ptr + 4, DB.ptr + 4,
                                             rows, C, 1e-5, None))
    dx = fetch(vh, DX, (rows * C + 1,))[1:].reshape(rows, C)
    dw = fetch(vh, DW, (C + 1,))[1:]
    cdx, cdw, _ = O.layernorm_backward(x, w, np.zeros(C, np.float32), dy, 1e-5)
    assert_parity(dx, cdx, name="dx")
    assert_parity(dw, cdw, name="dgamma")
    # rows == 0: zero gradients, as the reference returns.
    DW2, DB2 = dev(vh, np.ones(C, np.float32)), dev(vh, np.ones(C, np.float32))
    vh.check(vh.lib.vh_layernorm_bwd_noalloc(X.ptr, W.ptr, DY.ptr, DX.ptr, DW2.ptr, DB2.ptr, 0, C, 1e-5, None))
    assert not fetch(vh, DW2, (C,)).any() and not fetch(vh, DB2, (C,)).any()


def test_noalloc_rejects_scratch_beyond_limit(vh):
    # [4096, 2048] runs 256-thread workgroups (1024 of them): 16 MiB of
    # partials, past the 4 MiB device-resident scratch. Real buffers of the
    # claimed size, so a wrongly accepted call would still stay in bounds.
    rows, C = 4096, 2048
    assert vh.lib.vh_layernorm_bwd_scratch_bytes(rows, C) > 4 << 20
    X, DY, DX = out(vh, (rows, C)), out(vh, (rows, C)), out(vh, (rows, C))
    W, DW, DB = out(vh, (C,)), out(vh, (C,)), out(vh, (C,))
    rc = vh.lib.vh_layernorm_bwd_noalloc(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C, 1e-5, None)
    assert rc == vh.VH_ERR_UNSUPPORTED
    assert "device-resident scratch" in vh.last_error()
    rc = vh.lib.vh_layernorm_bwd_noalloc(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, -1, C, 1e-5, None)
    assert rc == vh.VH_ERR_INVALID
