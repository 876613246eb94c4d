"""LayerNorm and softmax over rows longer than the register-held row kernels
take (kernels/rowwide.h): the reference's CPU loops have no row-length limit
(crates/vearo-backend-cpu/src/lib.rs:499-563 softmax, 665-858 layernorm), so
neither may the slots. One workgroup per row streams the row; the LayerNorm
backward runs per-row statistics, column tiles over row blocks and the fixed
order column reduce. Against the oracle (and float64 for dgamma / dbeta),
128-bit and 32-bit forms, causal and dense softmax, y given or recomputed from
x, in place, deterministic, and the allocation-free LayerNorm backward on a
wide row (the same bits as vh_layernorm_bwd)."""
import numpy as np
import pytest

import oracle as O
from parity import assert_parity, dev, fetch, out

pytestmark = pytest.mark.gpu


def rng(k):
    return np.random.default_rng(0x5EED1000 + k)


# rows, C: 16384 floats or fewer fit the register kernels; these do not (or, as
# 20000 with 128-bit units, would need 24 floats of each row per lane).
LN_CASES = [(5, 20000), (3, 40000), (7, 33331), (2, 70000), (2, 65541)]


@pytest.mark.parametrize("rows,C", LN_CASES)
def test_layernorm_wide_rows(vh, rows, C):
    print(f"layernorm wide rows={rows} C={C}", flush=True)
    r = rng(C)
    x = r.normal(size=(rows, C)).astype(np.float32)
    w = (1 + 0.02 * r.normal(size=C)).astype(np.float32)
    b = (0.02 * r.normal(size=C)).astype(np.float32)
    dy = r.normal(size=(rows, C)).astype(np.float32)
    eps = 1e-5
    X, W, B, DY = dev(vh, x), dev(vh, w), dev(vh, b), dev(vh, dy)
    Y, DX, DW, DB = out(vh, (rows, C)), out(vh, (rows, C)), out(vh, (C,)), out(vh, (C,))
    vh.check(vh.lib.vh_layernorm_fwd(X.ptr, W.ptr, B.ptr, Y.ptr, rows, C, eps, None))
    vh.check(vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C, eps, None, 0, None))
    dx_cpu, dw_cpu, db_cpu = O.layernorm_backward(x, w, b, dy, eps)
    assert_parity(fetch(vh, Y, (rows, C)), O.layernorm(x, w, b, eps), name=f"wide y C={C}")
    dx = fetch(vh, DX, (rows, C))
    assert_parity(dx, dx_cpu, name=f"wide dx C={C}")
    x64, dy64 = x.astype(np.float64), dy.astype(np.float64)
    xh = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + eps)
    dw = fetch(vh, DW, (C,))
    assert_parity(dw, dw_cpu, (dy64 * xh).sum(0), name=f"wide dgamma C={C}")
    assert_parity(fetch(vh, DB, (C,)), db_cpu, dy64.sum(0), name=f"wide dbeta C={C}")
    # Deterministic: the same bits on a second call.
    DX2, DW2 = out(vh, (rows, C)), out(vh, (C,))
    vh.check(vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX2.ptr, DW2.ptr, DB.ptr, rows, C, eps, None, 0, None))
    np.testing.assert_array_equal(fetch(vh, DX2, (rows, C)), dx)
    np.testing.assert_array_equal(fetch(vh, DW2, (C,)), dw)
    # The allocation-free entry, where its device-resident scratch holds the plan.
    if vh.lib.vh_layernorm_bwd_scratch_bytes(rows, C) <= 4 << 20:
        DX3, DW3, DB3 = out(vh, (rows, C)), out(vh, (C,)), out(vh, (C,))
        vh.check(vh.lib.vh_layernorm_bwd_noalloc(X.ptr, W.ptr, DY.ptr, DX3.ptr, DW3.ptr, DB3.ptr, rows, C, eps, None))
        np.testing.assert_array_equal(fetch(vh, DX3, (rows, C)), dx)
        np.testing.assert_array_equal(fetch(vh, DW3, (C,)), dw)


def test_layernorm_wide_rows_many(vh):
    """More rows than one row block: several partial rows per column, summed
    by the column reduce in row-block order."""
    rows, C = 300, 20480
    r = rng(7)
    x = r.normal(size=(rows, C)).astype(np.float32)
    w = (1 + 0.02 * r.normal(size=C)).astype(np.float32)
    b = np.zeros(C, np.float32)
    dy = r.normal(size=(rows, C)).astype(np.float32)
    X, W, DY = dev(vh, x), dev(vh, w), dev(vh, dy)
    DX, DW, DB = out(vh, (rows, C)), out(vh, (C,)), out(vh, (C,))
    vh.check(vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C, 1e-5, None, 0, None))
    dx_cpu, dw_cpu, db_cpu = O.layernorm_backward(x, w, b, dy, 1e-5)
    x64, dy64 = x.astype(np.float64), dy.astype(np.float64)
    xh = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5)
    assert_parity(fetch(vh, DX, (rows, C)), dx_cpu, name="wide many dx")
    assert_parity(fetch(vh, DW, (C,)), dw_cpu, (dy64 * xh).sum(0), name="wide many dgamma")
    assert_parity(fetch(vh, DB, (C,)), db_cpu, dy64.sum(0), name="wide many dbeta")


# rows, T, causal: the forward holds rows of up to 65536 floats in registers,
# the backward 32768; causal rows r keep the columns [0, r % T].
SM_CASES = [(3, 70000, 0), (2, 65537, 0), (4, 40000, 0), (3, 33333, 0), (5, 40000, 1), (2, 70001, 1)]


@pytest.mark.parametrize("rows,T,causal", SM_CASES)
def test_softmax_wide_rows(vh, rows, T, causal):
    print(f"softmax wide rows={rows} T={T} causal={causal}", flush=True)
    r = rng(T + causal)
    x = (r.normal(size=(rows, T)) * 3).astype(np.float32)
    dy = r.normal(size=(rows, T)).astype(np.float32)
    xm = x.copy()
    if causal:
        for i in range(rows):
            xm[i, i % T + 1:] = -np.inf
    X, DY, Y, DX, DX2 = dev(vh, x), dev(vh, dy), out(vh, x.shape), out(vh, x.shape), out(vh, x.shape)
    vh.check(vh.lib.vh_softmax_fwd(X.ptr, Y.ptr, rows, T, causal, None))
    vh.check(vh.lib.vh_softmax_bwd(Y.ptr, DY.ptr, DX.ptr, rows, T, 0, causal, None))
    vh.check(vh.lib.vh_softmax_bwd(X.ptr, DY.ptr, DX2.ptr, rows, T, 1, causal, None))
    y = fetch(vh, Y, x.shape)
    assert_parity(y, O.softmax(xm, 1), name=f"wide y T={T}")
    if causal:
        for i in range(rows):
            assert np.all(y[i, i % T + 1:] == 0.0)
    dx_cpu = O.softmax_backward_composite(xm, dy, 1)
    if causal:  # the composite gives 0 * (dy - s) = 0 (or -0) on masked columns
        dx_cpu = np.where(np.isfinite(xm), dx_cpu, 0.0).astype(np.float32)
    dx = fetch(vh, DX, x.shape)
    assert_parity(dx, dx_cpu, name=f"wide dx(from y) T={T}")
    assert_parity(fetch(vh, DX2, x.shape), dx_cpu, name=f"wide dx(from x) T={T}")
    # In place: dx written over dy.
    vh.check(vh.lib.vh_softmax_bwd(Y.ptr, DY.ptr, DY.ptr, rows, T, 0, causal, None))
    np.testing.assert_array_equal(fetch(vh, DY, x.shape), dx)
