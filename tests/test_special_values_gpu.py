"""Special values through the hot-path kernels, against the oracle's
restatement of the reference's CPU loops: infinities, NaN, signed zeros,
f32 extremes, a fully masked (all -inf) softmax row, constant LayerNorm rows,
-inf logits. Non-finite results must sit where the oracle's are (NaN for NaN,
infinities with their sign), finite ones within the usual tolerance."""
import numpy as np
import pytest

import oracle as O
from parity import assert_parity, dev, fetch, ln64, out, softmax64

pytestmark = pytest.mark.gpu

SPECIAL = np.float32([0.0, -0.0, 1e-30, -1e-30, 1.0, -1.0, 5.0, -5.0, 10.0, -10.0, 20.0, -20.0, 1e10, -1e10,
                      3.4e38, -3.4e38, np.inf, -np.inf, np.nan, 1.4e-45])


def same(gpu, cpu, name, ref64=None):
    """NaN where the oracle has NaN, its infinities with their signs, and the
    finite elements to the usual bar (with the float64 fallback of
    assert_parity where a long f32 sum makes the oracle itself drift)."""
    gpu = np.asarray(gpu, np.float64)
    cpu = np.asarray(cpu, np.float64)
    assert gpu.shape == cpu.shape
    nan = np.isnan(cpu)
    assert np.array_equal(np.isnan(gpu), nan), f"{name}: NaN at {np.argwhere(np.isnan(gpu) != nan)[:5].tolist()}"
    inf = np.isinf(cpu)
    assert np.array_equal(gpu[inf], cpu[inf]) and not np.isinf(gpu[~inf]).any(), f"{name}: infinity mismatch"
    fin = np.isfinite(cpu)
    assert_parity(gpu[fin], cpu[fin], None if ref64 is None else np.asarray(ref64, np.float64)[fin], name=name)


def test_gelu_special_values(vh):
    x = np.tile(SPECIAL, 7)  # 140 elements: the vector and scalar tails of the kernels
    X, Y = dev(vh, x), out(vh, x.shape)
    vh.check(vh.lib.vh_gelu_fwd(X.ptr, Y.ptr, x.size, None))
    same(fetch(vh, Y, x.shape), O.gelu(x), "gelu")
    dy = np.ones_like(x)
    DY, DX = dev(vh, dy), out(vh, x.shape)
    vh.check(vh.lib.vh_gelu_grad_mul(X.ptr, DY.ptr, DX.ptr, x.size, None))
    same(fetch(vh, DX, x.shape), O.gelu_grad_mask(x) * dy, "gelu mask")
    rows, C = 7, SPECIAL.size
    b = np.linspace(-1, 1, C).astype(np.float32)
    Bb, Y2 = dev(vh, b), out(vh, (rows, C))
    vh.check(vh.lib.vh_gelu_bias_fwd(X.ptr, Bb.ptr, Y2.ptr, rows, C, None))
    same(fetch(vh, Y2, (rows, C)), O.gelu_bias_forward(x.reshape(rows, C), b), "gelu(x + b)")
    dy2 = np.linspace(-2, 2, x.size).astype(np.float32)
    DY2, DX2, DB2 = dev(vh, dy2), out(vh, (rows, C)), out(vh, (C,))
    vh.check(vh.lib.vh_gelu_bias_bwd(X.ptr, Bb.ptr, DY2.ptr, DX2.ptr, DB2.ptr, rows, C, None, 0, None))
    dx_cpu, db_cpu = O.gelu_bias_backward(x.reshape(rows, C), b, dy2.reshape(rows, C))
    same(fetch(vh, DX2, (rows, C)), dx_cpu, "gelu(x + b) dx")
    same(fetch(vh, DB2, (C,)), db_cpu, "gelu(x + b) dbias")


@pytest.mark.parametrize("C", [20, 768, 70000, 70002])
def test_layernorm_special_rows(vh, C):
    r = np.random.default_rng(5)
    x = r.normal(size=(6, C)).astype(np.float32)
    x[0] = 3.0                      # constant row: variance 0, x - mean = 0
    x[1] = -0.0
    x[2, 3] = np.inf                # an infinity: mean inf, x - mean NaN
    x[3, 5] = np.nan
    x[4, :] = 2.0 ** 60             # large constant row (exact sums: the mean is the value itself)
    x[5, ::2] = 1e-38               # tiny values
    w = r.normal(size=C).astype(np.float32)
    b = r.normal(size=C).astype(np.float32)
    dy = r.normal(size=(6, C)).astype(np.float32)
    X, W, B, Y = dev(vh, x), dev(vh, w), dev(vh, b), out(vh, x.shape)
    vh.check(vh.lib.vh_layernorm_fwd(X.ptr, W.ptr, B.ptr, Y.ptr, 6, C, 1e-5, None))
    y64, dx64 = ln64(x, w, b, 1e-5, dy)
    same(fetch(vh, Y, x.shape), O.layernorm(x, w, b, 1e-5), f"layernorm C={C}", y64)
    DY, DX, DW, DB = dev(vh, dy), out(vh, x.shape), out(vh, (C,)), out(vh, (C,))
    vh.check(vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, 6, C, 1e-5, None, 0, None))
    dx, dw, db = O.layernorm_backward(x, w, b, dy, 1e-5)
    same(fetch(vh, DX, x.shape), dx, "layernorm dx", dx64)
    same(fetch(vh, DW, (C,)), dw, "layernorm dgamma")
    same(fetch(vh, DB, (C,)), db, "layernorm dbeta")


@pytest.mark.parametrize("T", [8, 1024, 70000, 70002])
def test_softmax_special_rows(vh, T):
    r = np.random.default_rng(6)
    x = r.normal(size=(6, T)).astype(np.float32)
    x[0] = -np.inf                  # fully masked row
    x[1, 2] = np.inf                # a +inf entry
    x[2, 1] = np.nan
    x[3] = 0.0                      # uniform row
    x[4, ::2] = -np.inf             # half masked
    x[5, 0] = 80.0                  # one dominant entry (exp of the others underflows)
    x[5, 1:] = -80.0
    dy = r.normal(size=(6, T)).astype(np.float32)
    X, DY, Y, DX = dev(vh, x), dev(vh, dy), out(vh, x.shape), out(vh, x.shape)
    vh.check(vh.lib.vh_softmax_fwd(X.ptr, Y.ptr, 6, T, 0, None))
    y64, dx64 = softmax64(x, dy)
    same(fetch(vh, Y, x.shape), O.softmax(x, 1), f"softmax T={T}", y64)
    vh.check(vh.lib.vh_softmax_bwd(X.ptr, DY.ptr, DX.ptr, 6, T, 1, 0, None))
    same(fetch(vh, DX, x.shape), O.softmax_backward_composite(x, dy, 1), f"softmax bwd T={T}", dx64)


@pytest.mark.parametrize("V", [1000, 50257])
def test_cross_entropy_special_logits(vh, V):
    r = np.random.default_rng(7)
    B = 5
    logits = r.normal(size=(B, V)).astype(np.float32)
    logits[0, 10:] = -np.inf        # masked classes, target among the finite ones
    logits[1, :] = 0.0              # uniform: loss ln V
    logits[2, 3] = 1e30             # one huge logit
    logits[3, 0] = -1000.0          # the target far below the rest
    tg = np.float32([5, 17, 3, 0, V - 1])
    go = np.float32([1.0])
    L, T, GO = dev(vh, logits), dev(vh, tg), dev(vh, go)
    LOSS, DL = out(vh, (1,)), out(vh, (B, V))
    vh.check(vh.lib.vh_cross_entropy_fwd(L.ptr, T.ptr, LOSS.ptr, B, V, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_bwd(L.ptr, T.ptr, GO.ptr, DL.ptr, B, V, None))
    same(fetch(vh, LOSS, (1,)), O.cross_entropy(logits, tg), "loss")
    same(fetch(vh, DL, (B, V)), O.cross_entropy_backward(logits, tg, go), "dlogits")
