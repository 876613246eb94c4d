"""Routing sweep of the row kernels against the oracle.

For a row width the library picks a team (16, 32 or 64 lanes, or a 1024-thread
workgroup), units per lane, 128-bit or 32-bit units (by the width and the
16-byte alignment of every pointer) and, past 65536 floats, a streaming form.
Every width on a boundary of those choices runs here twice: with all buffers
16-byte aligned, and with every buffer one float past that (which forces the
32-bit forms). LayerNorm fwd/bwd, dense softmax fwd/bwd, GELU(+bias) fwd/bwd,
GELU and its gradient, and cross-entropy fwd/bwd, each against the oracle (with
the float64 fallback of assert_parity where long f32 sums make the oracle
drift). Each output has guard words on both sides that must come back
untouched. The causal softmax runs over whole T x T squares for the widths it
serves (T <= 1025), and the embedding gather and scatter-add over row widths
D of every class."""
import numpy as np
import pytest

import oracle as O
from parity import assert_parity, ln64, softmax64

pytestmark = pytest.mark.gpu

WIDTHS = [1, 2, 3, 4, 5, 7, 8, 12, 15, 16, 17, 20, 31, 32, 33, 36, 63, 64, 65, 68, 127, 128, 129, 132,
          255, 256, 257, 260, 511, 512, 513, 516, 767, 768, 1023, 1024, 1025, 1028, 2047, 2048, 2049, 2052,
          4095, 4096, 4097, 4100, 8192, 8195, 16384, 16388, 32768, 32769, 65536, 65537, 65540, 70000, 100003]
GUARD = 4
SENTINEL = np.float32(-12345.5)


class Buf:
    """A device copy of `a` starting `off` floats past a 16-byte boundary, with
    GUARD sentinel floats after it (and the `off` floats before it)."""

    def __init__(self, vh, a, off):
        a = np.ascontiguousarray(a, np.float32).reshape(-1)
        self.vh, self.off, self.n = vh, off, a.size
        full = np.concatenate([np.full(off, SENTINEL, np.float32), a, np.full(GUARD, SENTINEL, np.float32)])
        self.buf = vh.DeviceBuffer.from_array(full)
        self.ptr = self.buf.ptr + 4 * off

    def get(self, shape):
        self.vh.sync()
        full = self.buf.to_array((self.off + self.n + GUARD,))
        assert np.all(full[:self.off] == SENTINEL) and np.all(full[self.off + self.n:] == SENTINEL), \
            "a kernel wrote outside its output"
        return full[self.off:self.off + self.n].reshape(shape)


def outbuf(vh, shape, off):
    return Buf(vh, np.zeros(int(np.prod(shape)), np.float32), off)


def rows_for(C):
    return 5 if C <= 8192 else 2


@pytest.mark.parametrize("off", [0, 1])
@pytest.mark.parametrize("C", WIDTHS)
def test_row_kernels_sweep(vh, C, off):
    print(f"sweep C={C} off={off}", flush=True)
    R = rows_for(C)
    r = np.random.default_rng(1000 * C + off)
    eps = 1e-5

    # LayerNorm
    x = r.normal(size=(R, C)).astype(np.float32)
    w = (1 + 0.1 * r.normal(size=C)).astype(np.float32)
    b = (0.1 * r.normal(size=C)).astype(np.float32)
    dy = r.normal(size=(R, C)).astype(np.float32)
    X, W, B, DY = Buf(vh, x, off), Buf(vh, w, off), Buf(vh, b, off), Buf(vh, dy, off)
    Y, DX, DW, DB = outbuf(vh, (R, C), off), outbuf(vh, (R, C), off), outbuf(vh, (C,), off), outbuf(vh, (C,), off)
    vh.check(vh.lib.vh_layernorm_fwd(X.ptr, W.ptr, B.ptr, Y.ptr, R, C, eps, None))
    vh.check(vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, R, C, eps, None, 0, None))
    y64, dx64 = ln64(x, w, b, eps, dy)
    dx_cpu, dw_cpu, db_cpu = O.layernorm_backward(x, w, b, dy, eps)
    assert_parity(Y.get((R, C)), O.layernorm(x, w, b, eps), y64, name=f"ln y C={C} off={off}")
    assert_parity(DX.get((R, C)), dx_cpu, dx64, name=f"ln dx C={C} off={off}")
    x64 = x.astype(np.float64)
    xh = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + eps)
    assert_parity(DW.get((C,)), dw_cpu, (dy * xh).sum(0), name=f"ln dgamma C={C} off={off}")
    assert_parity(DB.get((C,)), db_cpu, dy.astype(np.float64).sum(0), name=f"ln dbeta C={C} off={off}")

    # Dense softmax (rows of width C), backward from x and from y
    s = (3 * r.normal(size=(R, C))).astype(np.float32)
    S, DS = Buf(vh, s, off), Buf(vh, dy, off)
    P, DP, DP2 = outbuf(vh, (R, C), off), outbuf(vh, (R, C), off), outbuf(vh, (R, C), off)
    vh.check(vh.lib.vh_softmax_fwd(S.ptr, P.ptr, R, C, 0, None))
    vh.check(vh.lib.vh_softmax_bwd(S.ptr, DS.ptr, DP.ptr, R, C, 1, 0, None))
    vh.check(vh.lib.vh_softmax_bwd(P.ptr, DS.ptr, DP2.ptr, R, C, 0, 0, None))
    p64, dp64 = softmax64(s, dy)
    dp_cpu = O.softmax_backward_composite(s, dy, 1)
    assert_parity(P.get((R, C)), O.softmax(s, 1), p64, name=f"softmax y C={C} off={off}")
    assert_parity(DP.get((R, C)), dp_cpu, dp64, name=f"softmax dx(from x) C={C} off={off}")
    assert_parity(DP2.get((R, C)), dp_cpu, dp64, name=f"softmax dx(from y) C={C} off={off}")

    # GELU(x + b) forward and backward (dbias over the rows), GELU and its mask
    g = (2 * r.normal(size=(R, C))).astype(np.float32)
    G = Buf(vh, g, off)
    GY, GDX, GDB = outbuf(vh, (R, C), off), outbuf(vh, (R, C), off), outbuf(vh, (C,), off)
    vh.check(vh.lib.vh_gelu_bias_fwd(G.ptr, B.ptr, GY.ptr, R, C, None))
    vh.check(vh.lib.vh_gelu_bias_bwd(G.ptr, B.ptr, DY.ptr, GDX.ptr, GDB.ptr, R, C, None, 0, None))
    gdx_cpu, gdb_cpu = O.gelu_bias_backward(g, b, dy)
    assert_parity(GY.get((R, C)), O.gelu_bias_forward(g, b), name=f"gelu(x+b) C={C} off={off}")
    assert_parity(GDX.get((R, C)), gdx_cpu, name=f"gelu(x+b) dx C={C} off={off}")
    assert_parity(GDB.get((C,)), gdb_cpu, name=f"gelu(x+b) dbias C={C} off={off}")
    E, EM = outbuf(vh, (R, C), off), outbuf(vh, (R, C), off)
    vh.check(vh.lib.vh_gelu_fwd(G.ptr, E.ptr, R * C, None))
    vh.check(vh.lib.vh_gelu_grad_mul(G.ptr, DY.ptr, EM.ptr, R * C, None))
    assert_parity(E.get((R, C)), O.gelu(g), name=f"gelu C={C} off={off}")
    assert_parity(EM.get((R, C)), O.gelu_grad_mask(g) * dy, name=f"gelu mask C={C} off={off}")

    # Cross-entropy over a vocabulary of C classes
    logits = (2 * r.normal(size=(R, C))).astype(np.float32)
    tg = r.integers(0, C, size=R).astype(np.float32)
    go = np.float32([0.7])
    L, TG, GO = Buf(vh, logits, off), Buf(vh, tg, off), Buf(vh, go, off)
    LOSS, DL = outbuf(vh, (1,), off), outbuf(vh, (R, C), off)
    vh.check(vh.lib.vh_cross_entropy_fwd(L.ptr, TG.ptr, LOSS.ptr, R, C, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_bwd(L.ptr, TG.ptr, GO.ptr, DL.ptr, R, C, None))
    l64 = logits.astype(np.float64)
    m = l64.max(1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(l64 - m).sum(1))
    t = tg.astype(np.int64)
    loss64 = np.float64((lse - l64[np.arange(R), t]).mean())
    sm64 = np.exp(l64 - m) / np.exp(l64 - m).sum(1, keepdims=True)
    oh = np.zeros_like(sm64)
    oh[np.arange(R), t] = 1
    assert_parity(LOSS.get((1,)), O.cross_entropy(logits, tg), np.float64([loss64]), name=f"ce loss C={C} off={off}")
    assert_parity(DL.get((R, C)), O.cross_entropy_backward(logits, tg, go), 0.7 * (sm64 - oh) / R,
                  name=f"ce dlogits C={C} off={off}")


@pytest.mark.parametrize("off", [0, 1])
@pytest.mark.parametrize("T", [w for w in WIDTHS if w <= 1025])
def test_causal_softmax_sweep(vh, T, off):
    """Whole T x T causal squares: row r reads its live prefix [0, r] and
    writes exact zeros past it."""
    print(f"causal sweep T={T} off={off}", flush=True)
    r = np.random.default_rng(2000 * T + off)
    x = (2 * r.normal(size=(T, T))).astype(np.float32)
    iu = np.triu_indices(T, 1)
    x[iu] = -np.inf
    dy = r.normal(size=(T, T)).astype(np.float32)
    X, DY = Buf(vh, x, off), Buf(vh, dy, off)
    Y, DX, DX2 = outbuf(vh, (T, T), off), outbuf(vh, (T, T), off), outbuf(vh, (T, T), off)
    vh.check(vh.lib.vh_softmax_fwd(X.ptr, Y.ptr, T, T, 1, None))
    vh.check(vh.lib.vh_softmax_bwd(X.ptr, DY.ptr, DX.ptr, T, T, 1, 1, None))
    vh.check(vh.lib.vh_softmax_bwd(Y.ptr, DY.ptr, DX2.ptr, T, T, 0, 1, None))
    y = Y.get((T, T))
    assert np.all(y[iu] == 0.0)
    assert_parity(y, O.softmax(x, 1), name=f"causal y T={T} off={off}")
    dx_cpu = O.softmax_backward_composite(x, dy, 1)
    dx = DX.get((T, T))
    assert np.all(dx[iu] == 0.0)
    assert_parity(dx, dx_cpu, name=f"causal dx(from x) T={T} off={off}")
    assert_parity(DX2.get((T, T)), dx_cpu, name=f"causal dx(from y) T={T} off={off}")


@pytest.mark.parametrize("off", [0, 1])
@pytest.mark.parametrize("D", [1, 3, 4, 5, 63, 64, 65, 68, 767, 768, 1023, 1024, 4097, 20000])
def test_embedding_sweep(vh, D, off):
    """Embedding rows of every width class, 128-bit and 32-bit forms: the
    forward's copy bit for bit, the backward's rows of tokens with at most 16
    hits bit for bit (the CPU loop's order) and the heavier ones (a token
    with 40 hits here) within tolerance; dW's untouched rows exactly 0."""
    from test_parity_gpu import check_embedding_grad
    print(f"embedding sweep D={D} off={off}", flush=True)
    r = np.random.default_rng(3000 * D + off)
    V, n = 300, 200
    ids = r.integers(0, V, size=n).astype(np.float32)
    ids[::5] = 7.0                                  # one heavy token (40 hits)
    W = r.normal(size=(V, D)).astype(np.float32)
    dy = r.normal(size=(n, D)).astype(np.float32)
    I, Wd, DY = Buf(vh, ids, off), Buf(vh, W, off), Buf(vh, dy, off)
    OUT, DW = outbuf(vh, (n, D), off), outbuf(vh, (V, D), off)
    vh.check(vh.lib.vh_embedding_fwd(I.ptr, Wd.ptr, OUT.ptr, n, V, D, None))
    vh.check(vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, DW.ptr, n, V, D, None, 0, None))
    np.testing.assert_array_equal(OUT.get((n, D)), O.embedding(ids, W))
    check_embedding_grad(DW.get((V, D)), ids, dy, V)
