"""Parity of every BASELINE config against both the CPU oracle and float64:
for each output, max-abs and max-rel of GPU - oracle, GPU - float64 and
oracle - float64, recorded through assert_parity (tests/parity.py; written as
JSON when VH_PARITY_REPORT names a file) and held to the north-star bar
|gpu - cpu| <= 1e-5 + 1e-4 |cpu| elementwise. The float64 references are the
closed forms written out in numpy here (an independent statement of each op).
Softmax runs on 2 of the 16 batches of cfg[2] (rows are independent; the
oracle and float64 on all 201M scores would take minutes); cross-entropy on
512 rows of cfg[4]'s logits; the other configs at full size."""
import numpy as np
import pytest

import oracle as O
from parity import assert_parity, dev, fetch, out

pytestmark = pytest.mark.gpu
SEED = 0x5EED0000


def ln64(x, w, b, eps):
    x = x.astype(np.float64)
    m = x.mean(1, keepdims=True)
    v = ((x - m) ** 2).mean(1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * w + b


def ln_bwd64(x, w, g, eps):
    x, g, w = x.astype(np.float64), g.astype(np.float64), w.astype(np.float64)
    C = x.shape[1]
    m = x.mean(1, keepdims=True)
    inv = 1.0 / np.sqrt(((x - m) ** 2).mean(1, keepdims=True) + eps)
    xh = (x - m) * inv
    gw = g * w
    dx = (C * gw - gw.sum(1, keepdims=True) - xh * (gw * xh).sum(1, keepdims=True)) * inv / C
    return dx, (g * xh).sum(0), g.sum(0)


@pytest.mark.parametrize("rows,C", [(2048, 128), (16384, 768)])
def test_report_layernorm(vh, rows, C):
    r = np.random.default_rng(SEED + 0)
    x = r.standard_normal((rows, C), dtype=np.float32)
    w = (1 + 0.02 * r.standard_normal(C)).astype(np.float32)
    b = (0.02 * r.standard_normal(C)).astype(np.float32)
    dy = r.standard_normal((rows, C), dtype=np.float32)
    X, W, Bb, DY = dev(vh, x), dev(vh, w), dev(vh, b), dev(vh, dy)
    Y, DX, DW, DB = out(vh, (rows, C)), out(vh, (rows, C)), out(vh, (C,)), out(vh, (C,))
    vh.check(vh.lib.vh_layernorm_fwd(X.ptr, W.ptr, Bb.ptr, Y.ptr, rows, C, 1e-5, None))
    vh.check(vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C, 1e-5, None, 0, None))
    cy = O.layernorm(x, w, b, 1e-5)
    cdx, cdw, cdb = O.layernorm_backward(x, w, b, dy, 1e-5)
    rdx, rdw, rdb = ln_bwd64(x, w, dy, 1e-5)
    tag = f"layernorm [{rows},{C}]"
    assert_parity(fetch(vh, Y, (rows, C)), cy, ln64(x, w, b, 1e-5), name=f"{tag} y")
    assert_parity(fetch(vh, DX, (rows, C)), cdx, rdx, name=f"{tag} dx")
    assert_parity(fetch(vh, DW, (C,)), cdw, rdw, name=f"{tag} dgamma")
    assert_parity(fetch(vh, DB, (C,)), cdb, rdb, name=f"{tag} dbeta")


def gelu64(x):
    x = x.astype(np.float64)
    return 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))


def gelu_grad64(x):
    x = x.astype(np.float64)
    k = np.sqrt(2 / np.pi)
    t = np.tanh(k * (x + 0.044715 * x ** 3))
    return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * k * (1 + 3 * 0.044715 * x * x)


def test_report_gelu_bias(vh):
    rows, C = 16384, 3072
    r = np.random.default_rng(SEED + 1)
    bias = (0.02 * r.standard_normal(C)).astype(np.float32)
    x = r.standard_normal((rows, C), dtype=np.float32) * np.float32(1.5)
    dy = r.standard_normal((rows, C), dtype=np.float32)
    X, Bi, DY = dev(vh, x), dev(vh, bias), dev(vh, dy)
    Y, DX, DB = out(vh, (rows, C)), out(vh, (rows, C)), out(vh, (C,))
    vh.check(vh.lib.vh_gelu_bias_fwd(X.ptr, Bi.ptr, Y.ptr, rows, C, None))
    vh.check(vh.lib.vh_gelu_bias_bwd(X.ptr, Bi.ptr, DY.ptr, DX.ptr, DB.ptr, rows, C, None, 0, None))
    cy = O.gelu_bias_forward(x, bias)
    cdx, cdb = O.gelu_bias_backward(x, bias, dy)
    xb = x.astype(np.float64) + bias
    rdx = dy * gelu_grad64(xb)
    assert_parity(fetch(vh, Y, (rows, C)), cy, gelu64(xb), name="gelu+bias [16384,3072] y")
    assert_parity(fetch(vh, DX, (rows, C)), cdx, rdx, name="gelu+bias [16384,3072] dx")
    assert_parity(fetch(vh, DB, (C,)), cdb, rdx.sum(0), name="gelu+bias [16384,3072] dbias")


def test_report_softmax_causal(vh):
    B, H, T = 2, 12, 1024
    r = np.random.default_rng(SEED + 2)
    s = r.standard_normal((B, H, T, T), dtype=np.float32) * np.float32(0.125)
    iu = np.triu_indices(T, 1)
    s[:, :, iu[0], iu[1]] = -np.inf
    g = r.standard_normal(s.shape, dtype=np.float32)
    S, G = dev(vh, s), dev(vh, g)
    P, D = out(vh, s.shape), out(vh, s.shape)
    rows = B * H * T
    vh.check(vh.lib.vh_softmax_fwd(S.ptr, P.ptr, rows, T, 1, None))
    vh.check(vh.lib.vh_softmax_bwd(S.ptr, G.ptr, D.ptr, rows, T, 1, 1, None))
    cp = O.softmax(s, 3)
    cd = O.softmax_backward_composite(s, g, 3)
    s64 = s.astype(np.float64)
    e = np.exp(s64 - s64.max(3, keepdims=True))
    p64 = e / e.sum(3, keepdims=True)
    d64 = p64 * (g - (g * p64).sum(3, keepdims=True))
    assert_parity(fetch(vh, P, s.shape), cp, p64, name="causal softmax [2,12,1024,1024] y")
    assert_parity(fetch(vh, D, s.shape), cd, d64, name="causal softmax [2,12,1024,1024] dx")


@pytest.mark.parametrize("dist", ["uniform", "zipf"])
def test_report_embedding(vh, dist):
    V, D, n = 50257, 768, 16384
    r = np.random.default_rng(SEED + 3)
    if dist == "uniform":
        ids = r.integers(0, V, size=n).astype(np.float32)
    else:
        ranks = np.arange(1, V + 1, dtype=np.float64)
        cdf = np.cumsum(ranks ** -1.1)
        ids = np.searchsorted(cdf / cdf[-1], r.random(n)).astype(np.float32)
    W = (0.02 * r.standard_normal((V, D))).astype(np.float32)
    dy = r.standard_normal((n, D), dtype=np.float32)
    I, Wd, DY = dev(vh, ids), dev(vh, W), dev(vh, dy)
    OUT, DW = out(vh, (n, D)), out(vh, (V, D))
    vh.check(vh.lib.vh_embedding_fwd(I.ptr, Wd.ptr, OUT.ptr, n, V, D, None))
    vh.check(vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, DW.ptr, n, V, D, None, 0, None))
    fwd = fetch(vh, OUT, (n, D))
    np.testing.assert_array_equal(fwd, O.embedding(ids, W))
    assert_parity(fwd, O.embedding(ids, W), W[ids.astype(np.int64)], name=f"embedding {dist} fwd (bit-exact)")
    tok = ids.astype(np.int64)
    ref64 = np.zeros((V, D))
    np.add.at(ref64, tok, dy.astype(np.float64))
    assert_parity(fetch(vh, DW, (V, D)), O.embedding_backward(ids, (V, D), dy), ref64,
                  name=f"embedding {dist} dW")


def test_report_cross_entropy(vh):
    B, V = 512, 50257
    r = np.random.default_rng(SEED + 4)
    lg = r.standard_normal((B, V), dtype=np.float32)
    tg = r.integers(0, V, size=B).astype(np.float32)
    L, T, GO = dev(vh, lg), dev(vh, tg), dev(vh, np.float32([1.0]))
    LOSS, DL = out(vh, (1,)), out(vh, (B, V))
    vh.check(vh.lib.vh_cross_entropy_fwd(L.ptr, T.ptr, LOSS.ptr, B, V, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_bwd(L.ptr, T.ptr, GO.ptr, DL.ptr, B, V, None))
    l64 = lg.astype(np.float64)
    m = l64.max(1, keepdims=True)
    lse = np.log(np.exp(l64 - m).sum(1, keepdims=True)) + m
    t = tg.astype(np.int64)
    loss64 = -(l64[np.arange(B), t] - lse[:, 0]).mean()
    p = np.exp(l64 - lse)
    p[np.arange(B), t] -= 1
    assert_parity(fetch(vh, LOSS, (1,)), np.float32([O.cross_entropy(lg, tg)]).reshape(1), np.array([loss64]),
                  name="cross-entropy [512,50257] loss")
    assert_parity(fetch(vh, DL, (B, V)), O.cross_entropy_backward(lg, tg, np.float32([1.0])), p / B,
                  name="cross-entropy [512,50257] dlogits")
