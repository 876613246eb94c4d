"""Full-size checks at BASELINE.json's largest single-GPU shapes:
size-independent properties and oracle parity on every row (the oracle runs
head by head / in row blocks, seconds of CPU each test).

* cfg[2] causal softmax [16, 12, 1024, 1024]: rows sum to 1, masked entries are
  exactly 0, backward rows sum to 0, every head matches the oracle (fwd and
  the 5-op backward composite).
* cfg[4] cross-entropy over [16384, 50257]: the loss matches the oracle's and
  a float64 log-sum-exp of all rows, gradient rows sum to 0 and the target
  entry is the only negative one, every row matches the oracle.
"""
import numpy as np
import pytest

import oracle as O
from parity import assert_parity, dev, fetch, out

pytestmark = pytest.mark.gpu


def test_softmax_cfg2_full(vh):
    B, H, T = 16, 12, 1024
    print("softmax cfg2 full", flush=True)
    r = np.random.default_rng(0x5EED0000 + 2)
    x = r.standard_normal(size=(B, H, T, T), dtype=np.float32) * np.float32(0.125)
    iu = np.triu_indices(T, 1)
    x[:, :, iu[0], iu[1]] = -np.inf
    dy = r.standard_normal(size=x.shape, dtype=np.float32)
    rows = B * H * T
    X, DY = dev(vh, x), dev(vh, dy)
    Y, DX = out(vh, x.shape), out(vh, x.shape)
    vh.check(vh.lib.vh_softmax_fwd(X.ptr, Y.ptr, rows, T, 1, None))
    vh.check(vh.lib.vh_softmax_bwd(X.ptr, DY.ptr, DX.ptr, rows, T, 1, 1, None))
    y = fetch(vh, Y, x.shape)
    del Y
    np.testing.assert_allclose(y.sum(axis=-1, dtype=np.float64), 1.0, atol=2e-5)
    assert np.all(y[:, :, iu[0], iu[1]] == 0.0)
    dx = fetch(vh, DX, x.shape)
    del DX
    np.testing.assert_allclose(dx.sum(axis=-1, dtype=np.float64), 0.0, atol=1e-4)
    assert np.all(dx[:, :, iu[0], iu[1]] == 0.0)
    for b in range(B):
        for h in range(H):
            assert_parity(y[b, h], O.softmax(x[b, h], 1), name=f"y[{b},{h}]")
            assert_parity(dx[b, h], O.softmax_backward_composite(x[b, h], dy[b, h], 1), name=f"dx[{b},{h}]")


def test_cross_entropy_cfg4_full(vh):
    B, V = 16384, 50257
    print("cross-entropy cfg4 full", flush=True)
    r = np.random.default_rng(0x5EED0000 + 4)
    logits = r.standard_normal(size=(B, V), dtype=np.float32)
    tg = r.integers(0, V, size=B).astype(np.float32)
    go = np.float32([1.0])
    L, T, GO = dev(vh, logits), dev(vh, tg), dev(vh, go)
    LOSS, DL = out(vh, (1,)), out(vh, (B, V))
    vh.check(vh.lib.vh_cross_entropy_fwd(L.ptr, T.ptr, LOSS.ptr, B, V, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_bwd(L.ptr, T.ptr, GO.ptr, DL.ptr, B, V, None))
    loss = fetch(vh, LOSS, (1,))[0]
    ls = np.empty(B)
    for i in range(0, B, 1024):
        blk = logits[i:i + 1024].astype(np.float64)
        m = blk.max(axis=1)
        lse = m + np.log(np.exp(blk - m[:, None]).sum(axis=1))
        ls[i:i + 1024] = blk[np.arange(len(blk)), tg[i:i + 1024].astype(np.int64)] - lse
    exact = -ls.sum() / B
    assert abs(loss - exact) <= 1e-5 + 1e-4 * abs(exact), (loss, exact)
    assert_parity(np.float32([loss]), O.cross_entropy(logits, tg), name="loss")
    dl = fetch(vh, DL, (B, V))
    # The row-statistics pair on the same logits: the same loss and dlogits bits.
    ST, LOSS2 = out(vh, (B, 2)), out(vh, (1,))
    vh.check(vh.lib.vh_cross_entropy_fwd_rs_ld(L.ptr, V, T.ptr, LOSS2.ptr, ST.ptr, B, V, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_bwd_rs_ld(L.ptr, V, T.ptr, ST.ptr, GO.ptr, DL.ptr, B, V, None))
    assert fetch(vh, LOSS2, (1,))[0] == loss
    assert np.array_equal(fetch(vh, DL, (B, V)), dl)
    del DL, L
    np.testing.assert_allclose(dl.sum(axis=1, dtype=np.float64), 0.0, atol=1e-9)
    ti = tg.astype(np.int64)
    assert np.all(dl[np.arange(B), ti] < 0)
    neg = (dl < 0).sum(axis=1)
    assert np.all(neg == 1)
    # The oracle on every row, in blocks of R rows: it divides by the batch it
    # is given, so grad_out carries R / B -- with B and R powers of two every
    # scaling is exact and each row gets the full batch's values.
    # (The oracle's C calls release the GIL, so blocks run on 8 threads.)
    from concurrent.futures import ThreadPoolExecutor
    R = 1024
    gb = go * np.float32(R) / np.float32(B)
    with ThreadPoolExecutor(8) as pool:
        refs = pool.map(lambda i: (i, O.cross_entropy_backward(logits[i:i + R], tg[i:i + R], gb)), range(0, B, R))
        for i, ref in refs:
            np.testing.assert_allclose(dl[i:i + R], ref, rtol=1e-4, atol=1e-12, err_msg=f"rows {i}..{i + R}")
