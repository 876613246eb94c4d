"""GPU parity: every hot-path entry point of libvearo_hip.so, called through the
C ABI, against the CPU oracle on identical seeded inputs. Embedding forward is
bit-exact, and so are embedding-gradient rows of tokens with at most 16 hits
(summed in the CPU's order); everything else within 1e-5 + 1e-4*|cpu|.
Shapes cover the BASELINE configs (or a row-subset of them where the oracle
would take minutes) plus the ragged / tiny / large-row variants of each kernel
family. Full-size properties of the biggest configs run in test_properties_gpu.py."""
import ctypes

import numpy as np
import pytest

import oracle as O
from parity import assert_parity, dev, fetch, out

pytestmark = pytest.mark.gpu


def rng(tag):
    return np.random.default_rng(0x5EED0000 + tag)


# ------------------------------------------------------------------ layernorm
# (33, 256), (9, 512), (16384, 768), (70, 1024): the full-row kernel forms
# (C = 64 lanes x 1..4 units x 4 floats), with ragged row counts.
LN_SHAPES = [(2048, 128), (16384, 768), (1, 5), (3, 33), (7, 64), (130, 100), (64, 1000),
             (17, 1030), (8, 4096), (4, 20000), (5, 1), (33, 256), (9, 512), (70, 1024)]


@pytest.mark.parametrize("rows,C", LN_SHAPES)
def test_layernorm_fwd_bwd(vh, rows, C):
    print(f"layernorm rows={rows} C={C}", flush=True)
    r = rng(0)
    x = r.normal(size=(rows, C)).astype(np.float32)
    w = (1 + 0.02 * r.normal(size=C)).astype(np.float32)
    b = (0.02 * r.normal(size=C)).astype(np.float32)
    dy = r.normal(size=(rows, C)).astype(np.float32)
    eps = 1e-5
    X, W, B, DY = dev(vh, x), dev(vh, w), dev(vh, b), dev(vh, dy)
    Y, DX, DW, DB = out(vh, (rows, C)), out(vh, (rows, C)), out(vh, (C,)), out(vh, (C,))
    vh.check(vh.lib.vh_layernorm_fwd(X.ptr, W.ptr, B.ptr, Y.ptr, rows, C, eps, None))
    vh.check(vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C, eps,
                                     None, 0, None))
    y_cpu = O.layernorm(x, w, b, eps)
    dx_cpu, dw_cpu, db_cpu = O.layernorm_backward(x, w, b, dy, eps)
    assert_parity(fetch(vh, Y, (rows, C)), y_cpu, name="y")
    assert_parity(fetch(vh, DX, (rows, C)), dx_cpu, name="dx")
    x64, dy64 = x.astype(np.float64), dy.astype(np.float64)
    xh = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + eps)
    assert_parity(fetch(vh, DW, (C,)), dw_cpu, (dy64 * xh).sum(0), name="dgamma")
    assert_parity(fetch(vh, DB, (C,)), db_cpu, dy64.sum(0), name="dbeta")


def test_layernorm_deterministic(vh):
    r = rng(1)
    rows, C = 4096, 768
    x = r.normal(size=(rows, C)).astype(np.float32)
    w = np.ones(C, np.float32)
    dy = r.normal(size=(rows, C)).astype(np.float32)
    X, W, DY = dev(vh, x), dev(vh, w), dev(vh, dy)
    res = []
    for _ in range(3):
        DX, DW, DB = out(vh, (rows, C)), out(vh, (C,)), out(vh, (C,))
        vh.check(vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C,
                                         1e-5, None, 0, None))
        res.append((fetch(vh, DW, (C,)), fetch(vh, DB, (C,))))
    for dw, db in res[1:]:
        np.testing.assert_array_equal(dw, res[0][0])
        np.testing.assert_array_equal(db, res[0][1])


def test_layernorm_explicit_scratch_and_errors(vh):
    rows, C = 300, 96
    need = vh.lib.vh_layernorm_bwd_scratch_bytes(rows, C)
    assert need > 0
    r = rng(2)
    x = r.normal(size=(rows, C)).astype(np.float32)
    w, dy = np.ones(C, np.float32), r.normal(size=(rows, C)).astype(np.float32)
    X, W, DY = dev(vh, x), dev(vh, w), dev(vh, dy)
    DX, DW, DB = out(vh, (rows, C)), out(vh, (C,)), out(vh, (C,))
    S = vh.DeviceBuffer(need)
    rc = vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C, 1e-5, S.ptr,
                                 256, None)
    assert rc == vh.VH_ERR_INVALID and "scratch buffer too small" in vh.last_error()
    vh.check(vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, rows, C, 1e-5,
                                     S.ptr, need, None))
    _, dw_cpu, db_cpu = O.layernorm_backward(x, w, np.zeros(C, np.float32), dy, 1e-5)
    assert_parity(fetch(vh, DB, (C,)), db_cpu, dy.astype(np.float64).sum(0), name="dbeta")
    assert vh.lib.vh_layernorm_fwd(X.ptr, W.ptr, W.ptr, DX.ptr, -1, C, 1e-5, None) == vh.VH_ERR_INVALID
    # Rows longer than int32 are refused before any launch, by both entries.
    big = 1 << 31
    assert vh.lib.vh_layernorm_fwd(X.ptr, W.ptr, W.ptr, DX.ptr, 1, big, 1e-5, None) == vh.VH_ERR_UNSUPPORTED
    for rc in (vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, 1, big, 1e-5, None, 0, None),
               vh.lib.vh_layernorm_bwd_noalloc(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr, 1, big, 1e-5, None)):
        assert rc == vh.VH_ERR_UNSUPPORTED and "C too large" in vh.last_error()


# ----------------------------------------------------------------------- gelu
# (2500, 768) and (20000, 192): row blocks of 3 and 20 rows (at most 1024
# dbias partials), so a block's rows end partway through a batch of loads.
# (5, 4097), (3, 20000), (2, 70001): rows wider than the forward's registers
# hold (4096 single floats, 16384 as 128-bit units) take its column-tile form.
@pytest.mark.parametrize("rows,C", [(16384, 3072), (3, 5), (33, 100), (7, 4096), (5, 5000), (2500, 768),
                                    (20000, 192), (5, 4097), (3, 20000), (2, 70001)])
def test_gelu_bias_fwd_bwd(vh, rows, C):
    print(f"gelu_bias rows={rows} C={C}", flush=True)
    r = rng(1)
    x = (1.5 * r.normal(size=(rows, C))).astype(np.float32)
    bias = (0.02 * r.normal(size=C)).astype(np.float32)
    dy = r.normal(size=(rows, C)).astype(np.float32)
    X, Bi, DY = dev(vh, x), dev(vh, bias), dev(vh, dy)
    Y, DX, DB = out(vh, (rows, C)), out(vh, (rows, C)), out(vh, (C,))
    vh.check(vh.lib.vh_gelu_bias_fwd(X.ptr, Bi.ptr, Y.ptr, rows, C, None))
    vh.check(vh.lib.vh_gelu_bias_bwd(X.ptr, Bi.ptr, DY.ptr, DX.ptr, DB.ptr, rows, C, None, 0, None))
    assert_parity(fetch(vh, Y, (rows, C)), O.gelu_bias_forward(x, bias), name="y")
    dx_cpu, db_cpu = O.gelu_bias_backward(x, bias, dy)
    assert_parity(fetch(vh, DX, (rows, C)), dx_cpu, name="dx")
    assert_parity(fetch(vh, DB, (C,)), db_cpu, dx_cpu.astype(np.float64).sum(0), name="dbias")


def test_gelu_bias_fwd_tile_form_same_bits(vh):
    """The column-tile forward (rows past the register form's width) gives the
    register form's bits: C = 4100 runs in registers as 128-bit units from
    aligned buffers and as column tiles of single floats one float past them."""
    r = rng(9)
    rows, C = 6, 4100
    x = (2.0 * r.normal(size=(rows, C))).astype(np.float32)
    bias = r.normal(size=C).astype(np.float32)
    X, Bi, Y = dev(vh, x), dev(vh, bias), out(vh, (rows, C))
    vh.check(vh.lib.vh_gelu_bias_fwd(X.ptr, Bi.ptr, Y.ptr, rows, C, None))
    X1 = dev(vh, np.concatenate([[0.0], x.reshape(-1)]))
    B1 = dev(vh, np.concatenate([[0.0], bias]))
    Y1 = out(vh, (rows * C + 1,))
    vh.check(vh.lib.vh_gelu_bias_fwd(X1.ptr + 4, B1.ptr + 4, Y1.ptr + 4, rows, C, None))
    a = fetch(vh, Y, (rows, C))
    b = fetch(vh, Y1, (rows * C + 1,))[1:].reshape(rows, C)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    assert_parity(a, O.gelu_bias_forward(x, bias), name="gelu(x + b) C=4100")


@pytest.mark.parametrize("n", [1, 7, 4096, 1000003])
def test_gelu_and_grad_mul(vh, n):
    r = rng(3)
    x = (2.0 * r.normal(size=n)).astype(np.float32)
    dy = r.normal(size=n).astype(np.float32)
    X, DY, Y, DX = dev(vh, x), dev(vh, dy), out(vh, (n,)), out(vh, (n,))
    vh.check(vh.lib.vh_gelu_fwd(X.ptr, Y.ptr, n, None))
    vh.check(vh.lib.vh_gelu_grad_mul(X.ptr, DY.ptr, DX.ptr, n, None))
    assert_parity(fetch(vh, Y, (n,)), O.gelu(x), name="gelu")
    assert_parity(fetch(vh, DX, (n,)), O.binary(2, dy, O.gelu_grad_mask(x)), name="gelu'")


# -------------------------------------------------------------------- softmax
def causal_scores(r, B, H, T):
    s = (r.normal(size=(B, H, T, T)) / 8.0).astype(np.float32)
    iu = np.triu_indices(T, 1)
    s[:, :, iu[0], iu[1]] = -np.inf
    return s


# (1, 1, 201): 201 one-float units on two-wave teams and an odd row count, so a
# workgroup's second team has no row; (1, 3, 600): 150 four-float units.
@pytest.mark.parametrize("B,H,T", [(2, 12, 1024), (1, 2, 37), (2, 3, 128), (1, 1, 1000),
                                   (1, 1, 2048), (1, 1, 5000), (1, 1, 201), (1, 3, 600), (2, 3, 1), (1, 1, 3)])
@pytest.mark.parametrize("causal", [0, 1])
def test_softmax_fwd_bwd(vh, B, H, T, causal):
    print(f"softmax B={B} H={H} T={T} causal={causal}", flush=True)
    r = rng(2)
    x = causal_scores(r, B, H, T)
    dy = r.normal(size=x.shape).astype(np.float32)
    rows = B * H * T
    X, DY, Y, DX, DX2 = dev(vh, x), dev(vh, dy), out(vh, x.shape), out(vh, x.shape), out(vh, x.shape)
    vh.check(vh.lib.vh_softmax_fwd(X.ptr, Y.ptr, rows, T, causal, None))
    vh.check(vh.lib.vh_softmax_bwd(Y.ptr, DY.ptr, DX.ptr, rows, T, 0, causal, None))
    vh.check(vh.lib.vh_softmax_bwd(X.ptr, DY.ptr, DX2.ptr, rows, T, 1, causal, None))
    y_cpu = O.softmax(x, 3)
    dx_cpu = O.softmax_backward_composite(x, dy, 3)
    y = fetch(vh, Y, x.shape)
    assert_parity(y, y_cpu, name="y")
    iu = np.triu_indices(T, 1)
    assert np.all(y[:, :, iu[0], iu[1]] == 0.0)
    assert_parity(fetch(vh, DX, x.shape), dx_cpu, name="dx(from y)")
    assert_parity(fetch(vh, DX2, x.shape), dx_cpu, name="dx(from x)")


def test_softmax_dense_rows(vh):
    r = rng(4)
    for rows, T in [(100, 1024), (5, 3), (9, 17), (3, 65536)]:
        x = r.normal(size=(rows, T)).astype(np.float32) * 3
        dy = r.normal(size=(rows, T)).astype(np.float32)
        X, DY, Y, DX = dev(vh, x), dev(vh, dy), out(vh, x.shape), out(vh, x.shape)
        vh.check(vh.lib.vh_softmax_fwd(X.ptr, Y.ptr, rows, T, 0, None))
        vh.check(vh.lib.vh_softmax_bwd(X.ptr, DY.ptr, DX.ptr, rows, T, 1, 0, None))
        assert_parity(fetch(vh, DX, x.shape), O.softmax_backward_composite(x, dy, 1), name=f"dx T={T}")
        assert_parity(fetch(vh, Y, x.shape), O.softmax(x, 1), name=f"y T={T}")


# ------------------------------------------------------------------ embedding
def zipf_ids(r, n, V, s=1.1):
    ranks = np.arange(1, V + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    return np.searchsorted(cdf, r.random(n)).astype(np.float32)


def check_embedding_grad(gpu, ids, dy, V):
    """Rows of tokens with <= 16 hits must equal the oracle bit for bit (same f32
    order as the CPU loop); rows of heavier tokens, summed in position chunks,
    must be within tolerance of it (checked against float64 as well)."""
    D = dy.shape[-1]
    ref = O.embedding_backward(ids, (V, D), dy)
    tok = np.floor(ids.reshape(-1).astype(np.float64) + 0.5).astype(np.int64)
    counts = np.bincount(tok, minlength=V)
    light = counts <= 16
    np.testing.assert_array_equal(gpu[light], ref[light])
    if (~light).any():
        ref64 = np.zeros((V, D))
        np.add.at(ref64, tok, dy.reshape(-1, D).astype(np.float64))
        assert_parity(gpu[~light], ref[~light], ref64[~light], name="heavy rows")


@pytest.mark.parametrize("dist", ["uniform", "zipf"])
def test_embedding_config3(vh, dist):
    print(f"embedding config3 {dist}", flush=True)
    r = rng(3)
    V, D, n = 50257, 768, 16384
    W = (0.02 * r.normal(size=(V, D))).astype(np.float32)
    ids = (r.integers(0, V, size=n).astype(np.float32) if dist == "uniform" else zipf_ids(r, n, V))
    dy = r.normal(size=(n, D)).astype(np.float32)
    I, Wd, DY = dev(vh, ids), dev(vh, W), dev(vh, dy)
    OUT, DW, DW2 = out(vh, (n, D)), out(vh, (V, D)), out(vh, (V, D))
    vh.check(vh.lib.vh_embedding_fwd(I.ptr, Wd.ptr, OUT.ptr, n, V, D, None))
    vh.check(vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, DW.ptr, n, V, D, None, 0, None))
    vh.check(vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, DW2.ptr, n, V, D, None, 0, None))
    np.testing.assert_array_equal(fetch(vh, OUT, (n, D)), O.embedding(ids, W))  # forward: bit-exact
    g = fetch(vh, DW, (V, D))
    np.testing.assert_array_equal(g, fetch(vh, DW2, (V, D)))                     # deterministic
    check_embedding_grad(g, ids, dy, V)


@pytest.mark.parametrize("n,V,D", [(1, 3, 2), (10, 4, 5), (300, 7, 64), (5000, 3, 33),
                                   (9000, 2, 8), (100, 100000, 1), (20000, 1, 1030), (640, 10, 4)])
def test_embedding_shapes(vh, n, V, D):
    r = rng(5)
    ids = r.integers(0, V, size=n).astype(np.float32) + r.uniform(-0.49, 0.49, size=n).astype(np.float32)
    ids = np.clip(ids, 0, V - 1).astype(np.float32)
    W = r.normal(size=(V, D)).astype(np.float32)
    dy = r.normal(size=(n, D)).astype(np.float32)
    I, Wd, DY = dev(vh, ids), dev(vh, W), dev(vh, dy)
    OUT, DW = out(vh, (n, D)), out(vh, (V, D))
    vh.check(vh.lib.vh_embedding_fwd(I.ptr, Wd.ptr, OUT.ptr, n, V, D, None))
    vh.check(vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, DW.ptr, n, V, D, None, 0, None))
    np.testing.assert_array_equal(fetch(vh, OUT, (n, D)), O.embedding(ids, W))
    check_embedding_grad(fetch(vh, DW, (V, D)), ids, dy, V)


def test_embedding_sorted_and_general_paths_agree(vh):
    """The same Zipf ids through the sorted path (V = 50257) and the general
    one (V = 70000 > 65534, the rows past 50257 unused): the same bits in the
    shared rows -- the same light-row order, 32-hit tasks and final grouping --
    and zeros past them."""
    r = rng(31)
    n, D = 16384, 768
    ids = zipf_ids(r, n, 50257)
    dy = r.normal(size=(n, D)).astype(np.float32)
    I, DY = dev(vh, ids), dev(vh, dy)
    A, B = out(vh, (50257, D)), out(vh, (70000, D))
    vh.check(vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, A.ptr, n, 50257, D, None, 0, None))
    vh.check(vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, B.ptr, n, 70000, D, None, 0, None))
    a, b = fetch(vh, A, (50257, D)), fetch(vh, B, (70000, D))
    np.testing.assert_array_equal(a, b[:50257])
    assert not b[50257:].any()
    check_embedding_grad(a, ids, dy, 50257)


def test_embedding_heavy_token_clustered(vh):
    # A heavy token whose hits all sit at the end of the positions: the chunks
    # before them hold nothing, the last chunks hold everything.
    n, V, D = 4096, 50, 96
    ids = np.concatenate([np.arange(n - 700) % 49 + 1, np.zeros(700)]).astype(np.float32)
    r = rng(8)
    dy = r.normal(size=(n, D)).astype(np.float32)
    I, DY, DW = dev(vh, ids), dev(vh, dy), out(vh, (V, D))
    vh.check(vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, DW.ptr, n, V, D, None, 0, None))
    check_embedding_grad(fetch(vh, DW, (V, D)), ids, dy, V)


@pytest.mark.parametrize("n,D,dist", [(40000, 96, "uniform"), (40000, 96, "zipf"), (82020, 64, "zipf")])
def test_embedding_many_tokens(vh, n, D, dist):
    """More positions than the sorted path takes (16384): the general path
    (token histogram, per-row position slots sorted in registers) -- light rows
    bit-exact, heavy rows within tolerance, two runs the same bits."""
    print(f"embedding many tokens n={n} D={D} {dist}", flush=True)
    r = rng(41)
    V = 50257
    ids = (r.integers(0, V, size=n).astype(np.float32) if dist == "uniform" else zipf_ids(r, n, V))
    dy = r.normal(size=(n, D)).astype(np.float32)
    I, DY = dev(vh, ids), dev(vh, dy)
    A, B = out(vh, (V, D)), out(vh, (V, D))
    vh.check(vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, A.ptr, n, V, D, None, 0, None))
    vh.check(vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, B.ptr, n, V, D, None, 0, None))
    a = fetch(vh, A, (V, D))
    np.testing.assert_array_equal(a, fetch(vh, B, (V, D)))
    check_embedding_grad(a, ids, dy, V)


def test_embedding_many_tokens_report_first_bad_id(vh):
    # Two bad ids far apart among 40000 positions: the panic names the first
    # one in position order, as the CPU loop would.
    n, V, D = 40000, 50257, 4
    ids = np.arange(n, dtype=np.float32) % V
    ids[35000], ids[20000] = -1.0, 60000.0
    I, DY, DW = dev(vh, ids), dev(vh, np.ones((n, D))), out(vh, (V, D))
    vh.check(vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, DW.ptr, n, V, D, None, 0, None))
    with pytest.raises(vh.DevicePanic) as ei:
        vh.sync()
    with pytest.raises(O.Panic) as eo:
        O.embedding(ids, np.ones((V, D), np.float32))
    assert ei.value.msg == str(eo.value) == "Token ID 60000 out of vocabulary bound 50257"
    vh.sync()


@pytest.mark.parametrize("bad,msg", [(-1.0, "Token ID cannot be negative: -1"),
                                     (7.0, "Token ID 7 out of vocabulary bound 5"),
                                     (4.5, "Token ID 5 out of vocabulary bound 5"),
                                     (float("nan"), "Token ID cannot be negative: NaN"),
                                     (-0.25, "Token ID cannot be negative: -0.25")])
def test_embedding_bad_ids_report_cpu_panic(vh, bad, msg):
    V, D = 5, 4
    ids = np.float32([1, 2, bad, 3, -2.0])
    I, Wd, DY = dev(vh, ids), dev(vh, np.ones((V, D))), dev(vh, np.ones((5, D)))
    OUT, DW = out(vh, (5, D)), out(vh, (V, D))
    for call in (lambda: vh.lib.vh_embedding_fwd(I.ptr, Wd.ptr, OUT.ptr, 5, V, D, None),
                 lambda: vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, DW.ptr, 5, V, D, None, 0, None)):
        vh.check(call())
        with pytest.raises(vh.DevicePanic) as ei:
            vh.sync()
        assert ei.value.msg == msg
        with pytest.raises(O.Panic) as eo:
            O.embedding(ids, np.ones((V, D), np.float32))
        assert str(eo.value) == msg
    vh.sync()  # the record is cleared once reported


# -------------------------------------------------------------- cross-entropy
# (1500, 3000): more rows than the GPU holds row-cached workgroups at once.
@pytest.mark.parametrize("B,V", [(512, 50257), (3, 5), (64, 1000), (7, 70000), (1, 1), (1500, 3000)])
def test_cross_entropy_fwd_bwd(vh, B, V):
    print(f"cross_entropy B={B} V={V}", flush=True)
    r = rng(4)
    logits = (2.0 * r.normal(size=(B, V))).astype(np.float32)
    tg = r.integers(0, V, size=B).astype(np.float32)
    go = np.float32([1.3])
    L, T, GO = dev(vh, logits), dev(vh, tg), dev(vh, go)
    LOSS, DL = out(vh, (1,)), out(vh, (B, V))
    vh.check(vh.lib.vh_cross_entropy_fwd(L.ptr, T.ptr, LOSS.ptr, B, V, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_bwd(L.ptr, T.ptr, GO.ptr, DL.ptr, B, V, None))
    assert_parity(fetch(vh, LOSS, (1,)), O.cross_entropy(logits, tg), name="loss")
    assert_parity(fetch(vh, DL, (B, V)), O.cross_entropy_backward(logits, tg, go), name="dlogits")


# (4, 4096) and (3, 8193): whole and ragged 4096-column chunks of the row-statistics backward.
@pytest.mark.parametrize("B,V", [(512, 50257), (3, 5), (64, 1000), (7, 70000), (1, 1), (1500, 3000),
                                 (4, 4096), (3, 8193)])
def test_cross_entropy_row_stats(vh, B, V):
    """The forward that keeps each row's (max, sum-exp) and the streaming
    backward from them: the loss bit-equal to vh_cross_entropy_fwd's, the max
    equal to the row's maximum, dlogits bit-equal to the recomputing backward
    (row-cached and streaming V alike), with a row stride, in place, with inf
    and NaN logits, and against the oracle."""
    print(f"cross_entropy row stats B={B} V={V}", flush=True)
    r = rng(41)
    logits = (2.0 * r.normal(size=(B, V))).astype(np.float32)
    if B >= 3 and V >= 3:
        logits[1, V // 2] = np.inf
        logits[2, 1] = np.nan
    tg = r.integers(0, V, size=B).astype(np.float32)
    go = np.float32([1.3])
    L, T, GO = dev(vh, logits), dev(vh, tg), dev(vh, go)
    LOSS, LOSS2, ST = out(vh, (1,)), out(vh, (1,)), out(vh, (B, 2))
    DL, DL2 = out(vh, (B, V)), out(vh, (B, V))
    vh.check(vh.lib.vh_cross_entropy_fwd(L.ptr, T.ptr, LOSS.ptr, B, V, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_bwd(L.ptr, T.ptr, GO.ptr, DL.ptr, B, V, None))
    vh.check(vh.lib.vh_cross_entropy_fwd_rs_ld(L.ptr, V, T.ptr, LOSS2.ptr, ST.ptr, B, V, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_bwd_rs_ld(L.ptr, V, T.ptr, ST.ptr, GO.ptr, DL2.ptr, B, V, None))
    np.testing.assert_array_equal(fetch(vh, LOSS2, (1,)), fetch(vh, LOSS, (1,)))
    st = fetch(vh, ST, (B, 2))
    # The reference's max skips NaN (`if l > max`, cpu:1102-1108).
    np.testing.assert_array_equal(st[:, 0], np.nanmax(logits, axis=1))
    want = fetch(vh, DL, (B, V))
    np.testing.assert_array_equal(fetch(vh, DL2, (B, V)), want)
    fin = np.isfinite(logits).all(axis=1)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = O.cross_entropy_backward(logits, tg, go)
    assert_parity(want[fin], ref[fin], name="dlogits")
    if fin.all():
        assert_parity(fetch(vh, LOSS2, (1,)), O.cross_entropy(logits, tg), name="loss")
    # Row stride ld > V (both buffers), then in place over the logits.
    ld = V + 7
    wide = np.full((B, ld), 5.0, np.float32)
    wide[:, :V] = logits
    LW, DW = dev(vh, wide), dev(vh, np.full((B, ld), -3.0, np.float32))
    vh.check(vh.lib.vh_cross_entropy_fwd_rs_ld(LW.ptr, ld, T.ptr, LOSS2.ptr, ST.ptr, B, V, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_bwd_rs_ld(LW.ptr, ld, T.ptr, ST.ptr, GO.ptr, DW.ptr, B, V, None))
    dw = fetch(vh, DW, (B, ld))
    np.testing.assert_array_equal(dw[:, :V], want)
    assert np.all(dw[:, V:] == -3.0)
    vh.check(vh.lib.vh_cross_entropy_bwd_rs_ld(LW.ptr, ld, T.ptr, ST.ptr, GO.ptr, LW.ptr, B, V, None))
    lw = fetch(vh, LW, (B, ld))
    np.testing.assert_array_equal(lw[:, :V], want)
    assert np.all(lw[:, V:] == 5.0)
    # Buffers 4 bytes past a 16-byte boundary: the 32-bit kernel.
    LO = dev(vh, np.concatenate([np.float32([7.0]), logits.ravel()]))
    DO = dev(vh, np.full(B * V + 1, -3.0, np.float32))
    vh.check(vh.lib.vh_cross_entropy_fwd_rs_ld(LO.ptr + 4, V, T.ptr, LOSS2.ptr, ST.ptr, B, V, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_bwd_rs_ld(LO.ptr + 4, V, T.ptr, ST.ptr, GO.ptr, DO.ptr + 4, B, V, None))
    do = fetch(vh, DO, (B * V + 1,))
    np.testing.assert_array_equal(do[1:].reshape(B, V), want)
    assert do[0] == -3.0


def test_cross_entropy_row_stats_errors(vh):
    """Argument errors and the invalid-target panic through the row-statistics
    entries, with the reference's messages."""
    L = dev(vh, np.zeros((2, 3), np.float32))
    LOSS, ST, GO, DL = out(vh, (1,)), out(vh, (2, 2)), dev(vh, np.float32([1.0])), out(vh, (2, 3))
    for tv, msg in [(-1.0, "Target class cannot be negative: -1"),
                    (3.0, "Target class 3 out of vocab bounds 3")]:
        T = dev(vh, np.float32([0.0, tv]))
        vh.check(vh.lib.vh_cross_entropy_fwd_rs_ld(L.ptr, 3, T.ptr, LOSS.ptr, ST.ptr, 2, 3, None, 0, None))
        with pytest.raises(vh.DevicePanic) as ei:
            vh.sync()
        assert ei.value.msg == msg
        vh.check(vh.lib.vh_cross_entropy_bwd_rs_ld(L.ptr, 3, T.ptr, ST.ptr, GO.ptr, DL.ptr, 2, 3, None))
        with pytest.raises(vh.DevicePanic) as ei:
            vh.sync()
        assert ei.value.msg == msg
    T = dev(vh, np.float32([0.0, 1.0]))
    rc = vh.lib.vh_cross_entropy_bwd_rs_ld(L.ptr, 3, T.ptr, ST.ptr, GO.ptr, DL.ptr, 0, 3, None)
    assert rc == vh.VH_ERR_INVALID and vh.last_error() == "Batch size must be greater than 0"
    rc = vh.lib.vh_cross_entropy_bwd_rs_ld(L.ptr, 2, T.ptr, ST.ptr, GO.ptr, DL.ptr, 2, 3, None)
    assert rc == vh.VH_ERR_INVALID and "row stride below V" in vh.last_error()
    rc = vh.lib.vh_cross_entropy_bwd_rs_ld(L.ptr, 3, T.ptr, ST.ptr + 4, GO.ptr, DL.ptr, 2, 3, None)
    assert rc == vh.VH_ERR_INVALID and "8-byte aligned" in vh.last_error()
    rc = vh.lib.vh_cross_entropy_fwd_rs_ld(L.ptr, 3, T.ptr, LOSS.ptr, None, 2, 3, None, 0, None)
    assert rc == vh.VH_ERR_INVALID and "null pointer" in vh.last_error()


def test_cross_entropy_kats_and_panics(vh):
    L, T = dev(vh, np.float32([[1000.0, -1000.0]])), dev(vh, np.float32([0.0]))
    LOSS = out(vh, (1,))
    vh.check(vh.lib.vh_cross_entropy_fwd(L.ptr, T.ptr, LOSS.ptr, 1, 2, None, 0, None))
    assert abs(fetch(vh, LOSS, (1,))[0]) < 1e-4  # cpu lib.rs:2902-2913
    L = dev(vh, np.zeros((2, 3), np.float32))
    for tv, msg in [(-1.0, "Target class cannot be negative: -1"),
                    (3.0, "Target class 3 out of vocab bounds 3")]:
        T = dev(vh, np.float32([tv, 0.0]))
        vh.check(vh.lib.vh_cross_entropy_fwd(L.ptr, T.ptr, LOSS.ptr, 2, 3, None, 0, None))
        with pytest.raises(vh.DevicePanic) as ei:
            vh.sync()
        assert ei.value.msg == msg
    rc = vh.lib.vh_cross_entropy_fwd(L.ptr, T.ptr, LOSS.ptr, 0, 3, None, 0, None)
    assert rc == vh.VH_ERR_INVALID and vh.last_error() == "Batch size must be greater than 0"


# --------------------------------------------------------- composites (a13)
def test_binary_row_broadcast(vh):
    """A contiguous operand against a vector over its last dim (a bias add, or
    the vector on the left of a sub/div) takes the row-broadcast stream: the
    same values as the broadcast rule, both operand orders, 16-byte and 4-byte
    units."""
    r = rng(16)
    for full_shape, vec_shape in (((64, 3072), (3072,)), ((4, 33, 769), (769,)), ((5, 7, 128), (1, 1, 128))):
        f = r.normal(size=full_shape).astype(np.float32)
        v = (r.normal(size=vec_shape) + 3).astype(np.float32)
        F, Vd = dev(vh, f), dev(vh, v)
        for op, fn in enumerate((np.add, np.subtract, np.multiply, np.divide)):
            for left in (False, True):
                OUT = out(vh, full_shape)
                a, al, b, bl = (Vd, v.shape, F, f.shape) if left else (F, f.shape, Vd, v.shape)
                vh.check(vh.lib.vh_binary(op, a.ptr, vh.layout(al), b.ptr, vh.layout(bl), OUT.ptr, None))
                want = fn(v, f) if left else fn(f, v)
                np.testing.assert_array_equal(fetch(vh, OUT, full_shape), want.astype(np.float32),
                                              err_msg=f"{full_shape} op={op} left={left}")



def test_binary_block_scalar_and_column_broadcast(vh):
    """The other broadcast streams the unfused attention and the Softmax arm
    drive: a vector over the output's trailing dims (the [S, S] mask on [B, H,
    S, S] scores), a single value (the scale), and a vector over the leading
    dims with size-1 trailing dims (dy - sum(dy * y, keep_dim)); both operand
    orders, every op, 16-byte and 4-byte units, the same bits as the oracle's
    broadcast rule (cpu:160-238)."""
    r = rng(17)
    cases = [((2, 3, 64, 64), (64, 64)), ((2, 3, 64, 64), (1, 1, 64, 64)), ((2, 3, 64, 64), (1,)),
             ((5, 7, 33), ()), ((2, 3, 64, 64), (2, 3, 64, 1)), ((4, 9, 30), (4, 9, 1)), ((6, 10), (6, 1)),
             ((3, 5, 8), (5, 8)), ((3, 5, 7), (3, 1, 1))]
    for fs, vs in cases:
        f = r.normal(size=fs).astype(np.float32)
        v = (r.normal(size=vs) + 3).astype(np.float32)
        F, Vd = dev(vh, f), dev(vh, v)
        for op in range(4):
            for left in (False, True):
                OUT = out(vh, fs)
                a, al, b, bl = (Vd, v.shape, F, f.shape) if left else (F, f.shape, Vd, v.shape)
                vh.check(vh.lib.vh_binary(op, a.ptr, vh.layout(al), b.ptr, vh.layout(bl), OUT.ptr, None))
                want = O.binary(op, v, f) if left else O.binary(op, f, v)
                np.testing.assert_array_equal(fetch(vh, OUT, fs), want, err_msg=f"{fs} {vs} op={op} left={left}")


def test_binary_broadcast_and_strided(vh):
    r = rng(6)
    cases = [((64, 3072), (3072,)), ((3, 1, 5), (4, 1)), ((16, 12, 128, 128), (16, 12, 128, 1)),
             ((1000,), (1000,)), ((7,), ())]
    for ls, rs in cases:
        a = r.normal(size=ls).astype(np.float32)
        b = (r.normal(size=rs) + 3).astype(np.float32)
        A, B = dev(vh, a), dev(vh, b)
        shape = np.broadcast_shapes(ls, rs)
        for op in range(4):
            OUT = out(vh, shape)
            vh.check(vh.lib.vh_binary(op, A.ptr, vh.layout(ls), B.ptr, vh.layout(rs), OUT.ptr, None))
            np.testing.assert_array_equal(fetch(vh, OUT, shape), O.binary(op, a, b))
    # Transposed (strided) operands, the backward's case.
    a = np.arange(9, dtype=np.float32).reshape(3, 3) + 1
    b = a[::-1].copy()
    A, B = dev(vh, a), dev(vh, b)
    OUT = out(vh, (3, 3))
    vh.check(vh.lib.vh_binary(0, A.ptr, vh.layout((3, 3)), B.ptr, vh.layout((3, 3), (1, 3)), OUT.ptr, None))
    np.testing.assert_array_equal(fetch(vh, OUT, (3, 3)), a + b.T)
    rc = vh.lib.vh_binary(0, A.ptr, vh.layout((2, 3)), B.ptr, vh.layout((4,)), OUT.ptr, None)
    assert rc == vh.VH_ERR_INVALID and vh.last_error() == "Shapes are not broadcastable"


def test_reduce_and_strided_copy(vh):
    r = rng(7)
    x = r.normal(size=(4, 6, 300)).astype(np.float32)
    X = dev(vh, x)
    for dim in range(3):
        for mean in (0, 1):
            shape = tuple(s for i, s in enumerate(x.shape) if i != dim)
            OUT = out(vh, shape)
            vh.check(vh.lib.vh_reduce(mean, X.ptr, vh.layout(x.shape), dim, OUT.ptr, None))
            assert_parity(fetch(vh, OUT, shape), O.reduce(x, dim, mean=bool(mean)),
                          x.astype(np.float64).mean(dim) if mean else x.astype(np.float64).sum(dim))
    # Column sums of a tall matrix (a bias gradient's reduce_to): the two-pass
    # row-group path, and the same sum with a leading 1 dim.
    y = r.normal(size=(3000, 70)).astype(np.float32)
    Y = dev(vh, y)
    for lay in ((3000, 70), (1, 3000, 70)):
        OUT = out(vh, (70,))
        dim = len(lay) - 2
        vh.check(vh.lib.vh_reduce(0, Y.ptr, vh.layout(lay), dim, OUT.ptr, None))
        assert_parity(fetch(vh, OUT, (70,)), O.reduce(y, 0), y.astype(np.float64).sum(0), name=f"col sum {lay}")
    # A transposed view [300, 6, 4] of the same buffer.
    dims, strides = (300, 6, 4), (1, 300, 1800)
    xt = np.transpose(x, (2, 1, 0))
    OUT = out(vh, xt.shape)
    vh.check(vh.lib.vh_strided_copy(X.ptr, vh.layout(dims, strides), OUT.ptr, None))
    np.testing.assert_array_equal(fetch(vh, OUT, xt.shape), np.ascontiguousarray(xt))
    OUT = out(vh, (300, 4))
    vh.check(vh.lib.vh_reduce(0, X.ptr, vh.layout(dims, strides), 1, OUT.ptr, None))
    np.testing.assert_array_equal(fetch(vh, OUT, (300, 4)), O.reduce(xt, 1))


def test_strided_copy_transposed_views(vh):
    """contiguous() of transposed views (a last dim with a stride, the one before
    it unit-stride; up to two leading dims) runs the LDS-tiled transpose:
    exact copies, edge tiles included."""
    r = rng(8)
    cases = [((777, 1000), None), ((3, 130, 67), (0, 2, 1)), ((3, 130, 67), (1, 0, 2)), ((2, 3, 65, 129), (0, 1, 3, 2)),
             ((64, 64), None), ((17, 5000), None),
             # 128-bit form (sizes and strides multiples of 4), edge tiles included
             ((768, 1024), None), ((68, 132), None), ((2, 3, 64, 132), (0, 1, 3, 2)), ((4, 36, 200), (0, 2, 1))]
    for shape, perm in cases:
        x = r.normal(size=shape).astype(np.float32)
        X = dev(vh, x)
        if perm is None:  # the 2-D transpose
            view = x.T
            dims, strides = view.shape, (1, shape[1])
        else:
            view = np.transpose(x, perm)
            cstr = [int(np.prod(shape[i + 1:])) for i in range(len(shape))]
            dims, strides = view.shape, tuple(cstr[p] for p in perm)
        OUT = out(vh, dims)
        vh.check(vh.lib.vh_strided_copy(X.ptr, vh.layout(dims, strides), OUT.ptr, None))
        np.testing.assert_array_equal(fetch(vh, OUT, dims), np.ascontiguousarray(view), err_msg=str(shape))


def test_arena_reuse_and_zeroing(vh):
    before = vh.mem_stats()
    bufs = [vh.DeviceBuffer(1 << 20, zero=True) for _ in range(4)]
    for b in bufs:
        assert not fetch(vh, b, (1 << 18,)).any()
        b.upload(np.ones(1 << 18, np.float32))
    for b in bufs:
        b.close()
    again = vh.DeviceBuffer(1 << 20, zero=True)
    assert not fetch(vh, again, (1 << 18,)).any()  # reused block comes back zeroed
    again.close()
    after = vh.mem_stats()
    assert after.live_bytes == before.live_bytes
    assert after.hip_bytes <= before.hip_bytes + 4 * (1 << 20)


@pytest.mark.parametrize("nbytes,soff,doff", [(16, 0, 0), (20, 0, 0), (4, 0, 0), (1_000_004, 0, 0),
                                              (64 * 2**20 + 12, 0, 0), (1000, 4, 0), (4096, 16, 32),
                                              (3 * 2**20, 8, 8)])
def test_device_copy_is_exact(vh, nbytes, soff, doff):
    """vh_d2d: 16-byte aligned copies through the library's streaming kernel
    (with the runtime's copy for a tail under 16 bytes), other alignments
    through the runtime's copy; bytes around the destination stay untouched."""
    r = np.random.default_rng(nbytes)
    src = r.integers(0, 256, size=nbytes + soff, dtype=np.uint8)
    guard = np.full(nbytes + doff + 64, 0xA5, np.uint8)
    S, D = vh.DeviceBuffer.from_array(src), vh.DeviceBuffer.from_array(guard)
    vh.check(vh.lib.vh_d2d(ctypes.c_void_p(D.ptr + doff), ctypes.c_void_p(S.ptr + soff), nbytes, None))
    vh.sync()
    got = D.to_array((guard.size,), np.uint8)
    assert got[doff:doff + nbytes].tobytes() == src[soff:].tobytes()
    assert (got[:doff] == 0xA5).all() and (got[doff + nbytes:] == 0xA5).all()
