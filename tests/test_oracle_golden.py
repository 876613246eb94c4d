"""Pins the CPU oracle (oracle/vearo_cpu_ref.c) before it is trusted as the
parity reference: against float64 torch golden vectors (tests/golden/), the
reference's own known-answer tests, its panic messages, and invariants the
mathematics fixes. CPU only."""
import math

import numpy as np
import pytest

import oracle as O


def close(a, b, rtol=1e-5, atol=1e-6):
    np.testing.assert_allclose(np.asarray(a, np.float64), np.asarray(b, np.float64), rtol=rtol, atol=atol)


# ------------------------------------------------------------------ layernorm
@pytest.mark.parametrize("tag", ["ln", "ln3d", "lnkat"])
def test_layernorm_matches_torch_f64(golden, tag):
    g = lambda k: golden[f"{tag}_{k}"]
    eps = float(g("eps"))
    y = O.layernorm(g("x"), g("w"), g("b"), eps)
    close(y, g("y"), rtol=1e-5, atol=2e-6)
    dx, dw, db = O.layernorm_backward(g("x"), g("w"), g("b"), g("dy"), eps)
    close(dx, g("dx"), rtol=1e-4, atol=2e-5)
    close(dw, g("dw"), rtol=1e-5, atol=2e-5)
    close(db, g("db"), rtol=1e-5, atol=2e-5)


def test_layernorm_invariants():
    rng = np.random.default_rng(1)
    x = rng.normal(size=(64, 96)).astype(np.float32) * 4 + 2
    w = (1 + 0.1 * rng.normal(size=96)).astype(np.float32)
    b = (0.1 * rng.normal(size=96)).astype(np.float32)
    dy = rng.normal(size=(64, 96)).astype(np.float32)
    y = O.layernorm(x, w, b, 1e-5)
    xhat = (y - b) / w
    close(xhat.mean(axis=1), 0.0, atol=1e-5)
    dx, dw, db = O.layernorm_backward(x, w, b, dy, 1e-5)
    close(dx.sum(axis=1), 0.0, atol=1e-4)          # d/dx of a normalised row sums to 0
    close(db, dy.astype(np.float64).sum(axis=0), rtol=1e-5, atol=1e-5)
    close(dw, (dy.astype(np.float64) * xhat).sum(axis=0), rtol=1e-4, atol=1e-4)


def test_layernorm_noncontiguous_and_empty():
    # cpu lib.rs:2847-2864: empty input keeps its shape; a transposed input works.
    w4, b4 = np.ones(4, np.float32), np.zeros(4, np.float32)
    assert O.layernorm(np.zeros((2, 0, 4), np.float32), w4, b4, 1e-5).shape == (2, 0, 4)
    x = np.arange(1, 9, dtype=np.float32).reshape(2, 4)
    xt = x.T  # [4, 2] strided view
    w2, b2 = np.ones(2, np.float32), np.zeros(2, np.float32)
    out = O.layernorm(xt, w2, b2, 1e-5)
    assert out.shape == (4, 2)
    np.testing.assert_array_equal(out, O.layernorm(np.ascontiguousarray(xt), w2, b2, 1e-5))


def test_layernorm_shape_panics():
    x = np.zeros((2, 3), np.float32)
    with pytest.raises(O.Panic, match="Weight dimension must match norm_dim"):
        O.layernorm(x, np.ones(4, np.float32), np.zeros(3, np.float32), 1e-5)
    with pytest.raises(O.Panic, match="LayerNorm weight must be rank 1"):
        O.layernorm(x, np.ones((1, 3), np.float32), np.zeros(3, np.float32), 1e-5)


# ----------------------------------------------------------------------- gelu
def test_gelu_matches_torch_tanh_gelu(golden):
    x = golden["gelu_x"]
    close(O.gelu(x), golden["gelu_y"], rtol=1e-5, atol=1e-6)
    close(O.gelu_grad_mask(x), golden["gelu_mask"], rtol=1e-5, atol=1e-6)


def test_gelu_special_values():
    assert O.gelu(np.float32([0.0]))[0] == 0.0
    assert O.gelu_grad_mask(np.float32([0.0]))[0] == 0.5
    big = O.gelu(np.float32([-20.0, 20.0]))
    assert big[0] == 0.0 or abs(big[0]) < 1e-30
    assert big[1] == np.float32(20.0)


def test_gelu_bias_composite(golden):
    y = O.gelu_bias_forward(golden["gb_x"], golden["gb_bias"])
    close(y, golden["gb_y"], rtol=1e-5, atol=1e-6)
    dx, db = O.gelu_bias_backward(golden["gb_x"], golden["gb_bias"], golden["gb_dy"])
    close(dx, golden["gb_dx"], rtol=1e-5, atol=1e-6)
    close(db, golden["gb_dbias"], rtol=1e-5, atol=1e-5)
    # The fused composite is exactly add -> gelu, and mask -> mul -> reduce_to.
    h = O.binary(0, golden["gb_x"], golden["gb_bias"])
    np.testing.assert_array_equal(y, O.gelu(h))
    g = O.binary(2, golden["gb_dy"], O.gelu_grad_mask(h))
    np.testing.assert_array_equal(dx, g)
    np.testing.assert_array_equal(db, O.reduce_to(g, [g.shape[1]]))


def test_gelu_noncontiguous():
    x = np.arange(-6, 6, dtype=np.float32).reshape(3, 4) * 0.5
    np.testing.assert_array_equal(O.gelu(x.T), O.gelu(np.ascontiguousarray(x.T)))


# -------------------------------------------------------------------- softmax
@pytest.mark.parametrize("tag", ["sm", "sm0", "smc", "smkat"])
def test_softmax_matches_torch(golden, tag):
    g = lambda k: golden[f"{tag}_{k}"]
    dim = int(g("dim"))
    y = O.softmax(g("x"), dim)
    close(y, g("y"), rtol=1e-5, atol=1e-7)
    dx = O.softmax_backward_composite(g("x"), g("dy"), dim)
    close(dx, g("dx"), rtol=1e-4, atol=1e-6)


def test_softmax_invariants(golden):
    x = golden["sm_x"]
    y = O.softmax(x, 1)
    close(y.sum(axis=1), 1.0, atol=1e-6)
    np.testing.assert_allclose(O.softmax(x + np.float32(3.0), 1), y, rtol=2e-6, atol=1e-7)
    yc = O.softmax(golden["smc_x"], 2)
    iu = np.triu_indices(8, 1)
    assert np.all(yc[:, iu[0], iu[1]] == 0.0)  # masked entries are exactly zero
    dx = O.softmax_backward_composite(x, golden["sm_dy"], 1)
    close(dx.sum(axis=1), 0.0, atol=1e-5)


def test_softmax_strided_axes():
    x = np.float32([[-2, -1, 0.5, 1], [2, 3, -0.5, 4], [-3, 0, 1.5, -1.5]])
    for d in (0, 1):
        np.testing.assert_array_equal(O.softmax(x.T, d), O.softmax(np.ascontiguousarray(x.T), d))
    with pytest.raises(O.Panic, match="Softmax dim out of range"):
        O.softmax(x, 2)


# ------------------------------------------------------------------ embedding
def test_embedding_matches_torch(golden):
    out = O.embedding(golden["emb_ids"], golden["emb_W"])
    np.testing.assert_array_equal(out, golden["emb_out"].astype(np.float32))  # a pure copy
    W = golden["emb_W"]
    for (i, j), t in np.ndenumerate(golden["emb_tok"]):
        np.testing.assert_array_equal(out[i, j], W[t])  # round half away from zero
    dW = O.embedding_backward(golden["emb_ids"], W.shape, golden["emb_dy"])
    close(dW, golden["emb_dW"], rtol=1e-6, atol=1e-6)
    close(dW.sum(axis=0), golden["emb_dy"].astype(np.float64).sum(axis=(0, 1)), atol=1e-5)


def test_embedding_kat(golden):
    out = O.embedding(golden["embkat_ids"], golden["embkat_W"])
    np.testing.assert_array_equal(out, golden["embkat_out"])
    dW = O.embedding_backward(golden["embkat_ids"], (2, 3), np.ones((2, 3), np.float32))
    np.testing.assert_array_equal(dW, golden["embkat_dW"])


def test_embedding_backward_sequential_order():
    # dW[t] accumulates dy rows in ascending position order, starting from 0.0.
    ids = np.float32([1, 0, 1, 1])
    dy = np.float32([[1e8], [5], [1], [-1e8]])
    dW = O.embedding_backward(ids, (2, 1), dy)
    expect = np.float32(np.float32(np.float32(np.float32(0) + np.float32(1e8)) + np.float32(1)) - np.float32(1e8))
    assert dW[1, 0] == expect and dW[0, 0] == 5.0


def test_embedding_panics():
    W = np.zeros((2, 3), np.float32)
    with pytest.raises(O.Panic, match=r"^Token ID cannot be negative: -1$"):
        O.embedding(np.float32([-1.0, 0.0]), W)  # cpu lib.rs:2866-2872
    with pytest.raises(O.Panic, match=r"^Token ID 2 out of vocabulary bound 2$"):
        O.embedding(np.float32([2.0, 0.0]), W)   # cpu lib.rs:2874-2880
    with pytest.raises(O.Panic, match=r"^Token ID cannot be negative: NaN$"):
        O.embedding(np.float32([np.nan]), W)
    with pytest.raises(O.Panic, match=r"^Token ID 2 out of vocabulary bound 2$"):
        O.embedding_backward(np.float32([1.5]), (2, 3), np.zeros((1, 3), np.float32))
    with pytest.raises(O.Panic, match="grad_out shape must be"):
        O.embedding_backward(np.float32([1.0]), (2, 3), np.zeros((1, 2), np.float32))


# -------------------------------------------------------------- cross-entropy
@pytest.mark.parametrize("tag", ["ce", "cekat", "cestab", "ceuni"])
def test_cross_entropy_matches_torch(golden, tag):
    g = lambda k: golden[f"{tag}_{k}"]
    loss = O.cross_entropy(g("logits"), g("targets"))
    close(loss, g("loss"), rtol=2e-6, atol=1e-6)
    dl = O.cross_entropy_backward(g("logits"), g("targets"), g("go"))
    close(dl, g("dl"), rtol=1e-5, atol=1e-7)
    close(dl.sum(axis=1), 0.0, atol=1e-6)


def test_cross_entropy_kats(golden):
    assert abs(O.cross_entropy(golden["cestab_logits"], golden["cestab_targets"])[0]) < 1e-4
    # Uniform logits: a single row gives exactly ln(V) in f32; three rows are
    # within the rounding of the sequential sum and the division by B.
    one = O.cross_entropy(golden["ceuni_logits"][:1], golden["ceuni_targets"][:1])[0]
    assert one == np.float32(math.log(50))
    three = O.cross_entropy(golden["ceuni_logits"], golden["ceuni_targets"])[0]
    assert abs(float(three) - math.log(50)) <= 4 * np.spacing(np.float32(4.0))


def test_cross_entropy_panics():
    logits = np.zeros((2, 3), np.float32)
    with pytest.raises(O.Panic, match=r"^Target class cannot be negative: -1$"):
        O.cross_entropy(logits, np.float32([-1.0, 0.0]))  # cpu lib.rs:2884-2890
    with pytest.raises(O.Panic, match=r"^Target class 3 out of vocab bounds 3$"):
        O.cross_entropy(logits, np.float32([3.0, 0.0]))  # cpu lib.rs:2892-2898
    with pytest.raises(O.Panic, match="grad_out must be a scalar"):
        O.cross_entropy_backward(logits, np.float32([0, 1]), np.float32([1, 1]))
    with pytest.raises(O.Panic, match="Batch size must be greater than 0"):
        O.cross_entropy(np.zeros((0, 3), np.float32), np.zeros(0, np.float32))


def test_cross_entropy_noncontiguous():
    base = np.float32([[1, 4], [2, 5], [3, 6]])
    tgt = np.float32([0, 2])
    np.testing.assert_array_equal(O.cross_entropy(base.T, tgt),
                                  O.cross_entropy(np.ascontiguousarray(base.T), tgt))


# ------------------------------------------------------- reductions / binary
def test_reductions_match_numpy(golden):
    x = golden["red_x"]
    for d in range(3):
        close(O.reduce(x, d), golden[f"red_sum{d}"], rtol=1e-6, atol=1e-6)
        close(O.reduce(x, d, mean=True), golden[f"red_mean{d}"], rtol=1e-6, atol=1e-6)
        assert O.reduce(x, d, keep_dim=True).shape[d] == 1


def test_reduction_kats():
    x = np.float32([[1, 2, 3], [4, 5, 6]])  # cpu lib.rs:2798-2830
    np.testing.assert_array_equal(O.reduce(x, 1), [6, 15])
    np.testing.assert_array_equal(O.reduce(x, 0), [5, 7, 9])
    np.testing.assert_array_equal(O.reduce(x, 1, mean=True), [2, 5])
    np.testing.assert_array_equal(O.reduce(x, 0, mean=True), [2.5, 3.5, 4.5])
    np.testing.assert_array_equal(O.reduce(x.T, 1), [5, 7, 9])


def test_binary_broadcast(golden):
    a, b = golden["bin_a"], golden["bin_b"]
    for op, key in enumerate(["add", "sub", "mul", "div"]):
        close(O.binary(op, a, b), golden[f"bin_{key}"], rtol=1e-6, atol=1e-7)
    with pytest.raises(O.Panic, match="Shapes are not broadcastable"):
        O.binary(0, np.zeros((2, 3), np.float32), np.zeros((4,), np.float32))


def test_reduce_to():
    g = np.arange(12, dtype=np.float32).reshape(4, 3)
    np.testing.assert_array_equal(O.reduce_to(g, [3]), g.sum(axis=0))
    np.testing.assert_array_equal(O.reduce_to(g, [4, 1]), g.sum(axis=1, keepdims=True))
    np.testing.assert_array_equal(O.reduce_to(g, [1, 3]), g.sum(axis=0, keepdims=True))
    np.testing.assert_array_equal(O.reduce_to(g, [4, 3]), g)


def test_format_f32_matches_rust_display():
    cases = {-1.0: "-1", 2.5: "2.5", -0.5: "-0.5", 0.1: "0.1", 1e20: "100000000000000000000",
             -3.25e-5: "-0.0000325", float("nan"): "NaN", float("-inf"): "-inf", 123456.0: "123456"}
    for v, s in cases.items():
        assert O.format_f32(v) == s, (v, O.format_f32(v), s)
