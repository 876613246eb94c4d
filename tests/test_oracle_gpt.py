"""Pins the oracle's second part (matmul, fused attention, AdamW, the SimpleGPT
step) before it is trusted as the GPU checker.

* Known answers from the reference's own tests: matmul 2-D and batched
  (cpu:2656-2672, 2730-2762), the transposed-rhs case (cuda:1676-1699), the
  fused-vs-unfused attention parity inputs and bounds
  (crates/vearo/tests/fused_attention_parity.rs), the GPT overfitting run
  (crates/vearo/tests/verification_harness.rs:184-237).
* Float64 torch references (tests/golden/golden.npz, gen_golden.py): matmul
  with broadcast batches, attention fwd/bwd with causal, dense-random and no
  mask, and a whole one-block SimpleGPT step -- loss, every parameter's
  gradient, and the loss after one AdamW step.
* Exact identities: integer matmuls are exact; the AVX2 fused-multiply-add
  block and the scalar fmaf chain give bit-identical elements; AdamW's first
  step has a closed form; the unfused attention equals its chain of single
  oracle ops bit for bit.
"""
import math
import os

import numpy as np
import pytest

import oracle as O

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))


def test_matmul_reference_kats():
    x = np.array([[1, 2], [3, 4]], np.float32)
    y = np.array([[5, 6], [7, 8]], np.float32)
    assert O.matmul(x, y).tolist() == [[19, 22], [43, 50]]
    xb = np.arange(1, 13, dtype=np.float32).reshape(2, 2, 3)
    yb = np.arange(1, 13, dtype=np.float32).reshape(2, 3, 2)
    assert O.matmul(xb, yb).reshape(-1).tolist() == [22, 28, 49, 64, 220, 244, 301, 334]
    a = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    b = np.arange(7, 13, dtype=np.float32).reshape(2, 3)
    assert O.matmul(a, b.T).tolist() == (a.astype(np.int64) @ b.T.astype(np.int64)).tolist()


def test_matmul_golden():
    for tag in ("mm2", "mm3", "mmb"):
        got = O.matmul(GOLD[f"{tag}_a"], GOLD[f"{tag}_b"])
        np.testing.assert_allclose(got, GOLD[f"{tag}_out"], rtol=1e-5, atol=1e-5, err_msg=tag)


def test_matmul_integers_exact():
    r = np.random.default_rng(1)
    a = r.integers(-8, 9, size=(3, 37, 61)).astype(np.float32)
    b = r.integers(-8, 9, size=(61, 45)).astype(np.float32)
    np.testing.assert_array_equal(O.matmul(a, b), (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))


def test_matmul_blocked_path_is_the_scalar_chain():
    # Rows 0-4 of a 6-row product run through the AVX2 6x16 block; a 5-row
    # product runs them through the scalar fmaf loop. Same chain, same bits.
    r = np.random.default_rng(2)
    a = r.standard_normal((6, 700), dtype=np.float32)
    b = r.standard_normal((700, 33), dtype=np.float32)
    full = O.matmul(a, b)
    np.testing.assert_array_equal(full[:5], O.matmul(a[:5], b))
    np.testing.assert_array_equal(full[:, :16], O.matmul(a, b[:, :16]))
    np.testing.assert_array_equal(full[:, :15], O.matmul(a, np.ascontiguousarray(b[:, :15])))


def test_matmul_thread_count_does_not_change_bits():
    r = np.random.default_rng(3)
    a = r.standard_normal((200, 300), dtype=np.float32)
    b = r.standard_normal((300, 260), dtype=np.float32)
    O.set_threads(1)
    one = O.matmul(a, b)
    O.set_threads(7)
    seven = O.matmul(a, b)
    O.set_threads(0)
    np.testing.assert_array_equal(one, seven)


@pytest.mark.parametrize("tag", ["attkat", "attc", "attm", "attn"])
def test_attention_golden(tag):
    q, k, v, go = (GOLD[f"{tag}_{n}"] for n in ("q", "k", "v", "go"))
    mask = GOLD[f"{tag}_mask"] if f"{tag}_mask" in GOLD.files else None
    out = O.fused_attention(q, k, v, mask)
    np.testing.assert_allclose(out, GOLD[f"{tag}_out"], rtol=1e-4, atol=1e-5)
    dq, dk, dv = O.fused_attention_backward(q, k, v, mask, go)
    for name, g in (("dq", dq), ("dk", dk), ("dv", dv)):
        ref = GOLD[f"{tag}_{name}"]
        np.testing.assert_allclose(g, ref, rtol=1e-4, atol=1e-5 * max(1.0, np.abs(ref).max()),
                                   err_msg=f"{tag} {name}")


def test_attention_fused_matches_unfused_composite():
    """fused_attention_parity.rs: the fused op against the unfused chain of
    backend ops and autograd arms (matmul, mul by scale, add mask, softmax,
    matmul), with the test's own bounds."""
    q, k, v, go, mask = (GOLD[f"attkat_{n}"] for n in ("q", "k", "v", "go", "mask"))
    scale = np.float32([1.0 / math.sqrt(q.shape[-1])])
    kt = np.ascontiguousarray(np.swapaxes(k, 2, 3))
    s_mm = O.matmul(q, kt)
    s_scaled = O.binary(2, s_mm, scale)
    scores = O.binary(0, s_scaled, mask)
    p = O.softmax(scores, 3)
    out_ref = O.matmul(p, v)
    out_fused = O.fused_attention(q, k, v, mask)
    assert np.abs(out_ref).max() > 1e-4
    assert np.abs(out_ref - out_fused).max() < 1e-5
    # Autograd arms of the unfused chain (autograd:481-519, 547-553).
    dp = O.matmul(go, np.ascontiguousarray(np.swapaxes(v, 2, 3)))
    dv_ref = O.matmul(np.ascontiguousarray(np.swapaxes(p, 2, 3)), go)
    ds = O.softmax_backward_composite(scores, dp, 3)
    dqk = O.binary(2, ds, scale)
    dq_ref = O.matmul(dqk, k)
    dk_ref = np.swapaxes(O.matmul(np.ascontiguousarray(np.swapaxes(q, 2, 3)), dqk), 2, 3)
    dq, dk, dv = O.fused_attention_backward(q, k, v, mask, go)
    assert np.abs(dq - dq_ref).max() < 1e-4
    assert np.abs(dk - dk_ref).max() < 1e-4
    assert np.abs(dv - dv_ref).max() < 1e-4


def _unfused_chain(q, k, v, mask, go):
    """MultiHeadAttention's unfused path (nn:603-613) and its tape's arms,
    spelled out with the oracle's single ops (as the fused parity test does)."""
    scale = np.float32([1.0 / math.sqrt(q.shape[-1])])
    s_scaled = O.binary(2, O.matmul(q, np.ascontiguousarray(np.swapaxes(k, 2, 3))), scale)
    scores = O.binary(0, s_scaled, mask) if mask is not None else s_scaled
    p = O.softmax(scores, 3)
    out = O.matmul(p, v)
    dp = O.matmul(go, np.ascontiguousarray(np.swapaxes(v, 2, 3)))
    dv = O.matmul(np.ascontiguousarray(np.swapaxes(p, 2, 3)), go)
    dqk = O.binary(2, O.softmax_backward_composite(scores, dp, 3), scale)
    dq = O.matmul(dqk, k)
    dk = np.swapaxes(O.matmul(np.ascontiguousarray(np.swapaxes(q, 2, 3)), dqk), 2, 3)
    return out, dq, dk, dv


@pytest.mark.parametrize("tag", ["attkat", "attc", "attm", "attn"])
def test_attention_unfused_is_the_op_chain(tag):
    """vo_attention_unfused(_backward) run exactly the single ops of the chain
    (same bits), and land on the float64 torch attention within the bar."""
    q, k, v, go = (GOLD[f"{tag}_{n}"] for n in ("q", "k", "v", "go"))
    mask = GOLD[f"{tag}_mask"] if f"{tag}_mask" in GOLD.files else None
    out = O.attention_unfused(q, k, v, mask)
    dq, dk, dv = O.attention_unfused_backward(q, k, v, mask, go)
    ref = _unfused_chain(q, k, v, mask, go)
    for name, got, want in zip(("out", "dq", "dk", "dv"), (out, dq, dk, dv), ref):
        np.testing.assert_array_equal(got, want, err_msg=f"{tag} {name}")
    if tag != "attkat":
        for name, got in (("out", out), ("dq", dq), ("dk", dk), ("dv", dv)):
            g = GOLD[f"{tag}_{name}"]
            np.testing.assert_allclose(got, g, rtol=1e-4, atol=1e-5 * max(1.0, np.abs(g).max()),
                                       err_msg=f"{tag} {name} vs float64")


def test_attention_rows_are_convex_combinations():
    # With v = identity-like one-hot rows, out rows are the probability rows:
    # non-negative, summing to 1, zero above the diagonal under the causal mask.
    S = 12
    r = np.random.default_rng(4)
    q = r.standard_normal((1, 1, S, S), dtype=np.float32)
    k = r.standard_normal((1, 1, S, S), dtype=np.float32)
    v = np.eye(S, dtype=np.float32).reshape(1, 1, S, S)
    m = np.zeros((S, S), np.float32)
    m[np.triu_indices(S, 1)] = -1e9
    p = O.fused_attention(q, k, v, m)[0, 0]
    assert np.all(p >= 0)
    np.testing.assert_allclose(p.sum(axis=1), 1.0, atol=1e-6)
    assert np.all(p[np.triu_indices(S, 1)] == 0.0)
    assert p[0, 0] == 1.0


def test_adamw_first_step_closed_form():
    r = np.random.default_rng(5)
    p0 = r.standard_normal(1000).astype(np.float32)
    g = (r.standard_normal(1000) * 0.1).astype(np.float32)
    g[:10] = 0.0
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    lr, b1, b2, eps, wd = 0.02, 0.9, 0.95, 1e-8, 0.01
    O.adamw_step(p, g, m, v, 1, lr, b1, b2, eps, wd)
    p64, g64 = p0.astype(np.float64), g.astype(np.float64)
    # t = 1: m_hat = g, v_hat = g^2 (up to f32 rounding of the moments).
    exp = p64 - lr * wd * p64 - lr * g64 / (np.abs(g64) + eps)
    np.testing.assert_allclose(p, exp, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(m, 0.1 * g64, rtol=1e-6)
    np.testing.assert_allclose(v, 0.05 * g64 * g64, rtol=1e-5)
    # Zero gradient: only the decoupled decay acts, p * (1 - lr*wd) in two steps.
    np.testing.assert_array_equal(p[:10], p0[:10] - np.float32(lr * wd) * p0[:10])
    # t = 2 against the float64 recurrence.
    g2 = (r.standard_normal(1000) * 0.1).astype(np.float32)
    O.adamw_step(p, g2, m, v, 2, lr, b1, b2, eps, wd)
    m64 = 0.9 * (0.1 * g64) + 0.1 * g2
    v64 = 0.95 * (0.05 * g64 * g64) + 0.05 * g2.astype(np.float64) ** 2
    np.testing.assert_allclose(m, m64, rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(v, v64, rtol=1e-4, atol=1e-12)


def _gpt_from_gold(tag):
    B, S, D, H, F, V, P = (int(x) for x in GOLD[f"{tag}_cfg"])
    cfg = O.GptConfig(B, S, D, H, F, V, P)
    params = [GOLD[f"{tag}_p{i}"].copy() for i in range(len(O.GPT_PARAM_NAMES))]
    return cfg, params, GOLD[f"{tag}_ids"], GOLD[f"{tag}_targets"]


def test_gpt_step_matches_float64_model():
    cfg, params, ids, tg = _gpt_from_gold("gpt")
    loss, grads = O.gpt_step(cfg, params, ids, tg)
    assert abs(loss - GOLD["gpt_loss"]) <= 1e-5 * abs(GOLD["gpt_loss"])
    for i, name in enumerate(O.GPT_PARAM_NAMES):
        ref = GOLD[f"gpt_g{i}"]
        if name == "k_b":
            # Adding a constant to every key shifts each score row by q.b, which
            # softmax ignores: the exact gradient is 0, f32 leaves rounding noise.
            assert np.abs(ref).max() < 1e-12 and np.abs(grads[i]).max() < 1e-6
            continue
        err = np.abs(grads[i] - ref).max() / np.abs(ref).max()
        assert err < 1e-4, (name, err)
    # One AdamW step on every parameter, then the loss again.
    for p, g in zip(params, grads):
        m, v = np.zeros_like(p), np.zeros_like(p)
        O.adamw_step(p, g, m, v, 1, 0.02, 0.9, 0.95, 1e-8, 0.01)
    loss1, _ = O.gpt_step(cfg, params, ids, tg, grads=False)
    assert abs(loss1 - GOLD["gpt_loss1"]) <= 1e-4 * abs(GOLD["gpt_loss1"]), (loss1, GOLD["gpt_loss1"])
    assert loss1 < loss


def test_gpt_step_unfused_attention_matches_float64_model():
    """The step with VEARO_USE_FUSED_ATTENTION=0's path: the same float64
    model (the two attention forms are the same mathematics), loss and every
    gradient to the same bar as the fused step, and close to the fused step."""
    cfg, params, ids, tg = _gpt_from_gold("gpt")
    loss, grads = O.gpt_step(cfg, params, ids, tg, fused_attention=False)
    floss, fgrads = O.gpt_step(cfg, params, ids, tg)
    assert abs(loss - GOLD["gpt_loss"]) <= 1e-5 * abs(GOLD["gpt_loss"])
    assert abs(loss - floss) <= 1e-5 * abs(floss)
    for i, name in enumerate(O.GPT_PARAM_NAMES):
        ref = GOLD[f"gpt_g{i}"]
        if name == "k_b":
            assert np.abs(grads[i]).max() < 1e-6
            continue
        assert np.abs(grads[i] - ref).max() / np.abs(ref).max() < 1e-4, name
        assert np.abs(grads[i] - fgrads[i]).max() / np.abs(ref).max() < 1e-4, name


def test_gpt_overfits_like_the_reference_test():
    """verification_harness.rs:184-237: SimpleGPT(vocab 8, seq 4, n_embd 8,
    2 heads, 1 layer, mlp 16), AdamW(0.02, 0.9, 0.95, 1e-8, 0.01), 150 steps
    must bring the loss under 0.05. Module init as nn:86-97 and nn:478-486
    (uniform in +-1/sqrt(fan_in)), from this test's own generator."""
    cfg = O.GptConfig(2, 4, 8, 2, 16, 8, 4)
    r = np.random.default_rng(42)
    params = []
    for i, sh in enumerate(O.gpt_param_shapes(cfg)):
        name = O.GPT_PARAM_NAMES[i]
        if name.startswith("ln") and name.endswith("_w"):
            params.append(np.ones(sh, np.float32))
        elif name.startswith("ln"):
            params.append(np.zeros(sh, np.float32))
        else:
            fan_in = sh[-1] if name.endswith("_w") and name not in ("wte", "wpe") else None
            if name in ("wte", "wpe"):
                bound = 1.0 / math.sqrt(sh[1])
            elif name.endswith("_b"):
                bound = 1.0 / math.sqrt(cfg.D if name != "fc2_b" else cfg.F)
            else:
                bound = 1.0 / math.sqrt(fan_in)
            params.append(r.uniform(-bound, bound, size=sh).astype(np.float32))
    ids = np.array([[0, 1, 2, 3], [1, 2, 3, 0]], np.float32)
    tg = np.array([[1, 2, 3, 0], [2, 3, 0, 1]], np.float32)
    ms = [np.zeros_like(p) for p in params]
    vs = [np.zeros_like(p) for p in params]
    loss = None
    for t in range(1, 151):
        loss, grads = O.gpt_step(cfg, params, ids, tg)
        for p, g, m, v in zip(params, grads, ms, vs):
            O.adamw_step(p, g, m, v, t, 0.02, 0.9, 0.95, 1e-8, 0.01)
    assert loss < 0.05, loss
