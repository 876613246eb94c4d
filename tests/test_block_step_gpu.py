"""The config[4] training step (include/vearo_block.h) against the oracle's
SimpleGPT step and the float64 torch model (tests/golden):

* the golden small model: loss, every parameter gradient, and the loss after
  one AdamW step;
* a medium model (multi-tile GEMMs, S = 128 attention) against the oracle;
* determinism: two identical steps give identical bits;
* the reference's GPT overfitting run (verification_harness.rs:184-237) on the
  device.
"""
import math
import os

import numpy as np
import pytest

import oracle as O
from parity import assert_parity

pytestmark = pytest.mark.gpu
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
ADAM = dict(lr=0.02, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.01)


def make(vh, cfg_tuple):
    from vearo_amd import _block
    cfg = _block.GptConfig(*cfg_tuple)
    return _block, _block.Gpt(cfg), O.GptConfig(*cfg_tuple)


def check_grads(got, ref, ref64=None, tag=""):
    for i, name in enumerate(O.GPT_PARAM_NAMES):
        if name == "k_b":  # exact gradient 0 (softmax ignores a per-row shift)
            assert np.abs(got[i]).max() < 1e-6, (tag, name)
            continue
        scale = np.abs(ref[i]).max()
        err = np.abs(got[i] - ref[i]).max()
        assert err <= 1e-4 * scale + 1e-9, (tag, name, err, scale)
        assert_parity(got[i], ref[i], None if ref64 is None else ref64[i], name=f"{tag} {name}")


def test_block_step_golden_model(vh):
    B, S, D, H, F, V, P = (int(x) for x in GOLD["gpt_cfg"])
    _b, g, ocfg = make(vh, (B, S, D, H, F, V, P))
    params = [GOLD[f"gpt_p{i}"] for i in range(21)]
    ids, tg = GOLD["gpt_ids"], GOLD["gpt_targets"]
    g.set_params(params)
    g.set_inputs(ids, tg)
    g.forward_backward(True)
    loss = g.loss()
    oloss, ograds = O.gpt_step(ocfg, params, ids, tg)
    assert abs(loss - oloss) <= 1e-5 + 1e-4 * abs(oloss), (loss, oloss)
    assert abs(loss - GOLD["gpt_loss"]) <= 1e-4 * GOLD["gpt_loss"]
    check_grads(g.grads(), ograds, [GOLD[f"gpt_g{i}"] for i in range(21)], "golden")
    g.adamw(**ADAM)
    g.forward_backward(False)
    loss1 = g.loss()
    assert abs(loss1 - GOLD["gpt_loss1"]) <= 1e-4 * GOLD["gpt_loss1"], (loss1, GOLD["gpt_loss1"])
    # The oracle's own step-1 loss from the same update.
    ps = [p.copy() for p in params]
    for p, gr in zip(ps, ograds):
        O.adamw_step(p, gr, np.zeros_like(p), np.zeros_like(p), 1, 0.02, 0.9, 0.95, 1e-8, 0.01)
    oloss1, _ = O.gpt_step(ocfg, ps, ids, tg, grads=False)
    assert abs(loss1 - oloss1) <= 1e-5 + 1e-4 * abs(oloss1), (loss1, oloss1)
    assert_parity(g.params()[20], ps[20], name="lm_w after AdamW")
    g.close()


def random_model(cfg_tuple, seed):
    B, S, D, H, F, V, P = cfg_tuple
    r = np.random.default_rng(seed)
    params = []
    for name, sh in zip(O.GPT_PARAM_NAMES, O.gpt_param_shapes(O.GptConfig(*cfg_tuple))):
        if name.startswith("ln") and name.endswith("_w"):
            params.append(np.ones(sh, np.float32))
        elif name.startswith("ln"):
            params.append(np.zeros(sh, np.float32))
        else:
            params.append((r.standard_normal(sh) * 0.02).astype(np.float32))
    ids = r.integers(0, V, size=(B, S)).astype(np.float32)
    tg = r.integers(0, V, size=(B, S)).astype(np.float32)
    return params, ids, tg


def test_block_step_medium_model(vh):
    cfg = (2, 128, 128, 4, 512, 1000, 128)
    print("block step medium", flush=True)
    _b, g, ocfg = make(vh, cfg)
    params, ids, tg = random_model(cfg, 11)
    g.set_params(params)
    g.set_inputs(ids, tg)
    g.forward_backward(True)
    loss = g.loss()
    oloss, ograds = O.gpt_step(ocfg, params, ids, tg)
    assert abs(loss - oloss) <= 1e-5 + 1e-4 * abs(oloss), (loss, oloss)
    assert abs(loss - math.log(1000)) < 0.05  # near-uniform logits at init
    grads = g.grads()
    check_grads(grads, ograds, tag="medium")
    # Determinism: the same step again gives the same bits.
    g.forward_backward(True)
    assert g.loss() == loss
    for a, b in zip(g.grads(), grads):
        np.testing.assert_array_equal(a, b)
    g.close()


def test_block_step_overfits_like_the_reference_test(vh):
    """verification_harness.rs:184-237 on the device: SimpleGPT(vocab 8, seq 4,
    n_embd 8, 2 heads, 1 layer, mlp 16), AdamW(0.02, 0.9, 0.95, 1e-8, 0.01),
    150 steps bring the loss under 0.05; the oracle runs the same 150 steps and
    the two loss curves agree."""
    cfg = (2, 4, 8, 2, 16, 8, 4)
    _b, g, ocfg = make(vh, cfg)
    r = np.random.default_rng(42)
    params = []
    for name, sh in zip(O.GPT_PARAM_NAMES, O.gpt_param_shapes(ocfg)):
        if name.startswith("ln") and name.endswith("_w"):
            params.append(np.ones(sh, np.float32))
        elif name.startswith("ln"):
            params.append(np.zeros(sh, np.float32))
        else:
            fan = sh[1] if len(sh) == 2 else (cfg[2] if name != "fc2_b" else cfg[4])
            bound = 1.0 / math.sqrt(fan)
            params.append(r.uniform(-bound, bound, size=sh).astype(np.float32))
    ids = np.array([[0, 1, 2, 3], [1, 2, 3, 0]], np.float32)
    tg = np.array([[1, 2, 3, 0], [2, 3, 0, 1]], np.float32)
    g.set_params(params)
    g.set_inputs(ids, tg)
    ps = [p.copy() for p in params]
    ms = [np.zeros_like(p) for p in ps]
    vs = [np.zeros_like(p) for p in ps]
    for t in range(1, 151):
        g.forward_backward(True)
        loss = g.loss()
        oloss, ograds = O.gpt_step(ocfg, ps, ids, tg)
        for p, gr, m, v in zip(ps, ograds, ms, vs):
            O.adamw_step(p, gr, m, v, t, 0.02, 0.9, 0.95, 1e-8, 0.01)
        if t <= 10:
            assert abs(loss - oloss) <= 1e-4 * max(1.0, abs(oloss)), (t, loss, oloss)
        g.adamw(**ADAM)
    assert loss < 0.05, loss
    g.close()
