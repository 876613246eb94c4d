"""The config[4] step issued op by op through the BackendOps mirror
(vb_dropin_*, include/vearo_block.h): the tape SimpleGPT::forward records
(crates/vearo-nn/src/lib.rs:584-621, 666-675, 745-791; the attention on its
fused path or, as with VEARO_USE_FUSED_ATTENTION=0, its unfused one), walked in reverse
through backward_impl's arms (crates/vearo-autograd/src/lib.rs:429-792), then
AdamW::step (crates/vearo-optim/src/lib.rs:105-123). Against the oracle's
SimpleGPT step and the golden float64 torch model: the loss, every parameter
gradient and the loss after one AdamW step; against the fused vb_gpt driver on
the same model; and the reference's GPT overfitting run
(crates/vearo/tests/verification_harness.rs:184-237) through the drop-in path.
"""
import math
import os

import numpy as np
import pytest

import oracle as O
from parity import assert_parity
from test_block_step_gpu import check_grads, random_model

pytestmark = pytest.mark.gpu
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))


def dropin(cfg_tuple):
    from vearo_amd import _block
    return _block.DropIn(_block.GptConfig(*cfg_tuple))


def adam_ref(params, grads, t=1, ms=None, vs=None):
    ps = [p.copy() for p in params]
    ms = ms or [np.zeros_like(p) for p in ps]
    vs = vs or [np.zeros_like(p) for p in ps]
    for p, gr, m, v in zip(ps, grads, ms, vs):
        O.adamw_step(p, gr, m, v, t, 0.02, 0.9, 0.95, 1e-8, 0.01)
    return ps


def test_dropin_golden_model(vh):
    cfg = tuple(int(x) for x in GOLD["gpt_cfg"])
    d = dropin(cfg)
    params = [GOLD[f"gpt_p{i}"] for i in range(21)]
    ids, tg = GOLD["gpt_ids"], GOLD["gpt_targets"]
    d.set_params(params)
    d.set_inputs(ids, tg)
    loss = d.step(backward=True)
    oloss, ograds = O.gpt_step(O.GptConfig(*cfg), params, ids, tg)
    assert abs(loss - oloss) <= 1e-5 + 1e-4 * abs(oloss), (loss, oloss)
    assert abs(loss - GOLD["gpt_loss"]) <= 1e-4 * GOLD["gpt_loss"]
    check_grads(d.grads(), ograds, [GOLD[f"gpt_g{i}"] for i in range(21)], "dropin golden")
    # Forward + backward + AdamW in one call, then the step-1 loss.
    d.set_params(params)
    d.step(backward=True, adamw=True)
    loss1 = d.step(backward=False)
    assert abs(loss1 - GOLD["gpt_loss1"]) <= 1e-4 * GOLD["gpt_loss1"], (loss1, GOLD["gpt_loss1"])
    ps = adam_ref(params, ograds)
    oloss1, _ = O.gpt_step(O.GptConfig(*cfg), ps, ids, tg, grads=False)
    assert abs(loss1 - oloss1) <= 1e-5 + 1e-4 * abs(oloss1), (loss1, oloss1)
    assert_parity(d.params()[20], ps[20], name="dropin lm_w after AdamW")
    d.close()


def test_dropin_medium_model_matches_oracle_and_fused_driver(vh):
    from vearo_amd import _block
    cfg = (2, 128, 128, 4, 512, 1000, 128)
    print("dropin medium", flush=True)
    params, ids, tg = random_model(cfg, 11)
    d = dropin(cfg)
    d.set_params(params)
    d.set_inputs(ids, tg)
    loss = d.step(backward=True, timing=True)
    ph = d.phase_ms()
    assert len(ph) == 23 and all(v >= 0 for v in ph.values()) and ph["fwd.matmul"] > 0
    assert ph["fwd.softmax"] == 0 and ph["bwd.softmax"] == 0  # the fused path
    assert ph["bwd.reduce_to"] > 0 and ph["bwd.grad_accumulate"] > 0, ph
    grads = d.grads()
    oloss, ograds = O.gpt_step(O.GptConfig(*cfg), params, ids, tg)
    assert abs(loss - oloss) <= 1e-5 + 1e-4 * abs(oloss), (loss, oloss)
    check_grads(grads, ograds, tag="dropin medium")
    # The fused driver on the same model: same loss and gradients to the same bar.
    g = _block.Gpt(_block.GptConfig(*cfg))
    g.set_params(params)
    g.set_inputs(ids, tg)
    g.forward_backward(True)
    assert abs(g.loss() - loss) <= 1e-5 + 1e-4 * abs(oloss)
    for i, (a, b) in enumerate(zip(g.grads(), grads)):
        if O.GPT_PARAM_NAMES[i] != "k_b":
            assert_parity(b, a, ograds[i].astype(np.float64), name=f"dropin vs fused {O.GPT_PARAM_NAMES[i]}")
    g.close()
    # Two AdamW steps against the oracle's.
    ms = [np.zeros_like(p) for p in params]
    vs = [np.zeros_like(p) for p in params]
    ps = [p.copy() for p in params]
    for t in (1, 2):
        d.step(backward=True, adamw=True, want_loss=False)
        _, og = O.gpt_step(O.GptConfig(*cfg), ps, ids, tg)
        for p, gr, m, v in zip(ps, og, ms, vs):
            O.adamw_step(p, gr, m, v, t, 0.02, 0.9, 0.95, 1e-8, 0.01)
    loss2 = d.step(backward=False)
    oloss2, _ = O.gpt_step(O.GptConfig(*cfg), ps, ids, tg, grads=False)
    assert abs(loss2 - oloss2) <= 1e-5 + 1e-4 * abs(oloss2), (loss2, oloss2)
    d.close()


def test_dropin_weight_gradient_fold_and_reference_arm(vh):
    """The Matmul arm's shared-weight gradient both ways: folded (the default,
    one product over all B*S rows) and the reference's own arm (per-batch
    product, then reduce_to over the batch, autograd:502-519, 316-361). Both
    against the oracle, on the medium model and on the golden one (B = 2), and
    against each other (the same sums in another grouping)."""
    from vearo_amd import _block
    for cfg, seed in (((2, 128, 128, 4, 512, 1000, 128), 17), (tuple(int(x) for x in GOLD["gpt_cfg"]), None)):
        if seed is None:
            params = [GOLD[f"gpt_p{i}"] for i in range(21)]
            ids, tg = GOLD["gpt_ids"], GOLD["gpt_targets"]
        else:
            params, ids, tg = random_model(cfg, seed)
        print(f"dropin fold cfg={cfg}", flush=True)
        oloss, ograds = O.gpt_step(O.GptConfig(*cfg), params, ids, tg)
        got = {}
        for fold in (True, False):
            d = _block.DropIn(_block.GptConfig(*cfg), fold_weight_grads=fold)
            assert d.fold_weight_grads == fold
            d.set_params(params)
            d.set_inputs(ids, tg)
            loss = d.step(backward=True, timing=True)
            ph = d.phase_ms()
            assert abs(loss - oloss) <= 1e-5 + 1e-4 * abs(oloss), (fold, loss, oloss)
            got[fold] = d.grads()
            check_grads(got[fold], ograds, tag=f"dropin fold={fold}")
            assert ph["bwd.matmul"] > 0 and ph["bwd.reduce_to"] > 0, ph
            d.close()
        for i, (a, b) in enumerate(zip(got[True], got[False])):
            if O.GPT_PARAM_NAMES[i] != "k_b":
                assert_parity(a, b, ograds[i].astype(np.float64), name=f"fold vs reference arm {O.GPT_PARAM_NAMES[i]}")
    d = _block.DropIn(_block.GptConfig(*cfg))
    assert d.fold_weight_grads  # the default
    d.close()


def test_dropin_unfused_attention(vh):
    """MultiHeadAttention's unfused path (VEARO_USE_FUSED_ATTENTION=0,
    crates/vearo-nn/src/lib.rs:603-613): scores through the matmul, mul, add
    and softmax slots, the backward through the Matmul, Softmax (five slot
    calls, autograd:547-553), Add, Mul and Transpose arms. Golden and medium
    models against the oracle's unfused step (and the golden float64 model),
    the losses after AdamW, and the environment switch itself."""
    from vearo_amd import _block
    cfg = tuple(int(x) for x in GOLD["gpt_cfg"])
    params = [GOLD[f"gpt_p{i}"] for i in range(21)]
    ids, tg = GOLD["gpt_ids"], GOLD["gpt_targets"]
    d = _block.DropIn(_block.GptConfig(*cfg), fused_attention=False)
    assert not d.fused_attention
    d.set_params(params)
    d.set_inputs(ids, tg)
    loss = d.step(backward=True)
    oloss, ograds = O.gpt_step(O.GptConfig(*cfg), params, ids, tg, fused_attention=False)
    assert abs(loss - oloss) <= 1e-5 + 1e-4 * abs(oloss), (loss, oloss)
    assert abs(loss - GOLD["gpt_loss"]) <= 1e-4 * GOLD["gpt_loss"]
    check_grads(d.grads(), ograds, [GOLD[f"gpt_g{i}"] for i in range(21)], "dropin unfused golden")
    d.set_params(params)
    d.step(backward=True, adamw=True)
    loss1 = d.step(backward=False)
    oloss1, _ = O.gpt_step(O.GptConfig(*cfg), adam_ref(params, ograds), ids, tg, grads=False, fused_attention=False)
    assert abs(loss1 - oloss1) <= 1e-5 + 1e-4 * abs(oloss1), (loss1, oloss1)
    d.close()

    cfg = (2, 128, 128, 4, 512, 1000, 128)
    print("dropin unfused medium", flush=True)
    params, ids, tg = random_model(cfg, 13)
    d = _block.DropIn(_block.GptConfig(*cfg), fused_attention=False)
    d.set_params(params)
    d.set_inputs(ids, tg)
    loss = d.step(backward=True, timing=True)
    ph = d.phase_ms()
    assert ph["fwd.fused_attention"] == 0 and ph["bwd.fused_attention"] == 0, ph
    for k in ("fwd.mul", "fwd.softmax", "bwd.mul", "bwd.softmax"):
        assert ph[k] > 0, (k, ph)
    oloss, ograds = O.gpt_step(O.GptConfig(*cfg), params, ids, tg, fused_attention=False)
    assert abs(loss - oloss) <= 1e-5 + 1e-4 * abs(oloss), (loss, oloss)
    check_grads(d.grads(), ograds, tag="dropin unfused medium")
    d.step(backward=True, adamw=True, want_loss=False)
    loss1 = d.step(backward=False)
    oloss1, _ = O.gpt_step(O.GptConfig(*cfg), adam_ref(params, ograds), ids, tg, grads=False, fused_attention=False)
    assert abs(loss1 - oloss1) <= 1e-5 + 1e-4 * abs(oloss1), (loss1, oloss1)
    d.close()

    # The reference's switch: the fused path unless the variable is "0" or "false".
    old = os.environ.get("VEARO_USE_FUSED_ATTENTION")
    try:
        for val, fused in (("0", False), ("false", False), ("1", True), ("no", True)):
            os.environ["VEARO_USE_FUSED_ATTENTION"] = val
            d = _block.DropIn(_block.GptConfig(*cfg))
            assert d.fused_attention == fused, val
            d.close()
        del os.environ["VEARO_USE_FUSED_ATTENTION"]
        d = _block.DropIn(_block.GptConfig(*cfg))
        assert d.fused_attention
        d.close()
    finally:
        if old is None:
            os.environ.pop("VEARO_USE_FUSED_ATTENTION", None)
        else:
            os.environ["VEARO_USE_FUSED_ATTENTION"] = old


def test_dropin_errors(vh):
    from vearo_amd import _block
    cfg = (1, 4, 8, 2, 16, 8, 4)
    d = dropin(cfg)
    with pytest.raises(vh.VhError, match="no gradient"):
        d.grads()
    with pytest.raises(vh.VhError, match="AdamW needs"):
        d.step(backward=False, adamw=True)
    with pytest.raises(vh.VhError, match="element count"):
        _block.check(_block.lib.vb_dropin_set_param(d.h, 0, np.zeros(3, np.float32).ctypes.data, 3))
    # A target outside the vocabulary: the cross-entropy slot's panic (cpu:1000-1006).
    d.set_inputs(np.zeros((1, 4), np.float32), np.full((1, 4), 9.0, np.float32))
    with pytest.raises(vh.VhError, match="Target class 9 out of vocab bounds 8"):
        d.step(backward=False)
    vh.sync()  # the panic was reported once and cleared
    d.close()
    with pytest.raises(vh.VhError, match="divisible"):
        dropin((1, 4, 9, 2, 16, 8, 4))


def test_dropin_overfits_like_the_reference_test(vh):
    """verification_harness.rs:184-237 through the drop-in path, which issues
    the reference's own op sequence: 150 AdamW steps bring the loss under 0.05,
    and the first ten losses follow the oracle's."""
    cfg = (2, 4, 8, 2, 16, 8, 4)
    ocfg = O.GptConfig(*cfg)
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
    d = dropin(cfg)
    d.set_params(params)
    d.set_inputs(ids, tg)
    ps = [p.copy() for p in params]
    ms = [np.zeros_like(p) for p in ps]
    vs = [np.zeros_like(p) for p in ps]
    for t in range(1, 151):
        loss = d.step(backward=True, adamw=True)
        if t <= 10:
            oloss, ograds = O.gpt_step(ocfg, ps, ids, tg)
            for p, gr, m, v in zip(ps, ograds, ms, vs):
                O.adamw_step(p, gr, m, v, t, 0.02, 0.9, 0.95, 1e-8, 0.01)
            assert abs(loss - oloss) <= 1e-4 * max(1.0, abs(oloss)), (t, loss, oloss)
    loss = d.step(backward=False)
    assert loss < 0.05, loss
    d.close()


def test_steps_do_not_grow_device_memory(vh):
    """The reference's memory-regression check (crates/vearo/tests/memory_regression.rs:
    103-137: slots must not grow over 25 training steps), for both step drivers
    on one device: after a few warm-up steps the library's live bytes and the
    bytes it holds from hipMalloc stay where they were over 25 more steps."""
    from vearo_amd import _block
    cfg = (2, 128, 128, 4, 512, 1000, 128)
    params, ids, tg = random_model(cfg, 5)
    for name, make, run in (
            ("dropin", lambda: dropin(cfg), lambda m: m.step(backward=True, adamw=True)),
            ("fused", lambda: _block.Gpt(_block.GptConfig(*cfg)), lambda m: (m.train_step(), m.loss()))):
        print("memory growth", name, flush=True)
        m = make()
        m.set_params(params)
        m.set_inputs(ids, tg)
        for _ in range(3):
            run(m)
        vh.sync()
        before = vh.mem_stats()
        for _ in range(25):
            run(m)
        vh.sync()
        after = vh.mem_stats()
        assert after.live_bytes == before.live_bytes, (name, before.live_bytes, after.live_bytes)
        assert after.hip_bytes <= before.hip_bytes, (name, before.hip_bytes, after.hip_bytes)
        m.close()
