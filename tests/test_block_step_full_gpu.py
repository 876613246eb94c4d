"""Config[4] at its real size (B=16, T=1024, C=768, H=12, MLP 3072, V=50257):
the device step against the CPU oracle's SimpleGPT step on identical inputs --
the step-0 loss, every parameter gradient, and the loss after one AdamW step,
for the fused driver (vb_gpt) and for the same step issued op by op through the
BackendOps mirror (vb_dropin) (north_star: "the full config[4] block step runs end to end with loss matching
the CPU backend"; loss within 1e-4 relative).

The oracle needs about 6 TFLOP here; it runs threaded (its results do not
depend on the thread count), a few tens of seconds on the GPU box's cores.
"""
import time

import numpy as np
import pytest

import oracle as O
from parity import assert_parity

pytestmark = pytest.mark.gpu

CFG = (16, 1024, 768, 12, 3072, 50257, 1024)
ADAM = (0.02, 0.9, 0.95, 1e-8, 0.01)  # verification_harness.rs:203-210


def full_model():
    B, S, D, H, F, V, P = CFG
    r = np.random.default_rng(0x5EED0000 + 4)
    params = []
    for name, sh in zip(O.GPT_PARAM_NAMES, O.gpt_param_shapes(O.GptConfig(*CFG))):
        if name.startswith("ln") and name.endswith("_w"):
            params.append(np.ones(sh, np.float32))
        elif name.startswith("ln"):
            params.append(np.zeros(sh, np.float32))
        else:
            params.append(r.standard_normal(sh, dtype=np.float32) * np.float32(0.02))
    ids = r.integers(0, V, size=(B, S)).astype(np.float32)
    tg = r.integers(0, V, size=(B, S)).astype(np.float32)
    return params, ids, tg


def test_block_step_full_size_matches_oracle(vh):
    from vearo_amd import _block
    params, ids, tg = full_model()

    g = _block.Gpt(_block.GptConfig(*CFG))
    g.set_params(params)
    g.set_inputs(ids, tg)
    g.forward_backward(True)
    loss0 = g.loss()
    grads = g.grads()
    g.adamw(*ADAM)
    g.forward_backward(False)
    loss1 = g.loss()
    g.close()
    print(f"device: loss0 {loss0:.7f} loss1 {loss1:.7f}", flush=True)
    assert np.isfinite(loss0) and np.isfinite(loss1)

    t0 = time.perf_counter()
    oloss0, ograds = O.gpt_step(O.GptConfig(*CFG), params, ids, tg)
    print(f"oracle forward+backward {time.perf_counter() - t0:.1f} s: loss0 {oloss0:.7f}", flush=True)
    assert abs(loss0 - oloss0) <= 1e-4 * abs(oloss0), (loss0, oloss0)
    for i, name in enumerate(O.GPT_PARAM_NAMES):
        if name == "k_b":  # exact gradient 0 (softmax ignores a per-row shift)
            assert np.abs(grads[i]).max() < 1e-6 and np.abs(ograds[i]).max() < 1e-6
            continue
        scale = np.abs(ograds[i]).max()
        err = np.abs(grads[i] - ograds[i]).max()
        print(f"  grad {name:6s} max|cpu| {scale:.3e} max|gpu-cpu| {err:.3e}", flush=True)
        assert err <= 1e-4 * scale, (name, err, scale)
        # Elementwise, the north-star bar |gpu - cpu| <= 1e-5 + 1e-4 |cpu| on every element.
        assert_parity(grads[i], ograds[i], name=f"full-size block-step grad {name}")
    # The same step issued op by op through the BackendOps mirror (vb_dropin),
    # the reference's own op order: loss, gradients, then AdamW.
    d = _block.DropIn(_block.GptConfig(*CFG))
    d.set_params(params)
    d.set_inputs(ids, tg)
    dloss0 = d.step(backward=True, adamw=True, lr=ADAM[0], beta1=ADAM[1], beta2=ADAM[2], eps=ADAM[3], wd=ADAM[4])
    print(f"drop-in: loss0 {dloss0:.7f}", flush=True)
    assert abs(dloss0 - oloss0) <= 1e-4 * abs(oloss0), (dloss0, oloss0)
    for i, dg in enumerate(d.grads()):
        if O.GPT_PARAM_NAMES[i] == "k_b":
            assert np.abs(dg).max() < 1e-6
            continue
        assert_parity(dg, ograds[i], name=f"full-size drop-in grad {O.GPT_PARAM_NAMES[i]}")
    dloss1 = d.step(backward=False)
    d.close()
    print(f"drop-in: loss1 {dloss1:.7f}", flush=True)
    # The reference's own Matmul arm (per-batch weight gradients, then reduce_to).
    d = _block.DropIn(_block.GptConfig(*CFG), fold_weight_grads=False)
    d.set_params(params)
    d.set_inputs(ids, tg)
    rloss0 = d.step(backward=True)
    assert abs(rloss0 - oloss0) <= 1e-4 * abs(oloss0), (rloss0, oloss0)
    for i, dg in enumerate(d.grads()):
        if O.GPT_PARAM_NAMES[i] != "k_b":
            assert_parity(dg, ograds[i], name=f"full-size drop-in (reference arm) grad {O.GPT_PARAM_NAMES[i]}")
    d.close()
    for p, gr in zip(params, ograds):
        O.adamw_step(p, gr, np.zeros_like(p), np.zeros_like(p), 1, *ADAM)
    t0 = time.perf_counter()
    oloss1, _ = O.gpt_step(O.GptConfig(*CFG), params, ids, tg, grads=False)
    print(f"oracle forward after AdamW {time.perf_counter() - t0:.1f} s: loss1 {oloss1:.7f}", flush=True)
    assert abs(loss1 - oloss1) <= 1e-4 * abs(oloss1), (loss1, oloss1)
    assert abs(dloss1 - oloss1) <= 1e-4 * abs(oloss1), (dloss1, oloss1)


def test_block_step_full_size_unfused_attention(vh):
    """The drop-in step with MultiHeadAttention's unfused path
    (VEARO_USE_FUSED_ATTENTION=0, nn:603-613) at the real size: the [16, 12,
    1024, 1024] scores go through the matmul, mul, add and softmax slots, and
    back through the Softmax arm's five slot calls. Step-0 loss, every
    gradient elementwise and the loss after AdamW against the oracle's unfused
    step on the same inputs."""
    from vearo_amd import _block
    params, ids, tg = full_model()
    d = _block.DropIn(_block.GptConfig(*CFG), fused_attention=False)
    d.set_params(params)
    d.set_inputs(ids, tg)
    dloss0 = d.step(backward=True, adamw=True, lr=ADAM[0], beta1=ADAM[1], beta2=ADAM[2], eps=ADAM[3], wd=ADAM[4])
    dgrads = d.grads()
    dloss1 = d.step(backward=False)
    d.close()
    print(f"drop-in unfused: loss0 {dloss0:.7f} loss1 {dloss1:.7f}", flush=True)
    t0 = time.perf_counter()
    oloss0, ograds = O.gpt_step(O.GptConfig(*CFG), params, ids, tg, fused_attention=False)
    print(f"oracle unfused forward+backward {time.perf_counter() - t0:.1f} s: loss0 {oloss0:.7f}", flush=True)
    assert abs(dloss0 - oloss0) <= 1e-4 * abs(oloss0), (dloss0, oloss0)
    for i, dg in enumerate(dgrads):
        if O.GPT_PARAM_NAMES[i] == "k_b":
            assert np.abs(dg).max() < 1e-6
            continue
        assert_parity(dg, ograds[i], name=f"full-size unfused drop-in grad {O.GPT_PARAM_NAMES[i]}")
    for p, gr in zip(params, ograds):
        O.adamw_step(p, gr, np.zeros_like(p), np.zeros_like(p), 1, *ADAM)
    oloss1, _ = O.gpt_step(O.GptConfig(*CFG), params, ids, tg, grads=False, fused_attention=False)
    print(f"oracle unfused loss1 {oloss1:.7f}", flush=True)
    assert abs(dloss1 - oloss1) <= 1e-4 * abs(oloss1), (dloss1, oloss1)
