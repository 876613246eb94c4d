"""Generate tests/golden/golden.npz: small inputs with float64 reference outputs.

The references are computed with torch in float64 on the CPU -- torch's own
layer_norm / gelu(approximate="tanh") / softmax / embedding / cross_entropy and
autograd -- which is an implementation independent of the C oracle, so a
dropped term, wrong sign or transposed operand in the oracle shows up as a
mismatch far above f32 rounding. Known-answer inputs from the reference's own
tests are included (crates/vearo-autograd/src/lib.rs:1253-1495 grad checks,
crates/vearo-backend-cpu/src/lib.rs:2902-2913 cross-entropy stability).

Run:  python tests/golden/gen_golden.py   (rewrites golden.npz next to this file)
"""
import math
import os

import numpy as np
import torch

torch.set_default_dtype(torch.float64)
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")
rng = np.random.default_rng(0x5EED)


def f32(a):
    return np.asarray(a, dtype=np.float32)


def t64(a, grad=False):
    t = torch.tensor(np.asarray(a, dtype=np.float64))
    if grad:
        t.requires_grad_(True)
    return t


def round_half_away(v):
    return int(math.copysign(math.floor(abs(v) + 0.5), v))


G = {}

# ---------------------------------------------------------------- layernorm
def add_layernorm(tag, x, w, b, dy, eps):
    x, w, b, dy = f32(x), f32(w), f32(b), f32(dy)
    X, W, B = t64(x, True), t64(w, True), t64(b, True)
    y = torch.nn.functional.layer_norm(X, (x.shape[-1],), W, B, eps)
    y.backward(t64(dy))
    G.update({f"{tag}_x": x, f"{tag}_w": w, f"{tag}_b": b, f"{tag}_dy": dy,
              f"{tag}_eps": np.float32(eps), f"{tag}_y": y.detach().numpy(),
              f"{tag}_dx": X.grad.numpy(), f"{tag}_dw": W.grad.numpy(),
              f"{tag}_db": B.grad.numpy()})


add_layernorm("ln", rng.normal(size=(7, 33)), 1 + 0.02 * rng.normal(size=33),
              0.02 * rng.normal(size=33), rng.normal(size=(7, 33)), 1e-5)
add_layernorm("ln3d", rng.normal(size=(2, 3, 16)) * 3 + 1, 1 + 0.1 * rng.normal(size=16),
              0.1 * rng.normal(size=16), rng.normal(size=(2, 3, 16)), 1e-5)
# Reference grad-check inputs (autograd lib.rs:1394-1429): upstream grad of sum = ones.
add_layernorm("lnkat", [[1.0, 2.0], [3.0, 4.0]], [0.5, 1.5], [0.1, -0.1], np.ones((2, 2)), 1e-5)

# --------------------------------------------------------------------- gelu
xg = np.concatenate([[-1.0, 0.0, 1.0, 2.0], rng.normal(size=253) * 3.0])
Xg = t64(f32(xg), True)
yg = torch.nn.functional.gelu(Xg, approximate="tanh")
yg.sum().backward()
G.update({"gelu_x": f32(xg), "gelu_y": yg.detach().numpy(), "gelu_mask": Xg.grad.numpy()})

xb, bb, dyb = rng.normal(size=(5, 40)) * 1.5, rng.normal(size=40) * 0.02, rng.normal(size=(5, 40))
Xb, Bb = t64(f32(xb), True), t64(f32(bb), True)
yb = torch.nn.functional.gelu(Xb + Bb, approximate="tanh")
yb.backward(t64(f32(dyb)))
G.update({"gb_x": f32(xb), "gb_bias": f32(bb), "gb_dy": f32(dyb), "gb_y": yb.detach().numpy(),
          "gb_dx": Xb.grad.numpy(), "gb_dbias": Bb.grad.numpy()})

# ------------------------------------------------------------------ softmax
def add_softmax(tag, x, dy, dim):
    x, dy = f32(x), f32(dy)
    X = t64(x, True)
    y = torch.softmax(X, dim)
    y.backward(t64(dy))
    G.update({f"{tag}_x": x, f"{tag}_dy": dy, f"{tag}_dim": np.int64(dim),
              f"{tag}_y": y.detach().numpy(), f"{tag}_dx": X.grad.numpy()})


add_softmax("sm", rng.normal(size=(6, 37)), rng.normal(size=(6, 37)), 1)
add_softmax("sm0", rng.normal(size=(5, 4, 3)), rng.normal(size=(5, 4, 3)), 0)
sc = rng.normal(size=(2, 8, 8)) / 8.0
sc[:, np.triu_indices(8, 1)[0], np.triu_indices(8, 1)[1]] = -np.inf
add_softmax("smc", sc, rng.normal(size=(2, 8, 8)), 2)
# Reference grad-check (autograd lib.rs:1358-1391): loss = sum(softmax(x) * target).
add_softmax("smkat", [[1.0, 2.0], [3.0, 4.0]], [[0.5, 0.5], [0.2, 0.8]], 1)

# ---------------------------------------------------------------- embedding
V, D = 11, 6
W = rng.normal(size=(V, D)) * 0.5
ids = np.array([[2.4, 0.0, 10.0, 2.5, 0.49], [3.0, 3.0, 7.5, 0.0, 2.0],
                [9.0, 1.0, 3.0, 3.0, 3.0], [5.0, 4.0, 6.0, 8.0, 2.0]])
tok = np.vectorize(round_half_away)(ids)
dyE = rng.normal(size=(4, 5, D))
Wt = t64(f32(W), True)
outE = torch.nn.functional.embedding(torch.tensor(tok), Wt)
outE.backward(t64(f32(dyE)))
G.update({"emb_ids": f32(ids), "emb_W": f32(W), "emb_dy": f32(dyE), "emb_tok": tok,
          "emb_out": outE.detach().numpy(), "emb_dW": Wt.grad.numpy()})
# Reference grad-check inputs (autograd lib.rs:1432-1463).
G.update({"embkat_ids": f32([0.0, 1.0]), "embkat_W": f32([[1, 2, 3], [4, 5, 6]]),
          "embkat_out": np.array([[1.0, 2, 3], [4, 5, 6]]), "embkat_dW": np.ones((2, 3))})

# ------------------------------------------------------------ cross-entropy
def add_ce(tag, logits, targets, go):
    logits = f32(logits)
    L = t64(logits, True)
    tg = torch.tensor([round_half_away(v) for v in np.asarray(targets, np.float64)])
    loss = torch.nn.functional.cross_entropy(L, tg)
    loss.backward(torch.tensor(float(np.float32(go))))
    G.update({f"{tag}_logits": logits, f"{tag}_targets": f32(targets), f"{tag}_go": f32([go]),
              f"{tag}_loss": loss.detach().numpy().reshape(1), f"{tag}_dl": L.grad.numpy()})


add_ce("ce", rng.normal(size=(9, 13)) * 2, rng.integers(0, 13, size=9).astype(float), 1.7)
add_ce("cekat", [[1.0, 2.0], [3.0, 4.0]], [1.0, 0.0], 1.0)  # autograd lib.rs:1466-1495
add_ce("cestab", [[1000.0, -1000.0]], [0.0], 1.0)           # cpu lib.rs:2902-2913
add_ce("ceuni", np.zeros((3, 50)), [0.0, 17.0, 49.0], 1.0)   # loss = ln 50 exactly

# ------------------------------------------------------- reductions / binary
xr = rng.normal(size=(3, 4, 5))
G["red_x"] = f32(xr)
for d in range(3):
    G[f"red_sum{d}"] = f32(xr).astype(np.float64).sum(axis=d)
    G[f"red_mean{d}"] = f32(xr).astype(np.float64).mean(axis=d)
a, b = rng.normal(size=(3, 1, 5)), rng.normal(size=(4, 1)) + 3.0
G.update({"bin_a": f32(a), "bin_b": f32(b)})
A, B = f32(a).astype(np.float64), f32(b).astype(np.float64)
G.update({"bin_add": A + B, "bin_sub": A - B, "bin_mul": A * B, "bin_div": A / B})

np.savez_compressed(OUT, **G)
print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(G)} arrays)")
