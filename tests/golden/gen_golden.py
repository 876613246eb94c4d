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

# ------------------------------------------------------------------- matmul
# Batched matmul with broadcast batch dims (cpu:266-417): torch.matmul in f64.
for tag, sa, sb in (("mm2", (5, 7), (7, 3)), ("mm3", (2, 5, 7), (7, 4)),
                    ("mmb", (2, 1, 4, 6), (3, 6, 5))):
    a, b = f32(rng.normal(size=sa)), f32(rng.normal(size=sb))
    G.update({f"{tag}_a": a, f"{tag}_b": b,
              f"{tag}_out": torch.matmul(t64(a), t64(b)).numpy()})


# ---------------------------------------------------------- fused attention
# Unfused reference formula in f64: softmax(q k^T / sqrt(dk) + mask) v, and its
# autograd gradients for an upstream gradient go.
def add_attention(tag, q, k, v, mask, go):
    q, k, v, go = f32(q), f32(k), f32(v), f32(go)
    Q, K, Vt = t64(q, True), t64(k, True), t64(v, True)
    s = Q @ K.transpose(-1, -2) / math.sqrt(q.shape[-1])
    if mask is not None:
        s = s + t64(f32(mask))
        G[f"{tag}_mask"] = f32(mask)
    out = torch.softmax(s, -1) @ Vt
    out.backward(t64(go))
    G.update({f"{tag}_q": q, f"{tag}_k": k, f"{tag}_v": v, f"{tag}_go": go,
              f"{tag}_out": out.detach().numpy(), f"{tag}_dq": Q.grad.numpy(),
              f"{tag}_dk": K.grad.numpy(), f"{tag}_dv": Vt.grad.numpy()})


def causal_mask(S):
    m = np.zeros((S, S))
    m[np.triu_indices(S, 1)] = -1e9
    return m


# Known-answer inputs of crates/vearo/tests/fused_attention_parity.rs:13-47:
# B=H=2, S=4, DK=8, q/k/v = fill(n, phase), upstream grad = sin(0.19 i) + 1.5.
def kat_fill(n, phase):
    x = np.arange(n, dtype=np.float32)
    return (np.sin(x * np.float32(0.37) + np.float32(phase)) * np.float32(0.5)
            + np.cos(x * np.float32(0.11) + np.float32(phase)) * np.float32(0.25)).astype(np.float32)


n_kat = 2 * 2 * 4 * 8
add_attention("attkat", kat_fill(n_kat, 0.0).reshape(2, 2, 4, 8), kat_fill(n_kat, 1.3).reshape(2, 2, 4, 8),
              kat_fill(n_kat, 2.7).reshape(2, 2, 4, 8), causal_mask(4),
              (np.sin(np.arange(n_kat, dtype=np.float32) * np.float32(0.19)) + np.float32(1.5)).reshape(2, 2, 4, 8))
add_attention("attc", rng.normal(size=(1, 3, 17, 16)), rng.normal(size=(1, 3, 17, 16)),
              rng.normal(size=(1, 3, 17, 16)), causal_mask(17), rng.normal(size=(1, 3, 17, 16)))
add_attention("attm", rng.normal(size=(2, 2, 9, 8)), rng.normal(size=(2, 2, 9, 8)),
              rng.normal(size=(2, 2, 9, 8)), rng.normal(size=(2, 1, 9, 9)), rng.normal(size=(2, 2, 9, 8)))
add_attention("attn", rng.normal(size=(1, 2, 6, 4)), rng.normal(size=(1, 2, 6, 4)),
              rng.normal(size=(1, 2, 6, 4)), None, rng.normal(size=(1, 2, 6, 4)))


# ----------------------------------------------------------- SimpleGPT step
# nn:666-791 with one block, written independently in torch f64: loss and the
# gradient of every parameter, then one AdamW step (tensor.rs:967-986) and the
# loss after it.
def gpt_forward(P, ids, targets, B, S, D, H):
    def ln(x, w, b):
        return torch.nn.functional.layer_norm(x, (D,), w, b, 1e-5)

    def lin(x, w, b=None):
        y = x @ w.T
        return y + b if b is not None else y

    (wte, wpe, l1w, l1b, qw, qb, kw, kb, vw, vb, ow, ob, l2w, l2b, f1w, f1b, f2w, f2b,
     lfw, lfb, lmw) = P
    h = wte[ids] + wpe[torch.arange(S)].unsqueeze(0)
    x1 = ln(h, l1w, l1b)

    def heads(t):
        return t.reshape(B, S, H, D // H).transpose(1, 2)

    q, k, v = heads(lin(x1, qw, qb)), heads(lin(x1, kw, kb)), heads(lin(x1, vw, vb))
    s = q @ k.transpose(-1, -2) / math.sqrt(D // H) + torch.tensor(causal_mask(S))
    a = (torch.softmax(s, -1) @ v).transpose(1, 2).reshape(B, S, D)
    h = h + lin(a, ow, ob)
    m = torch.nn.functional.gelu(lin(ln(h, l2w, l2b), f1w, f1b), approximate="tanh")
    h = h + lin(m, f2w, f2b)
    logits = lin(ln(h, lfw, lfb).reshape(B * S, D), lmw)
    return torch.nn.functional.cross_entropy(logits, targets.reshape(-1))


def add_gpt(tag, B, S, D, H, F, V, scale):
    shapes = [(V, D), (S, D), (D,), (D,), (D, D), (D,), (D, D), (D,), (D, D), (D,), (D, D), (D,),
              (D,), (D,), (F, D), (F,), (D, F), (D,), (D,), (D,), (V, D)]
    params = []
    for i, sh in enumerate(shapes):
        if i in (2, 12, 18):
            params.append(f32(1 + 0.1 * rng.normal(size=sh)))
        elif i in (3, 13, 19):
            params.append(f32(0.1 * rng.normal(size=sh)))
        else:
            params.append(f32(scale * rng.normal(size=sh)))
    ids = rng.integers(0, V, size=(B, S))
    tg = rng.integers(0, V, size=(B, S))
    P = [t64(p, True) for p in params]
    loss = gpt_forward(P, torch.tensor(ids), torch.tensor(tg), B, S, D, H)
    loss.backward()
    lr, b1, b2, eps, wd = 0.02, 0.9, 0.95, 1e-8, 0.01
    new = []
    for p in P:
        g = p.grad.detach()
        m, v = (1 - b1) * g, (1 - b2) * g * g
        mh, vh = m / (1 - b1), v / (1 - b2)
        q = p.detach() - lr * wd * p.detach()
        new.append(q - lr * mh / (vh.sqrt() + eps))
    loss1 = gpt_forward(new, torch.tensor(ids), torch.tensor(tg), B, S, D, H)
    G[f"{tag}_cfg"] = np.array([B, S, D, H, F, V, S], np.int64)
    G[f"{tag}_ids"] = f32(ids)
    G[f"{tag}_targets"] = f32(tg)
    G[f"{tag}_loss"] = np.float64(loss.item())
    G[f"{tag}_loss1"] = np.float64(loss1.item())
    for i, (p, t) in enumerate(zip(params, P)):
        G[f"{tag}_p{i}"] = p
        G[f"{tag}_g{i}"] = t.grad.numpy()


add_gpt("gpt", B=2, S=8, D=16, H=2, F=32, V=40, scale=0.3)

np.savez_compressed(OUT, **G)
print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(G)} arrays)")
