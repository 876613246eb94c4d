"""vh_adamw_step_multi: AdamW over many parameter tensors in one launch per
32 tensors (AdamW::step's loop over parameters, crates/vearo-optim/src/lib.rs:105-123).
Every element must get the bits the per-tensor vh_adamw_step gives it
(tensor.rs:967-986): sizes that take the 128-bit and the 32-bit units, empty
tensors, bases one float off 16-byte alignment, more tensors than one launch
holds, three steps in a row; and the oracle's AdamW on the same data."""
import ctypes

import numpy as np
import pytest

import oracle as O
from parity import assert_parity, dev, fetch

pytestmark = pytest.mark.gpu

HP = (0.02, 0.9, 0.95, 1e-8, 0.01)  # lr, beta1, beta2, eps, weight decay (verification_harness.rs:203-210)


def test_adamw_multi_matches_per_tensor_bits(vh):
    r = np.random.default_rng(77)
    sizes = [4096, 1, 0, 3, 5, 1000, 1000003, 768, 38597376 // 64] + [int(x) for x in r.integers(1, 5000, 31)]
    offs = [0, 0, 0, 0, 1, 0, 1, 0, 0] + [int(x) for x in r.integers(0, 2, 31)]
    print("adamw multi", len(sizes), "tensors", flush=True)
    host = []
    for n, off in zip(sizes, offs):
        p = r.standard_normal(n + off).astype(np.float32)
        host.append((n, off, p, (r.standard_normal((3, n + off)) * 0.1).astype(np.float32)))
    # Two device copies of every tensor: one stepped per tensor, one by the multi entry.
    def alloc():
        bufs = []
        for n, off, p, gs in host:
            bufs.append(dict(P=dev(vh, p), M=dev(vh, np.zeros(n + off, np.float32)),
                             V=dev(vh, np.zeros(n + off, np.float32)), G=[dev(vh, g) for g in gs]))
        return bufs
    one, multi = alloc(), alloc()
    at = lambda b, off: b.ptr + 4 * off
    for t in (1, 2, 3):
        for (n, off, _, _), b in zip(host, one):
            vh.check(vh.lib.vh_adamw_step(at(b["P"], off), at(b["G"][t - 1], off), at(b["M"], off), at(b["V"], off),
                                          n, t, *HP, None))
        k = len(host)
        arr = lambda xs: (ctypes.c_void_p * k)(*xs)
        ps = arr([at(b["P"], off) for (n, off, _, _), b in zip(host, multi)])
        gs = arr([at(b["G"][t - 1], off) for (n, off, _, _), b in zip(host, multi)])
        ms = arr([at(b["M"], off) for (n, off, _, _), b in zip(host, multi)])
        vs = arr([at(b["V"], off) for (n, off, _, _), b in zip(host, multi)])
        ns = (ctypes.c_int64 * k)(*[n for n, _, _, _ in host])
        vh.check(vh.lib.vh_adamw_step_multi(k, ps, gs, ms, vs, ns, t, *HP, None))
    for i, ((n, off, p, gs), a, b) in enumerate(zip(host, one, multi)):
        for key in ("P", "M", "V"):
            np.testing.assert_array_equal(fetch(vh, b[key], (n + off,)), fetch(vh, a[key], (n + off,)),
                                          err_msg=f"tensor {i} (n={n}) {key}")
        if n in (1000003, 5):
            pc, mc, vc = p[off:].copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
            for t in (1, 2, 3):
                O.adamw_step(pc, gs[t - 1][off:], mc, vc, t, *HP)
            assert_parity(fetch(vh, b["P"], (n + off,))[off:], pc, name=f"multi adamw p n={n}")


def test_adamw_multi_errors(vh):
    one = (ctypes.c_void_p * 1)(None)
    n1 = (ctypes.c_int64 * 1)(-1)
    with pytest.raises(vh.VhError, match="negative count"):
        vh.check(vh.lib.vh_adamw_step_multi(-1, None, None, None, None, None, 1, *HP, None))
    with pytest.raises(vh.VhError, match="null array"):
        vh.check(vh.lib.vh_adamw_step_multi(1, None, one, one, one, n1, 1, *HP, None))
    with pytest.raises(vh.VhError, match="negative size"):
        vh.check(vh.lib.vh_adamw_step_multi(1, one, one, one, one, n1, 1, *HP, None))
    with pytest.raises(vh.VhError, match="t must be >= 1"):
        vh.check(vh.lib.vh_adamw_step_multi(0, None, None, None, None, None, 0, *HP, None))
    vh.check(vh.lib.vh_adamw_step_multi(0, None, None, None, None, None, 1, *HP, None))  # nothing to do
