"""The persistent GEMM's wide tile (256 x 256, kernels/gemm_big.h). vh_gemm
picks it for long k loops (K >= 8192 in whole k tiles) over a row-contiguous
B with at least one full round of wide tiles -- the block step's lm_head dW
([50260, 768] = dlogits^T ln_f) -- and the WIDE engine forces it wherever the
persistent kernel runs, so these products stay small enough for the CPU
oracle. Every operand layout, edges in M and N, a k tail left to the tiled
kernel, bias / accumulate / alpha epilogues, operands only 4-byte aligned, and
the stream-K round with its fix-up (fixed order: the same bits on a second
call); against the oracle, float64 and the f32 error bound of a K-term sum."""
import ctypes

import numpy as np
import pytest

import oracle as O
from parity import assert_parity, dev, fetch, out
from test_block_ops_gpu import gemm_desc

pytestmark = pytest.mark.gpu

# a_scale 1e-2 keeps long sums at the magnitude of the block step's (activations
# times ~1e-4 dlogits), where the elementwise bar compares the products; the
# unscaled cases keep the check that holds at any scale, the f32 error bound.
#   name, M, N, K, A k-contiguous, B k-contiguous, epilogue, a_scale, offset
WIDE_CASES = [
    ("kk, edges, bias + residual", 520, 600, 2080, True, True, "bias_acc", 1e-2, 0),
    ("kn, lm_head dx shape, K tail", 512, 768, 50260, True, False, "", 1e-3, 0),
    ("kn, alpha, bases one float off, K tail", 300, 1001, 9000, True, False, "alpha", 1e-2, 1),
    ("mk, stream-K only", 1024, 768, 4096, False, True, "", 1.0, 0),
    ("mn, lm_head dW shape [V, D]", 1000, 768, 16384, False, False, "", 1e-2, 0),
    ("mn, odd M and N, 4-byte aligned", 1001, 777, 8192, False, False, "alpha_acc", 1e-2, 1),
    ("kn, full round of tiles", 4096, 4096, 512, True, False, "", 1.0, 0),
]


@pytest.mark.parametrize("case", WIDE_CASES, ids=[c[0] for c in WIDE_CASES])
def test_gemm_persistent_wide_tile(vh, case):
    name, M, N, K, akc, bkc, epi, a_scale, off = case
    print("wide tile", case, flush=True)
    r = np.random.default_rng(M * 5 + N * 3 + K)
    a = (r.standard_normal((M, K)) * a_scale).astype(np.float32)
    b = (r.standard_normal((K, N)) * 0.05).astype(np.float32)
    pad = np.zeros(off, np.float32)
    Abuf = dev(vh, np.concatenate([pad, (a if akc else a.T).reshape(-1)]))
    Bbuf = dev(vh, np.concatenate([pad, (b.T if bkc else b).reshape(-1)]))
    A, B = Abuf.ptr + 4 * off, Bbuf.ptr + 4 * off
    a_sm, a_sk = (K, 1) if akc else (1, M)
    b_sk, b_sn = (1, K) if bkc else (N, 1)
    ref = O.matmul(a, b)
    ref64 = a.astype(np.float64) @ b.astype(np.float64)
    kw = {"engine": vh.GEMM_ENGINE_WIDE}
    c0 = np.zeros((M, N), np.float32)
    want, want64 = ref, ref64
    keep = []
    if "alpha" in epi:
        kw["alpha"] = 0.75
        want, want64 = ref * np.float32(0.75), ref64 * 0.75
    if "bias" in epi:
        bias = (r.standard_normal(N) * 0.1).astype(np.float32)
        keep.append(dev(vh, bias))
        kw.update(e=keep[-1].ptr, e_sm=0, e_sn=1)
        want, want64 = want + bias, want64 + bias.astype(np.float64)
    if "acc" in epi:
        c0 = r.standard_normal((M, N), dtype=np.float32)
        kw["accumulate"] = 1
        want, want64 = c0 + want, c0.astype(np.float64) + want64
    C = dev(vh, c0)
    d = gemm_desc(vh, M, N, K, A, a_sm, a_sk, B, b_sk, b_sn, C.ptr, N, **kw)
    vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
    assert vh.lib.vh_gemm_last_path() == vh.GEMM_PATH_PERSISTENT, name
    got = fetch(vh, C, (M, N))
    assert_parity(got, want, want64, name=f"wide tile {name}")
    if not epi:
        u = 2.0 ** -24
        bound = (K * u / (1 - K * u)) * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
        assert np.all(np.abs(got - ref64) <= bound), f"wide tile {name}: f32 error bound"
    if not kw.get("accumulate"):
        C2 = out(vh, (M, N))
        d = gemm_desc(vh, M, N, K, A, a_sm, a_sk, B, b_sk, b_sn, C2.ptr, N, **kw)
        vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
        np.testing.assert_array_equal(fetch(vh, C2, (M, N)), got)


def test_gemm_wide_engine_is_checked(vh):
    X = dev(vh, np.ones((4, 4), np.float32))
    d = gemm_desc(vh, 4, 4, 4, X.ptr, 4, 1, X.ptr, 4, 1, X.ptr, 4, engine=4)
    with pytest.raises(vh.VhError, match="unknown engine"):
        vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
