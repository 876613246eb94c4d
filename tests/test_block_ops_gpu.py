"""GPU parity of the config[4] block-step ops against the CPU oracle:
matmul (vh_matmul / vh_gemm on the f32 matrix cores), fused attention forward
and backward, AdamW, and the row sum used for bias gradients.

Bar (north_star): |gpu - cpu| <= 1e-5 + 1e-4 |cpu| elementwise, or no further
from the float64 value than the oracle itself where one is available. Known
answers from the reference's own tests are exact on the GPU too.
"""
import ctypes
import math
import os

import numpy as np
import pytest

import oracle as O
from parity import assert_parity, dev, fetch, out

pytestmark = pytest.mark.gpu
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))


def run_matmul(vh, a, b, a_view=None, b_view=None, offset_floats=0):
    """vh_matmul on device copies of a and b. a_view/b_view: ("T",) to pass the
    transpose of the stored array as a strided view. offset_floats shifts both
    operands off 16-byte alignment."""
    def put(x, view):
        x = np.ascontiguousarray(x, np.float32)
        store = np.ascontiguousarray(np.swapaxes(x, -1, -2)) if view == "T" else x
        flat = np.concatenate([np.zeros(offset_floats, np.float32), store.reshape(-1)])
        buf = dev(vh, flat)
        dims = list(x.shape)
        if view == "T":
            st = [0] * store.ndim
            acc = 1
            for i in range(store.ndim - 1, -1, -1):
                st[i] = acc
                acc *= store.shape[i]
            strides = st[:-2] + [st[-1], st[-2]]
        else:
            strides = None
        return buf, vh.layout(dims, strides)
    A, al = put(a, a_view)
    B, bl = put(b, b_view)
    shape = np.broadcast_shapes(a.shape[:-2], b.shape[:-2]) + (a.shape[-2], b.shape[-1])
    C = out(vh, shape)
    pa = ctypes.c_void_p(A.ptr + 4 * offset_floats)
    pb = ctypes.c_void_p(B.ptr + 4 * offset_floats)
    vh.check(vh.lib.vh_matmul(pa, ctypes.byref(al), pb, ctypes.byref(bl), C.ptr, None))
    return fetch(vh, C, shape)


def test_matmul_reference_kats(vh):
    x = np.array([[1, 2], [3, 4]], np.float32)
    y = np.array([[5, 6], [7, 8]], np.float32)
    assert run_matmul(vh, x, y).tolist() == [[19, 22], [43, 50]]
    xb = np.arange(1, 13, dtype=np.float32).reshape(2, 2, 3)
    yb = np.arange(1, 13, dtype=np.float32).reshape(2, 3, 2)
    assert run_matmul(vh, xb, yb).reshape(-1).tolist() == [22, 28, 49, 64, 220, 244, 301, 334]
    # cuda:1676-1699: a transposed, non-contiguous rhs matches the CPU exactly.
    a = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    b = np.arange(7, 13, dtype=np.float32).reshape(2, 3)
    assert run_matmul(vh, a, b.T, b_view="T").tolist() == O.matmul(a, b.T).tolist()


# N <= 64 takes the 128 x 64 tile; with 128-bit loads its k tiles run two
# steps ahead in pairs: (128, 32, 64) one step, (256, 96, 64) and
# (384, 160, 64) odd step counts, (200, 288, 60) edge tiles with the checked loop.
@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (5, 7, 3), (128, 32, 128), (129, 33, 131),
                                   (300, 768, 200), (64, 1000, 96), (257, 64, 513),
                                   (300, 200, 64), (257, 96, 33), (1024, 1024, 64),
                                   (128, 32, 64), (256, 96, 64), (384, 160, 64), (200, 288, 60)])
def test_matmul_shapes(vh, M, K, N):
    """Parity at the block step's scale (activations ~N(0,1), weights
    ~N(0,0.02)); and, with both operands ~N(0,1), the error bound every f32
    sum of K products obeys whatever its order: |s - exact| <= gamma_K sum|a||b|
    with gamma_K = K u / (1 - K u), u = 2^-24 (Higham, Accuracy and Stability of
    Numerical Algorithms, eq. 3.5) -- the CPU chain and the matrix cores both
    meet it, and a wrong index or dropped term breaks it."""
    print("matmul", M, K, N, flush=True)
    r = np.random.default_rng(M * 1000 + K + N)
    a = r.standard_normal((M, K), dtype=np.float32)
    b = (r.standard_normal((K, N)) * 0.02).astype(np.float32)
    ref = O.matmul(a, b)
    ref64 = a.astype(np.float64) @ b.astype(np.float64)
    b1 = r.standard_normal((K, N), dtype=np.float32)
    exact1 = a.astype(np.float64) @ b1.astype(np.float64)
    u = 2.0 ** -24
    bound = (K * u / (1 - K * u)) * (np.abs(a).astype(np.float64) @ np.abs(b1).astype(np.float64))
    assert np.all(np.abs(O.matmul(a, b1) - exact1) <= bound)
    for av in (None, "T"):
        for bv in (None, "T"):
            for off in (0, 1):
                got = run_matmul(vh, a, b, av, bv, off)
                assert_parity(got, ref, ref64, name=f"{M}x{K}x{N} a={av} b={bv} off={off}")
                got1 = run_matmul(vh, a, b1, av, bv, off)
                assert np.all(np.abs(got1 - exact1) <= bound), f"{M}x{K}x{N} a={av} b={bv} off={off}: bound"


def test_matmul_batched_broadcast(vh):
    r = np.random.default_rng(7)
    a = r.standard_normal((2, 1, 37, 45), dtype=np.float32)
    b = (r.standard_normal((3, 45, 29)) * 0.02).astype(np.float32)
    assert_parity(run_matmul(vh, a, b), O.matmul(a, b), np.matmul(a.astype(np.float64), b), name="bcast")
    a5 = r.standard_normal((2, 2, 3, 9, 17), dtype=np.float32)  # three batch dims
    b5 = (r.standard_normal((17, 11)) * 0.02).astype(np.float32)
    assert_parity(run_matmul(vh, a5, b5), O.matmul(a5, b5), name="rank5")


def test_matmul_folds_shared_weight_batches(vh):
    """A [B, S, K] input times a weight shared by every batch (Linear::forward's
    input.matmul(weight.transpose(0, 1)), crates/vearo-nn/src/lib.rs:121-122)
    runs as one product over B*S rows, on the large-product kernel at this
    size; a left operand whose batches are not evenly spaced rows (its
    transposed view) stays a batched product (on the large-product kernel's
    batched walk at this size). Same results either way."""
    r = np.random.default_rng(12)
    a = r.standard_normal((4, 1024, 768), dtype=np.float32)
    w = (r.standard_normal((2304, 768)) * 0.02).astype(np.float32)
    ref = O.matmul(a, np.ascontiguousarray(w.T))
    ref64 = a.astype(np.float64) @ w.T.astype(np.float64)
    got = run_matmul(vh, a, w.T, b_view="T")
    assert vh.lib.vh_gemm_last_path() == vh.GEMM_PATH_PERSISTENT
    assert_parity(got, ref, ref64, name="folded batches")
    got_t = run_matmul(vh, a, w.T, a_view="T", b_view="T")
    assert vh.lib.vh_gemm_last_path() in (vh.GEMM_PATH_TILED, vh.GEMM_PATH_BATCHED, vh.GEMM_PATH_PERSISTENT)
    assert_parity(got_t, ref, ref64, name="batched")


def test_matmul_zero_k_and_errors(vh):
    a = np.zeros((3, 0), np.float32)
    b = np.zeros((0, 4), np.float32)
    A, B = out(vh, (1,)), out(vh, (1,))
    C = dev(vh, np.full((3, 4), 7.0, np.float32))
    vh.check(vh.lib.vh_matmul(A.ptr, ctypes.byref(vh.layout(a.shape)), B.ptr, ctypes.byref(vh.layout(b.shape)),
                              C.ptr, None))
    assert np.all(fetch(vh, C, (3, 4)) == 0.0)
    for la, lb, msg in (((2, 3), (4, 5), "Incompatible dimensions for matmul"),
                        ((3,), (3, 2), "Matmul requires rank >= 2"),
                        ((2, 2, 3), (3, 3, 2), "Batch shapes are not broadcastable")):
        with pytest.raises(vh.VhError, match=msg):
            vh.check(vh.lib.vh_matmul(A.ptr, ctypes.byref(vh.layout(la)), B.ptr, ctypes.byref(vh.layout(lb)),
                                      C.ptr, None))


def test_matmul_operands_broadcast_along_k(vh):
    """Operands whose k dim has stride 0 (a [M, 1] column and a [1, N] row
    broadcast to [M, K] and [K, N]) at a size the large-product kernel would
    take, with K % 32 != 0: the last k tile must not read the broadcast
    values again past K (each would add 32 - K % 32 extra products), so the
    partial tile goes to the kernel that tests k < K."""
    r = np.random.default_rng(31)
    M, N = 1024, 1024
    for K in (100, 1000):
        acol = r.standard_normal(M, dtype=np.float32)
        brow = (r.standard_normal(N) * 0.05).astype(np.float32)
        A, B, C = dev(vh, acol), dev(vh, brow), out(vh, (M, N))
        al = vh.layout((M, K), (1, 0))
        bl = vh.layout((K, N), (0, 1))
        vh.check(vh.lib.vh_matmul(A.ptr, ctypes.byref(al), B.ptr, ctypes.byref(bl), C.ptr, None))
        a = np.ascontiguousarray(np.broadcast_to(acol[:, None], (M, K)))
        b = np.ascontiguousarray(np.broadcast_to(brow[None, :], (K, N)))
        assert_parity(fetch(vh, C, (M, N)), O.matmul(a, b), a.astype(np.float64) @ b.astype(np.float64),
                      name=f"stride-0 k, K={K}")


def gemm_desc(vh, M, N, K, a, a_sm, a_sk, b, b_sk, b_sn, c, c_sm, **kw):
    d = vh.VhGemmDesc()
    d.M, d.N, d.K = M, N, K
    d.a, d.a_sm, d.a_sk = a, a_sm, a_sk
    d.b, d.b_sk, d.b_sn = b, b_sk, b_sn
    d.c, d.c_sm = c, c_sm
    d.batch[0] = d.batch[1] = 1
    d.alpha = kw.get("alpha", 1.0)
    d.accumulate = kw.get("accumulate", 0)
    d.causal = kw.get("causal", 0)
    if "e" in kw:
        d.e, d.e_sm, d.e_sn = kw["e"], kw["e_sm"], kw["e_sn"]
    if "batch" in kw:
        d.batch[0], d.batch[1] = kw["batch"]
        d.a_sb[0], d.a_sb[1] = kw["a_sb"]
        d.b_sb[0], d.b_sb[1] = kw["b_sb"]
        d.c_sb[0], d.c_sb[1] = kw["c_sb"]
        if "e_sb" in kw:
            d.e_sb[0], d.e_sb[1] = kw["e_sb"]
    d.engine = kw.get("engine", vh.GEMM_ENGINE_DEFAULT)
    return d


def test_gemm_epilogue_scale_bias_accumulate(vh):
    r = np.random.default_rng(8)
    M, K, N = 200, 96, 150
    a = r.standard_normal((M, K), dtype=np.float32)
    w = (r.standard_normal((N, K)) * 0.02).astype(np.float32)  # Linear weight [out, in]
    bias = (r.standard_normal(N) * 0.02).astype(np.float32)
    c0 = r.standard_normal((M, N), dtype=np.float32)
    A, W, BI, C = dev(vh, a), dev(vh, w), dev(vh, bias), dev(vh, c0)
    mm = O.matmul(a, np.ascontiguousarray(w.T))
    # y = x W^T + b (Linear, nn:120-128): B[k, n] = W[n, k].
    d = gemm_desc(vh, M, N, K, A.ptr, K, 1, W.ptr, 1, K, C.ptr, N, e=BI.ptr, e_sm=0, e_sn=1)
    vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
    assert_parity(fetch(vh, C, (M, N)), mm + bias, name="linear")
    # C = C + alpha * (A W^T), the gradient-accumulation form.
    C2 = dev(vh, c0)
    d = gemm_desc(vh, M, N, K, A.ptr, K, 1, W.ptr, 1, K, C2.ptr, N, alpha=0.125, accumulate=1)
    vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
    assert_parity(fetch(vh, C2, (M, N)), c0 + mm * np.float32(0.125), name="accumulate")


def test_gemm_causal_modes(vh):
    r = np.random.default_rng(9)
    S, D = 300, 40
    lower = np.tril(r.standard_normal((S, S), dtype=np.float32))
    upper = np.triu(r.standard_normal((S, S), dtype=np.float32))
    x = (r.standard_normal((S, D)) * 0.02).astype(np.float32)
    L, U, X = dev(vh, lower), dev(vh, upper), dev(vh, x)
    # K_LE_M: A[m, k] = 0 for k > m; K_GE_M: A[m, k] = 0 for k < m.
    for A_, a_np, mode in ((L, lower, vh.GEMM_K_LE_M), (U, upper, vh.GEMM_K_GE_M)):
        C = out(vh, (S, D))
        d = gemm_desc(vh, S, D, S, A_.ptr, S, 1, X.ptr, D, 1, C.ptr, D, causal=mode)
        vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
        assert_parity(fetch(vh, C, (S, D)), O.matmul(a_np, x), name=f"mode {mode}")
    # SKIP_UPPER: scores q k^T; entries on and below the diagonal are exact.
    q = r.standard_normal((S, D), dtype=np.float32)
    Q = dev(vh, q)
    C = out(vh, (S, S))
    d = gemm_desc(vh, S, S, D, Q.ptr, D, 1, X.ptr, 1, D, C.ptr, S, causal=vh.GEMM_SKIP_UPPER)
    vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
    got = fetch(vh, C, (S, S))
    ref = O.matmul(q, np.ascontiguousarray(x.T))
    il = np.tril_indices(S)
    assert_parity(got[il], ref[il], name="skip upper")


@pytest.mark.parametrize("akc,bkc", [(True, True), (True, False), (False, True), (False, False)])
def test_gemm_persistent_short_k(vh, akc, bkc):
    """Batched products with K <= 256 and 128-bit operand layouts run the
    persistent kernel (vh_gemmp_*, one workgroup per resident slot walking the
    tiles): edge tiles, a ragged last k tile, the causal triangle, an addend
    (per element and a broadcast bias), alpha and accumulation, and more work
    items than resident workgroups (the 120-batch cases)."""
    r = np.random.default_rng(11)
    cases = ((3, 5, 200, 300, 40, 0, "full", 0), (2, 3, 300, 300, 64, 1, None, 1),
             (6, 20, 384, 384, 64, 1, None, 0), (4, 30, 256, 384, 96, 0, "bias", 1),
             (2, 2, 256, 384, 64, 1, "full", 1))
    for B0, B1, M, N, K, causal, ekind, acc in cases:
        a = r.standard_normal((B0, B1, M, K), dtype=np.float32)
        b = (r.standard_normal((B0, B1, K, N)) * 0.1).astype(np.float32)
        c0 = r.standard_normal((B0, B1, M, N), dtype=np.float32)
        # A stored k-contiguous [.., M, K] or as its transpose [.., K, M]; B as
        # [.., N, K] (k-contiguous) or [.., K, N].
        A = dev(vh, a if akc else np.swapaxes(a, -1, -2))
        Bb = dev(vh, np.swapaxes(b, -1, -2) if bkc else b)
        C = dev(vh, c0)
        d = gemm_desc(vh, M, N, K, A.ptr, K if akc else 1, 1 if akc else M, Bb.ptr, 1 if bkc else N,
                      K if bkc else 1, C.ptr, N, alpha=0.125, accumulate=acc, causal=causal)
        d.batch[0], d.batch[1] = B0, B1
        d.a_sb[0], d.a_sb[1] = B1 * M * K, M * K
        d.b_sb[0], d.b_sb[1] = B1 * K * N, K * N
        d.c_sb[0], d.c_sb[1] = B1 * M * N, M * N
        e = np.zeros((B0, B1, M, N), np.float32)
        keep = None
        if ekind == "full":
            e = r.standard_normal((B0, B1, M, N), dtype=np.float32)
            keep = dev(vh, e)
            d.e, d.e_sm, d.e_sn = keep.ptr, N, 1
            d.e_sb[0], d.e_sb[1] = B1 * M * N, M * N
        elif ekind == "bias":
            bias = r.standard_normal(N, dtype=np.float32)
            e = np.broadcast_to(bias, (B0, B1, M, N))
            keep = dev(vh, bias)
            d.e, d.e_sm, d.e_sn = keep.ptr, 0, 1
        vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
        got = fetch(vh, C, (B0, B1, M, N))
        mm = O.matmul(a, b)
        cpu = mm * np.float32(0.125) + e
        ref64 = np.matmul(a.astype(np.float64), b) * 0.125 + e
        if acc:
            cpu = c0 + cpu
            ref64 = c0 + ref64
        name = f"persistent {B0}x{B1} {M}x{N}x{K} causal={causal} e={ekind} acc={acc} akc={akc} bkc={bkc}"
        if causal:  # entries on and below the diagonal are defined
            il = np.tril_indices(M, 0, N)
            got, cpu, ref64 = got[..., il[0], il[1]], cpu[..., il[0], il[1]], ref64[..., il[0], il[1]]
        assert_parity(got, cpu, ref64, name=name)
        del keep


def attention_gpu(vh, q, k, v, mask, causal, go=None, layout="bhsd"):
    """Fused attention fwd (and bwd when go is given) on the device. layout
    'bshd' stores q/k/v/out as [B, S, H, Dk] and passes [B, H, S, Dk] views."""
    B, H, S, Dk = q.shape
    def put(x):
        if layout == "bshd":
            store = np.ascontiguousarray(np.transpose(x, (0, 2, 1, 3)))
            return dev(vh, store), vh.layout((B, H, S, Dk), (S * H * Dk, Dk, H * Dk, 1))
        return dev(vh, x), vh.layout(x.shape)
    def empty():
        return out(vh, (B, H, S, Dk)), (vh.layout((B, H, S, Dk), (S * H * Dk, Dk, H * Dk, 1))
                                        if layout == "bshd" else vh.layout((B, H, S, Dk)))
    def get(buf):
        a = fetch(vh, buf, (B, S, H, Dk) if layout == "bshd" else (B, H, S, Dk))
        return np.transpose(a, (0, 2, 1, 3)) if layout == "bshd" else a
    Q, ql = put(q)
    K, kl = put(k)
    V, vl = put(v)
    Mk, ml = (dev(vh, mask), vh.layout(mask.shape)) if mask is not None else (None, None)
    mptr = Mk.ptr if Mk is not None else None
    mlp = ctypes.byref(ml) if ml is not None else None
    Ot, ol = empty()
    vh.check(vh.lib.vh_fused_attention_fwd(Q.ptr, ctypes.byref(ql), K.ptr, ctypes.byref(kl), V.ptr,
                                           ctypes.byref(vl), mptr, mlp, causal, Ot.ptr, ctypes.byref(ol),
                                           None, 0, None))
    res = [get(Ot)]
    if go is not None:
        G, gl = put(go)
        (DQ, dql), (DK, dkl), (DV, dvl) = empty(), empty(), empty()
        vh.check(vh.lib.vh_fused_attention_bwd(Q.ptr, ctypes.byref(ql), K.ptr, ctypes.byref(kl), V.ptr,
                                               ctypes.byref(vl), mptr, mlp, causal, G.ptr, ctypes.byref(gl),
                                               DQ.ptr, ctypes.byref(dql), DK.ptr, ctypes.byref(dkl), DV.ptr,
                                               ctypes.byref(dvl), None, 0, None))
        res += [get(DQ), get(DK), get(DV)]
    return res


def test_attention_backward_from_saved_probs(vh):
    """vh_fused_attention_bwd_probs on the probabilities left in the forward's
    scratch gives the same bits as the recomputing backward."""
    B, H, S, Dk = 2, 3, 200, 32
    r = np.random.default_rng(13)
    q, k, v, go = (r.standard_normal((B, H, S, Dk), dtype=np.float32) for _ in range(4))
    Q, K, V, G = (dev(vh, a) for a in (q, k, v, go))
    l = vh.layout((B, H, S, Dk))
    nsc = vh.lib.vh_fused_attention_scratch_bytes(B, H, S, 0)
    SC, WS = vh.DeviceBuffer(nsc), vh.DeviceBuffer(nsc)
    O_ = out(vh, q.shape)
    vh.check(vh.lib.vh_fused_attention_fwd(Q.ptr, ctypes.byref(l), K.ptr, ctypes.byref(l), V.ptr, ctypes.byref(l),
                                           None, None, 1, O_.ptr, ctypes.byref(l), SC.ptr, nsc, None))
    r1 = [out(vh, q.shape) for _ in range(3)]
    r2 = [out(vh, q.shape) for _ in range(3)]
    vh.check(vh.lib.vh_fused_attention_bwd(Q.ptr, ctypes.byref(l), K.ptr, ctypes.byref(l), V.ptr, ctypes.byref(l),
                                           None, None, 1, G.ptr, ctypes.byref(l), r1[0].ptr, ctypes.byref(l),
                                           r1[1].ptr, ctypes.byref(l), r1[2].ptr, ctypes.byref(l), None, 0, None))
    vh.check(vh.lib.vh_fused_attention_bwd_probs(SC.ptr, Q.ptr, ctypes.byref(l), K.ptr, ctypes.byref(l), V.ptr,
                                                 ctypes.byref(l), 1, G.ptr, ctypes.byref(l), r2[0].ptr,
                                                 ctypes.byref(l), r2[1].ptr, ctypes.byref(l), r2[2].ptr,
                                                 ctypes.byref(l), WS.ptr, nsc, None))
    for a, b in zip(r1, r2):
        np.testing.assert_array_equal(fetch(vh, a, q.shape), fetch(vh, b, q.shape))


@pytest.mark.parametrize("tag", ["attkat", "attc", "attm", "attn"])
def test_attention_golden(vh, tag):
    print("attention", tag, flush=True)
    q, k, v, go = (GOLD[f"{tag}_{n}"] for n in ("q", "k", "v", "go"))
    mask = GOLD[f"{tag}_mask"] if f"{tag}_mask" in GOLD.files else None
    ref = [O.fused_attention(q, k, v, mask)] + list(O.fused_attention_backward(q, k, v, mask, go))
    ref64 = [GOLD[f"{tag}_{n}"] for n in ("out", "dq", "dk", "dv")]
    causal_ok = tag in ("attkat", "attc")  # masks that are the causal -1e9 triangle
    variants = [(mask, 0)] + ([(mask, 1), (None, 1)] if causal_ok else [])
    for m, causal in variants:
        for lay in ("bhsd", "bshd"):
            got = attention_gpu(vh, q, k, v, m, causal, go, lay)
            for name, g, c, r64 in zip(("out", "dq", "dk", "dv"), got, ref, ref64):
                assert_parity(g, c, r64, name=f"{tag} {name} mask={m is not None} causal={causal} {lay}")


def test_attention_gpt_shape(vh):
    """[2, 12, 1024, 64] causal, q/k/v as [B, S, H, Dk] views (the model's
    layout); oracle on a sample of heads."""
    B, H, S, Dk = 2, 12, 1024, 64
    print("attention gpt shape", flush=True)
    r = np.random.default_rng(10)
    q, k, v, go = (r.standard_normal((B, H, S, Dk), dtype=np.float32) for _ in range(4))
    mask = np.zeros((S, S), np.float32)
    mask[np.triu_indices(S, 1)] = -1e9
    got = attention_gpu(vh, q, k, v, None, 1, go, "bshd")
    for b, h in ((0, 0), (1, 7), (1, 11)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        ref = [O.fused_attention(q[sl], k[sl], v[sl], mask)] + list(
            O.fused_attention_backward(q[sl], k[sl], v[sl], mask, go[sl]))
        for name, g, c in zip(("out", "dq", "dk", "dv"), got, ref):
            assert_parity(g[sl], c, name=f"{name}[{b},{h}]")


def mask_is_causal(vh, q, k, v, mask, go=None):
    """vh_attention_mask_is_causal on contiguous [B, H, S, Dk] operands."""
    l = vh.layout(q.shape)
    Q, K, V, M = dev(vh, q), dev(vh, k), dev(vh, v), dev(vh, mask)
    ml = vh.layout(mask.shape)
    G = dev(vh, go) if go is not None else None
    c = ctypes.c_int(-1)
    vh.check(vh.lib.vh_attention_mask_is_causal(Q.ptr, ctypes.byref(l), K.ptr, ctypes.byref(l), V.ptr,
                                                ctypes.byref(l), G.ptr if G else None,
                                                ctypes.byref(l) if G else None, M.ptr, ctypes.byref(ml),
                                                ctypes.byref(c), None))
    return c.value


@pytest.mark.parametrize("case,want", [
    ("tri -1e9", 1), ("tri -inf", 1), ("tri [1,1,S,S]", 1), ("tri [B,1,S,S]", 1), ("tri, bwd operands", 1),
    ("allowed entry 0.5", 0), ("masked entry -0.5", 0), ("masked entry 0", 0), ("masked entry NaN", 0),
    ("masked -1e3, scores ~1e4", 0), ("q holds inf", 0), ("v holds NaN", 0), ("dout holds inf", 0),
    ("row-broadcast mask [1,S]", 0), ("masked -1e3, small scores", 1)])
def test_attention_mask_probe(vh, case, want):
    """The probe that lets the BackendOps attention slots take the causal
    kernels: yes for the model's -1e9 (or -inf) triangle in any broadcast form
    with ordinary operands; no for any entry off the pattern, a masked value
    that small scores could overtake, or a non-finite operand (whose zero
    probabilities would still make NaN in the dense form). When it says yes the
    causal kernels give the dense masked form's bits."""
    B, H, S, Dk = 2, 3, 160, 32
    r = np.random.default_rng(abs(hash(case)) % 2**32)
    q, k, v, go = (r.standard_normal((B, H, S, Dk), dtype=np.float32) for _ in range(4))
    tri = np.zeros((S, S), np.float32)
    tri[np.triu_indices(S, 1)] = -1e9
    mask, g = tri, None
    if case == "tri -inf":
        mask = np.where(tri < 0, -np.inf, 0).astype(np.float32)
    elif case == "tri [1,1,S,S]":
        mask = tri[None, None]
    elif case == "tri [B,1,S,S]":
        mask = np.stack([tri, tri])[:, None]
    elif case == "tri, bwd operands":
        g = go
    elif case == "allowed entry 0.5":
        mask = tri.copy(); mask[7, 3] = 0.5
    elif case == "masked entry -0.5":
        mask = tri.copy(); mask[3, 7] = -0.5
    elif case == "masked entry 0":
        mask = tri.copy(); mask[3, 7] = 0.0
    elif case == "masked entry NaN":
        mask = tri.copy(); mask[3, 7] = np.nan
    elif case == "masked -1e3, scores ~1e4":
        mask = np.where(tri < 0, -1e3, 0).astype(np.float32)
        q, k = q * 10, k * 10
    elif case == "masked -1e3, small scores":
        mask = np.where(tri < 0, -1e3, 0).astype(np.float32)
    elif case == "q holds inf":
        q[1, 2, 3, 4] = np.inf
    elif case == "v holds NaN":
        v[0, 1, 150, 5] = np.nan
    elif case == "dout holds inf":
        g = go.copy(); g[1, 0, 0, 0] = -np.inf
    elif case == "row-broadcast mask [1,S]":
        mask = np.zeros((1, S), np.float32)
    print("mask probe", case, flush=True)
    assert mask_is_causal(vh, q, k, v, mask, g) == want
    gg = g if g is not None else go
    dense = attention_gpu(vh, q, k, v, mask, 0, gg)
    if want:
        causal = attention_gpu(vh, q, k, v, None, 1, gg)
        for name, a, b in zip(("out", "dq", "dk", "dv"), dense, causal):
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"{case} {name}")
    # VH_ATTN_CAUSAL_AUTO makes the same decision on the device (the launches
    # read its flag): the dense masked form's bits whatever it decides.
    auto = attention_gpu(vh, q, k, v, mask, 2, gg)
    for name, a, b in zip(("out", "dq", "dk", "dv"), dense, auto):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"{case} auto {name}")


def test_attention_mask_probe_under_graph_capture(vh):
    """The host-answer probe needs a host wait, which a capturing stream does
    not allow: there it answers 0 and launches nothing (the captured graph is
    empty)."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so.7")
    B, H, S, Dk = 1, 2, 64, 16
    r = np.random.default_rng(5)
    q, k, v = (r.standard_normal((B, H, S, Dk), dtype=np.float32) for _ in range(3))
    tri = np.zeros((S, S), np.float32)
    tri[np.triu_indices(S, 1)] = -1e9
    assert mask_is_causal(vh, q, k, v, tri, None) == 1
    Q, K, V, M = dev(vh, q), dev(vh, k), dev(vh, v), dev(vh, tri)
    ql, ml = vh.layout(q.shape), vh.layout(tri.shape)
    st = C.c_void_p()
    assert hip.hipStreamCreate(C.byref(st)) == 0
    vh.sync()
    assert hip.hipStreamBeginCapture(st, 2) == 0  # relaxed mode
    res = C.c_int(7)
    rc = vh.lib.vh_attention_mask_is_causal(Q.ptr, C.byref(ql), K.ptr, C.byref(ql), V.ptr, C.byref(ql), None, None,
                                            M.ptr, C.byref(ml), C.byref(res), st)
    graph = C.c_void_p()
    assert hip.hipStreamEndCapture(st, C.byref(graph)) == 0
    nodes = C.c_size_t(99)
    assert hip.hipGraphGetNodes(graph, None, C.byref(nodes)) == 0
    hip.hipGraphDestroy(graph)
    hip.hipStreamDestroy(st)
    vh.check(rc)
    assert res.value == 0 and nodes.value == 0


@pytest.mark.parametrize("n", [4096, 1000003])
def test_adamw_matches_oracle(vh, n):
    r = np.random.default_rng(n)
    p = r.standard_normal(n).astype(np.float32)
    P, M, V = dev(vh, p), dev(vh, np.zeros(n, np.float32)), dev(vh, np.zeros(n, np.float32))
    pc, mc, vc = p.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for t in (1, 2, 3):
        g = (r.standard_normal(n) * 0.1).astype(np.float32)
        Gd = dev(vh, g)
        vh.check(vh.lib.vh_adamw_step(P.ptr, Gd.ptr, M.ptr, V.ptr, n, t, 0.02, 0.9, 0.95, 1e-8, 0.01, None))
        O.adamw_step(pc, g, mc, vc, t, 0.02, 0.9, 0.95, 1e-8, 0.01)
        assert_parity(fetch(vh, P, (n,)), pc, name=f"p t={t}")
        assert_parity(fetch(vh, M, (n,)), mc, name=f"m t={t}")
        assert_parity(fetch(vh, V, (n,)), vc, name=f"v t={t}")


@pytest.mark.parametrize("rows,C", [(1, 5), (16384, 768), (1000, 3072), (37, 1)])
def test_sum_rows(vh, rows, C):
    r = np.random.default_rng(rows + C)
    x = r.standard_normal((rows, C), dtype=np.float32)
    X, OUT = dev(vh, x), out(vh, (C,))
    vh.check(vh.lib.vh_sum_rows(X.ptr, rows, C, OUT.ptr, None, 0, None))
    assert_parity(fetch(vh, OUT, (C,)), O.reduce_to(x, (C,)), x.astype(np.float64).sum(axis=0), name="sum_rows")


@pytest.mark.parametrize("M,N,K", [(64, 64, 8192), (200, 64, 4096), (200, 150, 8192), (768, 768, 16384)])
def test_gemm_split_k(vh, M, N, K):
    """Few C tiles over a long K (weight-gradient shapes) on the tiled kernel's
    split-K path, forced with the TILED engine and checked through
    vh_gemm_last_path: the K-range partials summed in a fixed order by
    vh_gemm_reduce, then alpha, a column bias and accumulation into C."""
    print("split-k", M, N, K, flush=True)
    r = np.random.default_rng(M + N + K)
    # dW = dy^T x as the block step issues it: A m-contiguous (dy [K, M]), B = x [K, N].
    dy = (r.standard_normal((K, M)) * 0.02).astype(np.float32)
    x = r.standard_normal((K, N), dtype=np.float32)
    bias = (r.standard_normal(N) * 0.02).astype(np.float32)
    c0 = r.standard_normal((M, N), dtype=np.float32)
    DY, X, BI = dev(vh, dy), dev(vh, x), dev(vh, bias)
    ref = O.matmul(np.ascontiguousarray(dy.T), x)
    ref64 = dy.T.astype(np.float64) @ x.astype(np.float64)
    tiled = vh.GEMM_ENGINE_TILED
    C = out(vh, (M, N))
    d = gemm_desc(vh, M, N, K, DY.ptr, 1, M, X.ptr, N, 1, C.ptr, N, engine=tiled)
    vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
    assert vh.lib.vh_gemm_last_path() == vh.GEMM_PATH_SPLIT_K
    got = fetch(vh, C, (M, N))
    assert_parity(got, ref, ref64, name="split-k plain")
    C2 = dev(vh, c0)
    d = gemm_desc(vh, M, N, K, DY.ptr, 1, M, X.ptr, N, 1, C2.ptr, N, alpha=0.5, accumulate=1,
                  e=BI.ptr, e_sm=0, e_sn=1, engine=tiled)
    vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
    assert vh.lib.vh_gemm_last_path() == vh.GEMM_PATH_SPLIT_K
    assert_parity(fetch(vh, C2, (M, N)), c0 + (ref * np.float32(0.5) + bias),
                  c0.astype(np.float64) + (ref64 * 0.5 + bias), name="split-k epilogue")
    # Deterministic: the same call gives the same bits.
    C3 = out(vh, (M, N))
    d = gemm_desc(vh, M, N, K, DY.ptr, 1, M, X.ptr, N, 1, C3.ptr, N, engine=tiled)
    vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
    np.testing.assert_array_equal(fetch(vh, C3, (M, N)), got)


# The persistent 256 x 192-tile kernel at the block step's shapes (fewer rows
# where the full product would keep the oracle busy): every layout pair, tile
# edges in M and N, a stream-K last round (tiles mod CUs != 0), a ragged K
# (50260 = 1570 x 32 + 20: the tiled kernel adds the tail), and the Linear
# epilogues (bias, bias + residual accumulation, alpha). A is N(0,1) times
# a_scale: lm_head dx's A is dlogits, whose entries are ~1e-4 (softmax over
# 50257 classes, divided by the row count), so a 50260-term row sum of it
# stays far from cancellation; the plain cases also meet the f32 error bound
# of a K-term sum in any order, which holds for any data.
#   name, M, N, K, A k-contiguous, B k-contiguous, epilogue, a_scale
PERSISTENT_CASES = [
    ("lm_head fwd", 1024, 50257, 768, True, True, "", 1.0),
    ("lm_head dx", 512, 768, 50260, True, False, "", 1e-3),
    ("lm_head dW", 50260, 768, 512, False, False, "", 1.0),
    ("qkv fwd + bias", 2048, 2304, 768, True, True, "bias", 1.0),
    ("fc2 fwd + bias + residual", 2048, 768, 3072, True, True, "bias_acc", 1.0),
    ("fc1 dW", 3072, 768, 2048, False, False, "", 1.0),
    ("m-contiguous A, k-contiguous B", 1000, 777, 1536, False, True, "alpha", 1.0),
    ("edges", 1000, 1001, 2052, True, True, "alpha_acc", 1.0),
    # Operands only 4-byte aligned (32-bit loads): the drop-in step's logits
    # gradient has rows of V = 50257 floats; bases one float off 16 bytes.
    ("lm_head dx, odd V", 512, 768, 50257, True, False, "", 1e-3, 0),
    ("lm_head dW^T, odd V", 768, 50257, 512, False, False, "", 1.0, 0),
    ("m-contiguous A, odd M", 1001, 777, 1536, False, True, "", 1.0, 0),
    ("edges, bases one float off", 1000, 1001, 2052, True, True, "alpha_acc", 1.0, 1),
    # k-contiguous B with rows 32 KB apart (its lines prefetched a k tile ahead)
    ("m-contiguous A, far-apart B rows", 1024, 768, 8192, False, True, "", 1.0, 0),
    ("far-apart A rows, bias", 1024, 776, 5000, True, False, "bias", 1.0, 0),
]


@pytest.mark.parametrize("case", PERSISTENT_CASES, ids=[c[0] for c in PERSISTENT_CASES])
def test_gemm_persistent_block_shapes(vh, case):
    name, M, N, K, akc, bkc, epi, a_scale = case[:8]
    off = case[8] if len(case) > 8 else 0  # floats before each operand's first element
    print("persistent", case, flush=True)
    r = np.random.default_rng(M * 7 + N * 3 + K)
    a = (r.standard_normal((M, K)) * a_scale).astype(np.float32)
    b = (r.standard_normal((K, N)) * 0.05).astype(np.float32)
    # Operands stored as the block step stores them: k-contiguous A is a [M, K]
    # row-major array; m-contiguous A is stored transposed ([K, M]); likewise B.
    pad = np.zeros(off, np.float32)
    Abuf = dev(vh, np.concatenate([pad, (a if akc else a.T).reshape(-1)]))
    Bbuf = dev(vh, np.concatenate([pad, (b.T if bkc else b).reshape(-1)]))

    class _At:  # device address `off` floats into the buffer
        def __init__(self, buf):
            self.ptr = buf.ptr + 4 * off
    A, B = _At(Abuf), _At(Bbuf)
    a_sm, a_sk = (K, 1) if akc else (1, M)
    b_sk, b_sn = (1, K) if bkc else (N, 1)
    ref = O.matmul(a, b)
    ref64 = a.astype(np.float64) @ b.astype(np.float64)
    kw = {}
    c0 = np.zeros((M, N), np.float32)
    want, want64 = ref, ref64
    alpha = np.float32(0.75) if "alpha" in epi else np.float32(1.0)
    if "alpha" in epi:
        kw["alpha"] = float(alpha)
        want, want64 = ref * alpha, ref64 * float(alpha)
    if "bias" in epi:
        bias = (r.standard_normal(N) * 0.1).astype(np.float32)
        BI = dev(vh, bias)
        kw.update(e=BI.ptr, e_sm=0, e_sn=1)
        want, want64 = want + bias, want64 + bias.astype(np.float64)
    if "acc" in epi:
        c0 = r.standard_normal((M, N), dtype=np.float32)
        kw["accumulate"] = 1
        want, want64 = c0 + want, c0.astype(np.float64) + want64
    C = dev(vh, c0)
    d = gemm_desc(vh, M, N, K, A.ptr, a_sm, a_sk, B.ptr, b_sk, b_sn, C.ptr, N, **kw)
    vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
    assert vh.lib.vh_gemm_last_path() == vh.GEMM_PATH_PERSISTENT, name
    got = fetch(vh, C, (M, N))
    assert_parity(got, want, want64, name=f"persistent {name}")
    if not epi:
        u = 2.0 ** -24
        bound = (K * u / (1 - K * u)) * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
        assert np.all(np.abs(got - ref64) <= bound), f"persistent {name}: f32 error bound"
    if not kw.get("accumulate"):
        # Deterministic (fixed stream-K split and fix-up order): same bits again.
        C2 = out(vh, (M, N))
        d = gemm_desc(vh, M, N, K, A.ptr, a_sm, a_sk, B.ptr, b_sk, b_sn, C2.ptr, N, **kw)
        vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
        np.testing.assert_array_equal(fetch(vh, C2, (M, N)), got)


def test_gemm_persistent_few_k_tiles_after_workspace_reuse(vh):
    """Stream-K with fewer k tiles than workgroups leaves some workgroups an
    empty run inside a split tile; the fix-up must skip their workspace slots,
    which hold whatever an earlier product left there. A product with many
    partial pieces first fills the (reused) workspace, then products with
    102 and 120 k tiles in their stream-K round run against the oracle."""
    r = np.random.default_rng(21)
    def prod(M, N, K):
        a = r.standard_normal((M, K), dtype=np.float32)
        b = (r.standard_normal((K, N)) * 0.05).astype(np.float32)
        A, B, C = dev(vh, a), dev(vh, np.ascontiguousarray(b.T)), out(vh, (M, N))
        d = gemm_desc(vh, M, N, K, A.ptr, K, 1, B.ptr, 1, K, C.ptr, N)
        vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
        assert vh.lib.vh_gemm_last_path() == vh.GEMM_PATH_PERSISTENT
        return fetch(vh, C, (M, N)), a, b
    prod(1024, 1000, 2048)  # 24 tiles x 64 k tiles split over every workgroup
    for M, N, K in ((256, 1000, 544), (300, 400, 640)):
        print("few k tiles", M, N, K, flush=True)
        got, a, b = prod(M, N, K)
        assert_parity(got, O.matmul(a, b), a.astype(np.float64) @ b.astype(np.float64), name=f"few k tiles {M}x{N}x{K}")


BATCHED_PERSISTENT_CASES = [
    # name, (B0, B1), M, N, K, akc, bkc, B shared over batches, epilogue
    ("drop-in weight gradients: x^T g per batch", (4, 1), 768, 768, 1024, False, False, False, ""),
    ("two batch dims, shared k-contiguous B, bias", (2, 3), 300, 200, 544, True, True, True, "bias"),
    ("k tail, accumulate, alpha", (3, 1), 256, 192, 1000, True, False, False, "acc alpha"),
    ("per-batch addend, stream-K remainder", (2, 1), 520, 400, 640, False, True, False, "full"),
]


@pytest.mark.parametrize("case", BATCHED_PERSISTENT_CASES, ids=[c[0] for c in BATCHED_PERSISTENT_CASES])
def test_gemm_persistent_batched(vh, case):
    """Batched dense products with k loops of 512 and more on the persistent
    kernel: the tile list runs over every batch (tile-major within a batch),
    each segment offsets A, B, C and the addend by its batch's strides, and a
    batch's k-contiguous tail past the whole k tiles goes through the tiled
    kernel. Against the oracle's batched matmul and float64, and the same bits
    on a second call."""
    name, (B0, B1), M, N, K, akc, bkc, shared, epi = case
    print("persistent batched", name, flush=True)
    r = np.random.default_rng(M + N + K)
    nb = B0 * B1
    a = r.standard_normal((B0, B1, M, K), dtype=np.float32)
    b = (r.standard_normal((1 if shared else B0, 1 if shared else B1, K, N)) * 0.05).astype(np.float32)
    A = dev(vh, np.ascontiguousarray(a if akc else np.swapaxes(a, 2, 3)))
    Bd = dev(vh, np.ascontiguousarray(np.swapaxes(b, 2, 3) if bkc else b))
    a_sm, a_sk = (K, 1) if akc else (1, M)
    b_sk, b_sn = (1, K) if bkc else (N, 1)
    kw = {}
    ref = O.matmul(a, b)
    ref64 = np.matmul(a.astype(np.float64), b.astype(np.float64))
    c0 = np.zeros((B0, B1, M, N), np.float32)
    keep = []
    if "alpha" in epi:
        kw["alpha"] = 0.5
        ref, ref64 = ref * np.float32(0.5), ref64 * 0.5
    if epi == "bias":
        bias = (r.standard_normal(N) * 0.1).astype(np.float32)
        keep.append(dev(vh, bias))
        kw.update(e=keep[-1].ptr, e_sm=0, e_sn=1)
        ref, ref64 = ref + bias, ref64 + bias
    if epi == "full":
        e = r.standard_normal((B0, B1, M, N), dtype=np.float32)
        keep.append(dev(vh, e))
        kw.update(e=keep[-1].ptr, e_sm=N, e_sn=1, e_sb=(B1 * M * N, M * N))
        ref, ref64 = ref + e, ref64 + e
    if "acc" in epi:
        c0 = r.standard_normal((B0, B1, M, N), dtype=np.float32)
        kw["accumulate"] = 1
        ref, ref64 = c0 + ref, c0 + ref64
    C = dev(vh, c0)
    bsb = (0, 0) if shared else (B1 * K * N, K * N)
    d = gemm_desc(vh, M, N, K, A.ptr, a_sm, a_sk, Bd.ptr, b_sk, b_sn, C.ptr, N, batch=(B0, B1),
                  a_sb=(B1 * M * K, M * K), b_sb=bsb, c_sb=(B1 * M * N, M * N), **kw)
    vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
    assert vh.lib.vh_gemm_last_path() == vh.GEMM_PATH_PERSISTENT, name
    got = fetch(vh, C, (B0, B1, M, N))
    assert_parity(got, ref, ref64, name=f"batched persistent {name}")
    if "acc" not in epi:
        C2 = out(vh, (B0, B1, M, N))
        d = gemm_desc(vh, M, N, K, A.ptr, a_sm, a_sk, Bd.ptr, b_sk, b_sn, C2.ptr, N, batch=(B0, B1),
                      a_sb=(B1 * M * K, M * K), b_sb=bsb, c_sb=(B1 * M * N, M * N), **kw)
        vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
        np.testing.assert_array_equal(fetch(vh, C2, (B0, B1, M, N)), got)


def test_gemm_library_engine_is_an_ab_only(vh):
    """The LIBRARY engine hands a large dense product to hipBLASLt (when it has
    an algorithm) and gives the same results to the parity bar; the default
    engine never does."""
    M, N, K = 1024, 1536, 768
    r = np.random.default_rng(5)
    a = r.standard_normal((M, K), dtype=np.float32)
    w = (r.standard_normal((N, K)) * 0.05).astype(np.float32)
    A, W, C = dev(vh, a), dev(vh, w), out(vh, (M, N))
    ref = O.matmul(a, np.ascontiguousarray(w.T))
    ref64 = a.astype(np.float64) @ w.T.astype(np.float64)
    d = gemm_desc(vh, M, N, K, A.ptr, K, 1, W.ptr, 1, K, C.ptr, N)
    vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
    assert vh.lib.vh_gemm_last_path() == vh.GEMM_PATH_PERSISTENT
    assert_parity(fetch(vh, C, (M, N)), ref, ref64, name="default engine")
    d = gemm_desc(vh, M, N, K, A.ptr, K, 1, W.ptr, 1, K, C.ptr, N, engine=vh.GEMM_ENGINE_LIBRARY)
    vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
    assert vh.lib.vh_gemm_last_path() in (vh.GEMM_PATH_LIBRARY, vh.GEMM_PATH_PERSISTENT)
    assert_parity(fetch(vh, C, (M, N)), ref, ref64, name="library engine")


def test_cross_entropy_row_stride(vh):
    B, V, ld = 37, 1001, 1004
    r = np.random.default_rng(12)
    logits = r.standard_normal((B, V), dtype=np.float32)
    tg = r.integers(0, V, size=B).astype(np.float32)
    padded = np.full((B, ld), 7.0, np.float32)
    padded[:, :V] = logits
    L, T, GO = dev(vh, padded), dev(vh, tg), dev(vh, np.float32([1.3]))
    LOSS = out(vh, (1,))
    DL = dev(vh, np.full((B, ld), -5.0, np.float32))
    vh.check(vh.lib.vh_cross_entropy_fwd_ld(L.ptr, ld, T.ptr, LOSS.ptr, B, V, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_bwd_ld(L.ptr, ld, T.ptr, GO.ptr, DL.ptr, B, V, None))
    assert_parity(fetch(vh, LOSS, (1,)), O.cross_entropy(logits, tg), name="loss")
    dl = fetch(vh, DL, (B, ld))
    assert_parity(dl[:, :V], O.cross_entropy_backward(logits, tg, np.float32([1.3])), name="dlogits")
    assert np.all(dl[:, V:] == -5.0)  # only the first V columns are written
    # Forward and backward in one pass: the same bits as the two passes.
    LOSS2, DL2 = out(vh, (1,)), dev(vh, np.full((B, ld), -5.0, np.float32))
    vh.check(vh.lib.vh_cross_entropy_fwd_bwd_ld(L.ptr, ld, T.ptr, GO.ptr, LOSS2.ptr, DL2.ptr, B, V, None, 0, None))
    np.testing.assert_array_equal(fetch(vh, LOSS2, (1,)), fetch(vh, LOSS, (1,)))
    np.testing.assert_array_equal(fetch(vh, DL2, (B, ld)), dl)
    # In place (dlogits == logits): the target logit is read before the row's
    # gradient stores, so the loss and gradients are the same bits again.
    LOSS3, IP = out(vh, (1,)), dev(vh, padded)
    vh.check(vh.lib.vh_cross_entropy_fwd_bwd_ld(IP.ptr, ld, T.ptr, GO.ptr, LOSS3.ptr, IP.ptr, B, V, None, 0, None))
    np.testing.assert_array_equal(fetch(vh, LOSS3, (1,)), fetch(vh, LOSS, (1,)))
    ip = fetch(vh, IP, (B, ld))
    np.testing.assert_array_equal(ip[:, :V], dl[:, :V])
    assert np.all(ip[:, V:] == 7.0)


@pytest.mark.parametrize("B,V", [(64, 50257), (48, 70001)])
def test_cross_entropy_fwd_bwd_in_place(vh, B, V):
    """The fused pass in place at the GPT-2 vocabulary (row-cached kernel) and
    past it (streaming kernels): loss and dlogits equal the out-of-place call's."""
    r = np.random.default_rng(B)
    logits = r.standard_normal((B, V), dtype=np.float32)
    tg = r.integers(0, V, size=B).astype(np.float32)
    L, T, GO = dev(vh, logits), dev(vh, tg), dev(vh, np.float32([1.0]))
    LOSS, DL, LOSS2 = out(vh, (1,)), out(vh, (B, V)), out(vh, (1,))
    vh.check(vh.lib.vh_cross_entropy_fwd_bwd_ld(L.ptr, V, T.ptr, GO.ptr, LOSS.ptr, DL.ptr, B, V, None, 0, None))
    vh.check(vh.lib.vh_cross_entropy_fwd_bwd_ld(L.ptr, V, T.ptr, GO.ptr, LOSS2.ptr, L.ptr, B, V, None, 0, None))
    np.testing.assert_array_equal(fetch(vh, LOSS2, (1,)), fetch(vh, LOSS, (1,)))
    np.testing.assert_array_equal(fetch(vh, L, (B, V)), fetch(vh, DL, (B, V)))
    assert_parity(fetch(vh, LOSS, (1,)), O.cross_entropy(logits, tg), name="loss")


ENGINES = [("default", 0), ("library", 2)]


@pytest.mark.parametrize("engine", ENGINES, ids=[e[0] for e in ENGINES])
@pytest.mark.parametrize("akc,bkc", [(True, True), (True, False), (False, False), (False, True)])
def test_plain_gemm_large(vh, akc, bkc, engine):
    """Large plain products (no batch, causal range, addend or accumulation)
    on the default engine (the persistent kernel) and on the LIBRARY engine
    (hipBLASLt, the benchmarks' A/B reference): the oracle's matmul within the
    parity bar at model scale, the f32 error bound against float64 with N(0,1)
    operands, and the same bits from a second call (determinism), for every
    operand layout."""
    M, N, K = 1024, 3000, 768
    eng = engine[1]
    print("plain gemm", akc, bkc, engine[0], flush=True)
    r = np.random.default_rng(int(akc) * 2 + int(bkc))
    a = r.standard_normal((M, K), dtype=np.float32)
    b = (r.standard_normal((K, N)) * 0.02).astype(np.float32)
    b1 = r.standard_normal((K, N), dtype=np.float32)
    # Store A as [M, K] (k-contiguous) or [K, M] (m-contiguous), B as [N, K] or [K, N].
    A = dev(vh, a if akc else np.ascontiguousarray(a.T))
    a_sm, a_sk = (K, 1) if akc else (1, M)
    for bb, name in ((b, "model scale"), (b1, "N(0,1)")):
        B = dev(vh, np.ascontiguousarray(bb.T) if bkc else bb)
        b_sk, b_sn = (1, K) if bkc else (N, 1)
        C, C2 = out(vh, (M, N)), out(vh, (M, N))
        d = gemm_desc(vh, M, N, K, A.ptr, a_sm, a_sk, B.ptr, b_sk, b_sn, C.ptr, N, engine=eng)
        vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
        if eng == vh.GEMM_ENGINE_DEFAULT:
            assert vh.lib.vh_gemm_last_path() == vh.GEMM_PATH_PERSISTENT
        d2 = gemm_desc(vh, M, N, K, A.ptr, a_sm, a_sk, B.ptr, b_sk, b_sn, C2.ptr, N, engine=eng)
        vh.check(vh.lib.vh_gemm(ctypes.byref(d2), None))
        got = fetch(vh, C, (M, N))
        np.testing.assert_array_equal(got, fetch(vh, C2, (M, N)))
        exact = a.astype(np.float64) @ bb.astype(np.float64)
        if bb is b:
            assert_parity(got, O.matmul(a, bb), exact, name=f"plain {akc} {bkc} {engine[0]}")
        else:
            u = 2.0 ** -24
            bound = (K * u / (1 - K * u)) * (np.abs(a).astype(np.float64) @ np.abs(bb).astype(np.float64))
            assert np.all(np.abs(got - exact) <= bound), f"plain {akc} {bkc}: f32 error bound"


@pytest.mark.parametrize("engine", ENGINES, ids=[e[0] for e in ENGINES])
@pytest.mark.parametrize("accumulate", [0, 1])
def test_linear_bias_and_residual(vh, accumulate, engine):
    """A large Linear forward: y = x W^T + b, and with accumulation
    h = h0 + (x W^T + b) (the residual form the block step uses), on both
    engines, against the oracle's matmul then add; determinism on a repeat."""
    M, K, N = 2048, 3072, 768
    r = np.random.default_rng(40 + accumulate)
    x = r.standard_normal((M, K), dtype=np.float32)
    w = (r.standard_normal((N, K)) * 0.02).astype(np.float32)  # Linear weight [out, in]
    bias = (r.standard_normal(N) * 0.02).astype(np.float32)
    h0 = r.standard_normal((M, N), dtype=np.float32)
    X, W, BI = dev(vh, x), dev(vh, w), dev(vh, bias)
    outs = []
    for _ in range(2):
        C = dev(vh, h0 if accumulate else np.zeros((M, N), np.float32))
        d = gemm_desc(vh, M, N, K, X.ptr, K, 1, W.ptr, 1, K, C.ptr, N, e=BI.ptr, e_sm=0, e_sn=1,
                      accumulate=accumulate, engine=engine[1])
        vh.check(vh.lib.vh_gemm(ctypes.byref(d), None))
        outs.append(fetch(vh, C, (M, N)))
    np.testing.assert_array_equal(outs[0], outs[1])
    lin = O.matmul(x, np.ascontiguousarray(w.T)) + bias
    lin64 = x.astype(np.float64) @ w.T.astype(np.float64) + bias
    ref = (h0 + lin) if accumulate else lin
    ref64 = (h0.astype(np.float64) + lin64) if accumulate else lin64
    assert_parity(outs[0], ref, ref64, name=f"linear {engine[0]} acc={accumulate}")
