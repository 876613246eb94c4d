"""Benchmark of the hot path on one MI355X.

Default workload (BASELINE.json's metric): one step is one pass of the path
over one synthetic batch at GPT-2-small shape,
  layernorm forward    x [16384, 768]                 (the cfg[4] layernorm shape)
  causal softmax fwd   scores [16, 12, 1024, 1024]    (cfg[2])
  causal softmax bwd   from the saved input x and dy, as the autograd arm does
  layernorm backward   (x, w, dy -> dx, dgamma, dbeta)
issued in that order on the runtime stream, as a training step meets them
(forward, then backward in reverse). After it, the default run measures the
other configs of BASELINE.json the same way and reports them in the same JSON
line under "configs" (gpt2_block -- config[4]'s training step, whose ms per
step is also the top-level "gpt2_block_ms" -- gelu_bias, embedding_uniform,
embedding_zipf, cross_entropy, cross_entropy_rowstats -- the same with the
backward streaming from the forward's row statistics -- softmax_dense -- the
dense form the BackendOps slot runs -- and layernorm_cfg0); --no-extra skips
them, --workload NAME
prints one config's own line. gpt2_block also carries "ab_library" (its dense
products on hipBLASLt), "dropin" (the same step op by op through the
BackendOps mirror, shared-weight gradients folded into one product),
"dropin_reference_arms" (the reference's own Matmul arm: per-batch products,
then reduce_to) and "dropin_unfused" (MultiHeadAttention's unfused path).

Inputs are resident in HBM before timing. Buffers that would otherwise stay in
the 256 MB MALL between uses alternate between two sets (or are flushed by the
step's own multi-GB traffic), so every kernel reads cold data.

value = algorithmic bytes per step / wall time per step (GB/s), over exactly
--steps steps issued back to back; algorithmic bytes count each necessary HBM
transfer once (the live causal triangle only for causal softmax reads, distinct
rows only for embedding gathers). Per kernel, "avg_us" is the op run alone
--steps times back to back between two HIP events on the runtime stream (its
average launch duration, the figure a kernel trace reports) and "in_step_us"
the HIP events around it inside a second pass of the steps (each event's own
cost included). `roofline` reports the longest kernel by avg_us, with
`traffic` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
(profiles/pmc_traffic.json, written by --pmc-summarize); every op with such a
record carries "traffic_bytes" and "traffic_ratio" (measured over
algorithmic). cpu_baseline times the CPU oracle (the C restatement of the
reference's CPU backend, one thread, as the reference's kernels are) on the
whole headline step at its own shapes, and on bounded samples for the other
configs; "host" records the CPU model, core count and glibc.

Warmup is at least --warmup steps and at least --min-warmup-ms of them: after
the second or so of host-side input generation the GPU has lowered its clocks,
and a few milliseconds of work do not bring them back (measured: the softmax
backward runs 262 us back to back, 270-336 us for the first ~10 ms after a 1 s
idle). The JSON's "warmup" is the requested --warmup and "warmup_steps_run"
the number of warmup steps actually run; the timed region is exactly --steps
steps either way.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--min-warmup-ms 1000] [--workload NAME]
                       [--no-cpu] [--no-extra] [--calibrate-copy] [--pmc-summarize DIR]
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "LayerNorm/softmax fwd+bwd HBM GB/s (% of ~8 TB/s peak); GPT block step ms"
PEAK_GBPS = 8000.0
PEAK_F32_MFMA_TFLOPS = 157.3  # MI355X dense f32 matrix peak
SEED = 0x5EED0000


def ln_bytes(rows, C):
    n = rows * C
    fwd = 4 * n + 4 * n + 8 * C           # R x, W y, R w,b
    bwd = 4 * n * 3 + 4 * C + 8 * C       # R x, R dy, W dx, R w, W dgamma,dbeta
    return fwd, bwd


def sm_bytes(B, H, T):
    rows = B * H * T
    live = B * H * T * (T + 1) // 2       # causal lower triangle incl. diagonal
    n = rows * T
    fwd = 4 * live + 4 * n                # R live x, W all y
    bwd = 4 * live * 2 + 4 * n            # R live x, R live dy, W all dx
    return fwd, bwd


class Hip:
    """The few HIP runtime calls bench needs (events on the runtime stream)."""

    def __init__(self):
        self.h = ctypes.CDLL("libamdhip64.so.7")
        self.h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.h.hipStreamSynchronize.argtypes = [ctypes.c_void_p]

    def event(self):
        e = ctypes.c_void_p()
        assert self.h.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.h.hipEventRecord(e, stream) == 0

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        assert self.h.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value

    def sync(self, stream):
        assert self.h.hipStreamSynchronize(stream) == 0


def causal_scores(r, B, H, T):
    s = r.standard_normal(size=(B, H, T, T), dtype=np.float32) * np.float32(0.125)
    iu = np.triu_indices(T, 1)
    s[:, :, iu[0], iu[1]] = -np.inf
    return s


def zipf_ids(r, n, V, s=1.1):
    ranks = np.arange(1, V + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    return np.searchsorted(cdf, r.random(n)).astype(np.float32)


def time_cpu(fn, budget_s):
    t, reps = 0.0, 0
    while t < budget_s or reps == 0:
        t0 = time.perf_counter()
        fn()
        t += time.perf_counter() - t0
        reps += 1
    return t, reps


# ---------------------------------------------------------------- workloads
# Each workload: setup(vh) -> (ops, info); ops is a list of (name, bytes, call(i)).

def wl_ln_softmax(vh):
    LN_ROWS, LN_C = 16384, 768
    SM_B, SM_H, SM_T = 16, 12, 1024
    r = np.random.default_rng(SEED + 4)
    w = (1 + 0.02 * r.standard_normal(LN_C)).astype(np.float32)
    b = (0.02 * r.standard_normal(LN_C)).astype(np.float32)
    W, Bi = vh.DeviceBuffer.from_array(w), vh.DeviceBuffer.from_array(b)
    sets = []
    for _ in range(2):
        x = r.standard_normal(size=(LN_ROWS, LN_C), dtype=np.float32)
        dy = r.standard_normal(size=(LN_ROWS, LN_C), dtype=np.float32)
        sets.append(dict(x=vh.DeviceBuffer.from_array(x), dy=vh.DeviceBuffer.from_array(dy),
                         y=vh.DeviceBuffer(x.nbytes), dx=vh.DeviceBuffer(x.nbytes),
                         dw=vh.DeviceBuffer(w.nbytes), db=vh.DeviceBuffer(w.nbytes)))
    nsc = vh.lib.vh_layernorm_bwd_scratch_bytes(LN_ROWS, LN_C)
    LNS = vh.DeviceBuffer(nsc)
    rs = np.random.default_rng(SEED + 2)
    s = causal_scores(rs, SM_B, SM_H, SM_T)
    S = vh.DeviceBuffer.from_array(s)
    del s
    G = vh.DeviceBuffer.from_array(rs.standard_normal(size=(SM_B, SM_H, SM_T, SM_T), dtype=np.float32))
    n_sm = SM_B * SM_H * SM_T * SM_T
    P, DS = vh.DeviceBuffer(4 * n_sm), vh.DeviceBuffer(4 * n_sm)
    rows_sm = SM_B * SM_H * SM_T
    lf, lb = ln_bytes(LN_ROWS, LN_C)
    sf, sb = sm_bytes(SM_B, SM_H, SM_T)
    L = lambda i: sets[i % 2]
    ops = [
        ("layernorm_fwd", lf, lambda i: vh.lib.vh_layernorm_fwd(L(i)["x"].ptr, W.ptr, Bi.ptr, L(i)["y"].ptr,
                                                                 LN_ROWS, LN_C, 1e-5, None)),
        ("softmax_fwd", sf, lambda i: vh.lib.vh_softmax_fwd(S.ptr, P.ptr, rows_sm, SM_T, 1, None)),
        # The autograd Softmax arm saves the input x and recomputes y from it
        # (crates/vearo-autograd/src/lib.rs:547-553); the fused kernel does the same.
        ("softmax_bwd", sb, lambda i: vh.lib.vh_softmax_bwd(S.ptr, G.ptr, DS.ptr, rows_sm, SM_T, 1, 1, None)),
        ("layernorm_bwd", lb, lambda i: vh.lib.vh_layernorm_bwd(
            L(i)["x"].ptr, W.ptr, L(i)["dy"].ptr, L(i)["dx"].ptr, L(i)["dw"].ptr, L(i)["db"].ptr,
            LN_ROWS, LN_C, 1e-5, LNS.ptr, nsc, None)),
    ]
    keep = (W, Bi, sets, LNS, S, G, P, DS)

    def cpu(budget):
        # The oracle on the headline shapes themselves: one whole step (LN
        # fwd+bwd [16384,768], causal softmax fwd + the autograd arm's composite
        # backward [16,12,1024,1024]), repeated while the budget lasts.
        import oracle
        rc = np.random.default_rng(SEED)
        x = rc.standard_normal(size=(LN_ROWS, LN_C), dtype=np.float32)
        dy = rc.standard_normal(size=(LN_ROWS, LN_C), dtype=np.float32)
        s = causal_scores(rc, SM_B, SM_H, SM_T)
        g = rc.standard_normal(size=s.shape, dtype=np.float32)

        def step():
            oracle.layernorm(x, w, b, 1e-5)
            oracle.softmax(s, 3)
            oracle.softmax_backward_composite(s, g, 3)
            oracle.layernorm_backward(x, w, b, dy, 1e-5)
        t, reps = time_cpu(step, budget)
        return (lf + lb + sf + sb) * reps / t, (f"the whole headline step at its own shapes (LN [{LN_ROWS},{LN_C}], "
                                                f"softmax [{SM_B},{SM_H},{SM_T},{SM_T}]), {reps} step(s) in {t:.1f} s, "
                                                f"single thread (the reference's CPU kernels spawn none)")

    info = {"workload": "layernorm fwd+bwd [16384,768] + causal softmax fwd+bwd [16,12,1024,1024]",
            "ln_shape": [LN_ROWS, LN_C], "softmax_shape": [SM_B, SM_H, SM_T, SM_T]}
    return ops, info, cpu, keep


def wl_layernorm_cfg0(vh):
    rows, C = 2048, 128
    r = np.random.default_rng(SEED + 0)
    x = r.standard_normal(size=(rows, C), dtype=np.float32)
    w = (1 + 0.02 * r.standard_normal(C)).astype(np.float32)
    b = (0.02 * r.standard_normal(C)).astype(np.float32)
    dy = r.standard_normal(size=(rows, C), dtype=np.float32)
    X, W, Bi, DY = (vh.DeviceBuffer.from_array(a) for a in (x, w, b, dy))
    Y, DX = vh.DeviceBuffer(x.nbytes), vh.DeviceBuffer(x.nbytes)
    DW, DB = vh.DeviceBuffer(w.nbytes), vh.DeviceBuffer(w.nbytes)
    lf, lb = ln_bytes(rows, C)
    ops = [("layernorm_fwd", lf, lambda i: vh.lib.vh_layernorm_fwd(X.ptr, W.ptr, Bi.ptr, Y.ptr, rows, C, 1e-5, None)),
           ("layernorm_bwd", lb, lambda i: vh.lib.vh_layernorm_bwd(X.ptr, W.ptr, DY.ptr, DX.ptr, DW.ptr, DB.ptr,
                                                                   rows, C, 1e-5, None, 0, None))]

    def cpu(budget):
        import oracle
        t, reps = time_cpu(lambda: (oracle.layernorm(x, w, b, 1e-5), oracle.layernorm_backward(x, w, b, dy, 1e-5)),
                           budget)
        return (lf + lb) * reps / t, f"layernorm fwd+bwd [{rows},{C}] (the whole config), {reps} reps, single thread"

    return ops, {"workload": "cfg[0] layernorm fwd+bwd [2048,128] (launch-bound, cache-resident)"}, cpu, \
        (X, W, Bi, DY, Y, DX, DW, DB)


def wl_gelu_bias(vh):
    rows, C = 16384, 3072
    r = np.random.default_rng(SEED + 1)
    bias = (0.02 * r.standard_normal(C)).astype(np.float32)
    Bi = vh.DeviceBuffer.from_array(bias)
    X = vh.DeviceBuffer.from_array(r.standard_normal(size=(rows, C), dtype=np.float32) * np.float32(1.5))
    DY = vh.DeviceBuffer.from_array(r.standard_normal(size=(rows, C), dtype=np.float32))
    Y, DX, DB = vh.DeviceBuffer(4 * rows * C), vh.DeviceBuffer(4 * rows * C), vh.DeviceBuffer(4 * C)
    n = rows * C
    fb, bb = 8 * n + 4 * C, 12 * n + 8 * C
    nsc = vh.lib.vh_gelu_bias_bwd_scratch_bytes(rows, C)
    SC = vh.DeviceBuffer(nsc)
    ops = [("gelu_bias_fwd", fb, lambda i: vh.lib.vh_gelu_bias_fwd(X.ptr, Bi.ptr, Y.ptr, rows, C, None)),
           ("gelu_bias_bwd", bb, lambda i: vh.lib.vh_gelu_bias_bwd(X.ptr, Bi.ptr, DY.ptr, DX.ptr, DB.ptr, rows, C,
                                                                   SC.ptr, nsc, None))]

    def cpu(budget):
        import oracle
        rc = np.random.default_rng(SEED + 1)
        sr = 512
        x = rc.standard_normal(size=(sr, C), dtype=np.float32) * np.float32(1.5)
        dy = rc.standard_normal(size=(sr, C), dtype=np.float32)
        t, reps = time_cpu(lambda: (oracle.gelu_bias_forward(x, bias), oracle.gelu_bias_backward(x, bias, dy)), budget)
        return (20 * sr * C + 12 * C) * reps / t, (f"bias add + gelu fwd and mask*dy + bias reduce_to on "
                                                   f"[{sr},{C}], {reps} reps, single thread")

    return ops, {"workload": "cfg[1] gelu(x+bias) fwd+bwd [16384,3072]"}, cpu, (Bi, X, DY, Y, DX, DB, SC)


def _embedding(vh, zipf):
    V, D, n = 50257, 768, 16384
    r = np.random.default_rng(SEED + 3)
    Wt = (0.02 * r.standard_normal(size=(V, D), dtype=np.float32))
    ids = zipf_ids(r, n, V) if zipf else r.integers(0, V, size=n).astype(np.float32)
    dy = r.standard_normal(size=(n, D), dtype=np.float32)
    U = len(np.unique(ids))
    I, Wd, DY = vh.DeviceBuffer.from_array(ids), vh.DeviceBuffer.from_array(Wt), vh.DeviceBuffer.from_array(dy)
    OUT, DW = vh.DeviceBuffer(4 * n * D), vh.DeviceBuffer(4 * V * D)
    nsc = vh.lib.vh_embedding_bwd_scratch_bytes(n, V, D)
    SC = vh.DeviceBuffer(nsc)
    fb = 4 * n + 4 * U * D + 4 * n * D
    bb = 4 * n + 4 * n * D + 4 * V * D
    ops = [("embedding_fwd", fb, lambda i: vh.lib.vh_embedding_fwd(I.ptr, Wd.ptr, OUT.ptr, n, V, D, None)),
           ("embedding_bwd", bb, lambda i: vh.lib.vh_embedding_bwd(I.ptr, DY.ptr, DW.ptr, n, V, D, SC.ptr, nsc, None))]

    def cpu(budget):
        import oracle
        t, reps = time_cpu(lambda: (oracle.embedding(ids, Wt), oracle.embedding_backward(ids, (V, D), dy)), budget)
        return (fb + bb) * reps / t, f"the whole config (n={n}, V={V}, D={D}), {reps} reps, single thread"

    kind = "Zipf(1.1)" if zipf else "uniform"
    return ops, {"workload": f"cfg[3] embedding fwd+bwd, {kind} ids, V=50257 D=768 n=16384",
                 "distinct_ids": U}, cpu, (I, Wd, DY, OUT, DW, SC)


def wl_embedding_uniform(vh):
    return _embedding(vh, False)


def wl_embedding_zipf(vh):
    return _embedding(vh, True)


def wl_cross_entropy(vh):
    B, V = 16384, 50257
    r = np.random.default_rng(SEED + 4)
    L = vh.DeviceBuffer.from_array(r.standard_normal(size=(B, V), dtype=np.float32))
    T = vh.DeviceBuffer.from_array(r.integers(0, V, size=B).astype(np.float32))
    GO = vh.DeviceBuffer.from_array(np.float32([1.0]))
    LOSS, DL = vh.DeviceBuffer(4), vh.DeviceBuffer(4 * B * V)
    nsc = vh.lib.vh_cross_entropy_fwd_scratch_bytes(B)
    SC = vh.DeviceBuffer(nsc)
    fb, bb = 4 * B * V + 8 * B, 8 * B * V + 8 * B
    ops = [("cross_entropy_fwd", fb, lambda i: vh.lib.vh_cross_entropy_fwd(L.ptr, T.ptr, LOSS.ptr, B, V, SC.ptr,
                                                                           nsc, None)),
           ("cross_entropy_bwd", bb, lambda i: vh.lib.vh_cross_entropy_bwd(L.ptr, T.ptr, GO.ptr, DL.ptr, B, V, None))]

    def cpu(budget):
        import oracle
        rc = np.random.default_rng(SEED + 4)
        sb_ = 64
        lg = rc.standard_normal(size=(sb_, V), dtype=np.float32)
        tg = rc.integers(0, V, size=sb_).astype(np.float32)
        go = np.float32([1.0])
        t, reps = time_cpu(lambda: (oracle.cross_entropy(lg, tg), oracle.cross_entropy_backward(lg, tg, go)), budget)
        return (12 * sb_ * V + 16 * sb_) * reps / t, f"cross-entropy fwd+bwd on [{sb_},{V}], {reps} reps, single thread"

    return ops, {"workload": "cross-entropy fwd+bwd over logits [16384,50257] (cfg[4] lm_head output)"}, cpu, \
        (L, T, GO, LOSS, DL, SC)


def wl_cross_entropy_rowstats(vh):
    """The same fwd+bwd with the forward keeping each row's (max, sum-exp) and
    the backward streaming from them (vh_cross_entropy_fwd_rs_ld /
    vh_cross_entropy_bwd_rs_ld): the same loss and dlogits bits as the slot
    pair above, for a caller that keeps per-row state between its forward and
    backward. Bytes: fwd R logits + W stats, bwd R logits + W dlogits + R stats
    (targets read by both)."""
    B, V = 16384, 50257
    r = np.random.default_rng(SEED + 4)
    L = vh.DeviceBuffer.from_array(r.standard_normal(size=(B, V), dtype=np.float32))
    T = vh.DeviceBuffer.from_array(r.integers(0, V, size=B).astype(np.float32))
    GO = vh.DeviceBuffer.from_array(np.float32([1.0]))
    LOSS, DL, ST = vh.DeviceBuffer(4), vh.DeviceBuffer(4 * B * V), vh.DeviceBuffer(8 * B)
    nsc = vh.lib.vh_cross_entropy_fwd_scratch_bytes(B)
    SC = vh.DeviceBuffer(nsc)
    fb, bb = 4 * B * V + 8 * B + 8 * B, 8 * B * V + 8 * B + 4 * B
    ops = [("cross_entropy_fwd_rs", fb, lambda i: vh.lib.vh_cross_entropy_fwd_rs_ld(
               L.ptr, V, T.ptr, LOSS.ptr, ST.ptr, B, V, SC.ptr, nsc, None)),
           ("cross_entropy_bwd_rs", bb, lambda i: vh.lib.vh_cross_entropy_bwd_rs_ld(
               L.ptr, V, T.ptr, ST.ptr, GO.ptr, DL.ptr, B, V, None))]
    return ops, {"workload": "cross-entropy fwd+bwd over logits [16384,50257], the backward from the "
                             "forward's row statistics"}, None, (L, T, GO, LOSS, DL, ST, SC)


def wl_softmax_dense(vh):
    """The softmax the BackendOps slot runs: vearo's attention adds the causal
    mask to the scores (scores.add(mask).softmax(3)), so the slot sees a plain
    [rows, T] softmax and reads every entry (causal = 0). Same scores (-inf
    above the diagonal), dense accounting: fwd R x + W y, bwd R x + R dy + W dx."""
    B, H, T = 16, 12, 1024
    rs = np.random.default_rng(SEED + 2)
    S = vh.DeviceBuffer.from_array(causal_scores(rs, B, H, T))
    G = vh.DeviceBuffer.from_array(rs.standard_normal(size=(B, H, T, T), dtype=np.float32))
    n = B * H * T * T
    P, DS = vh.DeviceBuffer(4 * n), vh.DeviceBuffer(4 * n)
    rows = B * H * T
    ops = [("softmax_dense_fwd", 8 * n, lambda i: vh.lib.vh_softmax_fwd(S.ptr, P.ptr, rows, T, 0, None)),
           ("softmax_dense_bwd", 12 * n, lambda i: vh.lib.vh_softmax_bwd(S.ptr, G.ptr, DS.ptr, rows, T, 1, 0, None))]

    def cpu(budget):
        import oracle
        rc = np.random.default_rng(SEED + 2)
        s = causal_scores(rc, 1, 2, T)
        g = rc.standard_normal(size=s.shape, dtype=np.float32)
        t, reps = time_cpu(lambda: (oracle.softmax(s, 3), oracle.softmax_backward_composite(s, g, 3)), budget)
        return 20 * s.size * reps / t, f"softmax fwd + composite bwd on [1,2,{T},{T}], {reps} reps, single thread"

    return ops, {"workload": "softmax fwd+bwd [16,12,1024,1024], dense (the BackendOps slot form)"}, cpu, \
        (S, G, P, DS)


def gpt_fwd_flops(B, S, D, H, F, V):
    R = B * S
    gemm = 2 * R * D * D * 4 + 2 * R * D * F * 2   # q, k, v, out; fc1, fc2
    attn = 2 * 2 * B * S * S * D                    # q k^T and p v over all heads (dense)
    head = 2 * R * D * V                            # lm_head
    return gemm + attn + head


def wl_gpt2_block(vh):
    """config[4]: SimpleGPT(V=50257, S=1024, D=768, H=12, 1 block, MLP 3072),
    B=16, one training step = forward + autograd backward + AdamW (lr 0.02,
    betas 0.9/0.95, eps 1e-8, wd 0.01, verification_harness.rs:203-210)."""
    from vearo_amd import _block
    cfg = (16, 1024, 768, 12, 3072, 50257, 1024)
    B, S, D, H, F, V, P = cfg
    g = _block.Gpt(_block.GptConfig(*cfg))
    r = np.random.default_rng(SEED + 4)
    params = []
    for name, sh in zip(_block.PARAM_NAMES, g.shapes):
        if name.startswith("ln") and name.endswith("_w"):
            params.append(np.ones(sh, np.float32))
        elif name.startswith("ln"):
            params.append(np.zeros(sh, np.float32))
        else:
            params.append(r.standard_normal(sh, dtype=np.float32) * np.float32(0.02))
    g.set_params(params)
    ids = r.integers(0, V, size=(B, S)).astype(np.float32)
    tg = r.integers(0, V, size=(B, S)).astype(np.float32)
    g.set_inputs(ids, tg)
    flops = 3 * gpt_fwd_flops(B, S, D, H, F, V)  # fwd + bwd (2x fwd), the usual accounting
    ops = [("train_step", flops, lambda i: _block.lib.vb_gpt_train_step(g.h, 0.02, 0.9, 0.95, 1e-8, 0.01))]
    # The dominant kernel, timed on its own after the timed loop: the lm_head
    # forward GEMM logits[16384, 50257] = lnf[16384, 768] W^T, through the same
    # vh_gemm path the step uses (this library's persistent kernel), on scratch
    # buffers of the same shapes.
    A = vh.DeviceBuffer.from_array(r.standard_normal((B * S, D), dtype=np.float32))
    W = vh.DeviceBuffer.from_array(params[20])
    C = vh.DeviceBuffer(4 * B * S * V)
    d = vh.VhGemmDesc()
    d.M, d.N, d.K = B * S, V, D
    d.a, d.a_sm, d.a_sk = A.ptr, D, 1
    d.b, d.b_sk, d.b_sn = W.ptr, 1, D
    d.c, d.c_sm = C.ptr, V
    d.batch[0] = d.batch[1] = 1
    d.alpha = 1.0
    probe = ("lm_head_gemm", 2 * B * S * D * V, lambda i: vh.lib.vh_gemm(ctypes.byref(d), None))
    # A/B reference: the same step and lm_head product with the dense products
    # on hipBLASLt (the LIBRARY engine), timed after the headline.
    dl = vh.VhGemmDesc.from_buffer_copy(d)
    dl.engine = vh.GEMM_ENGINE_LIBRARY

    def ab(hip, stream, steps):
        out = {}
        lp = lm_head_time(vh, hip, stream, lambda i: vh.lib.vh_gemm(ctypes.byref(dl), None), 2 * B * S * D * V)
        lp["path"] = {vh.GEMM_PATH_LIBRARY: "hipBLASLt"}.get(vh.lib.vh_gemm_last_path(), "fell back to own kernel")
        out["lm_head_gemm_library"] = lp
        g.set_gemm_engine(vh.GEMM_ENGINE_LIBRARY)
        try:
            step = lambda: vh.check(_block.lib.vb_gpt_train_step(g.h, 0.02, 0.9, 0.95, 1e-8, 0.01))
            for _ in range(2):
                step()
            vh.sync()
            e0, e1 = hip.event(), hip.event()
            hip.record(e0, stream)
            for _ in range(steps):
                step()
            hip.record(e1, stream)
            hip.sync(stream)
            out["gpt2_block_ms_library"] = round(hip.elapsed_ms(e0, e1) / steps, 3)
        finally:
            g.set_gemm_engine(vh.GEMM_ENGINE_DEFAULT)
        return out

    def dropin(hip, stream, steps, fused=True, fold=True):
        # The same step issued op by op through the BackendOps mirror, in the
        # reference's own order (forward tape, backward_impl arms, AdamW::step):
        # what a vearo program gets. Timed like the headline, then one step
        # with an event after every op for the per-phase breakdown.
        # fused=False: MultiHeadAttention's unfused path (the reference with
        # VEARO_USE_FUSED_ATTENTION=0), scores through the matmul, mul, add and
        # softmax slots and back through the Softmax arm's slot calls.
        # fold=False: the reference's own Matmul arm for the shared weights
        # (per-batch product, then reduce_to over the batch) instead of one
        # product over all rows.
        d = _block.DropIn(_block.GptConfig(*cfg), fused_attention=fused, fold_weight_grads=fold)
        try:
            d.set_params(params)
            d.set_inputs(ids, tg)
            step = lambda: d.step(backward=True, adamw=True, want_loss=False)
            for _ in range(2):
                step()
            vh.sync()
            e0, e1 = hip.event(), hip.event()
            hip.record(e0, stream)
            for _ in range(steps):
                step()
            hip.record(e1, stream)
            hip.sync(stream)
            ms = hip.elapsed_ms(e0, e1) / steps
            d.step(backward=True, adamw=True, want_loss=False, timing=True)
            ph = d.phase_ms()
            loss = d.step(backward=False)
        finally:
            d.close()
        return {"ms_per_step": round(ms, 3), "tflops": round(flops / ms / 1e9, 2), "steps": steps,
                "loss_after": round(loss, 6),
                "phases_ms": {k: round(v, 3) for k, v in ph.items()},
                "phases_sum_ms": round(sum(ph.values()), 3)}

    def cpu(budget):
        import oracle
        t0 = time.perf_counter()
        _, grads = oracle.gpt_step(oracle.GptConfig(*cfg), params, ids, tg)
        t_fb = time.perf_counter() - t0
        t0 = time.perf_counter()
        for p, gr in zip(params, grads):
            oracle.adamw_step(p.copy(), gr, np.zeros_like(p), np.zeros_like(p), 1, 0.02, 0.9, 0.95, 1e-8, 0.01)
        t_adam = time.perf_counter() - t0
        threads = int(os.environ.get("VO_THREADS") or os.environ.get("OMP_NUM_THREADS") or os.cpu_count())
        return (t_fb + t_adam) * 1e3, threads, (
            f"one whole config[4] step of the oracle (forward+backward {t_fb:.1f} s, AdamW over "
            f"{sum(p.size for p in params)} parameters {t_adam:.2f} s); matmuls threaded as the "
            f"reference's are, attention threaded over heads (the reference runs it on one thread)")

    info = {"workload": "cfg[4] GPT-2-small block training step: B=16, T=1024, C=768, H=12, MLP 3072, "
                        "V=50257, one block; fwd + backward + AdamW",
            "flops_per_step": flops, "_mode": "step_ms", "_probe": probe, "_ab": ab, "_dropin": dropin,
            "_dropin_unfused": lambda hip, stream, steps: dropin(hip, stream, steps, fused=False),
            "_dropin_reference_arms": lambda hip, stream, steps: dropin(hip, stream, steps, fold=False)}
    return ops, info, cpu, (g, A, W, C, d, dl)


def wl_lm_head_gemm(vh):
    """The dominant kernel of config[4] on its own (for counters and traces):
    logits[16384, 50257] = lnf[16384, 768] W^T through vh_gemm (this library's
    persistent kernel), the product the block step's roofline line reports.
    Algorithmic bytes: A, B read once and C written once."""
    B, S, D, V = 16, 1024, 768, 50257
    r = np.random.default_rng(SEED + 4)
    A = vh.DeviceBuffer.from_array(r.standard_normal((B * S, D), dtype=np.float32))
    W = vh.DeviceBuffer.from_array(r.standard_normal((V, D), dtype=np.float32) * np.float32(0.02))
    C = vh.DeviceBuffer(4 * B * S * V)
    d = vh.VhGemmDesc()
    d.M, d.N, d.K = B * S, V, D
    d.a, d.a_sm, d.a_sk = A.ptr, D, 1
    d.b, d.b_sk, d.b_sn = W.ptr, 1, D
    d.c, d.c_sm = C.ptr, V
    d.batch[0] = d.batch[1] = 1
    d.alpha = 1.0
    nb = 4 * (B * S * D + V * D + B * S * V)
    ops = [("lm_head_gemm", nb, lambda i: vh.lib.vh_gemm(ctypes.byref(d), None))]
    info = {"workload": "cfg[4] lm_head forward product [16384,768] x [768,50257] alone",
            "flops": 2 * B * S * D * V}
    return ops, info, None, (A, W, C, d)


PEAK_PCIE_GBPS = 64.0  # MI355X host link, PCIe 5.0 x16, one direction


def run_checkpoint(args, vh):
    """`.ve` checkpoint save + load (crates/vearo/src/checkpoint.rs:9-91) of
    the cfg[4] parameter set (SimpleGPT, 21 tensors, 85,070,592 floats) from
    and to device memory, through vb_gpt_save / vb_gpt_load. Both directions
    are synchronous calls: wall-clock time, file written to TMPDIR, then read.
    The oracle's save/load of the same host arrays is the CPU baseline."""
    import tempfile
    from vearo_amd import _block
    cfg = (16, 1024, 768, 12, 3072, 50257, 1024)
    g = _block.Gpt(_block.GptConfig(*cfg))
    r = np.random.default_rng(SEED + 4)
    params = [r.standard_normal(sh, dtype=np.float32) * np.float32(0.02) for sh in g.shapes]
    g.set_params(params)
    vh.sync()
    d = tempfile.mkdtemp(prefix="vearo_ckpt_")
    path = os.path.join(d, "gpt.ve")
    try:
        for _ in range(max(args.warmup, 1)):
            g.save(path)
            g.load(path)
        nbytes = os.path.getsize(path)
        ts, tl = [], []
        for _ in range(args.steps):
            t0 = time.perf_counter()
            g.save(path)
            t1 = time.perf_counter()
            g.load(path)
            t2 = time.perf_counter()
            ts.append(t1 - t0)
            tl.append(t2 - t1)
        back = g.params()
        assert all(a.tobytes() == b.tobytes() for a, b in zip(back, params)), "checkpoint round trip changed bits"
        cpu_res = None
        if not args.no_cpu:
            import oracle
            cpath = os.path.join(d, "oracle.ve")
            arrays = [p.copy() for p in params]
            t0 = time.perf_counter()
            oracle.checkpoint_save(cpath, params)
            t1 = time.perf_counter()
            oracle.checkpoint_load(cpath, arrays)
            t2 = time.perf_counter()
            os.remove(cpath)
            cpu_res = {"value": round(2 * nbytes / (t2 - t0) / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                       "sample": f"one save ({t1 - t0:.2f} s) and one load ({t2 - t1:.2f} s) of the same "
                                 f"{nbytes} B file from host arrays, one value per stdio call as the reference's "
                                 f"BufWriter/BufReader loop does"}
    finally:
        if os.path.exists(path):
            os.remove(path)
        os.rmdir(d)
        g.close()
    save_s, load_s = sum(ts) / len(ts), sum(tl) / len(tl)
    value = 2 * nbytes / (save_s + load_s) / 1e9
    kernels = {"save": {"avg_ms": round(save_s * 1e3, 2), "bytes": nbytes, "gbps": round(nbytes / save_s / 1e9, 2)},
               "load": {"avg_ms": round(load_s * 1e3, 2), "bytes": nbytes, "gbps": round(nbytes / load_s / 1e9, 2)}}
    dom = max(kernels, key=lambda k: kernels[k]["avg_ms"])
    res = {
        "metric": "checkpoint save+load GB/s (cfg[4] parameters as a .ve file)", "value": round(value, 2),
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round((save_s + load_s) * 1e3, 2), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (weights ~N(0,0.02))",
        "config": {"workload": "vb_gpt_save + vb_gpt_load of SimpleGPT cfg[4] (85,070,592 floats, "
                               f"{nbytes} B file in TMPDIR)", "bytes_per_step": 2 * nbytes},
        "kernels": kernels,
        "roofline": {"bound": "pcie", "kernel": dom, "achieved": kernels[dom]["gbps"], "peak": PEAK_PCIE_GBPS,
                     "unit": "GB/s", "frac": round(kernels[dom]["gbps"] / PEAK_PCIE_GBPS, 4), "traffic": None},
        "cpu_baseline": cpu_res,
    }
    print(json.dumps(res), flush=True)


WORKLOADS = {"ln_softmax": wl_ln_softmax, "gpt2_block": wl_gpt2_block, "layernorm_cfg0": wl_layernorm_cfg0,
             "gelu_bias": wl_gelu_bias, "embedding_uniform": wl_embedding_uniform,
             "embedding_zipf": wl_embedding_zipf, "cross_entropy": wl_cross_entropy,
             "cross_entropy_rowstats": wl_cross_entropy_rowstats,
             "softmax_dense": wl_softmax_dense, "lm_head_gemm": wl_lm_head_gemm, "checkpoint": run_checkpoint}

# The kernels each op launches (name patterns), per workload: the per-dispatch
# FETCH_SIZE / WRITE_SIZE averages of the matching kernels add up to the op's
# measured HBM traffic (--pmc-summarize). gpt2_block's entry is the fused
# cross-entropy pass of its step (the one kernel of its kind there).
_LN = {"layernorm_fwd": r"^vh_ln_fwd_", "layernorm_bwd": r"^vh_ln_bwd_|^vh_col_reduce$"}
PMC_KERNELS = {
    "ln_softmax": dict(_LN, softmax_fwd=r"^vh_sm_fwd_", softmax_bwd=r"^vh_sm_bwd_"),
    "layernorm_cfg0": _LN,
    "gelu_bias": {"gelu_bias_fwd": r"^vh_gelu_bias_fwd", "gelu_bias_bwd": r"^vh_gelu_bias_bwd|^vh_col_reduce$"},
    "embedding_uniform": {"embedding_fwd": r"^vh_emb_fwd", "embedding_bwd": r"^vh_emb_(sort|sum)"},
    "embedding_zipf": {"embedding_fwd": r"^vh_emb_fwd", "embedding_bwd": r"^vh_emb_(sort|sum)"},
    "cross_entropy": {"cross_entropy_fwd": r"^vh_xent_fwd|^vh_xent_reduce$", "cross_entropy_bwd": r"^vh_xent_bwd"},
    "cross_entropy_rowstats": {"cross_entropy_fwd_rs": r"^vh_xent_fwd|^vh_xent_reduce$",
                               "cross_entropy_bwd_rs": r"^vh_xent_bwd_rs"},
    "softmax_dense": {"softmax_dense_fwd": r"^vh_sm_fwd_", "softmax_dense_bwd": r"^vh_sm_bwd_"},
    "lm_head_gemm": {"lm_head_gemm": r"^vh_gemm"},
    "gpt2_block": {"cross_entropy_fused": r"^vh_xent_fb_|^vh_xent_reduce$"},
}
PMC_FILE = os.path.join(ROOT, "profiles", "pmc_traffic.json")


def pmc_traffic(workload):
    """{op: traffic record} for a workload from the committed counter summary."""
    if not os.path.exists(PMC_FILE):
        return {}
    with open(PMC_FILE) as f:
        return json.load(f).get("workloads", {}).get(workload, {})


def pmc_summarize(root):
    """Writes profiles/pmc_traffic.json from rocprofv3 --pmc runs under root:
    <workload>_fetch/ and <workload>_write/ (FETCH_SIZE, WRITE_SIZE) for each
    workload in PMC_KERNELS that has them, and copy_fetch/ + copy_write/
    (--calibrate-copy: 4 copies of 1 GiB each way) for the scale factors."""
    import csv
    import glob
    import re

    def per_kernel(d):
        files = glob.glob(os.path.join(root, d, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            return None
        agg, names = {}, {}
        for row in csv.DictReader(open(files[0])):
            k = int(row["Dispatch_Id"])
            agg[k] = agg.get(k, 0.0) + float(row["Counter_Value"])
            names[k] = row["Kernel_Name"]
        byk = {}
        for k in sorted(agg):
            byk.setdefault(names[k], []).append(agg[k])
        return byk

    cf, cw = per_kernel("copy_fetch"), per_kernel("copy_write")
    exp_kib = float(1 << 30) / 1024
    cfv = [v for n, vs in cf.items() if n == "vh_stream_copy" for v in vs]
    cwv = [v for n, vs in cw.items() if n == "vh_stream_copy" for v in vs]
    fmean, wmean = sum(cfv) / len(cfv), sum(cwv) / len(cwv)
    fscale, wscale = exp_kib / fmean, exp_kib / wmean
    out = {"note": "HBM bytes per op call = (FETCH_SIZE KiB x fetch_scale + WRITE_SIZE KiB x write_scale) x 1024, "
                   "per-dispatch averages of the op's kernels summed; the scales make a copy of 1 GiB read as "
                   "1 GiB each way",
           "commands": {
               "fetch": "cd /tmp && export TMPDIR=/tmp && rocprofv3 --pmc FETCH_SIZE --output-format csv -d "
                        "$DIR/<workload>_fetch -o pmc -- python3 $REPO/bench.py --workload <workload> --steps 3 "
                        "--warmup 1 --min-warmup-ms 0 --no-cpu --no-extra",
               "write": "the same with --pmc WRITE_SIZE into $DIR/<workload>_write",
               "copy": "rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) -d $DIR/copy_fetch (copy_write) -o pmc -- "
                       "python3 $REPO/bench.py --calibrate-copy",
               "summary": "python3 bench.py --pmc-summarize $DIR"},
           "calibration": {"copy_kernel": "vh_d2d of 1 GiB, 4 dispatches", "expected_kib_each_way": exp_kib,
                           "fetch_kib_measured": round(fmean, 1), "write_kib_measured": round(wmean, 1),
                           "fetch_scale": round(fscale, 4), "write_scale": round(wscale, 4)},
           "workloads": {}}
    for wl, pats in PMC_KERNELS.items():
        bf, bw = per_kernel(wl + "_fetch"), per_kernel(wl + "_write")
        if bf is None or bw is None:
            continue
        res = {}
        for op, pat in pats.items():
            syms = sorted(n for n in bf if re.search(pat, n))
            if not syms:
                continue
            f = sum(sum(bf[n]) / len(bf[n]) for n in syms)
            w = sum(sum(bw[n]) / len(bw[n]) for n in syms if n in bw)
            res[op] = {"symbols": syms, "fetch_kib": round(f, 1), "write_kib": round(w, 1),
                       "traffic_bytes": int(round((f * fscale + w * wscale) * 1024))}
        out["workloads"][wl] = res
    # Workloads not measured under root keep their earlier records (each was
    # scaled by the copy calibration of its own run).
    if os.path.exists(PMC_FILE):
        with open(PMC_FILE) as f:
            prev = json.load(f).get("workloads", {})
        for wl, rec in prev.items():
            out["workloads"].setdefault(wl, rec)
    with open(PMC_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps({wl: {op: v["traffic_bytes"] for op, v in r.items()} for wl, r in out["workloads"].items()}))
# Run by default after the headline, each reported under "configs" in the one line.
EXTRA = ["gpt2_block", "gelu_bias", "embedding_uniform", "embedding_zipf", "cross_entropy",
         "cross_entropy_rowstats", "softmax_dense", "layernorm_cfg0"]


def host_info():
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    try:
        glibc = os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        glibc = None
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "glibc": glibc}


def measure(vh, hip, stream, ops, K, warmup, min_warmup_ms):
    """Warm up (at least `warmup` steps and `min_warmup_ms`), time exactly K
    steps back to back (wall clock around them, synchronised on both sides),
    then per-op times two ways: HIP events between the ops of a second pass of
    K steps ("in_step": includes each event's own cost), and each op alone K
    times back to back between two events ("avg": the op's average launch
    duration, what a kernel trace reports plus the gap between launches)."""
    vh.sync()
    warm = 0
    t_w = time.perf_counter()
    while warm < warmup or time.perf_counter() - t_w < min_warmup_ms / 1e3:
        for _, _, call in ops:
            vh.check(call(warm))
        warm += 1
        if warm % 8 == 0:
            vh.sync()  # wall time then tracks the GPU's, not the launch queue's
    vh.sync()
    t0 = time.perf_counter()
    for i in range(K):
        for _, _, call in ops:
            vh.check(call(i))
    hip.sync(stream)
    wall = time.perf_counter() - t0
    vh.sync()
    ev = [[hip.event() for _ in range(len(ops) + 1)] for _ in range(K)]
    for i in range(K):
        e = ev[i]
        hip.record(e[0], stream)
        for j, (_, _, call) in enumerate(ops):
            vh.check(call(i))
            hip.record(e[j + 1], stream)
    hip.sync(stream)
    vh.sync()
    in_step = {n: sum(hip.elapsed_ms(ev[i][j], ev[i][j + 1]) for i in range(K)) / K
               for j, (n, _, _) in enumerate(ops)}
    avg = {}
    for n, _, call in ops:
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, stream)
        for i in range(K):
            vh.check(call(i))
        hip.record(e1, stream)
        hip.sync(stream)
        avg[n] = hip.elapsed_ms(e0, e1) / K
    vh.sync()
    return {"warmup": warm, "wall": wall, "in_step_ms": in_step, "avg_ms": avg}


def summarize_bytes(ops, m, K, workload):
    kernels = {}
    tk = pmc_traffic(workload)
    for n, nb, _ in ops:
        a_s, s_s = m["avg_ms"][n] / 1e3, m["in_step_ms"][n] / 1e3
        kernels[n] = {"avg_us": round(a_s * 1e6, 2), "in_step_us": round(s_s * 1e6, 2), "bytes": nb,
                      "gbps": round(nb / a_s / 1e9, 1), "frac": round(nb / a_s / 1e9 / PEAK_GBPS, 4)}
        if n in tk:
            kernels[n]["traffic_bytes"] = tk[n]["traffic_bytes"]
            kernels[n]["traffic_ratio"] = round(tk[n]["traffic_bytes"] / nb, 3)
    step_bytes = sum(o[1] for o in ops)
    ms = m["wall"] / K * 1e3
    return {"ms_per_step": round(ms, 4), "bytes_per_step": step_bytes,
            "gbps": round(step_bytes / (ms / 1e3) / 1e9, 1),
            "frac": round(step_bytes / (ms / 1e3) / 1e9 / PEAK_GBPS, 4), "kernels": kernels}


def lm_head_time(vh, hip, stream, pcall, pflops, reps=10):
    vh.check(pcall(0))
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    for i in range(reps):
        vh.check(pcall(i))
    hip.record(e1, stream)
    hip.sync(stream)
    p_s = hip.elapsed_ms(e0, e1) / reps / 1e3
    achieved = pflops / p_s / 1e12
    return {"avg_us": round(p_s * 1e6, 1), "flops": pflops, "tflops": round(achieved, 2),
            "frac": round(achieved / PEAK_F32_MFMA_TFLOPS, 4)}


def lm_head_probe(vh, hip, stream, info):
    pname, pflops, pcall = info.pop("_probe")
    res = lm_head_time(vh, hip, stream, pcall, pflops)
    res["path"] = {vh.GEMM_PATH_PERSISTENT: "own persistent kernel", vh.GEMM_PATH_LIBRARY: "hipBLASLt"}.get(
        vh.lib.vh_gemm_last_path(), "own tiled kernel")
    return pname, res


def run_one(name, vh, hip, stream, args, cpu_budget):
    """Set up one workload, measure it, time its CPU baseline; returns a summary."""
    ops, info, cpu, keep = WORKLOADS[name](vh)
    m = measure(vh, hip, stream, ops, args.steps, args.warmup, args.min_warmup_ms)
    K = args.steps
    if info.get("_mode") == "step_ms":
        info.pop("_mode")
        pname, probe = lm_head_probe(vh, hip, stream, info)
        ab = info.pop("_ab", None)
        dropin = info.pop("_dropin", None)
        dropin_unfused = info.pop("_dropin_unfused", None)
        dropin_ref = info.pop("_dropin_reference_arms", None)
        step_s = m["wall"] / K
        flops = info["flops_per_step"]
        # HBM traffic of the lm_head product (counters over the product alone,
        # workload lm_head_gemm) and of the step's fused cross-entropy pass.
        lt = pmc_traffic("lm_head_gemm").get("lm_head_gemm")
        if lt:
            probe["traffic_bytes"] = lt["traffic_bytes"]
        ce = pmc_traffic(name).get("cross_entropy_fused")
        res = {"ms_per_step": round(step_s * 1e3, 3), "tflops": round(flops / step_s / 1e12, 2),
               "frac_of_f32_mfma_peak": round(flops / step_s / 1e12 / PEAK_F32_MFMA_TFLOPS, 4),
               "kernels": {pname: probe}, "config": info,
               "roofline": {"bound": "mfma", "kernel": pname, "achieved": probe["tflops"],
                            "peak": PEAK_F32_MFMA_TFLOPS, "unit": "TFLOP/s", "frac": probe["frac"],
                            "traffic": lt["traffic_bytes"] if lt else None}}
        if ce:
            res["cross_entropy_fused_traffic_bytes"] = ce["traffic_bytes"]
        if ab is not None:
            res["ab_library"] = ab(hip, stream, max(3, min(K, 10)))
        if dropin is not None:
            res["dropin"] = dropin(hip, stream, max(3, min(K, 10)))
        if dropin_ref is not None:
            res["dropin_reference_arms"] = dropin_ref(hip, stream, max(3, min(K, 10)))
        if dropin_unfused is not None:
            res["dropin_unfused"] = dropin_unfused(hip, stream, max(3, min(K, 10)))
        if cpu_budget is not None:
            ms, threads, sample = cpu(cpu_budget)
            res["cpu_baseline"] = {"value": round(ms, 1), "unit": "ms per step", "cores": threads, "kind": "port",
                                   "sample": sample, "host": host_info()}
    else:
        res = summarize_bytes(ops, m, K, name)
        res["config"] = info
        if cpu_budget is not None and cpu is not None:
            rate, sample = cpu(cpu_budget)
            res["cpu_baseline"] = {"value": round(rate / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                                   "sample": sample + "; GB/s counts the same algorithmic bytes as the GPU figure"}
    res["warmup_steps"] = m["warmup"]
    del keep, ops
    vh.sync()
    vh.check(vh.lib.vh_empty_cache())
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--min-warmup-ms", type=float, default=1000.0,
                    help="keep warming up until this much wall time has passed (GPU clocks recover "
                         "from the idle of input generation)")
    ap.add_argument("--workload", default="ln_softmax", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline only (no other configs in the line)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--pmc-summarize", metavar="DIR",
                    help="only write profiles/pmc_traffic.json from the rocprofv3 --pmc runs under DIR "
                         "(no GPU use)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 4 device-to-device copies of 1 GiB (a copy kernel of known "
                         "size, used to scale rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.pmc_summarize:
        pmc_summarize(args.pmc_summarize)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from vearo_amd import _abi as vh

    vh.init(0)
    hip = Hip()
    stream = vh.lib.vh_stream()
    if args.calibrate_copy:
        # 1 GiB each way: four times the 256 MB last-level cache in front of
        # HBM, so the copies stream from and to HBM.
        nb = 1 << 30
        src, dst = vh.DeviceBuffer(nb, zero=True), vh.DeviceBuffer(nb)
        vh.sync()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, stream)
        for _ in range(4):
            vh.check(vh.lib.vh_d2d(dst.ptr, src.ptr, nb, None))
        hip.record(e1, stream)
        vh.sync()
        ms = hip.elapsed_ms(e0, e1)
        print(json.dumps({"calibrate_copy_bytes": nb, "copies": 4,
                          "copy_gbps": round(4 * 2 * nb / (ms / 1e3) / 1e9, 1)}), flush=True)
        return
    if args.workload == "checkpoint":
        run_checkpoint(args, vh)
        return

    cpu_budget = None if args.no_cpu else args.cpu_seconds
    head = run_one(args.workload, vh, hip, stream, args, cpu_budget)
    K = args.steps
    common = {"n_gpus": 1, "steps": K, "warmup": args.warmup, "warmup_steps_run": head.pop("warmup_steps"),
              "scaling": "weak", "vs_baseline": None, "dtype": "f32"}
    if args.workload == "gpt2_block":
        res = {"metric": "GPT block step ms (config[4]: fwd + bwd + AdamW)", "value": head["ms_per_step"],
               "unit": "ms", **common, "ms_per_step": head["ms_per_step"], "higher_is_better": False,
               "data": "synthetic (random ids/targets, weights ~N(0,0.02))", **head}
        print(json.dumps(res), flush=True)
        return
    kernels = head["kernels"]
    dom = max(kernels, key=lambda n: kernels[n]["avg_us"])
    roofline = {"bound": "hbm", "kernel": dom, "achieved": kernels[dom]["gbps"], "peak": PEAK_GBPS, "unit": "GB/s",
                "frac": kernels[dom]["frac"], "traffic": kernels[dom].get("traffic_bytes")}
    info = head["config"]
    info["bytes_per_step"] = head["bytes_per_step"]
    res = {"metric": METRIC if args.workload == "ln_softmax" else f"{args.workload} fwd+bwd HBM GB/s",
           "value": head["gbps"], "unit": "GB/s", **common, "ms_per_step": head["ms_per_step"],
           "higher_is_better": True, "data": "synthetic", "config": info, "frac_of_peak": head["frac"],
           "kernels": kernels, "roofline": roofline, "cpu_baseline": head.get("cpu_baseline")}
    if res["cpu_baseline"] is not None:
        res["cpu_baseline"]["host"] = host_info()
    if args.workload == "ln_softmax":
        lnk = [kernels["layernorm_fwd"], kernels["layernorm_bwd"]]
        ln_us = sum(k["avg_us"] for k in lnk)
        ln_b = sum(k["bytes"] for k in lnk)
        res["layernorm_fwd_bwd"] = {"avg_us": round(ln_us, 2), "bytes": ln_b, "gbps": round(ln_b / ln_us / 1e3, 1),
                                    "frac": round(ln_b / ln_us / 1e3 / PEAK_GBPS, 4)}
        smk = [kernels["softmax_fwd"], kernels["softmax_bwd"]]
        sm_us = sum(k["avg_us"] for k in smk)
        sm_b = sum(k["bytes"] for k in smk)
        res["softmax_fwd_bwd"] = {"avg_us": round(sm_us, 2), "bytes": sm_b, "gbps": round(sm_b / sm_us / 1e3, 1),
                                  "frac": round(sm_b / sm_us / 1e3 / PEAK_GBPS, 4)}
    if args.workload == "ln_softmax" and not args.no_extra:
        # The other configs of BASELINE.json, each measured the same way; their
        # CPU baselines are bounded samples (a few seconds each).
        configs = {}
        ebudget = None if args.no_cpu else min(3.0, args.cpu_seconds)
        for name in EXTRA:
            t0 = time.perf_counter()
            configs[name] = run_one(name, vh, hip, stream, args, ebudget)
            configs[name]["wall_s"] = round(time.perf_counter() - t0, 1)
            print(f"# {name} done ({configs[name]['wall_s']} s)", file=sys.stderr, flush=True)
        g = configs["gpt2_block"]
        res["gpt2_block_ms"] = g["ms_per_step"]
        res["gpt2_block_tflops"] = g["tflops"]
        res["gpt2_block_frac_of_f32_mfma_peak"] = g["frac_of_f32_mfma_peak"]
        res["gpt2_block_ms_hipblaslt_ab"] = g.get("ab_library", {}).get("gpt2_block_ms_library")
        res["gpt2_block_dropin_ms"] = g.get("dropin", {}).get("ms_per_step")
        res["gpt2_block_dropin_reference_arms_ms"] = g.get("dropin_reference_arms", {}).get("ms_per_step")
        res["gpt2_block_dropin_unfused_ms"] = g.get("dropin_unfused", {}).get("ms_per_step")
        res["configs"] = configs
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
