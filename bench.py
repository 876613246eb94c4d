"""Benchmark of the hot path on one MI355X.

A step is one pass of the path over one synthetic batch at GPT-2-small shape:
  layernorm forward    x [16384, 768]                 (cfg[4] shape; cfg[0'] in SURVEY)
  causal softmax fwd   scores [16, 12, 1024, 1024]    (cfg[2])
  causal softmax bwd   (from the saved input x and dy, as the autograd arm)
  layernorm backward   (x, w, dy -> dx, dgamma, dbeta)
issued in that order on the runtime stream, as a training step meets them
(forward, then backward in reverse). Inputs are resident in HBM before timing;
layernorm buffers alternate between two sets and the 3.2 GB softmax working set
flushes the 256 MB MALL between uses, so every kernel reads cold data.

value = algorithmic bytes per step / wall time per step (GB/s), where the
algorithmic bytes count each necessary HBM transfer once (the live causal
triangle only for softmax reads). Per-kernel durations come from HIP events on
the runtime stream around each launch; the roofline object reports the longest
kernel. cpu_baseline times the CPU oracle (the C restatement of the reference's
CPU backend, one thread) on a bounded row sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu]
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
LN_ROWS, LN_C = 16384, 768
SM_B, SM_H, SM_T = 16, 12, 1024


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
    bwd = 4 * live * 2 + 4 * n            # R live x (or y), R live dy, W all dx
    return fwd, bwd


class Hip:
    """The few HIP runtime calls bench needs (events on the runtime stream)."""

    def __init__(self):
        self.h = ctypes.CDLL("libamdhip64.so.7")
        self.h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
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
    s = (r.standard_normal(size=(B, H, T, T), dtype=np.float32) * np.float32(0.125))
    iu = np.triu_indices(T, 1)
    s[:, :, iu[0], iu[1]] = -np.inf
    return s


def cpu_baseline(budget_s):
    """The oracle (one thread) on a row sample of the same workload."""
    import oracle

    r = np.random.default_rng(0x5EED0000)
    ln_rows, sm_heads = 4096, 2
    x = r.standard_normal(size=(ln_rows, LN_C), dtype=np.float32)
    w = (1 + 0.02 * r.standard_normal(LN_C)).astype(np.float32)
    b = (0.02 * r.standard_normal(LN_C)).astype(np.float32)
    dy = r.standard_normal(size=(ln_rows, LN_C), dtype=np.float32)
    s = causal_scores(r, 1, sm_heads, SM_T)
    g = r.standard_normal(size=s.shape, dtype=np.float32)
    t_total, reps, sample_bytes = 0.0, 0, 0
    lf, lb = ln_bytes(ln_rows, LN_C)
    sf, sb = sm_bytes(1, sm_heads, SM_T)
    while t_total < budget_s or reps == 0:
        t0 = time.perf_counter()
        oracle.layernorm(x, w, b, 1e-5)
        oracle.softmax(s, 3)
        oracle.softmax_backward_composite(s, g, 3)
        oracle.layernorm_backward(x, w, b, dy, 1e-5)
        t_total += time.perf_counter() - t0
        reps += 1
        sample_bytes += lf + lb + sf + sb
    return {"value": round(sample_bytes / t_total / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"layernorm fwd+bwd [{ln_rows},{LN_C}] + causal softmax fwd + composite bwd "
                      f"[1,{sm_heads},{SM_T},{SM_T}], {reps} reps in {t_total:.1f} s, single thread; "
                      f"GB/s counts the same algorithmic bytes as the GPU figure"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 4 device-to-device copies of 256 MiB (a copy kernel of known "
                         "size, used to scale rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from vearo_amd import _abi as vh

    vh.init(0)
    hip = Hip()
    stream = vh.lib.vh_stream()
    if args.calibrate_copy:
        nb = 256 << 20
        src, dst = vh.DeviceBuffer(nb, zero=True), vh.DeviceBuffer(nb)
        for _ in range(4):
            vh.check(vh.lib.vh_d2d(dst.ptr, src.ptr, nb, None))
        vh.sync()
        print(json.dumps({"calibrate_copy_bytes": nb, "copies": 4}), flush=True)
        return
    r = np.random.default_rng(0x5EED0000 + 4)

    # ---- inputs, resident in HBM before the timed region
    ln_sets = []
    w = (1 + 0.02 * r.standard_normal(LN_C)).astype(np.float32)
    b = (0.02 * r.standard_normal(LN_C)).astype(np.float32)
    W, Bi = vh.DeviceBuffer.from_array(w), vh.DeviceBuffer.from_array(b)
    for _ in range(2):
        x = r.standard_normal(size=(LN_ROWS, LN_C), dtype=np.float32)
        dy = r.standard_normal(size=(LN_ROWS, LN_C), dtype=np.float32)
        ln_sets.append(dict(x=vh.DeviceBuffer.from_array(x), dy=vh.DeviceBuffer.from_array(dy),
                            y=vh.DeviceBuffer(x.nbytes), dx=vh.DeviceBuffer(x.nbytes),
                            dw=vh.DeviceBuffer(w.nbytes), db=vh.DeviceBuffer(w.nbytes)))
    ln_scratch_bytes = vh.lib.vh_layernorm_bwd_scratch_bytes(LN_ROWS, LN_C)
    LNS = vh.DeviceBuffer(ln_scratch_bytes)
    rs = np.random.default_rng(0x5EED0000 + 2)
    s = causal_scores(rs, SM_B, SM_H, SM_T)
    S = vh.DeviceBuffer.from_array(s)
    del s
    G = vh.DeviceBuffer.from_array(rs.standard_normal(size=(SM_B, SM_H, SM_T, SM_T), dtype=np.float32))
    n_sm = SM_B * SM_H * SM_T * SM_T
    P, DS = vh.DeviceBuffer(4 * n_sm), vh.DeviceBuffer(4 * n_sm)
    rows_sm = SM_B * SM_H * SM_T
    vh.sync()

    names = ["layernorm_fwd", "softmax_fwd", "softmax_bwd", "layernorm_bwd"]

    def step(i):
        L = ln_sets[i % 2]
        yield lambda: vh.lib.vh_layernorm_fwd(L["x"].ptr, W.ptr, Bi.ptr, L["y"].ptr, LN_ROWS, LN_C, 1e-5, None)
        yield lambda: vh.lib.vh_softmax_fwd(S.ptr, P.ptr, rows_sm, SM_T, 1, None)
        # The autograd Softmax arm saves the input x and recomputes y from it
        # (crates/vearo-autograd/src/lib.rs:547-553); the fused kernel does the same.
        yield lambda: vh.lib.vh_softmax_bwd(S.ptr, G.ptr, DS.ptr, rows_sm, SM_T, 1, 1, None)
        yield lambda: vh.lib.vh_layernorm_bwd(L["x"].ptr, W.ptr, L["dy"].ptr, L["dx"].ptr, L["dw"].ptr,
                                              L["db"].ptr, LN_ROWS, LN_C, 1e-5, LNS.ptr, ln_scratch_bytes, None)

    for i in range(args.warmup):
        for call in step(i):
            vh.check(call())
    vh.sync()

    K = args.steps
    ev = [[hip.event() for _ in range(len(names) + 1)] for _ in range(K)]
    hip.sync(stream)
    t0 = time.perf_counter()
    for i in range(K):
        e = ev[i]
        hip.record(e[0], stream)
        for j, call in enumerate(step(i)):
            vh.check(call())
            hip.record(e[j + 1], stream)
    hip.sync(stream)
    wall = time.perf_counter() - t0
    vh.sync()

    per = {n: 0.0 for n in names}
    for i in range(K):
        for j, n in enumerate(names):
            per[n] += hip.elapsed_ms(ev[i][j], ev[i][j + 1])
    lf, lbw = ln_bytes(LN_ROWS, LN_C)
    sf, sbw = sm_bytes(SM_B, SM_H, SM_T)
    nbytes = {"layernorm_fwd": lf, "softmax_fwd": sf, "softmax_bwd": sbw, "layernorm_bwd": lbw}
    kernels = {}
    for n in names:
        avg_s = per[n] / K / 1e3
        gbps = nbytes[n] / avg_s / 1e9
        kernels[n] = {"avg_us": round(avg_s * 1e6, 2), "bytes": nbytes[n], "gbps": round(gbps, 1),
                      "frac": round(gbps / PEAK_GBPS, 4)}
    step_bytes = sum(nbytes.values())
    ms_per_step = wall / K * 1e3
    value = step_bytes / (wall / K) / 1e9
    dom = max(names, key=lambda n: per[n])
    # HBM traffic per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    # passes over this same workload, scaled by the counters' reading of a copy of
    # known size (profiles/pmc_traffic_bench.json); null when absent.
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "pmc_traffic_bench.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tk = json.load(f).get("kernels", {})
        for n in names:
            if n in tk:
                kernels[n]["traffic_bytes"] = tk[n]["traffic_bytes"]
        traffic = tk.get(dom, {}).get("traffic_bytes")
    roofline = {"bound": "hbm", "kernel": dom, "achieved": kernels[dom]["gbps"], "peak": PEAK_GBPS,
                "unit": "GB/s", "frac": kernels[dom]["frac"], "traffic": traffic}
    res = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "layernorm fwd+bwd [16384,768] + causal softmax fwd+bwd [16,12,1024,1024]",
                   "ln_shape": [LN_ROWS, LN_C], "softmax_shape": [SM_B, SM_H, SM_T, SM_T],
                   "bytes_per_step": step_bytes},
        "frac_of_peak": round(value / PEAK_GBPS, 4),
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": None if args.no_cpu else cpu_baseline(args.cpu_seconds),
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
