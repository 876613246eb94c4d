"""The reference's own golden fixture, test_data/oracles.json (written by its
tests/generate_oracles.py:14-58 with NumPy; replayed by
crates/vearo/tests/verification_harness.rs:46-104 at |got - expected| <= 1e-5),
kept here as data (tests/golden/oracles.json, copied unchanged).

The CPU half pins the oracle's binary ops and matmul against it; the GPU half
replays every case through the C ABI: vh_binary (add, sub, mul, div, the
transposed and the broadcast add -- the transposed add also as a genuinely
strided view), vh_matmul (2-D and batched), and vh_strided_copy for reshape,
transpose(0, 1) and permute([2, 0, 1]), the reference's views made contiguous
as its assert does (verification_harness.rs:22)."""
import json
import os

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
OPS = {"add": 0, "add_transposed": 0, "add_broadcasted": 0, "sub": 1, "mul": 2, "div": 3}


def cases():
    with open(os.path.join(HERE, "golden", "oracles.json")) as f:
        return json.load(f)


def arrays(case):
    ins = [np.float32(t["data"]).reshape(t["shape"]) for t in case["inputs"]]
    out = np.float32(case["output"]["data"]).reshape(case["output"]["shape"])
    return ins, out


def close(got, want):
    assert got.shape == want.shape
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5), (got, want)


def test_fixture_covers_the_reference_cases():
    assert [c["op"] for c in cases()] == ["add", "add_transposed", "add_broadcasted", "sub", "mul", "div",
                                           "matmul_2d", "matmul_batched", "reshape", "transpose", "permute"]


@pytest.mark.parametrize("case", cases(), ids=lambda c: c["op"])
def test_oracle_matches_reference_fixture(case):
    ins, want = arrays(case)
    op = case["op"]
    if op in OPS:
        got = O.binary(OPS[op], ins[0], ins[1])
    elif op.startswith("matmul"):
        got = O.matmul(ins[0], ins[1])
    elif op == "reshape":
        got = ins[0].reshape(want.shape)
    elif op == "transpose":
        got = np.ascontiguousarray(ins[0].T)
    else:
        got = np.ascontiguousarray(np.transpose(ins[0], (2, 0, 1)))
    close(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("case", cases(), ids=lambda c: c["op"])
def test_device_matches_reference_fixture(vh, case):
    from parity import dev, fetch, out
    ins, want = arrays(case)
    op = case["op"]
    X = dev(vh, ins[0])
    if op in OPS or op.startswith("matmul"):
        Y = dev(vh, ins[1])
        OUT = out(vh, want.shape)
        lx, ly = vh.layout(ins[0].shape), vh.layout(ins[1].shape)
        if op in OPS:
            vh.check(vh.lib.vh_binary(OPS[op], X.ptr, lx, Y.ptr, ly, OUT.ptr, None))
        else:
            vh.check(vh.lib.vh_matmul(X.ptr, lx, Y.ptr, ly, OUT.ptr, None))
        close(fetch(vh, OUT, want.shape), want)
        if op == "add_transposed":
            # The same sum with x given as the transposed view of its [2, 3]
            # original (strides (1, 3)), the reference case's intent.
            X2 = dev(vh, np.ascontiguousarray(ins[0].T))
            OUT2 = out(vh, want.shape)
            vh.check(vh.lib.vh_binary(0, X2.ptr, vh.layout((3, 2), (1, 3)), Y.ptr, ly, OUT2.ptr, None))
            close(fetch(vh, OUT2, want.shape), want)
        return
    if op == "reshape":
        view = vh.layout(want.shape)
    elif op == "transpose":
        r, c = ins[0].shape
        view = vh.layout((c, r), (1, c))
    else:  # permute([2, 0, 1]) of [a, b, c] (strides (b c, c, 1)) -> [c, a, b]
        a, b, c = ins[0].shape
        view = vh.layout((c, a, b), (1, b * c, c))
    OUT = out(vh, want.shape)
    vh.check(vh.lib.vh_strided_copy(X.ptr, view, OUT.ptr, None))
    close(fetch(vh, OUT, want.shape), want)
