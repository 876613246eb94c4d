"""`.ve` checkpoints of device tensors (vh_checkpoint_save/load, vb_gpt_save/load)
against the CPU oracle (oracle/vearo_cpu_ckpt.c): the files the device writes
are byte for byte the oracle's, files the oracle writes load bit-exactly, and
the reference's panics and io errors come back with its texts
(crates/vearo/src/checkpoint.rs:9-91, tensor.rs:751-755, 816-826).
"""
import ctypes
import os

import numpy as np
import pytest

import oracle as O
from test_checkpoint_cpu import KAT, ref_tensors

pytestmark = pytest.mark.gpu


def dev(vh, a):
    a = np.ascontiguousarray(a, np.float32)
    return vh.DeviceBuffer.from_array(a) if a.size else vh.DeviceBuffer(4)


def fetch(vh, b, shape):
    vh.sync()
    return b.to_array(shape) if int(np.prod(shape)) else np.zeros(shape, np.float32)


def call(vh, fn, path, bufs, layouts):
    n = len(bufs)
    ptrs = (ctypes.c_void_p * max(n, 1))(*[b.ptr for b in bufs])
    lays = (vh.VhLayout * max(n, 1))(*layouts)
    return fn(os.fsencode(path), n, ptrs, lays, None)


def save(vh, path, bufs, layouts):
    vh.check(call(vh, vh.lib.vh_checkpoint_save, path, bufs, layouts))


def load_rc(vh, path, bufs, layouts):
    return call(vh, vh.lib.vh_checkpoint_load, path, bufs, layouts)


def test_device_save_writes_the_reference_test_file(vh, tmp_path):
    t = ref_tensors()
    p = tmp_path / "model_checkpoint.ve"
    save(vh, p, [dev(vh, a) for a in t], [vh.layout(a.shape) for a in t])
    assert p.read_bytes() == KAT


def test_device_load_of_the_reference_test_file(vh, tmp_path):
    p = tmp_path / "model_checkpoint.ve"
    p.write_bytes(KAT)
    bufs = [dev(vh, np.zeros((2, 2), np.float32)), dev(vh, np.zeros(2, np.float32))]
    vh.check(load_rc(vh, p, bufs, [vh.layout((2, 2)), vh.layout((2,))]))
    assert fetch(vh, bufs[0], (2, 2)).tolist() == [[1, 2], [3, 4]]
    assert fetch(vh, bufs[1], (2,)).tolist() == [-0.5, 0.5]


def multi_chunk_set():
    """Tensors larger than the 32 MiB staging buffers (several chunks, a
    ragged last one), small ones, a scalar and an empty tensor."""
    r = np.random.default_rng(5)
    return [r.standard_normal((3, 11_000_003), dtype=np.float32),
            r.standard_normal((768,), dtype=np.float32),
            np.array(np.float32(-3.25)),
            np.zeros((5, 0, 2), np.float32),
            r.standard_normal((8_388_608,), dtype=np.float32),
            r.standard_normal((17, 3), dtype=np.float32)]


def test_device_save_equals_oracle_save_across_chunks(vh, tmp_path):
    arrays = multi_chunk_set()
    print("checkpoint save", [a.shape for a in arrays], flush=True)
    p, q = tmp_path / "dev.ve", tmp_path / "oracle.ve"
    save(vh, p, [dev(vh, a) for a in arrays], [vh.layout(a.shape) for a in arrays])
    O.checkpoint_save(q, arrays)
    assert p.stat().st_size == q.stat().st_size
    assert p.read_bytes() == q.read_bytes()


def test_device_load_of_an_oracle_file_is_bit_exact(vh, tmp_path):
    arrays = multi_chunk_set()
    print("checkpoint load", [a.shape for a in arrays], flush=True)
    q = tmp_path / "oracle.ve"
    O.checkpoint_save(q, arrays)
    bufs = [dev(vh, np.full(a.shape, 9.0, np.float32)) for a in arrays]
    vh.check(load_rc(vh, q, bufs, [vh.layout(a.shape) for a in arrays]))
    for a, b in zip(arrays, bufs):
        assert fetch(vh, b, a.shape).tobytes() == a.tobytes()


def test_device_load_panics_and_io_errors(vh, tmp_path):
    p = tmp_path / "m.ve"
    p.write_bytes(KAT)
    b1, b2 = dev(vh, np.zeros((2, 2), np.float32)), dev(vh, np.zeros(2, np.float32))
    l1, l2 = vh.layout((2, 2)), vh.layout((2,))

    def expect(rc, code, text):
        assert rc == code, (rc, vh.last_error())
        assert text in vh.last_error()

    expect(load_rc(vh, p, [b1], [l1]), vh.VH_ERR_INVALID,
           "Checkpoint tensor count does not match model parameter count")
    expect(load_rc(vh, p, [b2, b1], [l2, l1]), vh.VH_ERR_INVALID, "Checkpoint shape does not match parameter shape")
    expect(load_rc(vh, p, [b1, b2], [vh.layout((2, 2), (1, 2)), l2]), vh.VH_ERR_INVALID,
           "copy_from_slice requires contiguous tensor")
    # The first tensor is loaded before the second one's shape check fails.
    expect(load_rc(vh, p, [b1, b2], [l1, vh.layout((3,))]), vh.VH_ERR_INVALID,
           "Checkpoint shape does not match parameter shape")
    assert fetch(vh, b1, (2, 2)).tolist() == [[1, 2], [3, 4]]
    p.write_bytes(bytes.fromhex("01000000" "01000000" "02000000" "03000000") + b"\0" * 12)
    expect(load_rc(vh, p, [b2], [l2]), vh.VH_ERR_INVALID, "Source slice length must match tensor numel")
    p.write_bytes(KAT[:-3])
    expect(load_rc(vh, p, [b1, b2], [l1, l2]), vh.VH_ERR_IO, "unexpected end of file")
    expect(load_rc(vh, tmp_path / "missing.ve", [b1], [l1]), vh.VH_ERR_IO, "missing.ve")
    rc = call(vh, vh.lib.vh_checkpoint_save, tmp_path / "t.ve", [b1], [vh.layout((2, 2), (1, 2))])
    expect(rc, vh.VH_ERR_INVALID, "to_vec_f32 requires contiguous tensor")
    assert not (tmp_path / "t.ve").exists()


def test_device_load_length_mismatch_after_a_multi_chunk_tensor(vh, tmp_path):
    """A first tensor of two staging chunks, then a second whose element count
    disagrees with its dims: the error comes back with the reference's text and
    the first tensor is fully loaded (its copies finish before the discarded
    block reuses the staging buffer)."""
    r = np.random.default_rng(9)
    big = r.standard_normal(12_000_000, dtype=np.float32)  # 48 MB: two 32 MiB chunks
    head = np.uint32([2, 1, big.size, big.size]).tobytes()
    # Second tensor: rank 1, dims [2], but a length field of 3 and three values.
    tail = np.uint32([1, 2, 3]).tobytes() + np.float32([1, 2, 3]).tobytes()
    p = tmp_path / "len.ve"
    p.write_bytes(head + big.tobytes() + tail)
    b1 = dev(vh, np.zeros(big.size, np.float32))
    b2 = dev(vh, np.zeros(2, np.float32))
    rc = load_rc(vh, p, [b1, b2], [vh.layout((big.size,)), vh.layout((2,))])
    assert rc == vh.VH_ERR_INVALID and "Source slice length must match tensor numel" in vh.last_error()
    assert fetch(vh, b1, (big.size,)).tobytes() == big.tobytes()


def test_gpt_checkpoint_round_trip(vh, tmp_path):
    """vb_gpt_save writes model.parameters() as the reference would; loading it
    back after a training step restores every parameter bit for bit."""
    from vearo_amd import _block
    cfg = (2, 16, 32, 4, 64, 50, 16)
    g = _block.Gpt(_block.GptConfig(*cfg))
    r = np.random.default_rng(9)
    params = [(r.standard_normal(sh) * 0.02).astype(np.float32) for sh in g.shapes]
    g.set_params(params)
    p = tmp_path / "gpt.ve"
    g.save(p)
    q = tmp_path / "oracle.ve"
    O.checkpoint_save(q, params)
    assert p.read_bytes() == q.read_bytes()
    ids = r.integers(0, cfg[5], size=(2, 16)).astype(np.float32)
    g.set_inputs(ids, ids)
    g.train_step()
    assert any(not np.array_equal(a, b) for a, b in zip(g.params(), params))
    g.load(p)
    for a, b in zip(g.params(), params):
        assert a.tobytes() == b.tobytes()
    # A checkpoint of another model size is refused with the reference's text.
    small = _block.Gpt(_block.GptConfig(2, 16, 32, 4, 64, 40, 16))
    with pytest.raises(vh.VhError, match="Checkpoint shape does not match parameter shape"):
        small.load(p)
    small.close()
    g.close()
