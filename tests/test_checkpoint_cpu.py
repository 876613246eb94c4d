"""The `.ve` checkpoint oracle (oracle/vearo_cpu_ckpt.c) pinned on the CPU.

The format is fixed by crates/vearo/src/checkpoint.rs:12-27: u32 count; per
tensor u32 rank, u32 dims, u32 element count, f32 data; little-endian. The
known answer below is the file the reference's own test
(checkpoint.rs:97-120: t1 = [[1, 2], [3, 4]], t2 = [-0.5, 0.5]) writes, spelled
out byte by byte from that layout. The error cases follow the reference's
asserts (checkpoint.rs:50-54, 64-68; tensor.rs:751-755, 816-826) and its
io::Errors (read_exact on a short file, File::open on a missing one).
"""
import ctypes
import os

import numpy as np
import pytest

import oracle as O
from conftest import ROOT

# checkpoint.rs:97-120's two tensors as a .ve file.
KAT = bytes.fromhex(
    "02000000"                                  # 2 tensors
    "02000000" "02000000" "02000000"            # rank 2, dims [2, 2]
    "04000000"                                  # 4 values
    "0000803f" "00000040" "00004040" "00008040"  # 1.0 2.0 3.0 4.0
    "01000000" "02000000"                       # rank 1, dims [2]
    "02000000"                                  # 2 values
    "000000bf" "0000003f")                      # -0.5 0.5


def ref_tensors():
    return [np.array([[1, 2], [3, 4]], np.float32), np.array([-0.5, 0.5], np.float32)]


def test_oracle_save_writes_the_reference_test_file(tmp_path):
    p = tmp_path / "model_checkpoint.ve"
    O.checkpoint_save(p, ref_tensors())
    assert p.read_bytes() == KAT


def test_oracle_load_restores_the_reference_test_tensors(tmp_path):
    p = tmp_path / "model_checkpoint.ve"
    p.write_bytes(KAT)
    t1, t2 = np.zeros((2, 2), np.float32), np.zeros(2, np.float32)
    O.checkpoint_load(p, [t1, t2])
    assert t1.tolist() == [[1, 2], [3, 4]] and t2.tolist() == [-0.5, 0.5]


def test_oracle_round_trip_keeps_every_bit(tmp_path):
    r = np.random.default_rng(3)
    arrays = [r.standard_normal((7, 5, 3), dtype=np.float32), np.array(np.float32(2.5)),
              np.zeros((4, 0), np.float32), np.array([np.nan, -0.0, np.inf, 1e-45], np.float32)]
    p = tmp_path / "m.ve"
    O.checkpoint_save(p, arrays)
    # Header + data sizes: 4 + sum(4 + 4 rank + 4 + 4 numel).
    assert p.stat().st_size == 4 + sum(8 + 4 * a.ndim + 4 * a.size for a in arrays)
    back = [np.full(a.shape, 7.0, np.float32) for a in arrays]
    O.checkpoint_load(p, back)
    for a, b in zip(arrays, back):
        assert a.tobytes() == b.tobytes()


def test_oracle_rank0_and_empty_tensors_encode_as_the_format_says(tmp_path):
    p = tmp_path / "m.ve"
    O.checkpoint_save(p, [np.array(np.float32(1.0)), np.zeros((3, 0), np.float32)])
    assert p.read_bytes() == bytes.fromhex(
        "02000000" "00000000" "01000000" "0000803f"     # rank 0, one value
        "02000000" "03000000" "00000000" "00000000")    # rank 2 [3, 0], no values


def test_oracle_load_panics_like_the_reference(tmp_path):
    p = tmp_path / "m.ve"
    p.write_bytes(KAT)
    t1, t2 = np.zeros((2, 2), np.float32), np.zeros(2, np.float32)
    with pytest.raises(O.Panic, match="^Checkpoint tensor count does not match model parameter count$"):
        O.checkpoint_load(p, [t1])
    with pytest.raises(O.Panic, match="^Checkpoint shape does not match parameter shape$"):
        O.checkpoint_load(p, [t2, t1])
    with pytest.raises(O.Panic, match="^Checkpoint shape does not match parameter shape$"):
        O.checkpoint_load(p, [np.zeros((1, 4), np.float32), t2])
    # Same dims, strided view: copy_from_slice's contiguity assert.
    with pytest.raises(O.Panic, match="^copy_from_slice requires contiguous tensor$"):
        O.checkpoint_load(p, [np.zeros((2, 2), np.float32).T, t2])
    # A value count that differs from the dims' product: copy_from_slice's length assert.
    p.write_bytes(bytes.fromhex("01000000" "01000000" "02000000" "03000000") + b"\0" * 12)
    with pytest.raises(O.Panic, match="^Source slice length must match tensor numel$"):
        O.checkpoint_load(p, [t2])


def test_oracle_load_tensors_before_a_failure_keep_their_values(tmp_path):
    p = tmp_path / "m.ve"
    p.write_bytes(KAT)
    t1 = np.zeros((2, 2), np.float32)
    with pytest.raises(O.Panic):
        O.checkpoint_load(p, [t1, np.zeros(3, np.float32)])
    assert t1.tolist() == [[1, 2], [3, 4]]


def test_oracle_io_errors(tmp_path):
    with pytest.raises(O.CheckpointIOError):
        O.checkpoint_load(tmp_path / "missing.ve", [np.zeros(2, np.float32)])
    p = tmp_path / "short.ve"
    p.write_bytes(KAT[:-3])  # the last value cut short: read_exact fails
    with pytest.raises(O.CheckpointIOError, match="unexpected end of file"):
        O.checkpoint_load(p, ref_tensors())
    # A short data block is an io error even when the count would also panic.
    p.write_bytes(bytes.fromhex("01000000" "01000000" "02000000" "03000000") + b"\0" * 8)
    with pytest.raises(O.CheckpointIOError):
        O.checkpoint_load(p, [np.zeros(2, np.float32)])
    with pytest.raises(O.CheckpointIOError):
        O.checkpoint_save(tmp_path / "no_such_dir" / "m.ve", ref_tensors())


def test_oracle_save_refuses_a_strided_tensor(tmp_path):
    with pytest.raises(O.Panic, match="^to_vec_f32 requires contiguous tensor$"):
        O.checkpoint_save(tmp_path / "m.ve", [np.zeros((2, 3), np.float32).T])


def test_block_library_exports_checkpoint_entries():
    lib = ctypes.CDLL(os.path.join(ROOT, "vearo_amd", "lib", "libvearo_backend.so"))
    for name in ("vb_gpt_save", "vb_gpt_load"):
        assert hasattr(lib, name)


def test_device_checkpoint_before_init_fails_cleanly(tmp_path):
    from vearo_amd import _abi

    if _abi._initialised:
        pytest.skip("runtime already initialised in this process")
    assert _abi.lib.vh_checkpoint_save(os.fsencode(tmp_path / "m.ve"), 0, None, None, None) == \
        _abi.VH_ERR_NOT_INIT
    assert not (tmp_path / "m.ve").exists()
