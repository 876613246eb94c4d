"""CPU-side checks of the C ABI boundary: libvearo_hip.so loads, exports every
function include/vearo_hip.h declares, refuses work before vh_init (no GPU
call is made), and its embedded gfx950 code object holds every kernel name the
host launcher can ask for."""
import ctypes
import os
import re
import struct

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "vearo_hip.h")
LIB = os.path.join(ROOT, "vearo_amd", "lib", "libvearo_hip.so")
CODE_OBJECT = os.path.join(ROOT, "vearo_amd", "csrc", "_build", "vearo_kernels.co")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_hot_path():
    names = declared_functions()
    for want in ["vh_layernorm_fwd", "vh_layernorm_bwd", "vh_softmax_fwd", "vh_softmax_bwd",
                 "vh_gelu_fwd", "vh_gelu_bias_fwd", "vh_gelu_bias_bwd", "vh_gelu_grad_mul",
                 "vh_embedding_fwd", "vh_embedding_bwd", "vh_cross_entropy_fwd",
                 "vh_cross_entropy_bwd", "vh_binary", "vh_reduce", "vh_strided_copy",
                 "vh_init", "vh_alloc", "vh_free", "vh_h2d", "vh_d2h", "vh_sync"]:
        assert want in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_every_declared_symbol():
    from vearo_amd import _abi

    assert sorted(_abi.SIGNATURES) == declared_functions()


def test_calls_before_init_fail_cleanly():
    from vearo_amd import _abi

    if _abi._initialised:
        pytest.skip("runtime already initialised in this process")
    p = ctypes.c_void_p()
    assert _abi.lib.vh_alloc(16, 0, ctypes.byref(p)) == _abi.VH_ERR_NOT_INIT
    assert "vh_init" in _abi.last_error()
    assert _abi.lib.vh_layernorm_fwd(None, None, None, None, 1, 1, 1e-5, None) == _abi.VH_ERR_NOT_INIT
    assert _abi.lib.vh_sync() == _abi.VH_ERR_NOT_INIT


def test_scratch_size_queries_are_host_only():
    from vearo_amd import _abi

    assert _abi.lib.vh_layernorm_bwd_scratch_bytes(16384, 768) >= 2 * 768 * 4
    assert _abi.lib.vh_layernorm_bwd_scratch_bytes(0, 768) == 0
    assert _abi.lib.vh_gelu_bias_bwd_scratch_bytes(16384, 3072) >= 3072 * 4
    assert _abi.lib.vh_embedding_bwd_scratch_bytes(16384, 50257, 768) >= 4 * (3 * 16384 + 2 * 50257)
    assert _abi.lib.vh_cross_entropy_fwd_scratch_bytes(16384) >= 16384 * 4
    assert _abi.lib.vh_sum_rows_scratch_bytes(16384, 768) >= 768 * 4
    assert _abi.lib.vh_fused_attention_scratch_bytes(16, 12, 1024, 0) >= 16 * 12 * 1024 * 1024 * 4
    assert _abi.lib.vh_fused_attention_scratch_bytes(16, 12, 1024, 1) >= 2 * 16 * 12 * 1024 * 1024 * 4


def elf_symbols(path):
    data = open(path, "rb").read()
    assert data[:4] == b"\x7fELF" and data[4] == 2, "expected a 64-bit ELF code object"
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", data, 0x3A)
    secs = [struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize) for i in range(shnum)]
    names = set()
    for s in secs:
        if s[1] in (2, 11):  # SHT_SYMTAB, SHT_DYNSYM
            strtab = secs[s[6]]
            for off in range(s[4], s[4] + s[5], 24):
                st_name, = struct.unpack_from("<I", data, off)
                end = data.index(b"\0", strtab[4] + st_name)
                names.add(data[strtab[4] + st_name:end].decode())
    return names


def launcher_kernel_names():
    """Every kernel name the host launcher (vearo_amd/csrc/runtime.cpp) can build."""
    nv = [1, 2, 3, 4, 6, 8, 12, 16]
    cfgs_all = [(16, 1), (32, 1)] + [(64, v) for v in nv] + [(1024, v) for v in nv]
    cfgs_small = [(t, v) for t, v in cfgs_all if v <= 8]
    names = set()
    multi = [(16, 1), (32, 1), (64, 1), (64, 2), (64, 3), (64, 4)]
    for vw in (1, 4):
        for t, v in cfgs_all:
            names |= {f"vh_ln_fwd_t{t}_n{v}_v{vw}_r1", f"vh_sm_fwd_t{t}_n{v}_v{vw}_r1"}
        for t, v in cfgs_small:
            names.add(f"vh_sm_bwd_t{t}_n{v}_v{vw}_r1")
            if not (t == 1024 and v * vw > 16):  # longer rows take the streaming kernels
                names.add(f"vh_ln_bwd_t{t}_n{v}_v{vw}_b{max(t, 256)}")
        names |= {f"vh_sm_fwd_wide_v{vw}", f"vh_sm_bwd_wide_v{vw}", f"vh_ln_fwd_wide_v{vw}",
                  f"vh_ln_stats_wide_v{vw}", f"vh_ln_tile_wide_v{vw}", f"vh_binary_rowbcast_v{vw}",
                  f"vh_binary_colbcast_v{vw}", f"vh_emb_sum_v{vw}"}
        for t, v in multi:
            names |= {f"vh_ln_fwd_t{t}_n{v}_v{vw}_r2", f"vh_ln_fwd_t{t}_n{v}_v{vw}_r4",
                      f"vh_sm_fwd_t{t}_n{v}_v{vw}_r2", f"vh_sm_bwd_t{t}_n{v}_v{vw}_r2"}
        for v in (1, 2, 3, 4):
            names.add(f"vh_ln_bwd_t64_n{v}_v{vw}_b512")
            if vw == 4:
                names |= {f"vh_ln_bwd_t64_n{v}_v4_b512_f", f"vh_ln_fwd_t64_n{v}_v4_r4_f"}
        for v in nv:
            names.add(f"vh_gelu_bias_fwd_n{v}_v{vw}")
        names |= {f"vh_gelu_bias_bwd_tile_v{vw}", f"vh_gelu_bias_fwd_tile_v{vw}"}
        names |= {f"vh_sm_fwd_t128_n2_v{vw}_r1", f"vh_sm_bwd_t128_n2_v{vw}_r1"}
        names |= {f"vh_gelu_fwd_v{vw}", f"vh_gelu_gradmul_v{vw}", f"vh_emb_fwd_v{vw}",
                  f"vh_emb_rows_v{vw}", f"vh_emb_heavy_final_v{vw}", f"vh_binary_contig_v{vw}"}
    for v in list(range(8, 129, 8)) + [99]:
        names |= {f"vh_xent_fwd_n{v}", f"vh_xent_bwd_n{v}", f"vh_xent_fb_n{v}"}
    names |= {"vh_xent_fwd_stream", "vh_xent_bwd_stream", "vh_xent_reduce", "vh_col_reduce",
              "vh_emb_tokens", "vh_emb_alloc", "vh_emb_place", "vh_fill", "vh_stream_copy",
              "vh_binary_strided_i32", "vh_binary_strided_i64", "vh_reduce_thread",
              "vh_reduce_wave", "vh_strided_copy_i32", "vh_strided_copy_i64", "vh_col_partial",
              "vh_adamw_v1", "vh_adamw_v4", "vh_adamw_multi", "vh_gemm_reduce", "vh_emb_sort",
              "vh_attn_probe", "vh_attn_decide", "vh_math_probe", "vh_transpose", "vh_transpose_v4"}
    for bn in (192, 256):
        names.add(f"vh_gemmb_fix_{bn}")
        for lay in ("kk", "kn", "mk", "mn"):
            names.add(f"vh_gemmb_{lay}_{bn}")
    for a in ("k4", "k1", "m4", "m1"):
        for b in ("k4", "k1", "n4", "n1"):
            names.add(f"vh_gemm_{a}_{b}")
            names.add(f"vh_gemm_{a}_{b}_t64")
    for a in ("k4", "m4"):
        for b in ("k4", "n4"):
            names.add(f"vh_gemmp_{a}_{b}")
    return names


def test_code_object_holds_every_launchable_kernel():
    if not os.path.exists(CODE_OBJECT):
        pytest.skip("code object not built in-tree")
    syms = elf_symbols(CODE_OBJECT)
    missing = sorted(launcher_kernel_names() - syms)
    assert not missing, missing


def test_embedded_code_object_matches_build():
    if not os.path.exists(CODE_OBJECT):
        pytest.skip("code object not built in-tree")
    blob = open(CODE_OBJECT, "rb").read()
    assert blob in open(LIB, "rb").read()


def test_gemm_desc_layout_matches_header(tmp_path):
    """vh_gemm_desc crosses the boundary by pointer: the ctypes mirror must have
    the C compiler's size and field offsets."""
    import shutil
    import subprocess
    from vearo_amd import _abi
    if shutil.which("gcc") is None:
        pytest.skip("no C compiler")
    fields = [f[0] for f in _abi.VhGemmDesc._fields_]
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "vearo_hip.h"\nint main(void){\n'
        + 'printf("%zu\\n", sizeof(vh_gemm_desc));\n'
        + "".join(f'printf("%zu\\n", offsetof(vh_gemm_desc, {f}));\n' for f in fields)
        + "return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True,
                                          text=True).stdout.split()]
    want = [ctypes.sizeof(_abi.VhGemmDesc)] + [getattr(_abi.VhGemmDesc, f).offset for f in fields]
    assert got == want


def test_hipblaslt_is_not_a_link_dependency():
    # The hipBLASLt A/B engine opens the library at its first use; the
    # product library itself must load where hipBLASLt is not installed.
    import subprocess

    out = subprocess.run(["readelf", "-d", LIB], capture_output=True, text=True, check=True).stdout
    needed = re.findall(r"\(NEEDED\)\s+Shared library: \[([^\]]+)\]", out)
    assert needed and not any("hipblas" in n for n in needed), needed
