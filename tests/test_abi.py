"""CPU tests of the C ABI boundary: load, exports, precondition errors.

No kernel is launched here: every call below fails its shape or argument check
before any HIP call, exactly where the reference's wrappers would exit(1).
"""
from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "rt4k.h"


def declared_c_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:const char\*|int)\s+(rt4_\w+)\(", text, flags=re.M)))


def test_header_and_binding_agree(rt4):
    assert declared_c_symbols() == sorted(rt4.C_EXPORTS)


def test_library_exports_every_declared_symbol(rt4):
    L = rt4.lib()
    for name in declared_c_symbols():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(rt4.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name in list(rt4.C_EXPORTS) + list(rt4.CXX_EXPORTS):
        assert name in exported, name
    # nothing but the ABI and the reference-compatible prototypes leaks out
    assert all(s.startswith("rt4_") or s.startswith("_Z") for s in exported)
    assert all(s in rt4.CXX_EXPORTS for s in exported if s.startswith("_Z"))


def test_abi_version(rt4):
    assert rt4.lib().rt4_abi_version() == 1


DUMMY = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first


@pytest.mark.parametrize("rows,N,K", [(5, 64, 256), (0, 64, 256), (4, 64, 200), (4, 0, 256)])
def test_gemv_shape_errors(rt4, rows, N, K):
    L = rt4.lib()
    rc = L.rt4_gemv_w4a8(DUMMY, DUMMY, DUMMY, DUMMY, rows, N, K, None)
    assert rc == 1  # RT4_E_SHAPE
    assert "k_gemv_w4a8" in L.rt4_last_error().decode()
    rc = L.rt4_gemv_w4a8_q(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, rows, N, K, None)
    assert rc == 1


def test_gemv_null_and_config_errors(rt4):
    L = rt4.lib()
    assert L.rt4_gemv_w4a8(None, DUMMY, DUMMY, DUMMY, 1, 64, 256, None) == 2
    assert L.rt4_gemv_w4a8_q_cfg(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 1, 64, 256, 3, 1, 0, 0, None) == 2
    assert L.rt4_gemv_w4a8_q_cfg(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 1, 64, 256, 2, 2, 0, 0, None) == 2
    assert L.rt4_gemv_w4a8_q_cfg(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 1, 64, 256, 14, 1, 0, 0, None) == 2
    assert L.rt4_gemv_w4a8_q_cfg(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 1, 64, 256, 2, 1, 65, 0, None) == 2
    assert L.rt4_gemv_w4a8_q_cfg(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 1, 64, 256, 2, 1, 0, 3, None) == 2
    assert "config" in L.rt4_last_error().decode()
    assert L.rt4_gemv_w4a4_q_cfg(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 1, 64, 256, 3, 0, 0, None) == 2
    assert L.rt4_gemv_w4a4_q_cfg(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 1, 64, 256, 2, 17, 0, None) == 2
    assert L.rt4_gemv_w4a4_q_cfg(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 1, 64, 256, 2, 1, 65, None) == 2
    assert "k_splits=65" in L.rt4_last_error().decode()


def test_quant_errors(rt4):
    L = rt4.lib()
    assert L.rt4_quant_act_a8(DUMMY, DUMMY, None, DUMMY, 1, 100, None) == 1
    assert L.rt4_quant_act_rowwise(DUMMY, DUMMY, None, DUMMY, 1, 100, 0, None) == 1
    assert L.rt4_quant_act_rowwise(DUMMY, DUMMY, None, DUMMY, 0, 256, 0, None) == 1
    assert L.rt4_quant_act_rowwise(DUMMY, DUMMY, None, DUMMY, 1, 256, 2, None) == 2
    assert "mode=2" in L.rt4_last_error().decode()
    assert L.rt4_quant_rows_a8(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 4, 256, 96, 0, 0, None) == 2
    assert L.rt4_quant_rows_a8(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 4, 200, 128, 0, 0, None) == 2
    assert L.rt4_quant_rows_a8(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 0, 256, 128, 0, 0, None) == 1
    assert L.rt4_quant_rows_i8(DUMMY, DUMMY, DUMMY, 4, 200, 0, 0, None) == 1
    assert L.rt4_quant_rows_a4(DUMMY, DUMMY, DUMMY, 4, 256, 12, 0, 0, None) == 2


def test_shim_exits_like_the_reference():
    """k_gemv_w4a8 with rows > 4 prints and exits(1) (src/k_gemv.hip:54), via a C++ caller."""
    src = ROOT / "tests" / "shim_caller.cpp"
    exe = ROOT / "tests" / "_shim_caller"
    lib = ROOT / "k100lc-rt4_amd" / "rt4_amd" / "lib"
    subprocess.run(["g++", "-std=c++17", "-I", str(ROOT / "include"), str(src), "-L", str(lib),
                    "-lrt4k", f"-Wl,-rpath,{lib}", "-o", str(exe)], check=True)
    try:
        r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    finally:
        exe.unlink(missing_ok=True)
    assert r.returncode == 1
    assert "k_gemv_w4a8" in r.stdout and "rows=5" in r.stdout


def test_shim_attention_decode_branch_uses_callers_decode_kernel():
    """k_attention hands the single-row decode branch to the executable's own
    k_attention_decode (src/k_fa.hip:282-292) with the reference's arguments."""
    src = ROOT / "tests" / "shim_decode_caller.cpp"
    exe = ROOT / "tests" / "_shim_decode_caller"
    lib = ROOT / "k100lc-rt4_amd" / "rt4_amd" / "lib"
    subprocess.run(["g++", "-std=c++17", "-I", str(ROOT / "include"), str(src), "-L", str(lib),
                    "-lrt4k", f"-Wl,-rpath,{lib}", "-o", str(exe)], check=True)
    try:
        r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    finally:
        exe.unlink(missing_ok=True)
    assert r.returncode == 7, (r.returncode, r.stdout, r.stderr)
    assert "decode n_kv=300 kv_cap=4096 n_heads=24 ratio=6 n_q=64 max_split=8" in r.stdout


def test_shim_attention_old_switch_takes_the_prefill_kernel():
    """RT_ATTN_OLD=1 sends the decode branch to the prefill kernel, as the reference
    dispatcher does (src/k_fa.hip:287), even when the executable defines its own
    decode routine: the prefill entry's argument check (null pointers) then ends
    the caller with the reference's exit(1), before any device work."""
    import os
    src = ROOT / "tests" / "shim_decode_caller.cpp"
    exe = ROOT / "tests" / "_shim_decode_caller_old"
    lib = ROOT / "k100lc-rt4_amd" / "rt4_amd" / "lib"
    subprocess.run(["g++", "-std=c++17", "-I", str(ROOT / "include"), str(src), "-L", str(lib),
                    "-lrt4k", f"-Wl,-rpath,{lib}", "-o", str(exe)], check=True)
    try:
        r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60,
                           env={**os.environ, "RT_ATTN_OLD": "1"})
    finally:
        exe.unlink(missing_ok=True)
    assert r.returncode == 1, (r.returncode, r.stdout, r.stderr)
    assert "k_attention" in r.stdout and "decode n_kv" not in r.stdout


def test_dropin_caller_is_built_and_links():
    """tests/_bin/dropin_caller (built by __graft_entry__.build()) resolves librt4k.so
    and the HIP runtime; with no arguments it prints its usage before any device work."""
    exe = ROOT / "tests" / "_bin" / "dropin_caller"
    assert exe.exists(), "built by __graft_entry__.build() (make -C tests dropin)"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stdout, (r.returncode, r.stdout, r.stderr)


def test_single_hip_runtime_in_process(rt4):
    """librt4k.so binds to the HIP runtime torch already loaded (one runtime per process)."""
    import torch  # noqa: F401
    rt4.lib()
    maps = {line.split()[-1] for line in open("/proc/self/maps") if "libamdhip64" in line}
    assert len(maps) == 1, maps


def test_gemv_scale_pointer_needs_4_bytes(rt4):
    """The GEMVs load fp16 scale pairs as dwords (every row of an even-K/128 scale
    matrix starts 4-byte aligned), so ws must be 4-byte aligned."""
    L = rt4.lib()
    W16, WS2 = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1002)
    assert L.rt4_gemv_w4a8_q(W16, W16, WS2, W16, W16, 4, 64, 256, None) == 2
    assert "ws 4" in L.rt4_last_error().decode()
    assert L.rt4_gemv_w4a8(W16, W16, WS2, W16, 4, 64, 256, None) == 2
    assert L.rt4_gemv_w4a8_cfg(W16, W16, WS2, W16, 4, 64, 256, 0, 0, 0, 0, None) == 2
    assert L.rt4_gemv_w4a8_groupsums(W16, W16, W16, WS2, W16, W16, 4, 64, 256, None) == 2
    assert L.rt4_gemv_w4a4_q(W16, W16, WS2, W16, W16, 4, 64, 256, None) == 2
    assert L.rt4_gemv_w4a4(W16, W16, WS2, W16, 4, 64, 256, None) == 2


@pytest.mark.parametrize("M,N,K", [(838861, 64, 5120), (128, 1677722, 5120), (128, 65536, 131072)])
def test_gemm_rejects_shapes_beyond_32bit_offsets(rt4, M, N, K):
    """The GEMM addresses rows of A (M*K bytes) and of W (N*K/2 bytes) with 32-bit
    offsets; larger operands are rejected instead of wrapping."""
    L = rt4.lib()
    W16 = ctypes.c_void_p(0x1000)
    assert L.rt4_gemm_w4a8_i8(W16, W16, W16, W16, W16, M, N, K, None) == 1
    assert "32-bit offset" in L.rt4_last_error().decode()
    assert L.rt4_gemm_w4a8_groupsums(W16, W16, W16, W16, W16, W16, M, N, K, None) == 1
    # the largest operands inside the range still pass the shape check (fail later on alignment)
    assert L.rt4_gemm_w4a8_i8(W16, ctypes.c_void_p(0x1004), W16, W16, W16, 838860, 64, 5120, None) == 2


def test_attention_rejects_caches_beyond_32bit_offsets(rt4):
    """One KV head's cache is addressed with 32-bit buffer offsets (kv_cap * 128 bytes
    of K codes): kv_cap above 2^24 - 64 is refused before any device work."""
    L = rt4.lib()
    P = ctypes.c_void_p(0x10000)
    args = lambda cap: (P, P, P, P, P, P, P, 64, 64, 0, 1, 8, 1, cap, 0, None)  # noqa: E731
    assert L.rt4_attention_prefill_cfg(*args(1 << 24)) == 1          # RT4_E_SHAPE
    assert "kv_cap" in L.rt4_last_error().decode()
    assert L.rt4_attention_prefill_cfg(*args((1 << 24) + 64)) == 1


def test_noalloc_gemv_rejects_beyond_its_static_scratch(rt4):
    """rt4_gemv_w4a8_noalloc has a fixed scratch (K <= 65536); larger K is an error, not an allocation."""
    L = rt4.lib()
    W16 = ctypes.c_void_p(0x1000)
    assert L.rt4_gemv_w4a8_noalloc(W16, W16, W16, W16, 4, 64, 65536 + 128, None) == 1
    assert "static scratch" in L.rt4_last_error().decode()
    assert L.rt4_gemv_w4a8_noalloc(W16, W16, W16, W16, 5, 64, 256, None) == 1
    assert L.rt4_gemv_w4a8_noalloc(W16, W16, ctypes.c_void_p(0x1002), W16, 4, 64, 256, None) == 2
