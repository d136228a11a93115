"""Shared test setup: import paths, the `gpu` marker, library fixtures."""
from __future__ import annotations

import ctypes
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "k100lc-rt4_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)

REF_HIP = ROOT / "oracle" / "_ref" / "libref_hip.so"
REF_CONVERT = ROOT / "oracle" / "_ref" / "convert"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def orc():
    from oracle import rt4_oracle
    rt4_oracle.lib()
    return rt4_oracle


@pytest.fixture(scope="session")
def rt4():
    import rt4_amd
    rt4_amd.lib()
    return rt4_amd


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    torch.cuda.init()
    return torch


@pytest.fixture(scope="session")
def ref_hip(torch_gpu):
    """The reference's own activation quantizers built for gfx950 (oracle/_ref), if present."""
    if not REF_HIP.exists():
        pytest.skip("oracle/_ref/libref_hip.so not built (needs /root/reference at build time)")
    L = ctypes.CDLL(str(REF_HIP))
    P, I = ctypes.c_void_p, ctypes.c_int
    L.ref_quant_act.argtypes = [P, P, P, P, P, I, I]
    L.ref_quant_rows_a8.argtypes = [P, P, P, P, P, I, I, I, I, I]
    L.ref_quant_rows.argtypes = [P, P, P, I, I, I, I, I]
    L.ref_quant_act4.argtypes = [P, P, P, I, I]
    L.ref_sync.argtypes = []
    L.ref_fa_int4.argtypes = [P] * 7 + [I] * 7
    for f in ("ref_quant_act", "ref_quant_rows_a8", "ref_quant_rows", "ref_quant_act4", "ref_sync", "ref_fa_int4"):
        getattr(L, f).restype = None
    return L


def rel_l2(got, ref) -> float:
    import numpy as np
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))
