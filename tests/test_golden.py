"""Golden fixtures (tests/golden/rt4_golden.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture bit for bit, so a change to the checker
itself shows up here.  GPU: the HIP kernels reproduce the fixtures -- quantized
codes, scales and per-group int32 dot products bit-exact, fp32 outputs within a
relative L2 error of 1e-6 (the order of the fp32 sum over groups differs from
the oracle's fp64 fold).
"""
from __future__ import annotations

import pathlib

import numpy as np
import pytest

from conftest import rel_l2
from rt4_amd import layout

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "rt4_golden.npz"
TIGHT = 1e-6


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ------------------------------------------------------------------ CPU side --

def test_oracle_reproduces_quant_act(orc, g):
    q, sa, asu = orc.quant_act(g["qa_x"])
    assert np.array_equal(q, g["qa_q"]) and np.array_equal(sa, g["qa_sa"]) and np.array_equal(asu, g["qa_asu"])
    assert np.all(g["qa_q"][1, 128:256] == 0) and g["qa_sa"][1, 1] == 1.0      # zero group: s = 1
    assert g["qa_q"][2, 5] == 127                                              # outlier -> +127


def test_oracle_reproduces_gemv(orc, g):
    qg, sag, _ = orc.quant_act(g["gv_x"])
    I = orc.gemv_groupsums(g["gv_wq"], qg)
    assert np.array_equal(I, g["gv_I"])
    assert np.array_equal(orc.gemv_fold(I, g["gv_ws"], sag).astype(np.float32), g["gv_y"])
    # brute force on the unpacked codes (independent of the oracle's packed reader)
    codes = layout.unpack_rt4(g["gv_wq"]).astype(np.int64).reshape(48, 3, 128)
    brute = np.einsum("ngk,mgk->mng", codes, qg.astype(np.int64).reshape(4, 3, 128))
    assert np.array_equal(brute, g["gv_I"])


@pytest.mark.parametrize("G", [128, 64])
def test_oracle_reproduces_quant_rows_a8(orc, g, G):
    qh, ql, sc, sc16 = orc.quant_rows_a8(g["qr_x"], 5, 256, G)
    for name, v in (("qh", qh), ("ql", ql), ("sc", sc), ("sc16", sc16)):
        assert np.array_equal(v, g[f"qr{G}_{name}"]), name
    h = layout.unpack_rt4(g[f"qr{G}_qh"]).astype(np.int32)
    low = layout.unpack_rt4(g[f"qr{G}_ql"]).astype(np.int32)
    q8 = 16 * h + low
    assert q8.min() >= -128 and q8.max() <= 119 and np.all(q8[4, :128] == 0)


def test_oracle_reproduces_gemm(orc, g):
    M, N, K = 8, 32, 256
    qh, ql, sc, sc16 = orc.quant_rows_a8(g["gm_x"], M, K)
    mi = np.repeat(np.arange(M), N).astype(np.int32)
    ni = np.tile(np.arange(N), M).astype(np.int32)
    c, Ig = orc.gemm_w4a8_points(g["gm_wq"], g["gm_sb"], qh, ql, sc, sc16, M, N, K, mi, ni)
    assert np.array_equal(Ig.reshape(M, N, -1), g["gm_I"]) and np.array_equal(c.reshape(M, N), g["gm_c"])


def test_oracle_reproduces_weight_quantizer(orc, g):
    wq, ws = orc.quant_weight_rows(g["wc_w"])
    assert np.array_equal(wq, g["wc_wq"]) and np.array_equal(ws, g["wc_ws"])
    assert np.all(g["wc_wq"][1, :16] == 0) and g["wc_ws"][1, 0] == 0x3C00


# ------------------------------------------------------------------ GPU side --

def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    return t.detach().cpu().numpy()


def _wq_dev(torch, wq):
    return _dev(torch, wq.view(np.int32))


@pytest.mark.gpu
def test_kernels_reproduce_decode_fixtures(rt4, torch_gpu, g):
    print("case golden decode", flush=True)
    torch = torch_gpu
    xq, sa, asu = rt4.quant_act_a8(_dev(torch, g["qa_x"]), want_sums=True)
    torch.cuda.synchronize()
    assert np.array_equal(layout.deinterleave(_host(xq)), g["qa_q"])
    assert np.array_equal(_host(sa), g["qa_sa"]) and np.array_equal(_host(asu), g["qa_asu"])
    wq, ws = _wq_dev(torch, g["gv_wq"]), _dev(torch, g["gv_ws"].view(np.int16))
    xq, sa = rt4.quant_act_a8(_dev(torch, g["gv_x"]))
    y, gs = rt4.gemv_w4a8_groupsums(wq, ws, xq, sa)
    y2 = rt4.gemv_w4a8(wq, ws, _dev(torch, g["gv_x"]))
    torch.cuda.synchronize()
    assert np.array_equal(_host(gs), g["gv_I"])
    assert rel_l2(_host(y), g["gv_y"]) < TIGHT
    assert np.array_equal(_host(y2), _host(y))


@pytest.mark.gpu
def test_kernels_reproduce_prefill_fixtures(rt4, torch_gpu, g):
    print("case golden prefill", flush=True)
    torch = torch_gpu
    for G in (128, 64):
        qh, ql, sc, sc16 = rt4.quant_rows_a8(_dev(torch, g["qr_x"]), G=G)
        torch.cuda.synchronize()
        for name, v in (("qh", qh), ("ql", ql), ("sc", sc), ("sc16", sc16)):
            want = g[f"qr{G}_{name}"]
            got = _host(v)
            assert np.array_equal(got.view(want.dtype).reshape(want.shape), want), (G, name)
    M, N, K = 8, 32, 256
    wq = _wq_dev(torch, g["gm_wq"])
    sb = rt4.make_group_major(_dev(torch, g["gm_ws"].view(np.int16)), K)
    torch.cuda.synchronize()
    assert np.array_equal(_host(sb), g["gm_sb"])
    xq, sc = rt4.quant_rows_i8(_dev(torch, g["gm_x"]))
    c, gs = rt4.gemm_w4a8_groupsums(wq, sb, xq, sc)
    torch.cuda.synchronize()
    assert np.array_equal(_host(gs), g["gm_I"])
    assert rel_l2(_host(c), g["gm_c"]) < TIGHT
