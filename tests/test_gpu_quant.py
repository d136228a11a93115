"""GPU parity of the prefill-side quantizers (bit-exact against the oracle and,
where built, against the reference's own k_quant_rows_a8 / k_quant_rows)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from rt4_amd import layout, workload
from test_gpu_decode import dev, host

pytestmark = pytest.mark.gpu
P = ctypes.c_void_p


@pytest.mark.parametrize("rows,K,G", [(128, 5120, 128), (256, 17408, 128), (64, 1024, 64),
                                      (32, 2048, 256), (8, 512, 512), (16, 256, 8)])
def test_quant_rows_a8_bit_exact(rt4, orc, torch_gpu, rows, K, G):
    print(f"case quant_rows_a8 rows={rows} K={K} G={G}", flush=True)
    x = workload.acts_np(np.random.default_rng(rows + K + G), rows, K, outliers=True)
    x[0, :G] = 0.0
    qh, ql, sc, sc16 = rt4.quant_rows_a8(dev(torch_gpu, x), G=G)
    torch_gpu.cuda.synchronize()
    oh, ol, osc, osc16 = orc.quant_rows_a8(x, rows, K, G)
    assert np.array_equal(host(qh).view(np.uint32), oh)
    assert np.array_equal(host(ql).view(np.uint32), ol)
    assert np.array_equal(host(sc).view(np.uint32), osc.view(np.uint32))
    assert np.array_equal(host(sc16).view(np.uint32), osc16.view(np.uint32))


def test_quant_rows_a8_stride_offset(rt4, orc, torch_gpu):
    rows, K, stride, off = 128, 5120, 12288, 1024 + 4  # off not 16-byte aligned
    buf = workload.acts_np(np.random.default_rng(5), rows, stride)
    qh, ql, sc, sc16 = rt4.quant_rows_a8(dev(torch_gpu, buf), rows=rows, K=K, in_stride=stride, in_off=off)
    torch_gpu.cuda.synchronize()
    oh, ol, osc, _ = orc.quant_rows_a8(buf, rows, K, 128, stride, off)
    assert np.array_equal(host(qh).view(np.uint32), oh) and np.array_equal(host(ql).view(np.uint32), ol)
    assert np.array_equal(host(sc), osc)


def test_quant_rows_i8_and_digit_recombination(rt4, orc, torch_gpu):
    rows, K = 256, 5120
    x = workload.acts_np(np.random.default_rng(6), rows, K, outliers=True)
    xd = dev(torch_gpu, x)
    xq, sc = rt4.quant_rows_i8(xd)
    qh, ql, sc2, _ = rt4.quant_rows_a8(xd)
    xq2 = rt4.digits_to_i8(qh, ql)
    torch_gpu.cuda.synchronize()
    q8, osc = orc.quant_rows_i8(x, rows, K)
    assert np.array_equal(layout.deinterleave(host(xq)), q8)
    assert np.array_equal(host(xq2), host(xq))
    assert np.array_equal(host(sc), osc) and np.array_equal(host(sc2), osc)


def test_digits_to_i8_exhaustive(rt4, torch_gpu):
    """Every (h, l) digit pair the quantizer can emit maps to 16h + l."""
    h = np.repeat(np.arange(-8, 8), 16)
    l = np.tile(np.arange(-8, 8), 16)
    q8 = 16 * h + l
    keep = (q8 >= -128) & (q8 <= 119)
    h, l, q8 = h[keep], l[keep], q8[keep]
    n = (len(h) + 7) // 8 * 8
    hp = np.zeros(n, np.int8)
    lp = np.zeros(n, np.int8)
    hp[:len(h)], lp[:len(l)] = h, l
    qh = layout.pack_rt4(hp.reshape(1, n))
    ql = layout.pack_rt4(lp.reshape(1, n))
    out = rt4.digits_to_i8(dev(torch_gpu, qh), dev(torch_gpu, ql))
    torch_gpu.cuda.synchronize()
    got = layout.deinterleave(host(out))[0, :len(q8)]
    assert np.array_equal(got.astype(int), q8)


@pytest.mark.parametrize("rows,K,G", [(128, 5120, 128), (64, 512, 32)])
def test_quant_rows_a4_bit_exact(rt4, orc, torch_gpu, rows, K, G):
    x = workload.acts_np(np.random.default_rng(7), rows, K)
    q, sc = rt4.quant_rows_a4(dev(torch_gpu, x), G=G)
    torch_gpu.cuda.synchronize()
    oq, osc = orc.quant_rows_a4(x, rows, K, G)
    assert np.array_equal(host(q).view(np.uint32), oq) and np.array_equal(host(sc), osc)


def test_make_group_major(rt4, orc, torch_gpu):
    c = workload.gemv_case(9, 1, 17408, 5120)
    gm = rt4.make_group_major(dev(torch_gpu, c["ws"]), 5120)
    torch_gpu.cuda.synchronize()
    assert np.array_equal(host(gm), orc.make_group_major(c["ws"]))


def test_quantizers_against_reference_kernels(rt4, orc, torch_gpu, ref_hip):
    rows, K, G = 256, 5120, 128
    x = workload.acts_np(np.random.default_rng(8), rows, K, outliers=True)
    xd = dev(torch_gpu, x)
    f = lambda *s: torch_gpu.empty(s, dtype=torch_gpu.int32, device="cuda")  # noqa: E731
    rh, rl, rq = f(rows, K // 8), f(rows, K // 8), f(rows, K // 8)
    rsc = torch_gpu.empty((K // G, rows), dtype=torch_gpu.float32, device="cuda")
    rsc16, rsc4 = torch_gpu.empty_like(rsc), torch_gpu.empty_like(rsc)
    torch_gpu.cuda.synchronize()
    ref_hip.ref_quant_rows_a8(P(rh.data_ptr()), P(rl.data_ptr()), P(rsc.data_ptr()), P(rsc16.data_ptr()),
                              P(xd.data_ptr()), rows, K, G, 0, 0)
    ref_hip.ref_quant_rows(P(rq.data_ptr()), P(rsc4.data_ptr()), P(xd.data_ptr()), rows, K, G, 0, 0)
    ref_hip.ref_sync()
    qh, ql, sc, sc16 = rt4.quant_rows_a8(xd)
    q4, sc4 = rt4.quant_rows_a4(xd)
    torch_gpu.cuda.synchronize()
    oh, ol, osc, osc16 = orc.quant_rows_a8(x, rows, K, G)
    for ours, theirs, orac in [(qh, rh, oh), (ql, rl, ol)]:
        assert np.array_equal(host(theirs).view(np.uint32), orac)
        assert np.array_equal(host(ours).view(np.uint32), orac)
    assert np.array_equal(host(rsc), osc) and np.array_equal(host(rsc16), osc16)
    assert np.array_equal(host(sc), osc) and np.array_equal(host(sc16), osc16)
    oq4, osc4 = orc.quant_rows_a4(x, rows, K, G)
    assert np.array_equal(host(rq).view(np.uint32), oq4) and np.array_equal(host(q4).view(np.uint32), oq4)
    assert np.array_equal(host(rsc4), osc4) and np.array_equal(host(sc4), osc4)
