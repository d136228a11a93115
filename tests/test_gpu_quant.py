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


# workgroups of 320 / 128 / 128 / 256 / 64 / 256 (partial) / 448 / 192 lanes
@pytest.mark.parametrize("rows,K,G", [(128, 5120, 128), (256, 17408, 128), (64, 1024, 64),
                                      (32, 2048, 256), (8, 512, 512), (16, 256, 8), (16, 3584, 128),
                                      (8, 4608, 64)])
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


def test_digits_to_i8_tail_and_unaligned(rt4, torch_gpu):
    """Four digit dwords per lane with the last ndw % 4 by one lane, and the
    one-dword form for planes that are not 16-byte aligned: both equal 16h + l."""
    rng = np.random.default_rng(8)
    rows, K = 3, 40                       # 15 digit dwords: three whole quads and three more
    h = rng.integers(-7, 7, size=(rows, K)).astype(np.int8)     # 16h + l stays in int8
    l = rng.integers(-8, 8, size=(rows, K)).astype(np.int8)
    want = 16 * h.astype(int) + l
    qh, ql = layout.pack_rt4(h), layout.pack_rt4(l)
    out = rt4.digits_to_i8(dev(torch_gpu, qh), dev(torch_gpu, ql))
    bh = torch_gpu.zeros(qh.size + 1, dtype=torch_gpu.int32, device="cuda")
    bl = torch_gpu.zeros(ql.size + 1, dtype=torch_gpu.int32, device="cuda")
    bh[1:].copy_(dev(torch_gpu, qh).view(-1))
    bl[1:].copy_(dev(torch_gpu, ql).view(-1))
    out_u = rt4.digits_to_i8(bh[1:].view(rows, K // 8), bl[1:].view(rows, K // 8))   # 4-byte offset
    torch_gpu.cuda.synchronize()
    assert np.array_equal(layout.deinterleave(host(out)).astype(int), want)
    assert np.array_equal(host(out_u), host(out))


@pytest.mark.parametrize("rows,K,G", [(128, 5120, 128), (64, 512, 32), (16, 3584, 128), (8, 384, 32)])
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


def _special_acts(M, K):
    """Activations with IEEE special values in separate groups: +-Inf, NaN (alone
    and beside Inf), subnormals, +-FLT_MAX, -0.0 and tiny normals."""
    rng = np.random.default_rng(71)
    x = rng.standard_normal((M, K)).astype(np.float32)
    big = np.finfo(np.float32).max
    x[0, 5], x[0, 200] = np.inf, -np.inf
    x[1 % M, 130] = np.nan
    x[1 % M, 256:384] = np.float32(1e-40) * rng.standard_normal(128).astype(np.float32)
    x[2 % M, 384:512] = big * rng.choice(np.array([-1, 1], np.float32), 128)
    x[2 % M, 512:640] = -0.0
    x[3 % M, 640:768] = np.float32(1e-30) * rng.standard_normal(128).astype(np.float32)
    x[3 % M, 768], x[3 % M, 769] = np.nan, np.inf
    return x


def test_special_values_match_reference_kernels(rt4, torch_gpu, ref_hip):
    """IEEE special inputs: the float-to-int conversion of NaN and the scale of an
    Inf or subnormal group are the GPU's own behaviour, so the check is against
    the reference's quantizers built for gfx950 on the same card (codes, scales
    and sums bit for bit), and the one-launch GEMV against quantizer + GEMV."""
    M, K = 4, 1024
    x_np = _special_acts(M, K)
    x = dev(torch_gpu, x_np)
    # decode int8 (quant_act, /127 per 128)
    ae = torch_gpu.empty((M, K // 2), dtype=torch_gpu.int8, device="cuda")
    ao = torch_gpu.empty_like(ae)
    asc = torch_gpu.empty((M, K // 128), dtype=torch_gpu.float32, device="cuda")
    asu = torch_gpu.empty((M, K // 128), dtype=torch_gpu.int32, device="cuda")
    torch_gpu.cuda.synchronize()
    ref_hip.ref_quant_act(P(x.data_ptr()), P(ae.data_ptr()), P(ao.data_ptr()), P(asc.data_ptr()),
                          P(asu.data_ptr()), M, K)
    ref_hip.ref_sync()
    xq, sa, su = rt4.quant_act_a8(x, want_sums=True)
    torch_gpu.cuda.synchronize()
    q = layout.deinterleave(host(xq))
    assert np.array_equal(q[:, 0::2], host(ae)) and np.array_equal(q[:, 1::2], host(ao))
    assert np.array_equal(host(sa).view(np.uint32), host(asc).view(np.uint32))
    assert np.array_equal(host(su), host(asu))
    # the one-launch GEMV quantizes in registers: same y as quantizer + GEMV
    c = workload.gemv_case(seed=72, M=M, N=64, K=K)
    wq, ws = dev(torch_gpu, c["wq"]), dev(torch_gpu, c["ws"])
    y1 = rt4.gemv_w4a8(wq, ws, x, groups_per_wave=2, waves=4)
    y2 = rt4.gemv_w4a8_q(wq, ws, xq, sa, groups_per_wave=2, waves=4)
    torch_gpu.cuda.synchronize()
    assert np.array_equal(host(y1).view(np.uint32), host(y2).view(np.uint32))
    # decode int4 (quant_act4, /7 per 32)
    aq_r = torch_gpu.zeros((M, K // 2), dtype=torch_gpu.uint8, device="cuda")
    sa_r = torch_gpu.zeros((M, K // 32), dtype=torch_gpu.float32, device="cuda")
    torch_gpu.cuda.synchronize()
    ref_hip.ref_quant_act4(P(x.data_ptr()), P(aq_r.data_ptr()), P(sa_r.data_ptr()), M, K)
    ref_hip.ref_sync()
    aq4, sa4 = rt4.quant_act_a4(x)
    torch_gpu.cuda.synchronize()
    assert np.array_equal(host(aq4).view(np.uint8), host(aq_r))
    assert np.array_equal(host(sa4).view(np.uint32), host(sa_r).view(np.uint32))
    # prefill (/119 digits and /7), G = 128
    rows = 128
    xp_np = np.tile(x_np, (rows // M, 1))
    xp = dev(torch_gpu, xp_np)
    f = lambda *s: torch_gpu.empty(s, dtype=torch_gpu.int32, device="cuda")  # noqa: E731
    rh, rl, rq = f(rows, K // 8), f(rows, K // 8), f(rows, K // 8)
    rsc = torch_gpu.empty((K // 128, rows), dtype=torch_gpu.float32, device="cuda")
    rsc16, rsc4 = torch_gpu.empty_like(rsc), torch_gpu.empty_like(rsc)
    torch_gpu.cuda.synchronize()
    ref_hip.ref_quant_rows_a8(P(rh.data_ptr()), P(rl.data_ptr()), P(rsc.data_ptr()), P(rsc16.data_ptr()),
                              P(xp.data_ptr()), rows, K, 128, 0, 0)
    ref_hip.ref_quant_rows(P(rq.data_ptr()), P(rsc4.data_ptr()), P(xp.data_ptr()), rows, K, 128, 0, 0)
    ref_hip.ref_sync()
    qh, ql, sc, sc16 = rt4.quant_rows_a8(xp)
    q4, sc4 = rt4.quant_rows_a4(xp)
    torch_gpu.cuda.synchronize()
    for ours, theirs in [(qh, rh), (ql, rl), (sc, rsc), (sc16, rsc16), (q4, rq), (sc4, rsc4)]:
        assert np.array_equal(host(ours).view(np.uint32), host(theirs).view(np.uint32))
