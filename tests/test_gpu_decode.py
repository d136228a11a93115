"""GPU parity of the decode path: activation quantizer + W4A8 MFMA GEMV.

Bar: integer codes, scales and per-group int32 dot products bit-exact against
the CPU oracle; fp32 outputs within 1e-3 relative L2 of the oracle's fp64 fold
(the test also records the much tighter level actually reached).  Where the
reference's own quantizer is built (oracle/_ref/libref_hip.so), it is run on
the same inputs and compared as a third party.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
from rt4_amd import layout, workload

pytestmark = pytest.mark.gpu

TOL = 1e-3          # north-star bound for fp32 outputs (relative L2)
TIGHT = 2e-6        # what an exact-int + fp32-fold kernel actually reaches


def dev(torch, a: np.ndarray):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def host(t) -> np.ndarray:
    return t.cpu().numpy()


def edge_acts(rng, M, K):
    x = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
    x[0, :128] = 0.0
    x[-1, 128:256] = np.float32(2.5)
    x[-1, 300] = np.float32(-40.0)
    x[0, 512:640] = np.arange(128, dtype=np.float32) - np.float32(63.5)
    x[0, 639] = np.float32(127.0)
    return x


@pytest.mark.parametrize("M,K", [(1, 5120), (4, 5120), (4, 17408), (3, 1024)])
def test_quant_act_bit_exact(rt4, orc, torch_gpu, M, K):
    print(f"case quant_act M={M} K={K}", flush=True)
    x = edge_acts(np.random.default_rng(100 + K + M), M, K)
    xq, sa, asu = rt4.quant_act_a8(dev(torch_gpu, x), want_sums=True)
    torch_gpu.cuda.synchronize()
    q, sa_o, asu_o = orc.quant_act(x)
    assert np.array_equal(layout.deinterleave(host(xq)), q)
    assert np.array_equal(host(sa).view(np.uint32), sa_o.view(np.uint32))
    assert np.array_equal(host(asu), asu_o)


def test_quant_act_unaligned_with_sums(rt4, orc, torch_gpu):
    """Input rows not 16-byte aligned, group sums wanted: the scalar-load instance
    with sums, bit-identical to the oracle (edge values included)."""
    M, K = 3, 2048
    print(f"case quant_act unaligned M={M} K={K}", flush=True)
    x = edge_acts(np.random.default_rng(301), M, K)
    buf = torch_gpu.empty(M * K + 1, dtype=torch_gpu.float32, device="cuda")
    xd = buf[1:].view(M, K)
    xd.copy_(dev(torch_gpu, x))
    assert xd.data_ptr() % 16 != 0
    xq, sa, asu = rt4.quant_act_a8(xd, want_sums=True)
    torch_gpu.cuda.synchronize()
    q, sa_o, asu_o = orc.quant_act(x)
    assert np.array_equal(layout.deinterleave(host(xq)), q)
    assert np.array_equal(host(sa).view(np.uint32), sa_o.view(np.uint32))
    assert np.array_equal(host(asu), asu_o)


def _gemv_inputs(torch, seed, M, N, K):
    c = workload.gemv_case(seed, M, N, K)
    return c, dev(torch, c["wq"]), dev(torch, c["ws"]), dev(torch, c["x"])


@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (2, 40, 512), (3, 96, 1024), (4, 200, 2048),
                                   (4, 17, 128), (4, 1024, 5120), (3, 33, 384), (2, 48, 1920),
                                   (4, 64, 40960), (1, 16, 128), (3, 65560, 384), (4, 70000, 256),
                                   (1, 1001, 8192), (1, 5120, 5120)])
def test_gemv_groupsums_bit_exact(rt4, orc, torch_gpu, M, N, K):
    print(f"case gemv_groupsums M={M} N={N} K={K} plan={rt4.gemv_launch_plan(M, N, K)}", flush=True)
    c, wq, ws, x = _gemv_inputs(torch_gpu, 7, M, N, K)
    xq, sa = rt4.quant_act_a8(x)
    y, gs = rt4.gemv_w4a8_groupsums(wq, ws, xq, sa)
    torch_gpu.cuda.synchronize()
    q, sa_o, _ = orc.quant_act(c["x"])
    I = orc.gemv_groupsums(c["wq"], q)
    assert np.array_equal(host(gs), I)
    ref = orc.gemv_fold(I, c["ws"], sa_o)
    assert rel_l2(host(y), ref) < TIGHT


def test_gemv_default_row_blocks(rt4, torch_gpu):
    """Two 16-row blocks per tile only for 3-4 activation rows and where each CU
    has at least 320 (32-row tile x K group) units: the LM head, not the 27B MLP
    shapes."""
    cus = torch_gpu.cuda.get_device_properties(0).multi_processor_count
    for M, N, K in [(4, 17408, 5120), (4, 5120, 17408), (4, 248320, 5120), (1, 248320, 5120),
                    (3, 40960, 17408), (2, 248320, 5120), (1, 5120, 17408)]:
        if M == 1 and K % 256 == 0 and K <= 8192 and (N + 15) // 16 <= 16 * cus:
            want = 0                                  # the one-row dot-product form
        else:
            want = 2 if M >= 3 and (N + 31) // 32 * (K // 128) >= 320 * cus else 1
        assert rt4.gemv_launch_plan(M, N, K)["row_blocks"] == want, (M, N, K, cus)


@pytest.mark.parametrize("N,K", [(1, 256), (3, 512), (100, 768), (5121, 5120), (257, 8192), (4096, 2048)])
def test_gemv_one_row_dot_form(rt4, orc, torch_gpu, N, K):
    """One activation row, K a multiple of 256 up to 8192: the default launch is the
    row-contiguous dot-product form (two weight rows per wave, a short last wave at
    odd N, partly used load instructions where a wave's rows are not a multiple of
    1 KB).  Against the oracle and a tiled matrix-core launch of the same shape (the
    fp32 group sums in another order), and repeatable bit for bit."""
    print(f"case gemv_dot N={N} K={K}", flush=True)
    plan = rt4.gemv_launch_plan(1, N, K)
    assert plan["groups_per_wave"] == 0 and plan["row_blocks"] == 0, plan
    c, wq, ws, x = _gemv_inputs(torch_gpu, 21, 1, N, K)
    xq, sa = rt4.quant_act_a8(x)
    y = rt4.gemv_w4a8_q(wq, ws, xq, sa)
    y2 = rt4.gemv_w4a8_q(wq, ws, xq, sa)
    ym = rt4.gemv_w4a8_q(wq, ws, xq, sa, groups_per_wave=2)
    torch_gpu.cuda.synchronize()
    ref = orc.gemv_w4a8(c["wq"], c["ws"], c["x"])
    assert rel_l2(host(y), ref) < TIGHT
    assert rel_l2(host(y), host(ym)) < TIGHT
    assert np.array_equal(host(y).view(np.uint32), host(y2).view(np.uint32))


@pytest.mark.parametrize("M,N,K,gpw,waves", [(4, 300, 3072, 4, 6), (1, 17, 128, 2, 1), (2, 40, 512, 4, 1),
                                             (3, 1000, 5120, 4, 8), (4, 4176, 8192, 4, 8), (1, 520, 2944, 10, 2),
                                             (4, 64, 40960, 8, 16), (2, 48, 1920, 12, 1), (4, 33, 1408, 6, 2)])
def test_gemv_row_blocks(rt4, orc, torch_gpu, M, N, K, gpw, waves):
    """Tiles of two 16-row blocks: whole tiles give y bit-identical to one block
    per tile (same per-lane and per-wave sum order); with leftover tiles cut along
    K the result stays within the bar of the oracle and repeats exactly."""
    print(f"case gemv_rb M={M} N={N} K={K} gpw={gpw} waves={waves}", flush=True)
    c, wq, ws, x = _gemv_inputs(torch_gpu, 12, M, N, K)
    xq, sa = rt4.quant_act_a8(x)
    kw = dict(groups_per_wave=gpw, waves=waves)
    y1 = rt4.gemv_w4a8_q(wq, ws, xq, sa, k_splits=1, row_blocks=1, **kw)
    y2 = rt4.gemv_w4a8_q(wq, ws, xq, sa, k_splits=1, row_blocks=2, **kw)
    ys = rt4.gemv_w4a8_q(wq, ws, xq, sa, k_splits=64, row_blocks=2, **kw)
    ys2 = rt4.gemv_w4a8_q(wq, ws, xq, sa, k_splits=64, row_blocks=2, **kw)
    torch_gpu.cuda.synchronize()
    assert np.array_equal(host(y1).view(np.uint32), host(y2).view(np.uint32))
    ref = orc.gemv_w4a8(c["wq"], c["ws"], c["x"])
    assert rel_l2(host(y2), ref) < TIGHT
    assert rel_l2(host(ys), ref) < TIGHT
    assert np.array_equal(host(ys), host(ys2))


@pytest.mark.parametrize("gpw,waves", [(2, 1), (2, 12), (4, 3), (4, 6), (6, 4), (8, 2), (10, 3), (12, 1),
                                       (12, 2)])
def test_gemv_every_config(rt4, orc, torch_gpu, gpw, waves):
    M, N, K = 4, 300, 3072
    print(f"case gemv_cfg gpw={gpw} waves={waves}", flush=True)
    c, wq, ws, x = _gemv_inputs(torch_gpu, 8, M, N, K)
    xq, sa = rt4.quant_act_a8(x)
    y = rt4.gemv_w4a8_q(wq, ws, xq, sa, groups_per_wave=gpw, waves=waves)
    torch_gpu.cuda.synchronize()
    ref = orc.gemv_w4a8(c["wq"], c["ws"], c["x"])
    assert rel_l2(host(y), ref) < TIGHT


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("waves,splits", [(2, 1), (3, 1), (4, 1), (4, 4)])
def test_gemv_hoisted_scales(rt4, orc, torch_gpu, M, waves, splits):
    """Two groups per wave with 3-8 chunks per wave and at most 4 waves: the launch
    that loads each wave's weight scales once before its chunk loop (K = 3072: 12
    chunks; with 4 K-pieces per leftover tile a piece's waves have fewer chunks
    than the scale registers cover)."""
    N, K = 4100, 3072
    print(f"case gemv_hs M={M} waves={waves} splits={splits}", flush=True)
    c, wq, ws, x = _gemv_inputs(torch_gpu, 15, M, N, K)
    xq, sa = rt4.quant_act_a8(x)
    y = rt4.gemv_w4a8_q(wq, ws, xq, sa, groups_per_wave=2, waves=waves, k_splits=splits)
    y2 = rt4.gemv_w4a8_q(wq, ws, xq, sa, groups_per_wave=2, waves=waves, k_splits=splits)
    torch_gpu.cuda.synchronize()
    ref = orc.gemv_w4a8(c["wq"], c["ws"], c["x"])
    assert rel_l2(host(y), ref) < TIGHT
    assert torch_gpu.equal(y, y2)


@pytest.mark.parametrize("M,N,K,splits", [(4, 300, 3072, 8), (1, 300, 3072, 64), (4, 4176, 8192, 1),
                                           (4, 4176, 8192, 2), (2, 4176, 8192, 5), (3, 4176, 8192, 64),
                                           (4, 4176, 8192, 0), (1, 4100, 17408, 0)])
def test_gemv_k_split(rt4, orc, torch_gpu, M, N, K, splits):
    """Leftover tiles cut along K (pieces combined by the last to finish) against
    whole tiles and the oracle; the combine only changes the fp32 sum order."""
    print(f"case gemv_split M={M} N={N} K={K} k_splits={splits}", flush=True)
    c, wq, ws, x = _gemv_inputs(torch_gpu, 9, M, N, K)
    xq, sa = rt4.quant_act_a8(x)
    y = rt4.gemv_w4a8_q(wq, ws, xq, sa, k_splits=splits)
    y2 = rt4.gemv_w4a8_q(wq, ws, xq, sa, k_splits=splits)    # counters were left at zero
    torch_gpu.cuda.synchronize()
    ref = orc.gemv_w4a8(c["wq"], c["ws"], c["x"])
    assert rel_l2(host(y), ref) < TIGHT
    assert np.array_equal(host(y), host(y2))


def fused_edge_acts(rng, M, K):
    """edge_acts plus groups that take every branch of the in-GEMV quantizer: all
    zero (s = 1), tiny and huge magnitudes (scale outside [2^-96, 2^100]: IEEE
    division), exact rounding ties v/s = k + 1/2 (power-of-two scale), denormals."""
    x = edge_acts(rng, M, K)
    NG = K // 128
    for r in range(M):
        g = (3 * r) % NG
        x[r, g * 128:(g + 1) * 128] = rng.standard_normal(128).astype(np.float32) * np.float32(1e-33)
        g = (3 * r + 1) % NG
        x[r, g * 128:(g + 1) * 128] = rng.standard_normal(128).astype(np.float32) * np.float32(1e33)
        g = (3 * r + 2) % NG
        e = float(rng.integers(-20, 20))
        k = rng.integers(-127, 127, 128).astype(np.float32)
        x[r, g * 128:(g + 1) * 128] = np.ldexp(k + np.float32(0.5), int(e)).astype(np.float32)
        x[r, g * 128] = np.float32(np.ldexp(127.0, int(e)))          # amax: s = 2^e exactly
    if NG > 4:
        x[0, 4 * 128:4 * 128 + 64] = np.float32(1e-40)                # denormal inputs
    return x


@pytest.mark.parametrize("M,N,K,cfg", [(1, 5120, 5120, None), (2, 1000, 5120, None), (3, 2064, 17408, None),
                                       (4, 17408, 5120, None), (4, 5120, 17408, None), (4, 300, 3072, (2, 12, 1, 0)),
                                       (4, 300, 3072, (6, 4, 3, 0)), (1, 520, 2944, (10, 2, 0, 0)),
                                       (2, 64, 40960, (8, 16, 8, 0)), (3, 96, 1920, (12, 1, 1, 0)),
                                       (4, 300, 3072, (4, 6, 1, 2)), (4, 1000, 5120, (4, 8, 0, 2)),
                                       (1, 520, 2944, (10, 2, 4, 2))])
def test_gemv_fused_quant_equals_two_launches(rt4, orc, torch_gpu, M, N, K, cfg):
    """The one-launch linear (activations quantized in the GEMV's registers) against
    rt4_quant_act_a8 + the GEMV on the same config: outputs identical bit for bit
    (same codes, scales and sum order), and within the bar of the oracle."""
    print(f"case gemv_fused M={M} N={N} K={K} cfg={cfg}", flush=True)
    rng = np.random.default_rng(M * 7 + N + K)
    c = workload.gemv_case(N=N, K=K, M=M, seed=int(rng.integers(1 << 30)))
    x_np = fused_edge_acts(rng, M, K)
    wq, ws, x = dev(torch_gpu, c["wq"]), dev(torch_gpu, c["ws"]), dev(torch_gpu, x_np)
    g, w, s, rb = cfg or (0, 0, 0, 0)
    y = rt4.gemv_w4a8(wq, ws, x, groups_per_wave=g, waves=w, k_splits=s, row_blocks=rb)
    xq, sa = rt4.quant_act_a8(x)
    y2 = rt4.gemv_w4a8_q(wq, ws, xq, sa, groups_per_wave=g, waves=w, k_splits=s, row_blocks=rb)
    torch_gpu.cuda.synchronize()
    if cfg is None and rt4.gemv_launch_plan(M, N, K)["groups_per_wave"] == 0:
        # the two-launch default is the one-row dot-product form, which the fused
        # launch (a matrix-core form) does not share: same codes, other sum order
        assert rel_l2(host(y), host(y2)) < TIGHT
    else:
        assert np.array_equal(host(y).view(np.uint32), host(y2).view(np.uint32))
    if N * K <= 5120 * 5120:
        ref = orc.gemv_w4a8(c["wq"], c["ws"], x_np)
        assert rel_l2(host(y), ref) < TIGHT


def test_gemv_unaligned_activations(rt4, orc, torch_gpu):
    """x not 16-byte aligned: the drop-in quantizes separately; the fused config
    entry refuses it."""
    M, N, K = 2, 256, 1024
    print(f"case gemv_unaligned M={M} N={N} K={K}", flush=True)
    c, wq, ws, _ = _gemv_inputs(torch_gpu, 11, M, N, K)
    buf = torch_gpu.zeros(M * K + 1, dtype=torch_gpu.float32, device="cuda")
    x = buf[1:].view(M, K)
    x.copy_(torch_gpu.from_numpy(c["x"]).cuda())
    y = rt4.gemv_w4a8(wq, ws, x)
    torch_gpu.cuda.synchronize()
    assert rel_l2(host(y), orc.gemv_w4a8(c["wq"], c["ws"], c["x"])) < TIGHT
    with pytest.raises(rt4.RT4Error, match="misaligned"):
        rt4.gemv_w4a8(wq, ws, x, groups_per_wave=4)


@pytest.mark.parametrize("name", ["c0", "c1_gate_up", "c1_down"])
def test_gemv_benchmark_shapes(rt4, orc, torch_gpu, name):
    M, N, K = workload.GEMV_SHAPES[name]
    print(f"case gemv {name} M={M} N={N} K={K}", flush=True)
    c, wq, ws, x = _gemv_inputs(torch_gpu, 0, M, N, K)
    y = rt4.gemv_w4a8(wq, ws, x)                      # the drop-in entry (quant + GEMV)
    xq, sa = rt4.quant_act_a8(x)
    _, gs = rt4.gemv_w4a8_groupsums(wq, ws, xq, sa)
    torch_gpu.cuda.synchronize()
    q, sa_o, _ = orc.quant_act(c["x"])
    I = orc.gemv_groupsums(c["wq"], q)
    assert np.array_equal(host(gs), I)
    ref = orc.gemv_fold(I, c["ws"], sa_o)
    err = rel_l2(host(y), ref)
    print(f"  rel_l2 = {err:.3e}")
    assert err < TOL and err < TIGHT


def test_gemv_lm_head_full(rt4, orc, torch_gpu):
    """C3: M=4, K=5120, N=248320 (0.64 GB of weights), full output vs the oracle."""
    M, N, K = workload.GEMV_SHAPES["c3_lm_head"]
    print(f"case gemv lm_head M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(3)
    wq_np = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint32)  # uniform nibbles
    ws_np = (np.abs(rng.standard_normal((N, K // 128))) * 0.01 + 1e-3).astype(np.float16).view(np.uint16)
    x_np = workload.acts_np(rng, M, K)
    y = rt4.gemv_w4a8(dev(torch_gpu, wq_np), dev(torch_gpu, ws_np), dev(torch_gpu, x_np))
    torch_gpu.cuda.synchronize()
    ref = orc.gemv_w4a8(wq_np, ws_np, x_np)
    err = rel_l2(host(y), ref)
    print(f"  rel_l2 = {err:.3e}")
    assert err < TOL and err < TIGHT


def test_gemv_repeat_and_rows_change(rt4, orc, torch_gpu):
    """The drop-in entry reuses grown scratch: alternate row counts and K."""
    for (M, N, K) in [(4, 256, 5120), (1, 128, 1024), (3, 64, 17408), (2, 256, 5120)]:
        c, wq, ws, x = _gemv_inputs(torch_gpu, M * 31 + K, M, N, K)
        y = rt4.gemv_w4a8(wq, ws, x)
        torch_gpu.cuda.synchronize()
        assert rel_l2(host(y), orc.gemv_w4a8(c["wq"], c["ws"], c["x"])) < TIGHT


def test_quant_act_against_reference_kernel(rt4, orc, torch_gpu, ref_hip):
    """The reference's quant_act (built for gfx950) on the same inputs: its even/odd
    codes, scales and sums equal the oracle's and ours bit for bit."""
    import ctypes
    P = ctypes.c_void_p
    for (M, K) in [(1, 5120), (4, 5120), (4, 17408), (2, 1024)]:
        print(f"case ref quant_act M={M} K={K}", flush=True)
        x_np = edge_acts(np.random.default_rng(40 + M + K), M, K)
        x = dev(torch_gpu, x_np)
        ae = torch_gpu.empty((M, K // 2), dtype=torch_gpu.int8, device="cuda")
        ao = torch_gpu.empty_like(ae)
        asc = torch_gpu.empty((M, K // 128), dtype=torch_gpu.float32, device="cuda")
        asu = torch_gpu.empty((M, K // 128), dtype=torch_gpu.int32, device="cuda")
        torch_gpu.cuda.synchronize()
        ref_hip.ref_quant_act(P(x.data_ptr()), P(ae.data_ptr()), P(ao.data_ptr()), P(asc.data_ptr()),
                              P(asu.data_ptr()), M, K)
        ref_hip.ref_sync()
        q_ref = np.empty((M, K), np.int8)
        q_ref[:, 0::2], q_ref[:, 1::2] = host(ae), host(ao)
        q, sa_o, asu_o = orc.quant_act(x_np)
        assert np.array_equal(q_ref, q)
        assert np.array_equal(host(asc).view(np.uint32), sa_o.view(np.uint32))
        assert np.array_equal(host(asu), asu_o)
        xq, sa, asu_g = rt4.quant_act_a8(x, want_sums=True)
        torch_gpu.cuda.synchronize()
        assert np.array_equal(layout.deinterleave(host(xq)), q_ref)
        assert np.array_equal(host(sa).view(np.uint32), host(asc).view(np.uint32))
        assert np.array_equal(host(asu_g), host(asu))
