"""GPU parity of the W4A4 siblings (the reference's RT_ACT4 path): the decode
int4 activation quantizer, the W4A4 GEMV and the int4 x int4 prefill GEMM.

Bar: int4 codes and scales bit-exact against the CPU oracle and against the
reference's own quant_act4 built for gfx950; per-group int32 dot products of the
GEMM bit-exact; fp32 outputs within 1e-3 relative L2 of the oracle's fp64 fold
(the tests record the much tighter level reached: exact integers, fp32 folds).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
from rt4_amd import layout, workload
from test_gpu_decode import dev, edge_acts, host

pytestmark = pytest.mark.gpu

TOL = 1e-3
TIGHT = 2e-6


def _acts4(rng, M, K):
    """Activations with the int4 quantizer's edge cases: a zero 32-subgroup, exact
    ties at s = 1, an outlier; plus edge_acts' cases when K is large enough."""
    if K >= 640:
        x = edge_acts(rng, M, K)
    else:
        x = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
    x[-1, 32:64] = 0.0
    x[0, 64:96] = np.minimum(np.arange(32, dtype=np.float32) * np.float32(0.5) - np.float32(7.0), np.float32(7.0))
    x[-1, K - 1] = np.float32(-30.0)
    return x


@pytest.mark.parametrize("M,K", [(1, 5120), (4, 5120), (4, 17408), (3, 1024), (2, 672)])
def test_quant_act_a4_bit_exact(rt4, orc, torch_gpu, M, K):
    print(f"case quant_act_a4 M={M} K={K}", flush=True)
    x = _acts4(np.random.default_rng(200 + M + K), M, K)
    aq, sa = rt4.quant_act_a4(dev(torch_gpu, x))
    torch_gpu.cuda.synchronize()
    aq_o, sa_o = orc.quant_act4(x)
    assert np.array_equal(host(aq).view(np.uint32), aq_o)
    assert np.array_equal(host(sa).view(np.uint32), sa_o.view(np.uint32))


def test_quant_act_a4_against_reference_kernel(rt4, orc, torch_gpu, ref_hip):
    """The reference's quant_act4 (kernels/gemv_w4a4_core.h:22-44) built for gfx950."""
    import ctypes
    P = ctypes.c_void_p
    for M, K in [(1, 5120), (4, 5120), (4, 17408), (2, 1024)]:
        print(f"case ref quant_act4 M={M} K={K}", flush=True)
        x_np = _acts4(np.random.default_rng(60 + M + K), M, K)
        x = dev(torch_gpu, x_np)
        aq_r = torch_gpu.zeros((M, K // 2), dtype=torch_gpu.uint8, device="cuda")
        sa_r = torch_gpu.zeros((M, K // 32), dtype=torch_gpu.float32, device="cuda")
        torch_gpu.cuda.synchronize()
        ref_hip.ref_quant_act4(P(x.data_ptr()), P(aq_r.data_ptr()), P(sa_r.data_ptr()), M, K)
        ref_hip.ref_sync()
        aq_o, sa_o = orc.quant_act4(x_np)
        assert np.array_equal(host(aq_r).view(np.uint32), aq_o)
        assert np.array_equal(host(sa_r).view(np.uint32), sa_o.view(np.uint32))
        aq, sa = rt4.quant_act_a4(x)
        torch_gpu.cuda.synchronize()
        assert np.array_equal(host(aq).view(np.uint8), host(aq_r))
        assert np.array_equal(host(sa).view(np.uint32), host(sa_r).view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (2, 40, 512), (3, 96, 1024), (4, 200, 2048), (4, 17, 128),
                                   (4, 1024, 5120), (3, 33, 384), (2, 48, 1920), (4, 64, 17408), (1, 16, 128)])
def test_gemv_w4a4_against_oracle(rt4, orc, torch_gpu, M, N, K):
    print(f"case gemv_w4a4 M={M} N={N} K={K}", flush=True)
    c = workload.gemv_case(seed=41, M=M, N=N, K=K)
    x = _acts4(np.random.default_rng(41), M, K)
    wq, ws = dev(torch_gpu, c["wq"]), dev(torch_gpu, c["ws"])
    aq, sa = rt4.quant_act_a4(dev(torch_gpu, x))
    y = rt4.gemv_w4a4_q(wq, ws, aq, sa)
    y2 = rt4.gemv_w4a4(wq, ws, dev(torch_gpu, x))       # the drop-in k_gemv_w4a4 call
    torch_gpu.cuda.synchronize()
    ref = orc.gemv_w4a4(c["wq"], c["ws"], x)
    err = rel_l2(host(y), ref)
    print(f"  rel_l2 = {err:.3e}")
    assert err < TOL and err < TIGHT
    assert np.array_equal(host(y).view(np.uint32), host(y2).view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(4, 200, 2048), (3, 33, 384), (1, 48, 1920), (2, 40, 128), (4, 64, 17408),
                                   (4, 4176, 8192), (1, 4100, 17408)])
def test_gemv_w4a4_configs_agree(rt4, orc, torch_gpu, M, N, K):
    """Every launch configuration (groups per wave 2 or 4, 1..16 waves, leftover
    tiles whole or cut along K) meets the oracle; odd group counts and chunks cut
    by the end of K included.  The configurations differ only in the order of the
    fp32 sums over groups; one configuration repeats bit for bit (a split launch
    leaves its counters at zero for the next)."""
    print(f"case gemv_w4a4 configs M={M} N={N} K={K}", flush=True)
    c = workload.gemv_case(seed=45, M=M, N=N, K=K)
    x = _acts4(np.random.default_rng(45), M, K)
    wq, ws = dev(torch_gpu, c["wq"]), dev(torch_gpu, c["ws"])
    aq, sa = rt4.quant_act_a4(dev(torch_gpu, x))
    ref = orc.gemv_w4a4(c["wq"], c["ws"], x)
    for g, w, s in [(2, 1, 1), (2, 2, 0), (2, 3, 5), (2, 8, 64), (2, 16, 2), (4, 1, 0), (4, 2, 64), (4, 3, 1),
                    (4, 8, 3), (4, 16, 0)]:
        y = rt4.gemv_w4a4_q(wq, ws, aq, sa, groups_per_wave=g, waves=w, k_splits=s)
        y2 = rt4.gemv_w4a4_q(wq, ws, aq, sa, groups_per_wave=g, waves=w, k_splits=s)
        torch_gpu.cuda.synchronize()
        assert rel_l2(host(y), ref) < TIGHT, (g, w, s)
        assert np.array_equal(host(y).view(np.uint32), host(y2).view(np.uint32)), (g, w, s)


@pytest.mark.parametrize("name", ["c0", "c1_gate_up", "c1_down"])
def test_gemv_w4a4_benchmark_shapes(rt4, orc, torch_gpu, name):
    M, N, K = workload.GEMV_SHAPES[name]
    print(f"case gemv_w4a4 {name} M={M} N={N} K={K}", flush=True)
    c = workload.gemv_case(seed=0, M=M, N=N, K=K)
    y = rt4.gemv_w4a4(dev(torch_gpu, c["wq"]), dev(torch_gpu, c["ws"]), dev(torch_gpu, c["x"]))
    torch_gpu.cuda.synchronize()
    err = rel_l2(host(y), orc.gemv_w4a4(c["wq"], c["ws"], c["x"]))
    print(f"  rel_l2 = {err:.3e}")
    assert err < TOL and err < TIGHT


@pytest.mark.parametrize("M,N,K", [(128, 256, 512), (256, 320, 1024), (128, 64, 128), (384, 512, 2048)])
def test_gemm_w4a4_against_oracle(rt4, orc, torch_gpu, M, N, K):
    print(f"case gemm_w4a4 M={M} N={N} K={K}", flush=True)
    c = workload.gemm_case(43, M, N, K)
    wq, ws = dev(torch_gpu, c["wq"]), dev(torch_gpu, c["ws"])
    x = dev(torch_gpu, c["x"])
    aq, sc = rt4.quant_rows_a4(x)                       # k_quant_rows, G = 128
    sb = rt4.make_group_major(ws, K)
    out = rt4.gemm_w4a4(wq, sb, aq, sc)
    # the per-group integers: the same codes, sign-extended, through the group-sum hook
    a_codes = layout.unpack_rt4(host(aq).view(np.uint32))
    xq = dev(torch_gpu, layout.interleave(a_codes.astype(np.int8)))
    _, gs = rt4.gemm_w4a8_groupsums(wq, sb, xq, sc)
    torch_gpu.cuda.synchronize()
    aq_o, sc_o = orc.quant_rows_a4(c["x"], M, K, 128)
    assert np.array_equal(host(aq).view(np.uint32), aq_o)
    sb_o = orc.make_group_major(c["ws"])
    mi = np.repeat(np.arange(M), N).astype(np.int32)
    ni = np.tile(np.arange(N), M).astype(np.int32)
    ref, Ig = orc.gemm_w4a4_points(c["wq"], sb_o, aq_o, sc_o, M, N, K, mi, ni)
    assert np.array_equal(Ig.reshape(M, N, -1), host(gs))
    err = rel_l2(host(out).ravel(), ref)
    print(f"  rel_l2 = {err:.3e}")
    assert err < TOL and err < TIGHT


def test_gemm_w4a4_benchmark_shape_sampled(rt4, orc, torch_gpu):
    M, N, K = workload.GEMM_SHAPES["c2_gate_up"]
    print(f"case gemm_w4a4 c2 M={M} N={N} K={K}", flush=True)
    c = workload.gemm_case(0, M, N, K)
    wq, ws, x = dev(torch_gpu, c["wq"]), dev(torch_gpu, c["ws"]), dev(torch_gpu, c["x"])
    aq, sc = rt4.quant_rows_a4(x)
    out = rt4.gemm_w4a4(wq, rt4.make_group_major(ws, K), aq, sc)
    torch_gpu.cuda.synchronize()
    rng = np.random.default_rng(3)
    mi = rng.integers(0, M, 4096).astype(np.int32)
    ni = rng.integers(0, N, 4096).astype(np.int32)
    aq_o, sc_o = orc.quant_rows_a4(c["x"], M, K, 128)
    ref, _ = orc.gemm_w4a4_points(c["wq"], orc.make_group_major(c["ws"]), aq_o, sc_o, M, N, K, mi, ni)
    got = host(out)[mi, ni]
    err = rel_l2(got, ref)
    print(f"  rel_l2 = {err:.3e}")
    assert err < TOL and err < TIGHT


def test_w4a4_preconditions(rt4, torch_gpu):
    z = torch_gpu.zeros(1 << 16, dtype=torch_gpu.int32, device="cuda")
    f = torch_gpu.zeros(1 << 16, dtype=torch_gpu.float32, device="cuda")
    with pytest.raises(rt4.RT4Error, match="rows=5"):
        rt4.gemv_w4a4(z[:64 * 32].view(64, 32), z[:64].view(torch_gpu.int16).view(64, 2)[:, :2], f[:5 * 256].view(5, 256))
    with pytest.raises(rt4.RT4Error, match="BM=128"):
        rt4.gemm_w4a4(z[:64 * 16].view(64, 16), f[:64], z[:100 * 16].view(100, 16), f[:100])
