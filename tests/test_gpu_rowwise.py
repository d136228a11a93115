"""GPU parity of the per-row (G = K) quantizer mode and of the GEMV / GEMM fed by it.

The mode has no counterpart in the reference (which quantizes per (row, 128-group));
its checker is the numpy oracle's G = K restatement, pinned on the CPU by brute
force and by agreement with the per-group oracle (tests/test_rowwise_oracle.py).
Bar: codes, scales and group sums bit-exact; the kernel equals the per-group
kernel bit for bit on rows whose every group reaches the row's max-abs; GEMV and
GEMM outputs within 1e-6 relative L2 of the fp64 fold of the exact group sums.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
from oracle import np_ref
from rt4_amd import layout, workload
from test_gpu_decode import dev, host

pytestmark = pytest.mark.gpu

TIGHT = 1e-6


def _acts(seed, M, K, zero_row=False):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, K)) * np.exp2(rng.integers(-4, 5, (M, 1)))).astype(np.float32)
    x[0, rng.integers(0, K)] = 37.0 * (1 + np.abs(x[0]).max())     # one outlier sets row 0's scale
    if zero_row and M > 1:
        x[M - 1] = 0.0
    return x


@pytest.mark.parametrize("M,K", [(1, 5120), (4, 5120), (4, 17408), (3, 256), (2, 128)])
def test_rowwise_gemv_form_bit_exact(rt4, torch_gpu, M, K):
    print(f"case rowwise mode 0 M={M} K={K}", flush=True)
    x = _acts(61 + K, M, K, zero_row=True)
    xq, sa, asu = rt4.quant_act_rowwise(dev(torch_gpu, x), mode=0, want_sums=True)
    torch_gpu.cuda.synchronize()
    q, s, a = np_ref.quant_act(x, G=K)
    assert np.array_equal(layout.deinterleave(host(xq)), q)
    assert np.array_equal(host(sa), np.repeat(s, K // 128, axis=1))
    assert np.array_equal(host(asu), a)


@pytest.mark.parametrize("M,K", [(256, 5120), (100, 17408), (5, 384)])
def test_rowwise_gemm_form_bit_exact(rt4, torch_gpu, M, K):
    print(f"case rowwise mode 1 M={M} K={K}", flush=True)
    x = _acts(67 + M, M, K, zero_row=True)
    xq, sc = rt4.quant_act_rowwise(dev(torch_gpu, x), mode=1)
    torch_gpu.cuda.synchronize()
    q8, s8 = np_ref.quant_rows_i8(x, G=K)
    assert np.array_equal(layout.deinterleave(host(xq)), q8)
    assert np.array_equal(host(sc), np.repeat(s8, K // 128, axis=1).T)


def test_rowwise_kernel_equals_per_group_kernel_when_groups_reach_the_row_max(rt4, torch_gpu):
    """Where every 128-group of a row holds the row's max-abs, per-row and per-group
    quantization are the same computation: both kernels must write the same bits."""
    M, K = 4, 5120
    print(f"case rowwise vs per-group kernels M={M} K={K}", flush=True)
    rng = np.random.default_rng(71)
    x = rng.standard_normal((M, K)).astype(np.float32)
    top = np.abs(x).max(axis=1) * np.float32(2.0)
    for m in range(M):
        for g in range(K // 128):
            x[m, 128 * g + rng.integers(0, 128)] = top[m] * (1 if (g + m) % 2 else -1)
    xd = dev(torch_gpu, x)
    r = rt4.quant_act_rowwise(xd, mode=0, want_sums=True)
    p = rt4.quant_act_a8(xd, want_sums=True)
    for a, b in zip(r, p):
        assert np.array_equal(host(a), host(b))
    r8, rs8 = rt4.quant_act_rowwise(xd, mode=1)
    p8, ps8 = rt4.quant_rows_i8(xd)
    assert np.array_equal(host(r8), host(p8)) and np.array_equal(host(rs8), host(ps8))


@pytest.mark.parametrize("M,N,K", [(1, 5120, 5120), (4, 17408, 5120), (4, 5120, 17408)])
def test_gemv_on_rowwise_activations(rt4, orc, torch_gpu, M, N, K):
    print(f"case gemv rowwise M={M} N={N} K={K}", flush=True)
    c = workload.gemv_case(seed=73, M=M, N=N, K=K)
    xq, sa = rt4.quant_act_rowwise(dev(torch_gpu, c["x"]), mode=0)
    y = rt4.gemv_w4a8_q(dev(torch_gpu, c["wq"]), dev(torch_gpu, c["ws"]), xq, sa)
    torch_gpu.cuda.synchronize()
    q, s, _ = np_ref.quant_act(c["x"], G=K)
    I = orc.gemv_groupsums(c["wq"], q)
    ref = orc.gemv_fold(I, c["ws"], np.repeat(s, K // 128, axis=1))
    err = rel_l2(host(y), ref)
    print(f"  rel_l2 = {err:.3e}")
    assert err < TIGHT


def test_gemm_on_rowwise_activations(rt4, orc, torch_gpu):
    M, N, K = 256, 512, 1024
    print(f"case gemm rowwise M={M} N={N} K={K}", flush=True)
    c = workload.gemm_case(79, M, N, K)
    sb = rt4.make_group_major(dev(torch_gpu, c["ws"]), K)
    xq, sc = rt4.quant_act_rowwise(dev(torch_gpu, c["x"]), mode=1)
    out = rt4.gemm_w4a8_i8(dev(torch_gpu, c["wq"]), sb, xq, sc)
    torch_gpu.cuda.synchronize()
    q8, s8 = np_ref.quant_rows_i8(c["x"], G=K)
    I = orc.gemv_groupsums(c["wq"], q8).astype(np.float64)            # [M, N, NG]
    sbo = orc.make_group_major(c["ws"]).astype(np.float64)             # [NG, N]
    ref = np.einsum("mng,gn->mn", I, sbo) * s8[:, 0:1].astype(np.float64)
    err = rel_l2(host(out).ravel(), ref.ravel())
    print(f"  rel_l2 = {err:.3e}")
    assert err < TIGHT


@pytest.mark.parametrize("mode", [0, 1])
def test_rowwise_unaligned_input_matches_aligned(rt4, torch_gpu, mode):
    """x 4 bytes off 16-byte alignment takes the element-load path: same bits."""
    M, K = 3, 5120
    print(f"case rowwise unaligned mode={mode}", flush=True)
    x = _acts(83, M, K, zero_row=True)
    xa = dev(torch_gpu, x)
    buf = torch_gpu.empty(M * K + 1, dtype=torch_gpu.float32, device="cuda")
    xu = buf[1:].view(M, K)
    xu.copy_(xa)
    assert xu.data_ptr() % 16 != 0
    ra = rt4.quant_act_rowwise(xa, mode=mode)
    ru = rt4.quant_act_rowwise(xu, mode=mode)
    torch_gpu.cuda.synchronize()
    for a, b in zip(ra, ru):
        assert np.array_equal(host(a), host(b))
