"""GPU parity of the prefill path: int8 quantizer + W4A8 MFMA GEMM.

Bar: per-group int32 dot products bit-exact against the CPU oracle; fp32 outputs
within 1e-3 relative L2 of the oracle's fp64 restatement of k_gemm_i4_a8
(src/k_gemm.hip:22-34: Σ_g sb*(sc16*I_h + sc*I_l)); the reference's own
harness criterion (bench/int4_gemm2.cpp:104-123: worst |err| / rms|c| < 1e-5 on
sampled outputs) is checked as well.  At the benchmark sizes the oracle is
evaluated at sampled points, and size-independent properties are checked in
full: the drop-in digit-plane entry and the int8 entry give bit-identical
outputs, and a full-K tile's group sums are exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
from rt4_amd import layout, workload
from test_gpu_decode import dev, host

pytestmark = pytest.mark.gpu

TOL = 1e-3
TIGHT = 1e-6


def _case(torch, seed, M, N, K):
    c = workload.gemm_case(seed, M, N, K)
    wq, ws = dev(torch, c["wq"]), dev(torch, c["ws"])
    x = dev(torch, c["x"])
    return c, wq, ws, x


def _oracle_points(orc, c, M, N, K, mi, ni):
    qh, ql, sc, sc16 = orc.quant_rows_a8(c["x"], M, K)
    sb = orc.make_group_major(c["ws"])
    return orc.gemm_w4a8_points(c["wq"], sb, qh, ql, sc, sc16, M, N, K, mi, ni)


@pytest.mark.parametrize("M,N,K", [(128, 256, 512), (256, 320, 1024), (100, 64, 256), (1, 300, 128),
                                   (384, 512, 2048)])
def test_gemm_groupsums_bit_exact(rt4, orc, torch_gpu, M, N, K):
    print(f"case gemm_groupsums M={M} N={N} K={K}", flush=True)
    c, wq, ws, x = _case(torch_gpu, 17, M, N, K)
    xq, sc = rt4.quant_rows_i8(x)
    sb = rt4.make_group_major(ws, K)
    out, gs = rt4.gemm_w4a8_groupsums(wq, sb, xq, sc)
    torch_gpu.cuda.synchronize()
    q8, sc_o = orc.quant_rows_i8(c["x"], M, K)
    assert np.array_equal(layout.deinterleave(host(xq)), q8)
    assert np.array_equal(host(gs), orc.gemv_groupsums(c["wq"], q8))
    mi = np.repeat(np.arange(M), N).astype(np.int32)
    ni = np.tile(np.arange(N), M).astype(np.int32)
    ref, Ig = _oracle_points(orc, c, M, N, K, mi, ni)
    assert np.array_equal(Ig.reshape(M, N, -1), host(gs))  # 16*I_h + I_l == Σ code*q8
    err = rel_l2(host(out).ravel(), ref)
    print(f"  rel_l2 = {err:.3e}")
    assert err < TIGHT


@pytest.mark.parametrize("name", ["c2_gate_up", "c2_down"])
def test_gemm_benchmark_shapes(rt4, orc, torch_gpu, name):
    M, N, K = workload.GEMM_SHAPES[name]
    print(f"case gemm {name} M={M} N={N} K={K}", flush=True)
    c, wq, ws, x = _case(torch_gpu, 2, M, N, K)
    sb = rt4.make_group_major(ws, K)
    # drop-in path: digit planes, as k_quant_rows_a8 + k_gemm_i4_a8
    qh, ql, sc, sc16 = rt4.quant_rows_a8(x)
    y = rt4.gemm_w4a8(wq, sb, qh, ql, sc, sc16)
    # int8 path: fused quantizer + GEMM
    xq, sc8 = rt4.quant_rows_i8(x)
    y8 = rt4.gemm_w4a8_i8(wq, sb, xq, sc8)
    # one full-K tile with its group sums
    _, gs = rt4.gemm_w4a8_groupsums(wq[:256].contiguous(), sb[:, :256].contiguous(), xq[:128].contiguous(),
                                    sc8[:, :128].contiguous())
    torch_gpu.cuda.synchronize()
    y_h, y8_h = host(y), host(y8)
    assert np.array_equal(y_h.view(np.uint32), y8_h.view(np.uint32)), "digit-plane and int8 entries differ"
    q8, _ = orc.quant_rows_i8(c["x"], 128, K)
    assert np.array_equal(host(gs), orc.gemv_groupsums(c["wq"][:256], q8))
    rng = np.random.default_rng(5)
    P = 4096
    mi = rng.integers(0, M, P).astype(np.int32)
    ni = rng.integers(0, N, P).astype(np.int32)
    mi[:4], ni[:4] = [0, M - 1, 0, M - 1], [0, 0, N - 1, N - 1]
    ref, _ = _oracle_points(orc, c, M, N, K, mi, ni)
    got = y_h[mi, ni]
    err = rel_l2(got, ref)
    rms = float(np.sqrt(np.mean(ref ** 2)))
    worst = float(np.abs(got - ref).max()) / rms
    print(f"  rel_l2 = {err:.3e}  worst/rms = {worst:.3e}")
    assert err < TOL and err < TIGHT
    assert worst < 1e-5  # bench/int4_gemm2.cpp:104-123


def test_gemm_reference_benchmark_shape(rt4, orc, torch_gpu):
    """The reference's own benchmark shape, M=2048 tokens x gate/up (bench/int4_gemm2.cpp:
    4-9): sampled outputs against the fp64 oracle with the reference's criterion
    (worst |err| / rms|c| < 1e-5), and the drop-in entry bit-identical to the int8 one."""
    M, N, K = workload.GEMM_REF_SHAPE
    print(f"case gemm reference shape M={M} N={N} K={K}", flush=True)
    c, wq, ws, x = _case(torch_gpu, 3, M, N, K)
    sb = rt4.make_group_major(ws, K)
    xq, sc8 = rt4.quant_rows_i8(x)
    y8 = host(rt4.gemm_w4a8_i8(wq, sb, xq, sc8))
    qh, ql, sc, sc16 = rt4.quant_rows_a8(x)
    y = host(rt4.gemm_w4a8(wq, sb, qh, ql, sc, sc16))
    assert np.array_equal(y.view(np.uint32), y8.view(np.uint32)), "digit-plane and int8 entries differ"
    rng = np.random.default_rng(9)
    P = 4096
    mi = rng.integers(0, M, P).astype(np.int32)
    ni = rng.integers(0, N, P).astype(np.int32)
    mi[:4], ni[:4] = [0, M - 1, 0, M - 1], [0, 0, N - 1, N - 1]
    ref, _ = _oracle_points(orc, c, M, N, K, mi, ni)
    got = y8[mi, ni]
    err = rel_l2(got, ref)
    worst = float(np.abs(got - ref).max()) / float(np.sqrt(np.mean(ref ** 2)))
    print(f"  rel_l2 = {err:.3e}  worst/rms = {worst:.3e}")
    assert err < TIGHT and worst < 1e-5


def test_gemm_dropin_small_c2_uses_library_scratch(rt4, orc, torch_gpu):
    """4*N < K: the recombined codes do not fit in c2, library scratch is used."""
    M, N, K = 128, 64, 1024
    c, wq, ws, x = _case(torch_gpu, 23, M, N, K)
    sb = rt4.make_group_major(ws, K)
    qh, ql, sc, sc16 = rt4.quant_rows_a8(x)
    y = rt4.gemm_w4a8(wq, sb, qh, ql, sc, sc16)
    torch_gpu.cuda.synchronize()
    mi = np.repeat(np.arange(M), N).astype(np.int32)
    ni = np.tile(np.arange(N), M).astype(np.int32)
    ref, _ = _oracle_points(orc, c, M, N, K, mi, ni)
    assert rel_l2(host(y).ravel(), ref) < TIGHT


def test_gemm_repeat_shapes(rt4, orc, torch_gpu):
    """Back-to-back calls with changing shapes (scratch reuse, tails in N and M)."""
    for (M, N, K) in [(256, 1024, 5120), (128, 64, 256), (512, 832, 1024), (131, 200, 384)]:
        print(f"case gemm repeat M={M} N={N} K={K}", flush=True)
        c, wq, ws, x = _case(torch_gpu, M + N + K, M, N, K)
        sb = rt4.make_group_major(ws, K)
        xq, sc = rt4.quant_rows_i8(x)
        y = rt4.gemm_w4a8_i8(wq, sb, xq, sc)
        torch_gpu.cuda.synchronize()
        rng = np.random.default_rng(M)
        mi = rng.integers(0, M, 2048).astype(np.int32)
        ni = rng.integers(0, N, 2048).astype(np.int32)
        ref, _ = _oracle_points(orc, c, M, N, K, mi, ni)
        assert rel_l2(host(y)[mi, ni], ref) < TIGHT


@pytest.mark.parametrize("entry,M,N,K", [
    ("i8", 1000, 17408, 5120),     # the reference's own prefill shape (docs/FORMAT.md:129)
    ("dropin", 1024, 5184, 5120),  # N % 256 == 64: every column block ends in a partial tile
    ("i8", 1000, 8320, 1024),      # M and N tails, 264 tiles: workgroups run on past whole tail tiles
])
def test_gemm_tail_tiles_with_continuing_workgroups(rt4, orc, torch_gpu, entry, M, N, K):
    """Shapes whose workgroups own whole partial tiles (rows beyond M, columns beyond N)
    and then continue with the next tile: the next tile's operands must have landed
    whatever number of C stores the partial tile issued.  Sampled outputs against the
    fp64 oracle; a second call is bitwise equal to the first."""
    print(f"case gemm tails entry={entry} M={M} N={N} K={K}", flush=True)
    c, wq, ws, x = _case(torch_gpu, 31, M, N, K)
    sb = rt4.make_group_major(ws, K)
    if entry == "i8":
        xq, sc8 = rt4.quant_rows_i8(x)
        run = lambda: rt4.gemm_w4a8_i8(wq, sb, xq, sc8)  # noqa: E731
    else:
        qh, ql, sc, sc16 = rt4.quant_rows_a8(x)
        run = lambda: rt4.gemm_w4a8(wq, sb, qh, ql, sc, sc16)  # noqa: E731
    y1 = host(run())
    y2 = host(run())
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), "repeated call differs"
    rng = np.random.default_rng(7)
    P = 6144
    mi = rng.integers(0, M, P).astype(np.int32)
    ni = rng.integers(0, N, P).astype(np.int32)
    # every corner, and rows / columns of the last partial tiles
    m_t, n_t = min((M // 128) * 128, M - 1), min((N // 256) * 256, N - 1)
    mi[:8] = [0, M - 1, 0, M - 1, M - 1, M - 2, m_t, M - 1]
    ni[:8] = [0, 0, N - 1, N - 1, n_t, N - 1, N - 1, max(n_t - 1, 0)]
    tail = rng.integers(0, P, 1024)
    mi[tail] = rng.integers((M - 1) // 128 * 128, M, 1024)
    ref, _ = _oracle_points(orc, c, M, N, K, mi, ni)
    got = y1[mi, ni]
    err = rel_l2(got, ref)
    rms = float(np.sqrt(np.mean(ref ** 2)))
    worst = float(np.abs(got - ref).max()) / rms
    print(f"  rel_l2 = {err:.3e}  worst/rms = {worst:.3e}")
    assert err < TIGHT and worst < 1e-5


@pytest.mark.parametrize("entry", ["i8", "w4a4"])
def test_gemm_single_group_matches_fp32_fold_bitwise(rt4, orc, torch_gpu, entry):
    """One 128-wide group (K = 128): every tile is a single unit, so C is one fold
    step.  The reference folds acc = fmaf((float)I, SA*SB, acc) from acc = 0
    (kernels/gemm_core.h:176-183), i.e. f32(I) * f32(sa * sb) with one rounding of
    each product.  The kernel forms sa*sb as one fp32 product on the matrix core
    and folds 16*I (exact), scaled by 1/16 at the end (exact), so its output must
    carry exactly those bits -- for the int8 entry and for the W4A4 one, whose
    fold is literally the reference's gemm_w4a4."""
    M, N, K = 256, 512, 128
    print(f"case gemm single group entry={entry} M={M} N={N} K={K}", flush=True)
    c, wq, ws, x = _case(torch_gpu, 53, M, N, K)
    sb = rt4.make_group_major(ws, K)
    if entry == "i8":
        xq, sa = rt4.quant_rows_i8(x)
        out = rt4.gemm_w4a8_i8(wq, sb, xq, sa)
        q, sa_o = orc.quant_rows_i8(c["x"], M, K)
    else:
        aq, sa = rt4.quant_rows_a4(x)
        out = rt4.gemm_w4a4(wq, sb, aq, sa)
        aq_o, sa_o = orc.quant_rows_a4(c["x"], M, K, 128)
        q = layout.unpack_rt4(aq_o).astype(np.int8)
    torch_gpu.cuda.synchronize()
    sb_o = orc.make_group_major(c["ws"])
    I = orc.gemv_groupsums(c["wq"], q)[:, :, 0]
    S = sa_o[0][:, None] * sb_o[0][None, :]                  # fp32 products, round to nearest
    want = I.astype(np.float32) * S
    got = host(out)
    diff = int(np.count_nonzero(got.view(np.uint32) != want.view(np.uint32)))
    print(f"  outputs differing from f32(I) * f32(sa * sb): {diff} of {M * N}")
    assert diff == 0


def test_gemm_scale_products_over_wide_exponent_range(rt4, orc, torch_gpu):
    """The scale products sa*sb are single fp32 products on the matrix core.
    Activation scales spanning 2^-40 .. 2^40 across rows and groups exercise a wide
    range of exponents; each row must match the fp64 oracle to fp32 accuracy on its
    own (a per-row relative L2, so small rows are not hidden behind large ones), for
    both entries."""
    M, N, K = 256, 320, 1024
    print(f"case gemm scale range M={M} N={N} K={K}", flush=True)
    c = workload.gemm_case(41, M, N, K)
    rng = np.random.default_rng(41)
    er = rng.integers(-40, 41, M).astype(np.float64)
    eg = rng.integers(-8, 9, K // 128).astype(np.float64)
    c["x"] = (c["x"] * np.exp2(er)[:, None] * np.repeat(np.exp2(eg), 128)[None, :]).astype(np.float32)
    wq, ws, x = dev(torch_gpu, c["wq"]), dev(torch_gpu, c["ws"]), dev(torch_gpu, c["x"])
    sb = rt4.make_group_major(ws, K)
    xq, sc8 = rt4.quant_rows_i8(x)
    y8 = host(rt4.gemm_w4a8_i8(wq, sb, xq, sc8))
    qh, ql, sc, sc16 = rt4.quant_rows_a8(x)
    y = host(rt4.gemm_w4a8(wq, sb, qh, ql, sc, sc16))
    assert np.array_equal(y.view(np.uint32), y8.view(np.uint32)), "digit-plane and int8 entries differ"
    mi = np.repeat(np.arange(M), N).astype(np.int32)
    ni = np.tile(np.arange(N), M).astype(np.int32)
    ref, _ = _oracle_points(orc, c, M, N, K, mi, ni)
    ref = ref.reshape(M, N)
    worst = max(rel_l2(y8[m], ref[m]) for m in range(M))
    print(f"  worst per-row rel_l2 = {worst:.3e}")
    assert worst < TIGHT


def test_gemm_full_precision_fp32_weight_scales(rt4, orc, torch_gpu):
    """wsc_gm holding arbitrary fp32 values (24 significant bits, not the fp16 values
    make_group_major produces) over a wide exponent range: the scale products are
    single fp32 products of the full scales, so every row matches the fp64 oracle
    to fp32 accuracy, for the int8 and the drop-in digit-plane entries alike."""
    M, N, K = 256, 320, 1024
    print(f"case gemm fp32 weight scales M={M} N={N} K={K}", flush=True)
    c = workload.gemm_case(43, M, N, K)
    rng = np.random.default_rng(43)
    G = K // 128
    sb_h = (rng.uniform(1, 2, (G, N)) * np.exp2(rng.integers(-30, 31, (G, N)))).astype(np.float32)
    assert np.any(sb_h.astype(np.float16).astype(np.float32) != sb_h)   # not fp16-representable
    wq, x = dev(torch_gpu, c["wq"]), dev(torch_gpu, c["x"])
    sb = dev(torch_gpu, sb_h)
    xq, sc8 = rt4.quant_rows_i8(x)
    y8 = host(rt4.gemm_w4a8_i8(wq, sb, xq, sc8))
    qh, ql, sc, sc16 = rt4.quant_rows_a8(x)
    y = host(rt4.gemm_w4a8(wq, sb, qh, ql, sc, sc16))
    assert np.array_equal(y.view(np.uint32), y8.view(np.uint32)), "digit-plane and int8 entries differ"
    qh_o, ql_o, sc_o, sc16_o = orc.quant_rows_a8(c["x"], M, K)
    mi = np.repeat(np.arange(M), N).astype(np.int32)
    ni = np.tile(np.arange(N), M).astype(np.int32)
    ref, _ = orc.gemm_w4a8_points(c["wq"], sb_h, qh_o, ql_o, sc_o, sc16_o, M, N, K, mi, ni)
    ref = ref.reshape(M, N)
    worst = max(rel_l2(y8[m], ref[m]) for m in range(M))
    print(f"  worst per-row rel_l2 = {worst:.3e}")
    assert worst < TIGHT
