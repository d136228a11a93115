"""CPU tests pinning the oracle (oracle/rt4_oracle.c) before it is trusted.

Each function of the oracle is checked by something other than itself:
known-answer values from the reference, textbook results (IEEE binary16),
an independent numpy restatement, brute force on tiny inputs, and the
algebraic identities the reference relies on.
"""
from __future__ import annotations

import numpy as np
import pytest

from rt4_amd import layout
from oracle import np_ref


# ------------------------------------------------------------------ KATs ----
def test_dot8_known_answers(orc):
    # bench/bench_isa2.cpp:128-145, docs/DESIGN-INT4.md:40-44: nibbles 0..7 (low
    # nibble first) against all ones give 28; all 0xF (signed -1) give -8.
    assert orc.dot8_i4(0x76543210, 0x11111111) == 28
    assert orc.dot8_i4(0xFFFFFFFF, 0x11111111) == -8
    assert orc.dot8_i4(0x76543210, 0x11111111, 5) == 33


def test_nibble_order_matches_kat():
    # the same KAT fixes the packing: nibble e of the dword is element e, signed
    assert layout.unpack_rt4(np.array([0x76543210], np.uint32)).tolist() == list(range(8))
    assert layout.unpack_rt4(np.array([0xFFFFFFFF], np.uint32)).tolist() == [-1] * 8
    assert layout.unpack_rt4(np.array([0x89ABCDEF], np.uint32)).tolist() == [-1, -2, -3, -4, -5, -6, -7, -8]


def test_pack_unpack_roundtrip():
    rng = np.random.default_rng(3)
    c = rng.integers(-8, 8, size=(7, 256), dtype=np.int8)
    w = layout.pack_rt4(c)
    assert w.dtype == np.uint32 and w.shape == (7, 32)
    assert np.array_equal(layout.unpack_rt4(w), c)
    # byte view: low nibble holds the even element (docs/FORMAT.md:61-73)
    b = w.view(np.uint8)
    assert np.array_equal(np_ref.unpack_bytes(b), c.astype(np.int16))


def test_interleave_roundtrip():
    rng = np.random.default_rng(4)
    c = rng.integers(-128, 128, size=(3, 64), dtype=np.int8)
    iv = layout.interleave(c)
    assert np.array_equal(iv[0, :8], c[0, [0, 2, 4, 6, 1, 3, 5, 7]])
    assert np.array_equal(layout.deinterleave(iv), c)


def test_f16_decode_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    got_np = np_ref.f16_bits_to_f32(h)
    assert np.array_equal(got_np[finite].view(np.uint32), ref[finite].view(np.uint32))
    sample = h[finite][::97]
    got_c = np.array([orc.f16_to_f32(int(v)) for v in sample], np.float32)
    assert np.array_equal(got_c.view(np.uint32), sample.view(np.float16).astype(np.float32).view(np.uint32))


# ------------------------------------------------------------- quantizers ---
def _edge_acts(rng, M, K):
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0, :128] = 0.0                                      # all-zero group -> s = 1, q = 0
    x[0, 128:256] = np.float32(3.0)                       # constant group -> all +127
    x[-1, 256:384] *= np.float32(1e-20)                   # tiny magnitudes
    x[-1, 384] = np.float32(50.0)                         # an outlier
    # exact half-way points: amax 127 -> s = 1 -> x = k + 0.5 must round to even
    x[1 % M, 512:640] = np.arange(128, dtype=np.float32) - np.float32(63.5)
    x[1 % M, 512 + 127] = np.float32(127.0)
    return x


def test_quant_act_matches_numpy_and_invariants(orc):
    rng = np.random.default_rng(11)
    x = _edge_acts(rng, 4, 1024)
    q, sa, asu = orc.quant_act(x)
    q2, sa2, asu2 = np_ref.quant_act(x)
    assert np.array_equal(q, q2) and np.array_equal(sa.view(np.uint32), sa2.view(np.uint32))
    assert np.array_equal(asu, asu2)
    assert np.abs(q.astype(int)).max() <= 127
    assert sa[0, 0] == 1.0 and not q[0, :128].any()
    assert (q[0, 128:256] == 127).all()
    # every group's max-|x| element maps to +-127
    g = np.abs(x.reshape(4, 8, 128)).argmax(axis=2)
    qq = q.reshape(4, 8, 128)
    for m in range(4):
        for j in range(8):
            if sa[m, j] != 1.0 or x[m, 128 * j:128 * j + 128].any():
                assert abs(int(qq[m, j, g[m, j]])) == 127
    assert np.array_equal(asu, q.reshape(4, 8, 128).astype(np.int32).sum(axis=2))
    # half-way points round to even: values -63.5..63.5 with s == 1
    assert sa[1, 4] == 1.0
    assert q[1, 512] == -64 and q[1, 513] == -62 and q[1, 514] == -62


def test_quant_act_brute_force_tiny(orc):
    # restatement in plain python with float32 scalar ops
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1, 128)).astype(np.float32)
    amax = np.float32(0)
    for v in x[0]:
        amax = max(amax, np.float32(abs(v)))
    s = np.float32(amax / np.float32(127))
    expect = [max(-128, min(127, int(np.rint(np.float32(v / s))))) for v in x[0]]
    q, sa, _ = orc.quant_act(x)
    assert q[0].tolist() == expect and sa[0, 0] == s


@pytest.mark.parametrize("G", [64, 128, 256])
def test_quant_rows_a8_matches_numpy(orc, G):
    rng = np.random.default_rng(12)
    rows, K = 6, 1024
    x = rng.standard_normal((rows, K)).astype(np.float32) * 3
    x[2, :G] = 0
    qh, ql, sc, sc16 = orc.quant_rows_a8(x, rows, K, G)
    q8, s = np_ref.quant_rows_i8(x, G)
    h, l = np_ref.digits(q8)
    assert np.array_equal(layout.unpack_rt4(qh), h) and np.array_equal(layout.unpack_rt4(ql), l)
    assert np.array_equal(sc.T.view(np.uint32), s.view(np.uint32))
    assert np.array_equal(sc16, sc * np.float32(16))
    # exact digit identity and ranges (src/k_new.hip:286-287)
    hh, ll = layout.unpack_rt4(qh).astype(int), layout.unpack_rt4(ql).astype(int)
    assert np.array_equal(16 * hh + ll, q8.astype(int))
    assert hh.min() >= -8 and hh.max() <= 7 and ll.min() >= -8 and ll.max() <= 7
    assert q8.max() <= 119 and q8.min() >= -128
    q8c, scc = orc.quant_rows_i8(x, rows, K, G)
    assert np.array_equal(q8c, q8) and np.array_equal(scc, sc)


def test_quant_rows_a8_stride_offset(orc):
    rng = np.random.default_rng(13)
    rows, K, stride, off = 3, 256, 640, 96
    buf = rng.standard_normal((rows, stride)).astype(np.float32)
    qh, ql, sc, sc16 = orc.quant_rows_a8(buf, rows, K, 128, stride, off)
    qh2, ql2, sc2, _ = orc.quant_rows_a8(np.ascontiguousarray(buf[:, off:off + K]), rows, K, 128)
    assert np.array_equal(qh, qh2) and np.array_equal(ql, ql2) and np.array_equal(sc, sc2)


def test_quant_rows_a4(orc):
    rng = np.random.default_rng(14)
    rows, K = 4, 512
    x = rng.standard_normal((rows, K)).astype(np.float32)
    q, sc = orc.quant_rows_a4(x, rows, K, 128)
    c = layout.unpack_rt4(q).astype(int)
    amax = np.abs(x.reshape(rows, 4, 128)).max(axis=2)
    s = (amax / np.float32(7)).astype(np.float32)
    expect = np.clip(np.rint(x.reshape(rows, 4, 128) / s[:, :, None]), -8, 7).reshape(rows, K)
    assert np.array_equal(c, expect) and np.array_equal(sc.T, s)


def test_make_group_major(orc):
    rng = np.random.default_rng(15)
    ws = (np.abs(rng.standard_normal((40, 8))) * 0.01 + 1e-3).astype(np.float16)
    gm = orc.make_group_major(ws.view(np.uint16))
    assert np.array_equal(gm, ws.astype(np.float32).T)


# ------------------------------------------------------------------ GEMV ----
def test_gemv_groupsums_match_blas(orc):
    rng = np.random.default_rng(21)
    M, N, K = 4, 96, 1024
    codes = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    q = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    I = orc.gemv_groupsums(layout.pack_rt4(codes), q)
    assert np.array_equal(I, np_ref.gemv_groupsums(codes, q))
    # brute force one element
    assert I[2, 5, 3] == int((codes[5, 384:512].astype(int) * q[2, 384:512].astype(int)).sum())


def _u_form(wq_row, ae, ao, asu, g, correct_sign_flip=True):
    """Σu·a - 8Σa with u = code+8 obtained as nibble ^ 8 (kernels/gemv_w4a8_core.h:149-150)."""
    tot = 0
    for d in range(16 * g, 16 * g + 16):
        w = int(wq_row[d])
        for j in range(4):
            lo = (w >> (8 * j)) & 0xF
            hi = (w >> (8 * j + 4)) & 0xF
            if correct_sign_flip:
                lo ^= 8
                hi ^= 8
            tot += lo * int(ae[4 * d + j]) + hi * int(ao[4 * d + j])
    return tot - 8 * int(asu[g])


def test_gemv_u_form_identity_and_planted_mistake(orc):
    # kernels/gemv_int4.hip:317-336: Σcode·a == Σu·a - 8Σa.  The reference notes that
    # omitting the ^8 gives an error of the order of Σa (docs/GEMV.md:33); the
    # identity test must catch that mistake.
    rng = np.random.default_rng(22)
    K = 512
    x = rng.standard_normal((1, K)).astype(np.float32)
    q, sa, asu = orc.quant_act(x)
    codes = rng.integers(-8, 8, size=(1, K), dtype=np.int8)
    wq = layout.pack_rt4(codes)
    I = orc.gemv_groupsums(wq, q)
    ae, ao = q[0, 0::2], q[0, 1::2]
    for g in range(K // 128):
        assert _u_form(wq[0], ae, ao, asu[0], g) == I[0, 0, g]
    bad = [_u_form(wq[0], ae, ao, asu[0], g, correct_sign_flip=False) for g in range(K // 128)]
    assert any(b != I[0, 0, g] for g, b in enumerate(bad))


def test_gemv_fold_matches_dequant_matmul(orc):
    rng = np.random.default_rng(23)
    M, N, K = 3, 64, 768
    codes = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    ws = (np.abs(rng.standard_normal((N, K // 128))) * 0.01 + 1e-3).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float32)
    wq = layout.pack_rt4(codes)
    y = orc.gemv_w4a8(wq, ws.view(np.uint16), x)
    # float64 dequant of both operands, one matmul
    q, sa, _ = np_ref.quant_act(x)
    a = q.reshape(M, K // 128, 128).astype(np.float64) * sa[:, :, None].astype(np.float64)
    w = codes.reshape(N, K // 128, 128).astype(np.float64) * ws.astype(np.float64)[:, :, None]
    ref = a.reshape(M, K) @ w.reshape(N, K).T
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ GEMM ----
def test_gemm_points_digit_identity(orc):
    rng = np.random.default_rng(31)
    M, N, K = 8, 16, 512
    codes = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    wq = layout.pack_rt4(codes)
    ws = (np.abs(rng.standard_normal((N, K // 128))) * 0.01 + 1e-3).astype(np.float16)
    sb = orc.make_group_major(ws.view(np.uint16))
    x = rng.standard_normal((M, K)).astype(np.float32) * 2
    qh, ql, sc, sc16 = orc.quant_rows_a8(x, M, K)
    q8, _ = orc.quant_rows_i8(x, M, K)
    mi = np.repeat(np.arange(M), N).astype(np.int32)
    ni = np.tile(np.arange(N), M).astype(np.int32)
    c, Ig = orc.gemm_w4a8_points(wq, sb, qh, ql, sc, sc16, M, N, K, mi, ni)
    # per-group int = 16 I_h + I_l must equal the int8-code dot exactly
    I_exact = np_ref.gemv_groupsums(codes, q8)  # [M, N, NG]
    assert np.array_equal(Ig.reshape(M, N, -1), I_exact)
    ref = np.einsum("mng,gm,gn->mn", I_exact.astype(np.float64), sc.astype(np.float64),
                    sb.astype(np.float64))
    assert np.allclose(c.reshape(M, N), ref, rtol=1e-12, atol=1e-12)


def test_gemm_w4a4_points(orc):
    rng = np.random.default_rng(32)
    M, N, K = 4, 8, 256
    codes = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    wq = layout.pack_rt4(codes)
    sb = np.abs(rng.standard_normal((K // 128, N))).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    aq, sa = orc.quant_rows_a4(x, M, K)
    mi = np.repeat(np.arange(M), N).astype(np.int32)
    ni = np.tile(np.arange(N), M).astype(np.int32)
    c, Ig = orc.gemm_w4a4_points(wq, sb, aq, sa, M, N, K, mi, ni)
    I = np_ref.gemv_groupsums(codes, layout.unpack_rt4(aq))
    assert np.array_equal(Ig.reshape(M, N, -1), I)


# ------------------------------------------------------------- W4A4 GEMV ----
def _np_quant_act4(x):
    """quant_act4 (kernels/gemv_w4a4_core.h:22-44) in numpy: per 32 elements
    s = amax/7 (fp32 division), q = clip(rint(x/s), -8, 7) (round half to even)."""
    M, K = x.shape
    xg = x.reshape(M, K // 32, 32)
    amax = np.abs(xg).max(axis=2)
    s = np.where(amax > 0, (amax / np.float32(7)).astype(np.float32), np.float32(1)).astype(np.float32)
    q = np.clip(np.rint((xg / s[:, :, None]).astype(np.float32)), -8, 7).astype(np.int8).reshape(M, K)
    return q, s


def test_quant_act4_matches_numpy_and_invariants(orc):
    rng = np.random.default_rng(31)
    M, K = 4, 512
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0, :32] = 0.0                                        # zero subgroup -> s = 1, q = 0
    x[1, 32:64] = np.float32(-2.0)                          # constant subgroup -> all -7
    x[2, 64:96] = np.minimum(np.arange(32, dtype=np.float32) * np.float32(0.5) - np.float32(7.0),
                             np.float32(7.0))               # amax 7 -> s = 1: half-way points round to even
    x[3, 96:128] *= np.float32(1e-30)
    aq, sa = orc.quant_act4(x)
    q = layout.unpack_rt4(aq)
    q2, s2 = _np_quant_act4(x)
    assert np.array_equal(q, q2) and np.array_equal(sa.view(np.uint32), s2.view(np.uint32))
    assert sa[0, 0] == 1.0 and not q[0, :32].any()
    assert (q[1, 32:64] == -7).all()
    assert sa[2, 2] == 1.0
    assert q[2, 64 + 1] == -6 and q[2, 64 + 3] == -6 and q[2, 64 + 5] == -4   # -6.5 -> -6, -5.5 -> -6, -4.5 -> -4
    g = np.abs(x.reshape(M, K // 32, 32)).argmax(axis=2)
    qq = q.reshape(M, K // 32, 32)
    for m in range(M):
        for j in range(K // 32):
            if x[m, 32 * j:32 * j + 32].any():
                assert abs(int(qq[m, j, g[m, j]])) == 7


def test_quant_act4_brute_force_tiny(orc):
    rng = np.random.default_rng(32)
    x = rng.standard_normal((1, 32)).astype(np.float32)
    amax = np.float32(0)
    for v in x[0]:
        amax = max(amax, np.float32(abs(v)))
    s = np.float32(amax / np.float32(7))
    expect = [max(-8, min(7, int(np.rint(np.float32(v / s))))) for v in x[0]]
    aq, sa = orc.quant_act4(x)
    assert layout.unpack_rt4(aq)[0].tolist() == expect and sa[0, 0] == s


def test_gemv_w4a4_sums_and_fold(orc):
    rng = np.random.default_rng(33)
    M, N, K = 3, 48, 640
    codes = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    ws = (np.abs(rng.standard_normal((N, K // 128))) * 0.01 + 1e-3).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float32)
    wq = layout.pack_rt4(codes)
    aq, sa = orc.quant_act4(x)
    a = layout.unpack_rt4(aq).astype(np.int64)
    I = orc.gemv_w4a4_sums(wq, aq)
    brute = np.einsum("mjk,njk->mnj", a.reshape(M, K // 32, 32), codes.astype(np.int64).reshape(N, K // 32, 32))
    assert np.array_equal(I, brute)
    y = orc.gemv_w4a4(wq, ws.view(np.uint16), x)
    deq_a = a.reshape(M, K // 32, 32).astype(np.float64) * sa[:, :, None].astype(np.float64)
    deq_w = codes.reshape(N, K // 128, 128).astype(np.float64) * ws.astype(np.float64)[:, :, None]
    ref = deq_a.reshape(M, K) @ deq_w.reshape(N, K).T
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)
    assert np.array_equal(orc.gemv_w4a4_fold(I, ws.view(np.uint16), sa), y)
    # a plausible mistake -- one activation scale per 128 instead of per 32 -- must show
    sa_bad = np.repeat(sa[:, ::4], 4, axis=1)
    assert not np.allclose(orc.gemv_w4a4_fold(I, ws.view(np.uint16), sa_bad), y, rtol=1e-6)
