"""int4-KV FlashAttention prefill and its feeders (attention row of the RT4 path).

Oracle: oracle/rt4_oracle.c -- the feeders restated bit for bit (src/k_new.hip:
228-399), the kernel's fixed-point algorithm in fp64 (ref_alg,
kernels/flash_attn_int4.hip:175-217) and the exact softmax over the same
quantized values (ref_rows, :146-170).

CPU tests pin the oracle: numpy restatements of the feeders and of the exact
softmax, a numpy restatement of the tile algorithm, the split-append
invariance of the V stage, and a case where the fixed-point algorithm is exact.

GPU tests: feeders bit-exact against the oracle and against the reference's
own feeder kernels built for gfx950; the prefill kernel against the algorithm
model (rel. L2 < 1e-4: the same algorithm in fp32, where an fp32 score may
round a P code differently than fp64 does) on edge shapes and on sampled rows
of the full configs[4] shape.  Against the exact softmax the algorithm itself
deviates (int4 P): the kernel's deviation must equal the algorithm model's.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
from rt4_amd import workload

HD, BN = 256, 64


# ------------------------------------------------------------------ helpers --

def nibbles(w: np.ndarray) -> np.ndarray:
    """uint32 [..., n] -> int codes [..., n, 8] (low nibble first, two's complement)."""
    nib = (w[..., None].astype(np.uint32) >> (4 * np.arange(8, dtype=np.uint32))) & 0xF
    return np.where(nib >= 8, nib.astype(np.int64) - 16, nib.astype(np.int64))


def np_quant4(x: np.ndarray, G: int):
    """s = amax/7 per G-group (fp32 division), codes = clip(rint(x/s)) -- lrintf semantics."""
    xg = x.reshape(*x.shape[:-1], -1, G)
    amax = np.abs(xg).max(-1)
    s = np.where(amax > 0, (amax / np.float32(7.0)).astype(np.float32), np.float32(1.0)).astype(np.float32)
    c = np.clip(np.rint((xg / s[..., None]).astype(np.float32)), -8, 7).astype(np.int64)
    return c.reshape(x.shape), s


def pack8(c: np.ndarray) -> np.ndarray:
    c = (c.astype(np.int64) & 0xF).astype(np.uint32).reshape(*c.shape[:-1], -1, 8)
    return np.bitwise_or.reduce(c << (4 * np.arange(8, dtype=np.uint32)), axis=-1).astype(np.uint32)


def build_cache(orc, q, k, v, TP, kv_cap):
    T, H, D = q.shape
    n_kv, KVH, _ = k.shape
    qq, qs = orc.attn_q_quant(q, TP)
    kc = np.zeros((KVH, kv_cap, D // 8), np.uint32)
    ksc = np.ones((KVH, D // 128, kv_cap), np.float32)
    orc.kv_append_k(kc, ksc, k, 0)
    vc = np.zeros((KVH, kv_cap // 8, D), np.uint32)
    vsc = np.ones((KVH, kv_cap // BN, D), np.float32)
    stage = np.zeros((KVH, BN, D), np.float32)
    orc.kv_append_v(vc, vsc, stage, v, 0, kv_cap)
    return qq, qs, kc, ksc, vc, vsc, stage


def dequant(qq, qs, kc, ksc, vc, vsc, head, ratio):
    vh = head // ratio
    Q = nibbles(qq[head]).reshape(qq.shape[1], HD) * np.repeat(qs[head].T, 128, axis=1)
    K = nibbles(kc[vh]).reshape(kc.shape[1], HD) * np.repeat(ksc[vh].T, 128, axis=1)
    Vcode = nibbles(vc[vh]).transpose(0, 2, 1).reshape(-1, HD)        # [kv/8, D, 8] -> [kv, D]
    V = Vcode * np.repeat(vsc[vh], BN, axis=0)
    return Q, K, V


def small_case(seed=3, n_q=64, n_kv=320, H=2, KVH=1, scale=True):
    rng = np.random.default_rng(seed)
    q, k, v = workload.attn_np(rng, n_q, n_kv, H, KVH)
    if not scale:
        q = q * np.float32(16.0)
    return q, k, v


# ------------------------------------------------------------------ CPU side --

def test_feeders_match_numpy(orc):
    q, k, v = small_case(n_q=48, n_kv=200)
    q[5, 1, :128] = 0.0                                   # zero group -> s = 1
    qq, qs = orc.attn_q_quant(q, 64)
    c, s = np_quant4(q, 128)
    assert np.array_equal(qq[:, :48], pack8(c).transpose(1, 0, 2))
    assert np.array_equal(qs[:, :, :48], s.transpose(1, 2, 0))
    assert np.all(qq[:, 48:] == 0) and np.all(qs[:, :, 48:] == 1.0)       # rows >= T untouched
    assert qs[1, 0, 5] == 1.0
    kc = np.zeros((1, 256, 32), np.uint32)
    ksc = np.ones((1, 2, 256), np.float32)
    orc.kv_append_k(kc, ksc, k, 0)
    c, s = np_quant4(k, 128)
    assert np.array_equal(kc[:, :200], pack8(c).transpose(1, 0, 2))
    assert np.array_equal(ksc[:, :, :200], s.transpose(1, 2, 0))


def test_v_append_tiles_and_split_invariance(orc):
    _, _, v = small_case(n_kv=200)
    cap = 256
    one = [np.zeros((1, cap // 8, HD), np.uint32), np.ones((1, cap // BN, HD), np.float32),
           np.zeros((1, BN, HD), np.float32)]
    orc.kv_append_v(*one, v, 0, cap)
    two = [np.zeros((1, cap // 8, HD), np.uint32), np.ones((1, cap // BN, HD), np.float32),
           np.zeros((1, BN, HD), np.float32)]
    for a, b in ((0, 37), (37, 100), (100, 101), (101, 200)):          # appends crossing tiles
        orc.kv_append_v(*two, v[a:b], a, cap)
    assert np.array_equal(one[0], two[0]) and np.array_equal(one[1], two[1])
    # each tile is the per-(tile, dim) quantization of its valid keys, zero codes after
    for t in range(4):
        blk = np.zeros((BN, HD), np.float32)
        n = max(0, min(200 - BN * t, BN))
        blk[:n] = v[BN * t:BN * t + n, 0]
        amax = np.abs(blk[:n]).max(0) if n else np.zeros(HD, np.float32)
        s = np.where(amax > 0, amax / np.float32(7.0), np.float32(1.0)).astype(np.float32)
        if n == 0:
            continue
        c = np.clip(np.rint(blk / s), -8, 7).astype(np.int64)
        c[n:] = 0
        assert np.array_equal(one[1][0, t], s)
        got = nibbles(one[0][0, 8 * t:8 * t + 8]).transpose(0, 2, 1).reshape(BN, HD)
        assert np.array_equal(got, c)


def test_exact_softmax_oracle_matches_numpy(orc):
    q, k, v = small_case()
    n_q, n_kv, ratio = 64, 320, 2
    qq, qs, kc, ksc, vc, vsc, _ = build_cache(orc, q, k, v, n_q, n_kv)
    off = n_kv - n_q
    rows = np.arange(n_q, dtype=np.int32)
    for head in (0, 1):
        got = orc.fa_rows(qq, qs, kc, ksc, vc, vsc, n_q, n_kv, off, n_kv, ratio, head, rows, 0)
        Q, K, V = dequant(qq, qs, kc, ksc, vc, vsc, head, ratio)
        S = Q @ K.T
        mask = np.arange(n_kv)[None, :] > (off + rows)[:, None]
        S[mask] = -np.inf
        P = np.exp(S - S.max(1, keepdims=True))
        ref = (P @ V) / P.sum(1, keepdims=True)
        assert rel_l2(got, ref) < 1e-12


def np_tile_algorithm(Q, K, V, rows, off, n_kv):
    """The fixed-point online softmax of fa_int4, written out in numpy (fp64).  V is
    read per whole 8-key group, as the reference kernel loads it
    (kernels/flash_attn_core.h:150-152): keys of a partial last group get V = 0."""
    V = V.copy()
    V[n_kv // 8 * 8:] = 0.0
    out = []
    for i in rows:
        pos = min(off + i, n_kv - 1)
        s = K[:pos + 1] @ Q[i]
        O, L, r = np.zeros(HD), 0.0, -np.inf
        for j0 in range(0, pos + 1, BN):
            st = s[j0:pos + 1][:BN]
            mt = st.max()
            p = np.floor(7.0 * np.exp(st - mt) + 0.5)
            rn = max(r, mt)
            a, b = np.exp(r - rn), np.exp(mt - rn) / 7.0
            O = O * a + b * (p @ V[j0:j0 + len(st)])
            L = L * a + b * p.sum()
            r = rn
        out.append(O / L)
    return np.array(out)


def test_algorithm_oracle_matches_numpy_restatement(orc):
    for scale in (True, False):
        q, k, v = small_case(seed=5, scale=scale)
        n_q, n_kv, ratio = 64, 320, 2
        qq, qs, kc, ksc, vc, vsc, _ = build_cache(orc, q, k, v, n_q, n_kv)
        off = n_kv - n_q
        rows = np.arange(0, n_q, 3, dtype=np.int32)
        got = orc.fa_rows(qq, qs, kc, ksc, vc, vsc, n_q, n_kv, off, n_kv, ratio, 1, rows, 1)
        Q, K, V = dequant(qq, qs, kc, ksc, vc, vsc, 1, ratio)
        assert rel_l2(got, np_tile_algorithm(Q, K, V, rows, off, n_kv)) < 1e-12


def test_algorithm_ragged_kv_follows_the_kernel_loads(orc):
    """n_kv not a multiple of 8 (nor of 64): the tile algorithm matches the numpy
    restatement with the reference kernel's load rule, and the V codes of the
    partial 8-key group do not reach the output (planted: set them to the extreme
    code) while their probabilities still count in L."""
    for n_kv in (300, 197, 64 * 4 + 3):
        q, k, v = small_case(seed=8, n_kv=n_kv, scale=True)
        n_q, ratio = 64, 2
        cap = (n_kv + BN - 1) // BN * BN
        qq, qs, kc, ksc, vc, vsc, _ = build_cache(orc, q, k, v, n_q, cap)
        off = n_kv - n_q
        rows = np.arange(n_q, dtype=np.int32)
        got = orc.fa_rows(qq, qs, kc, ksc, vc, vsc, n_q, n_kv, off, cap, ratio, 1, rows, 1)
        Q, K, V = dequant(qq, qs, kc, ksc, vc, vsc, 1, ratio)
        assert rel_l2(got, np_tile_algorithm(Q, K, V[:n_kv], rows, off, n_kv)) < 1e-12
        vc2 = vc.copy()
        g = n_kv // 8
        vc2[:, g] = 0x77777777                               # partial group: codes 7 everywhere
        got2 = orc.fa_rows(qq, qs, kc, ksc, vc2, vsc, n_q, n_kv, off, cap, ratio, 1, rows, 1)
        assert np.array_equal(got, got2)
        # the exact softmax does read those keys' V
        e1 = orc.fa_rows(qq, qs, kc, ksc, vc, vsc, n_q, n_kv, off, cap, ratio, 1, rows, 0)
        e2 = orc.fa_rows(qq, qs, kc, ksc, vc2, vsc, n_q, n_kv, off, cap, ratio, 1, rows, 0)
        assert not np.array_equal(e1, e2)


def test_algorithm_is_exact_when_scores_are_equal(orc):
    """Q = 0: every visible score is 0, P = 7 everywhere, the fixed-point algorithm
    reduces to the plain mean of the visible V rows = the exact softmax."""
    q, k, v = small_case(seed=6)
    q[:] = 0.0
    n_q, n_kv = 64, 320
    qq, qs, kc, ksc, vc, vsc, _ = build_cache(orc, q, k, v, n_q, n_kv)
    rows = np.arange(n_q, dtype=np.int32)
    e = orc.fa_rows(qq, qs, kc, ksc, vc, vsc, n_q, n_kv, n_kv - n_q, n_kv, 2, 0, rows, 0)
    a = orc.fa_rows(qq, qs, kc, ksc, vc, vsc, n_q, n_kv, n_kv - n_q, n_kv, 2, 0, rows, 1)
    assert rel_l2(a, e) < 1e-13


def test_algorithm_error_vs_exact_is_the_reference_scheme(orc):
    """The int4-P scheme's own distance from the exact softmax: small for sharp
    softmax (unscaled scores, the reference harness's data: ~1e-2 at 5 tiles and
    ~2e-3 at 64 tiles, kernels/flash_attn_int4.hip:330-395), large for the flat
    softmax of 1/sqrt(D)-scaled queries.  Recorded, not a kernel property."""
    out = {}
    for scale, n_kv in ((False, 320), (False, 4096), (True, 4096)):
        q, k, v = small_case(seed=7, n_kv=n_kv, scale=scale)
        qq, qs, kc, ksc, vc, vsc, _ = build_cache(orc, q, k, v, 64, n_kv)
        rows = np.arange(0, 64, 9, dtype=np.int32)
        e = orc.fa_rows(qq, qs, kc, ksc, vc, vsc, 64, n_kv, n_kv - 64, n_kv, 2, 0, rows, 0)
        a = orc.fa_rows(qq, qs, kc, ksc, vc, vsc, 64, n_kv, n_kv - 64, n_kv, 2, 0, rows, 1)
        out[(scale, n_kv)] = rel_l2(a, e)
    assert out[(False, 4096)] < out[(False, 320)] < 0.05
    assert out[(False, 4096)] < 5e-3
    assert out[(True, 4096)] > 0.05


# ------------------------------------------------------------------ GPU side --

def dev(torch, a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def host(t):
    return t.detach().cpu().numpy()


def gpu_cache(rt4, torch, q, k, v, TP, kv_cap, steps=None):
    T, H, D = q.shape
    n_kv, KVH, _ = k.shape
    qq, qs = rt4.attn_q_quant(dev(torch, q), TP)
    kc = torch.zeros((KVH, kv_cap, D // 8), dtype=torch.int32, device="cuda")
    ksc = torch.ones((KVH, D // 128, kv_cap), dtype=torch.float32, device="cuda")
    vc = torch.zeros((KVH, kv_cap // 8, D), dtype=torch.int32, device="cuda")
    vsc = torch.ones((KVH, kv_cap // BN, D), dtype=torch.float32, device="cuda")
    stage = torch.zeros((KVH, BN, D), dtype=torch.float32, device="cuda")
    kd, vd = dev(torch, k), dev(torch, v)
    for a, b in (steps or [(0, n_kv)]):
        rt4.kv_append_k(kc, ksc, kd[a:b].contiguous(), a)
        rt4.kv_append_v(vc, vsc, stage, vd[a:b].contiguous(), a)
    torch.cuda.synchronize()
    return qq, qs, kc, ksc, vc, vsc, stage


def test_tile_offsets_at_the_largest_cache_stay_in_range():
    """The prefill kernel addresses one KV head's cache with 32-bit buffer offsets: per
    tile t a scalar offset t * 64 keys * 128 bytes (K codes) and t * 8 * 256 * 4 bytes
    (V codes), formed in unsigned 32-bit arithmetic, and prefetches up to three tiles
    past the last.  At the largest cache the C ABI accepts, every such offset must not
    wrap (so the buffer's range check sees it beyond the resource and returns the
    zero codes), and the in-range ones must address the whole cache."""
    import re
    from conftest import PKG_DIR
    src = (PKG_DIR / "csrc" / "attn.hip").read_text()
    capi = (PKG_DIR / "csrc" / "capi.hip").read_text()
    const = {k: int(re.search(rf"constexpr int {k} = (\d+);", src).group(1)) for k in ("HD", "BNK")}
    HD, BNK = const["HD"], const["BNK"]
    KDW = HD // 8
    m = re.search(r"constexpr int kMaxKvCap = \(1 << (\d+)\) - (\d+);", capi)
    cap = (1 << int(m.group(1))) - int(m.group(2))
    n_tile = cap // BNK
    for t in range(n_tile - 2, n_tile + 3):          # the last tiles and the prefetch beyond
        sk = (t * BNK * KDW * 4) % 2 ** 32             # uint32 product, as the kernel forms it
        sv = (t * (BNK // 8) * HD * 4) % 2 ** 32
        assert sk == t * BNK * KDW * 4 and sv == t * (BNK // 8) * HD * 4, "offset wraps"
        k_bytes, v_bytes = cap * KDW * 4, (cap // 8) * HD * 4   # resource sizes at n_kv = cap
        assert (sk + 31 * 16 < k_bytes) == (t < n_tile) and (sv < v_bytes) == (t < n_tile)
    # the K offset of the farthest prefetched tile is at least 2^31: beyond int, hence uint32
    assert (n_tile + 2) * BNK * KDW * 4 >= 2 ** 31


@pytest.mark.gpu
@pytest.mark.parametrize("T,n_kv,H,KVH,steps", [(48, 200, 3, 1, [(0, 37), (37, 100), (100, 200)]),
                                                (64, 1024, 24, 4, [(0, 1024)]),
                                                (5, 4096, 6, 2, [(0, 4000), (4000, 4096)])])
def test_feeders_bit_exact(rt4, orc, torch_gpu, T, n_kv, H, KVH, steps):
    print(f"case feeders T={T} n_kv={n_kv} H={H} KVH={KVH}", flush=True)
    rng = np.random.default_rng(11)
    q, k, v = workload.attn_np(rng, T, n_kv, H, KVH)
    q[0, 0, :128] = 0.0
    TP = (T + 63) // 64 * 64
    cap = (n_kv + 63) // 64 * 64
    g = gpu_cache(rt4, torch_gpu, q, k, v, TP, cap, steps)
    c = [np.zeros((H, TP, 32), np.uint32), np.ones((H, 2, TP), np.float32)]
    orc.attn_q_quant(q, TP, qq=c[0], qs=c[1])
    kc = np.zeros((KVH, cap, 32), np.uint32)
    ksc = np.ones((KVH, 2, cap), np.float32)
    vc = np.zeros((KVH, cap // 8, HD), np.uint32)
    vsc = np.ones((KVH, cap // BN, HD), np.float32)
    st = np.zeros((KVH, BN, HD), np.float32)
    for a, b in steps:
        orc.kv_append_k(kc, ksc, k[a:b], a)
        orc.kv_append_v(vc, vsc, st, v[a:b], a, cap)
    for got, want in zip(g, (c[0], c[1], kc, ksc, vc, vsc, st)):
        assert np.array_equal(host(got).view(want.dtype), want)


@pytest.mark.gpu
def test_q_quant_unaligned_input(rt4, orc, torch_gpu):
    """Q rows that are not 16-byte aligned (the scalar-load instance of the Q
    quantizer): codes and scales bit-identical to the oracle, tiny and zero groups
    included (they take the division path)."""
    print("case attn_q_quant unaligned", flush=True)
    torch = torch_gpu
    rng = np.random.default_rng(21)
    T, H = 70, 3
    q = rng.standard_normal((T, H, HD)).astype(np.float32)
    q[0, 0, :128] = 0.0
    q[1, 1, 128:] *= np.float32(1e-30)
    TP = (T + 63) // 64 * 64
    buf = torch.empty(T * H * HD + 1, dtype=torch.float32, device="cuda")
    qd = buf[1:].view(T, H, HD)
    qd.copy_(dev(torch, q))
    assert qd.data_ptr() % 16 != 0
    qq, qs = rt4.attn_q_quant(qd, TP)
    c = [np.zeros((H, TP, 32), np.uint32), np.ones((H, 2, TP), np.float32)]
    orc.attn_q_quant(q, TP, qq=c[0], qs=c[1])
    assert np.array_equal(host(qq).view(np.uint32), c[0])
    assert np.array_equal(host(qs).view(np.uint32), c[1].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("BG,D", [(32, 256), (64, 200), (128, 256)])
def test_kv_append_v_other_tiles(rt4, orc, torch_gpu, BG, D):
    """V tiles other than 64 keys (the generic kernels) and a dim count that is not
    a multiple of 64 (the 64-key kernels' tail lanes), in several appends."""
    print(f"case kv_append_v BG={BG} D={D}", flush=True)
    rng = np.random.default_rng(17 + BG)
    KVH, n_kv = 2, 300
    cap = (n_kv + BG - 1) // BG * BG
    v = rng.standard_normal((n_kv, KVH, D)).astype(np.float32)
    v[5:9, 0, :] = 0.0
    vc = torch_gpu.zeros((KVH, cap // 8, D), dtype=torch_gpu.int32, device="cuda")
    vsc = torch_gpu.ones((KVH, cap // BG, D), dtype=torch_gpu.float32, device="cuda")
    stage = torch_gpu.zeros((KVH, BG, D), dtype=torch_gpu.float32, device="cuda")
    vc_o = np.zeros((KVH, cap // 8, D), np.uint32)
    vsc_o = np.ones((KVH, cap // BG, D), np.float32)
    st_o = np.zeros((KVH, BG, D), np.float32)
    vd = dev(torch_gpu, v)
    for a, b in [(0, 7), (7, 70), (70, 71), (71, 300)]:
        rt4.kv_append_v(vc, vsc, stage, vd[a:b].contiguous(), a)
        orc.kv_append_v(vc_o, vsc_o, st_o, v[a:b], a, cap)
    torch_gpu.cuda.synchronize()
    assert np.array_equal(host(vc).view(np.uint32), vc_o)
    assert np.array_equal(host(vsc).view(np.uint32), vsc_o.view(np.uint32))
    assert np.array_equal(host(stage).view(np.uint32), st_o.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("special", [False, True])
def test_feeders_against_reference_kernels(rt4, orc, torch_gpu, ref_hip, special):
    """The reference's own k_attn_q_quant / k_kv_append_k / k_kv_append_v built for gfx950;
    `special` plants IEEE special values (+-Inf, NaN, subnormals, FLT_MAX, -0.0) in Q, K
    and V, whose handling is the GPU's own and so is checked against these kernels."""
    print(f"case feeders vs reference kernels special={special}", flush=True)
    import ctypes
    torch = torch_gpu
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    for fn, args in (("ref_attn_q_quant", [ctypes.c_void_p] * 3 + [ctypes.c_int] * 5),
                     ("ref_kv_append_k", [ctypes.c_void_p] * 3 + [ctypes.c_int] * 6),
                     ("ref_kv_append_v", [ctypes.c_void_p] * 4 + [ctypes.c_int] * 6)):
        getattr(ref_hip, fn).argtypes = args
        getattr(ref_hip, fn).restype = None
    rng = np.random.default_rng(12)
    T, n_kv, H, KVH = 100, 700, 6, 2
    q, k, v = workload.attn_np(rng, T, n_kv, H, KVH)
    if special:
        big = np.finfo(np.float32).max
        q[3, 1, 5], q[10, 2, 130], q[30, 4, 0] = np.inf, np.nan, -np.inf
        q[20, 0, :128] = np.float32(1e-40)
        k[50, 0, 7], k[60, 1, 200] = np.inf, np.nan
        k[100:110, 0, :] = big
        k[400, 1, :128] = -0.0
        v[70, 0, 3], v[80, 1, 9], v[650, 1, 255] = np.inf, np.nan, -np.inf
        v[300, 0, :] = np.float32(1e-40)
        v[200:264, 1, 17] = -big
    TP, cap = 128, 704
    steps = [(0, 333), (333, 334), (334, 700)]
    ours = gpu_cache(rt4, torch, q, k, v, TP, cap, steps)
    qq = torch.zeros((H, TP, 32), dtype=torch.int32, device="cuda")
    qs = torch.ones((H, 2, TP), dtype=torch.float32, device="cuda")
    ref_hip.ref_attn_q_quant(P(qq), P(qs), P(dev(torch, q)), T, H, HD, 128, TP)
    kc = torch.zeros((KVH, cap, 32), dtype=torch.int32, device="cuda")
    ksc = torch.ones((KVH, 2, cap), dtype=torch.float32, device="cuda")
    vc = torch.zeros((KVH, cap // 8, HD), dtype=torch.int32, device="cuda")
    vsc = torch.ones((KVH, cap // BN, HD), dtype=torch.float32, device="cuda")
    st = torch.zeros((KVH, BN, HD), dtype=torch.float32, device="cuda")
    kd, vd = dev(torch, k), dev(torch, v)
    for a, b in steps:
        ref_hip.ref_kv_append_k(P(kc), P(ksc), P(kd[a:b].contiguous()), a, b - a, KVH, HD, 128, cap)
        ref_hip.ref_kv_append_v(P(vc), P(vsc), P(st), P(vd[a:b].contiguous()), a, b - a, KVH, HD, BN, cap)
    ref_hip.ref_sync()
    for got, want in zip(ours, (qq, qs, kc, ksc, vc, vsc, st)):
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))     # bit patterns (NaN too)


def check_attention(rt4, orc, torch, q, k, v, ratio, off, n_kv, kv_cap, rows_per_head, heads, splits=(0,)):
    T, H, _ = q.shape
    TP = (T + 63) // 64 * 64
    g = gpu_cache(rt4, torch, q, k, v, TP, kv_cap)

    def run(s):
        # a NaN-filled output, so that a row the kernel does not write cannot pass
        o = torch.full((H, TP, HD), float("nan"), dtype=torch.float32, device="cuda")
        return host(rt4.attention_prefill(*g[:6], n_kv=n_kv, off=off, ratio=ratio, kv_splits=s, out=o))

    outs = []
    for s in splits:
        o1, o2 = run(s), run(s)
        # the split combines re-arm their counters: a second call gives the same bits
        assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32)), f"kv_splits={s}: second call differs"
        outs.append(o1)
    out = outs[0]
    for s, o in zip(splits[1:], outs[1:]):            # KV splits change only the fp32 rounding
        e = rel_l2(o, out)
        print(f"  kv_splits={s}: vs first {e:.2e}")
        assert e < 1e-5
    c = [host(t).view(np.uint32) if t.dtype == torch.int32 else host(t) for t in g[:6]]
    worst = 0.0
    for h in heads:
        rows = rows_per_head(h)
        alg = orc.fa_rows(*c, TP, n_kv, off, kv_cap, ratio, h, rows, 1)
        exact = orc.fa_rows(*c, TP, n_kv, off, kv_cap, ratio, h, rows, 0)
        got = out[h, rows].astype(np.float64)
        e_alg = rel_l2(got, alg)
        e_exact, a_exact = rel_l2(got, exact), rel_l2(alg, exact)
        print(f"  head {h}: kernel vs algorithm {e_alg:.2e}; vs exact {e_exact:.3e} (algorithm itself {a_exact:.3e})")
        assert e_alg < 1e-4
        assert abs(e_exact - a_exact) <= 1e-4 + 0.01 * a_exact
        worst = max(worst, e_alg)
    return out, worst


@pytest.mark.gpu
@pytest.mark.parametrize("T,n_kv,off,H,KVH,cap,scale", [
    (64, 64, 0, 2, 1, 64, False),          # one tile, square causal
    (64, 320, 256, 2, 1, 320, False),      # the reference harness's check shape family
    (128, 200, 72, 4, 2, 256, True),       # n_kv not a multiple of 64, kv_cap > n_kv
    (192, 1000, 808, 6, 1, 1024, True),    # ratio 6, partial last tile
    (64, 2048, 1984, 1, 1, 4096, False),   # no GQA, long-ish
    (128, 300, 172, 6, 2, 320, True),      # GQA ratio 3 over two KV heads; n_kv % 8 != 0: partial V group
    (64, 520, 456, 8, 2, 576, True),       # ratio 4 over two KV heads
])
def test_attention_against_oracle(rt4, orc, torch_gpu, T, n_kv, off, H, KVH, cap, scale):
    print(f"case attention T={T} n_kv={n_kv} off={off} H={H} KVH={KVH} cap={cap}", flush=True)
    rng = np.random.default_rng(13)
    q, k, v = workload.attn_np(rng, T, n_kv, H, KVH)
    if not scale:
        q = q * np.float32(16.0)
    ratio = H // KVH
    all_rows = np.arange(T, dtype=np.int32)
    check_attention(rt4, orc, torch_gpu, q, k, v, ratio, off, n_kv, cap, lambda h: all_rows, range(H),
                    splits=(0, 1, 2, 3, 7))


@pytest.mark.gpu
@pytest.mark.parametrize("T,n_kv,off,H,KVH,cap", [
    (64, 64, 0, 2, 1, 64),                 # one tile
    (128, 200, 72, 4, 2, 256),             # n_kv not a multiple of 64, kv_cap > n_kv
    (128, 300, 172, 6, 2, 320),            # partial 8-key V group
    (192, 1000, 808, 6, 1, 1024),          # GQA 6, partial last tile
    (64, 520, 456, 8, 2, 576),             # GQA 4 over two KV heads
])
def test_attention_staged_copy_matches_in_kernel_staging(rt4, torch_gpu, T, n_kv, off, H, KVH, cap):
    """The prefill stages K/V once per call into a copy that the workgroups DMA into
    LDS.  Captured into a graph with no room for that copy (scratch released), every
    workgroup stages its own tiles instead.  Both forms put the same operand bytes in
    LDS, so the outputs must be bit-identical (one split: the automatic count also
    falls back to one split under capture without workspace)."""
    torch = torch_gpu
    print(f"case staged copy vs in-kernel staging T={T} n_kv={n_kv} off={off} H={H} KVH={KVH} cap={cap}", flush=True)
    rng = np.random.default_rng(29)
    q, k, v = workload.attn_np(rng, T, n_kv, H, KVH)
    TP = (T + 63) // 64 * 64
    g = gpu_cache(rt4, torch, q, k, v, TP, cap)
    kw = dict(n_kv=n_kv, off=off, ratio=H // KVH)
    eager = host(rt4.attention_prefill(*g[:6], kv_splits=1, **kw))
    for s in (1, 0):
        torch.cuda.synchronize()
        rt4.release_scratch()
        out = torch.full((H, TP, HD), float("nan"), dtype=torch.float32, device="cuda")
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            rt4.attention_prefill(*g[:6], kv_splits=s, out=out, **kw)
        for _ in range(2):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(host(out).view(np.uint32), eager.view(np.uint32)), f"kv_splits={s}"
        del graph
        print(f"  captured kv_splits={s} (in-kernel staging) = eager (staged copy), bit for bit", flush=True)


@pytest.mark.gpu
def test_attention_benchmark_shape_sampled(rt4, orc, torch_gpu):
    """24 heads, GQA 6:1, 1024 queries over a 32768-token cache."""
    c4 = workload.ATTN_C4
    n_q, ctx = c4["n_q"], c4["ctx"]
    n_kv = ctx + n_q
    print(f"case attention C4 n_q={n_q} n_kv={n_kv}", flush=True)
    rng = np.random.default_rng(14)
    q, k, v = workload.attn_np(rng, n_q, n_kv, c4["H"], c4["KVH"])
    rows = np.array([0, 1, 63, 64, 511, 1000, 1023], np.int32)
    out, _ = check_attention(rt4, orc, torch_gpu, q, k, v, c4["H"] // c4["KVH"], ctx, n_kv, n_kv,
                             lambda h: rows, (0, 5, 6, 23))
    assert np.isfinite(out).all()


@pytest.mark.gpu
def test_attention_reference_long_context_sampled(rt4, orc, torch_gpu):
    """The reference's own benchmark shape (docs/FLASH-ATTN.md:78-80): 24 heads, GQA
    6:1, 1024 queries over a 131072-token cache, sampled rows of the first and last
    query head against the fp64 algorithm model."""
    c = workload.ATTN_REF
    n_q, ctx = c["n_q"], c["ctx"]
    n_kv = ctx + n_q
    print(f"case attention reference shape n_q={n_q} n_kv={n_kv}", flush=True)
    rng = np.random.default_rng(15)
    q, k, v = workload.attn_np(rng, n_q, n_kv, c["H"], c["KVH"])
    rows = np.array([0, 511, 1023], np.int32)
    out, _ = check_attention(rt4, orc, torch_gpu, q, k, v, c["H"] // c["KVH"], ctx, n_kv, n_kv,
                             lambda h: rows, (0, 23))
    assert np.isfinite(out).all()


@pytest.mark.gpu
def test_graph_keeps_workspace_when_scratch_grows(rt4, torch_gpu):
    """A HIP graph captured on the split-KV path holds the address of the library's
    partial-sum workspace.  A later, larger call grows that workspace; the graph's
    buffer must stay allocated, so its replays still give the eager result."""
    torch = torch_gpu
    print("case graph replay after scratch growth", flush=True)
    rng = np.random.default_rng(23)
    q, k, v = workload.attn_np(rng, 64, 640, 2, 1)
    g = gpu_cache(rt4, torch, q, k, v, 64, 640)
    kw = dict(n_kv=640, off=576, ratio=2, kv_splits=2)
    ref = host(rt4.attention_prefill(*g[:6], **kw))
    out = torch.empty((2, 64, HD), dtype=torch.float32, device="cuda")
    rt4.attention_prefill(*g[:6], out=out, **kw)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rt4.attention_prefill(*g[:6], out=out, **kw)
    # grow the workspace: 64 splits x 24 heads x 256 rows x 1 KB of partials
    q2, k2, v2 = workload.attn_np(rng, 256, 640, 24, 4)
    g2 = gpu_cache(rt4, torch, q2, k2, v2, 256, 640)
    rt4.attention_prefill(*g2[:6], n_kv=640, off=384, ratio=6, kv_splits=64)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("T,n_kv,off,H,KVH,cap,scale", [
    (64, 320, 256, 2, 1, 320, True),       # the verdict's small shape: 5 whole tiles
    (64, 320, 256, 2, 1, 320, False),      # unscaled Q: sharp softmax, the running max moves
    (128, 300, 172, 6, 2, 320, True),      # GQA 3, ragged n_kv (partial 8-key V group)
    (192, 1000, 808, 6, 1, 1024, True),    # GQA 6, partial last tile
])
def test_attention_against_reference_kernel(rt4, orc, torch_gpu, ref_hip, T, n_kv, off, H, KVH, cap, scale):
    """The reference's own fa_int4 (kernels/flash_attn_core.h:74-435, launched as
    src/k_fa.hip:294-296), built for gfx950 from its source, on the same quantized
    cache: first against the CPU algorithm model (pins the model: tile max vs running
    max, alpha/beta, P rounding), then our kernel against it."""
    import ctypes
    torch = torch_gpu
    print(f"case attention vs reference fa_int4 T={T} n_kv={n_kv} off={off} H={H} KVH={KVH}", flush=True)
    ref_hip.ref_fa_int4.argtypes = [ctypes.c_void_p] * 7 + [ctypes.c_int] * 7
    ref_hip.ref_fa_int4.restype = None
    rng = np.random.default_rng(29)
    q, k, v = workload.attn_np(rng, T, n_kv, H, KVH)
    if not scale:
        q = q * np.float32(16.0)
    ratio = H // KVH
    TP = (T + 63) // 64 * 64
    g = gpu_cache(rt4, torch, q, k, v, TP, cap)
    n_tile = (n_kv + BN - 1) // BN
    ref_out = torch.zeros((H, TP, HD), dtype=torch.float32, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    torch.cuda.synchronize()
    ref_hip.ref_fa_int4(P(g[0]), P(g[1]), P(g[2]), P(g[3]), P(g[4]), P(g[5]), P(ref_out), T, n_kv, off, n_tile,
                        H, ratio, cap)
    ref_hip.ref_sync()
    ours = host(rt4.attention_prefill(*g[:6], n_kv=n_kv, off=off, ratio=ratio))
    torch.cuda.synchronize()
    ref_o = host(ref_out)
    c = [host(t).view(np.uint32) if t.dtype == torch.int32 else host(t) for t in g[:6]]
    rows = np.arange(T, dtype=np.int32)
    for h in range(H):
        alg = orc.fa_rows(*c, TP, n_kv, off, cap, ratio, h, rows, 1)
        e_model = rel_l2(ref_o[h, :T], alg)
        e_ours = rel_l2(ours[h, :T], ref_o[h, :T])
        print(f"  head {h}: reference kernel vs algorithm model {e_model:.2e}; ours vs reference kernel {e_ours:.2e}")
        assert e_model < 1e-4
        assert e_ours < 1e-4


@pytest.mark.gpu
def test_attention_benchmark_shape_against_reference_kernel(rt4, orc, torch_gpu, ref_hip):
    """configs[4] in full: every output of our kernel against the reference's fa_int4
    (built for gfx950) on the same quantized cache, plus sampled rows of the reference
    kernel against the CPU algorithm model."""
    import ctypes
    torch = torch_gpu
    c4 = workload.ATTN_C4
    n_q, ctx, H, KVH = c4["n_q"], c4["ctx"], c4["H"], c4["KVH"]
    n_kv = ctx + n_q
    ratio = H // KVH
    print(f"case attention C4 vs reference fa_int4 n_q={n_q} n_kv={n_kv}", flush=True)
    rng = np.random.default_rng(31)
    q, k, v = workload.attn_np(rng, n_q, n_kv, H, KVH)
    g = gpu_cache(rt4, torch, q, k, v, n_q, n_kv)
    ref_out = torch.zeros((H, n_q, HD), dtype=torch.float32, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    torch.cuda.synchronize()
    ref_hip.ref_fa_int4(P(g[0]), P(g[1]), P(g[2]), P(g[3]), P(g[4]), P(g[5]), P(ref_out), n_q, n_kv, ctx,
                        n_kv // BN, H, ratio, n_kv)
    ref_hip.ref_sync()
    ours = rt4.attention_prefill(*g[:6], n_kv=n_kv, off=ctx, ratio=ratio)
    torch.cuda.synchronize()
    e_all = float((ours.double() - ref_out.double()).norm() / ref_out.double().norm())
    print(f"  all {H}x{n_q}x{HD} outputs: ours vs reference kernel {e_all:.2e}")
    ref_o, our_o = host(ref_out), host(ours)
    c = [host(t).view(np.uint32) if t.dtype == torch.int32 else host(t) for t in g[:6]]
    rows = np.array([0, 63, 64, 700, 1023], np.int32)
    worst = 0.0
    for h in (0, 11, 23):
        alg = orc.fa_rows(*c, n_q, n_kv, ctx, n_kv, ratio, h, rows, 1)
        e_ref, e_our = rel_l2(ref_o[h, rows], alg), rel_l2(our_o[h, rows], alg)
        print(f"  head {h}: vs the fp64 algorithm model: reference kernel {e_ref:.2e}, ours {e_our:.2e}")
        worst = max(worst, e_ref, e_our)
    # Every row where the two kernels differ by more than 1e-4, against the fp64 model:
    # such a row holds a 3-bit P code that a kernel's fp32 scores put on the other side
    # of a rounding edge from the model.  Both kernels do this on a few rows (seed 31:
    # 118 rows of 24576 differ; ours is off the model on 58, the reference kernel on 62,
    # both on 2), so ours must flip no more rows than the reference kernel, give or take
    # a few, and by no larger an error.
    d = np.linalg.norm(our_o - ref_o, axis=2) / np.maximum(np.linalg.norm(ref_o, axis=2), 1e-30)   # [H, n_q]
    rows_off = np.argwhere(d > 1e-4)
    print(f"  rows where the kernels differ by more than 1e-4: {len(rows_off)} of {H * n_q}")
    assert len(rows_off) <= 256
    ours_off = ref_off = both_off = 0
    worst_row_ours = worst_row_ref = 0.0
    for h in np.unique(rows_off[:, 0]):
        rr = rows_off[rows_off[:, 0] == h, 1].astype(np.int32)
        alg = orc.fa_rows(*c, n_q, n_kv, ctx, n_kv, ratio, int(h), rr, 1).reshape(len(rr), HD)
        for i, r in enumerate(rr):
            e_ref, e_our = rel_l2(ref_o[h, r], alg[i]), rel_l2(our_o[h, r], alg[i])
            ours_off += e_our > 1e-4
            ref_off += e_ref > 1e-4
            both_off += (e_our > 1e-4) and (e_ref > 1e-4)
            worst_row_ours, worst_row_ref = max(worst_row_ours, e_our), max(worst_row_ref, e_ref)
    print(f"  of those, off the fp64 model by more than 1e-4: ours {ours_off}, the reference kernel "
          f"{ref_off}, both {both_off}; worst row: ours {worst_row_ours:.2e}, reference {worst_row_ref:.2e}")
    assert ours_off <= ref_off + 8
    assert worst_row_ours <= max(worst_row_ref, 2e-2)
    # each fp32 kernel is within 1e-4 of the fp64 model (a score that lands on a
    # rounding edge of a 3-bit P code may round either way in fp32); the two
    # kernels' outputs may then differ by up to the sum of their deviations
    assert worst < 1e-4
    assert e_all < 5e-4
