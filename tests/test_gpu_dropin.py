"""The RT4 path driven the way the reference runtime drives it, from C++.

tests/_bin/dropin_caller (tests/dropin_caller.cpp, built by tests/Makefile from
include/rt4_kernels.h and librt4k.so only) repeats src/model.cpp's sequences:

* Model::linear_quant (src/model.cpp:1010-1026): M <= 4 -> k_gemv_w4a8; M > 4 ->
  M padded to a multiple of 128, k_quant_rows_a8, k_gemm_i4_a8;
* the attention prefill (src/model.cpp:1077-1081, :1140-1142): k_attn_q_quant,
  k_kv_append_k / k_kv_append_v at seq_len, k_attention(n_q = TP, n_row = T).

Each case writes its inputs as raw files, runs the program as a child process and
checks what it wrote against the golden fixtures or the CPU oracle:
GEMV/GEMM outputs within 1e-6 relative L2 of the oracle's fp64 restatement (the
fp32 sum order is the only difference) and the reference harness's worst/rms
< 1e-5; the quantized Q and KV cache bit-exact; attention outputs within 1e-4
relative L2 of the oracle's model of the kernel's fixed-point algorithm.
"""
from __future__ import annotations

import pathlib
import subprocess

import numpy as np
import pytest

from conftest import ROOT, rel_l2
from rt4_amd import workload

pytestmark = pytest.mark.gpu

EXE = ROOT / "tests" / "_bin" / "dropin_caller"
GOLDEN = ROOT / "tests" / "golden" / "rt4_golden.npz"
TIGHT = 1e-6


def run_caller(tmp: pathlib.Path, *args) -> None:
    if not EXE.exists():
        pytest.fail(f"{EXE} is missing: __graft_entry__.build() builds it (make -C tests dropin)")
    argv = [str(EXE), str(tmp)] + [str(a) for a in args]
    print("  run", " ".join(argv[2:]), flush=True)
    r = subprocess.run(argv, capture_output=True, text=True, timeout=120)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)


def put(tmp: pathlib.Path, name: str, a: np.ndarray) -> None:
    np.ascontiguousarray(a).tofile(tmp / name)


def get(tmp: pathlib.Path, name: str, dtype, shape) -> np.ndarray:
    return np.fromfile(tmp / name, dtype=dtype).reshape(shape)


def test_linear_quant_decode_golden(tmp_path):
    """M = 4 (the GEMV branch) on the golden decode fixture."""
    print("case dropin linear_quant golden decode M=4 N=48 K=384", flush=True)
    with np.load(GOLDEN, allow_pickle=False) as z:
        wq, ws, x, want = z["gv_wq"], z["gv_ws"], z["gv_x"], z["gv_y"]
    put(tmp_path, "wq.u32", wq)
    put(tmp_path, "ws.u16", ws)
    put(tmp_path, "x.f32", x)
    run_caller(tmp_path, "gemv", 4, 48, 384)
    y = get(tmp_path, "y.f32", np.float32, (4, 48))
    assert rel_l2(y, want) < TIGHT


@pytest.mark.parametrize("M,N,K", [(1, 4096, 5120), (3, 1024, 17408)])
def test_linear_quant_decode(orc, tmp_path, M, N, K):
    print(f"case dropin linear_quant decode M={M} N={N} K={K}", flush=True)
    c = workload.gemv_case(31, M, N, K)
    put(tmp_path, "wq.u32", c["wq"])
    put(tmp_path, "ws.u16", c["ws"])
    put(tmp_path, "x.f32", c["x"])
    run_caller(tmp_path, "gemv", M, N, K)
    y = get(tmp_path, "y.f32", np.float32, (M, N))
    ref = orc.gemv_w4a8(c["wq"], c["ws"], c["x"])
    err = rel_l2(y, ref)
    print(f"  rel_l2 = {err:.3e}")
    assert err < TIGHT


@pytest.mark.parametrize("M,N,K,full", [(5, 256, 512, True), (1000, 1024, 5120, False)])
def test_linear_quant_prefill(orc, tmp_path, M, N, K, full):
    """M > 4: padded to 128 rows, quantized, GEMM; the padding rows are whatever the
    activation buffer holds (random here) and are computed like the others."""
    Mp = (M + 127) // 128 * 128
    print(f"case dropin linear_quant prefill M={M} (Mp={Mp}) N={N} K={K}", flush=True)
    c = workload.gemm_case(41, Mp, N, K)
    put(tmp_path, "wq.u32", c["wq"])
    put(tmp_path, "wsgm.f32", orc.make_group_major(c["ws"]))
    put(tmp_path, "x.f32", c["x"])
    run_caller(tmp_path, "gemm", M, N, K)
    out = get(tmp_path, "c.f32", np.float32, (Mp, N))
    if full:
        mi = np.repeat(np.arange(Mp), N).astype(np.int32)
        ni = np.tile(np.arange(N), Mp).astype(np.int32)
    else:
        rng = np.random.default_rng(9)
        P = 8192
        mi = rng.integers(0, Mp, P).astype(np.int32)
        ni = rng.integers(0, N, P).astype(np.int32)
        mi[:6], ni[:6] = [0, M - 1, M, Mp - 1, 0, Mp - 1], [0, N - 1, 0, N - 1, N - 1, 0]
    qh, ql, sc, sc16 = orc.quant_rows_a8(c["x"], Mp, K)
    sb = orc.make_group_major(c["ws"])
    ref, _ = orc.gemm_w4a8_points(c["wq"], sb, qh, ql, sc, sc16, Mp, N, K, mi, ni)
    got = out[mi, ni]
    err = rel_l2(got, ref)
    worst = float(np.abs(got - ref).max()) / float(np.sqrt(np.mean(ref ** 2)))
    print(f"  rel_l2 = {err:.3e}  worst/rms = {worst:.3e}")
    assert err < TIGHT and worst < 1e-5


@pytest.mark.parametrize("T,H,KVH,seq_len,cap", [(100, 8, 2, 300, 512), (64, 24, 4, 0, 64)])
def test_attention_prefill_chunk(orc, tmp_path, T, H, KVH, seq_len, cap):
    """A prefill chunk of T rows after seq_len cached keys (T not a multiple of 64)."""
    TP = (T + 63) // 64 * 64
    n_kv = seq_len + T
    print(f"case dropin attention T={T} H={H} KVH={KVH} seq_len={seq_len} cap={cap}", flush=True)
    rng = np.random.default_rng(77)
    q, k, v = workload.attn_np(rng, T, n_kv, H, KVH)
    put(tmp_path, "q.f32", q)
    put(tmp_path, "kold.f32", k[:seq_len])
    put(tmp_path, "vold.f32", v[:seq_len])
    put(tmp_path, "knew.f32", k[seq_len:])
    put(tmp_path, "vnew.f32", v[seq_len:])
    run_caller(tmp_path, "attn", T, H, KVH, seq_len, cap)

    qq, qs = orc.attn_q_quant(q, TP)
    kc = np.zeros((KVH, cap, 32), np.uint32)
    ksc = np.ones((KVH, 2, cap), np.float32)
    vc = np.zeros((KVH, cap // 8, 256), np.uint32)
    vsc = np.ones((KVH, cap // 64, 256), np.float32)
    stage = np.zeros((KVH, 64, 256), np.float32)
    orc.kv_append_k(kc, ksc, k[:seq_len], 0)
    orc.kv_append_v(vc, vsc, stage, v[:seq_len], 0, cap)
    orc.kv_append_k(kc, ksc, k[seq_len:], seq_len)
    orc.kv_append_v(vc, vsc, stage, v[seq_len:], seq_len, cap)
    for name, want in (("qq.u32", qq), ("qs.f32", qs), ("kc.u32", kc), ("ksc.f32", ksc), ("vc.u32", vc),
                       ("vsc.f32", vsc)):
        got = get(tmp_path, name, want.dtype, want.shape)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name

    out = get(tmp_path, "out.f32", np.float32, (H, TP, 256))
    rows = np.arange(T, dtype=np.int32)
    worst = 0.0
    for h in range(H):
        alg = orc.fa_rows(qq, qs, kc, ksc, vc, vsc, TP, n_kv, seq_len, cap, H // KVH, h, rows, 1)
        worst = max(worst, rel_l2(out[h, :T].astype(np.float64), alg))
    print(f"  worst head rel_l2 vs the algorithm model = {worst:.2e}")
    assert worst < 1e-4
