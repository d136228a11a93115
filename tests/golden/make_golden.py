#!/usr/bin/env python3
"""Writes the golden fixtures of the RT4 path into tests/golden/rt4_golden.npz.

Inputs are small seeded tensors with the edge cases of the path (an all-zero
activation group, a 20-sigma outlier, a ragged row count, the most negative
weight code -8); outputs come from the CPU oracle (oracle/rt4_oracle.c, which
cites the reference file:line of every step).  tests/test_golden.py checks the
oracle against these files on the CPU (any change to the oracle's results is a
visible diff) and the HIP kernels against them on the GPU.

    python tests/golden/make_golden.py        # rewrites rt4_golden.npz
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "k100lc-rt4_amd"))

from oracle import rt4_oracle as orc  # noqa: E402
from rt4_amd import layout  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent / "rt4_golden.npz"


def make() -> dict:
    rng = np.random.default_rng(20260101)
    f = {}
    # --- decode quantizer (quant_act): 3 rows x 384, an all-zero group, an outlier, ties
    x = rng.standard_normal((3, 384)).astype(np.float16).astype(np.float32)
    x[1, 128:256] = 0.0
    x[2, 5] = 20.0
    x[0, 256:384] = np.round(x[0, 256:384] * 4) / 4
    q, sa, asu = orc.quant_act(x)
    f.update(qa_x=x, qa_q=q, qa_sa=sa, qa_asu=asu)
    # --- decode GEMV: M=4 rows, N=48, K=384; codes in [-8, 7] (the -8 corner included)
    M, N, K = 4, 48, 384
    codes = rng.integers(-8, 8, size=(N, K)).astype(np.int8)
    codes[0, :8] = -8
    wq = layout.pack_rt4(codes)
    ws = layout.f16_bits((np.abs(rng.standard_normal((N, K // 128))) * 0.01 + 1e-3).astype(np.float32))
    xg = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
    qg, sag, _ = orc.quant_act(xg)
    I = orc.gemv_groupsums(wq, qg)
    y = orc.gemv_fold(I, ws, sag).astype(np.float32)
    f.update(gv_wq=wq, gv_ws=ws, gv_x=xg, gv_I=I, gv_y=y)
    # --- prefill quantizer (quant_rows_a8), ragged rows, G=128 and G=64
    xr = rng.standard_normal((5, 256)).astype(np.float16).astype(np.float32)
    xr[4, :128] = 0.0
    xr[3, 77] = -20.0
    for G in (128, 64):
        qh, ql, sc, sc16 = orc.quant_rows_a8(xr, 5, 256, G)
        f.update({f"qr{G}_qh": qh, f"qr{G}_ql": ql, f"qr{G}_sc": sc, f"qr{G}_sc16": sc16})
    f["qr_x"] = xr
    # --- prefill GEMM: M=8 (not a multiple of the tile), N=32, K=256, full output
    M, N, K = 8, 32, 256
    codes = rng.integers(-8, 8, size=(N, K)).astype(np.int8)
    wq = layout.pack_rt4(codes)
    ws = layout.f16_bits((np.abs(rng.standard_normal((N, K // 128))) * 0.01 + 1e-3).astype(np.float32))
    xm = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
    xm[rng.random((M, K)) < 0.01] *= 20.0
    qh, ql, sc, sc16 = orc.quant_rows_a8(xm, M, K)
    sb = orc.make_group_major(ws)
    mi = np.repeat(np.arange(M), N).astype(np.int32)
    ni = np.tile(np.arange(N), M).astype(np.int32)
    c, Ig = orc.gemm_w4a8_points(wq, sb, qh, ql, sc, sc16, M, N, K, mi, ni)
    f.update(gm_wq=wq, gm_ws=ws, gm_x=xm, gm_sb=sb, gm_I=Ig.reshape(M, N, K // 128),
             gm_c=c.reshape(M, N))
    # --- converter weight quantizer (tools/convert.c:338-360)
    w = (rng.standard_normal((4, 256)) * 0.02).astype(np.float32)
    w[1, :128] = 0.0
    wq4, ws4 = orc.quant_weight_rows(w)
    f.update(wc_w=w, wc_wq=wq4, wc_ws=ws4)
    return f


def main() -> int:
    f = make()
    np.savez_compressed(OUT, **f)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(f)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
