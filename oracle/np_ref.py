"""Independent numpy restatement of the RT4 path, and the numpy CPU baseline.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Two uses:
 1. A second, vectorised restatement written from the format spec
    (docs/FORMAT.md:61-93) and the reference quantizers, used to cross-check
    the C oracle (rt4_oracle.c): two restatements that agree bit for bit on the
    codes pin each other against transcription slips.
 2. The CPU baseline of the benchmark: the reference's own CPU path, i.e. the
    RT4 dequantisation of tools/rt4_io.py:40-52 (codes * repeat(scale, 128) in
    fp32) followed by a float matmul, chunked by 8192 output rows for the LM
    head as tools/ref_full.py:113-117 does.  numpy's BLAS does the matmul.
"""
from __future__ import annotations

import numpy as np

GROUP = 128


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    """tools/rt4_io.py:8-18: binary16 bits -> float32 without numpy's float16."""
    h = np.asarray(h, dtype=np.uint16)
    sg = (h >> 15) & 1
    ex = ((h >> 10) & 0x1F).astype(np.int32)
    ma = (h & 0x3FF).astype(np.float32)
    out = np.where(ex == 0, np.ldexp(ma / np.float32(1024.0), -14),
                   np.ldexp(np.float32(1.0) + ma / np.float32(1024.0), ex - 15))
    return np.where(sg == 1, -out, out).astype(np.float32)


def unpack_bytes(qbytes: np.ndarray) -> np.ndarray:
    """RT4 byte view [N, K/2] -> int16 codes [N, K] (low nibble = even k), tools/rt4_io.py:47-51."""
    lo = (qbytes & 0x0F).astype(np.int16)
    hi = ((qbytes >> 4) & 0x0F).astype(np.int16)
    N = qbytes.shape[0]
    out = np.empty((N, qbytes.shape[1] * 2), np.int16)
    out[:, 0::2] = np.where(lo >= 8, lo - 16, lo)
    out[:, 1::2] = np.where(hi >= 8, hi - 16, hi)
    return out


def _group_amax(x: np.ndarray, G: int) -> np.ndarray:
    M, K = x.shape
    return np.abs(x.reshape(M, K // G, G)).max(axis=2)


def quant_act(x: np.ndarray, G: int = GROUP):
    """Decode-side quantizer (kernels/gemv_w4a8_core.h:34-66), vectorised, per (row,
    G).  The reference's G is 128; G = K is the per-row mode (one scale per row),
    which has no reference counterpart: its scale s[:, 0] is the row's scale and Σq
    is still returned per 128-group, the layouts the library writes."""
    x = np.asarray(x, np.float32)
    M, K = x.shape
    amax = _group_amax(x, G)
    s = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.rint(x.reshape(M, K // G, G) / s[:, :, None])
    q = np.clip(q, -128, 127).astype(np.int8).reshape(M, K)
    asu = q.reshape(M, K // GROUP, GROUP).astype(np.int32).sum(axis=2)
    return q, s, asu


def quant_rows_i8(x: np.ndarray, G: int = GROUP):
    """Prefill-side quantizer's code (src/k_new.hip:268-301): q8 and s, per (row, G)."""
    x = np.asarray(x, np.float32)
    M, K = x.shape
    amax = _group_amax(x, G)
    s = np.where(amax > 0, amax / np.float32(119.0), np.float32(1.0)).astype(np.float32)
    q = np.rint(x.reshape(M, K // G, G) / s[:, :, None])
    q = np.clip(q, -128, 119).astype(np.int8).reshape(M, K)
    return q, s


def digits(q8: np.ndarray):
    """q8 -> (h, l) with q8 = 16h + l, h = floor((q8+8)/16) (src/k_new.hip:286-287)."""
    q = q8.astype(np.int32)
    h = (q + 8) >> 4
    return h.astype(np.int8), (q - 16 * h).astype(np.int8)


def gemv_groupsums(codes: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Exact int group dots via float64 BLAS (integers < 2^53 are exact)."""
    N, K = codes.shape
    M = q.shape[0]
    NG = K // GROUP
    c = codes.astype(np.float64).reshape(N, NG, GROUP).transpose(1, 0, 2)   # [NG, N, 128]
    a = q.astype(np.float64).reshape(M, NG, GROUP).transpose(1, 2, 0)       # [NG, 128, M]
    I = np.matmul(c, a)                                                     # [NG, N, M]
    return np.rint(I).astype(np.int64).transpose(2, 1, 0).astype(np.int32)  # [M, N, NG]


# ------------------------------------------------------------ CPU baseline --
def dequant(wq_bytes: np.ndarray, ws_bits: np.ndarray) -> np.ndarray:
    """RT4.dequant (tools/rt4_io.py:40-52): fp32 W [N, K] = code * repeat(scale, 128)."""
    N = wq_bytes.shape[0]
    K = wq_bytes.shape[1] * 2
    s = f16_bits_to_f32(ws_bits).reshape(N, K // GROUP)
    w = unpack_bytes(wq_bytes).astype(np.float32)
    w *= np.repeat(s, GROUP, axis=1)
    return w


def fake_quant_act(x: np.ndarray) -> np.ndarray:
    """Activations as the GEMV sees them: q * sa per (row, group), fp32."""
    q, s, _ = quant_act(x)
    M, K = q.shape
    return (q.reshape(M, K // GROUP, GROUP).astype(np.float32) * s[:, :, None]).reshape(M, K)


def cpu_linear(wq_bytes: np.ndarray, ws_bits: np.ndarray, xf: np.ndarray, chunk: int = 8192):
    """Dequantise chunk by chunk and multiply (tools/ref_full.py:113-117): y [M, N] fp32."""
    N = wq_bytes.shape[0]
    y = np.empty((xf.shape[0], N), np.float32)
    for c0 in range(0, N, chunk):
        c1 = min(c0 + chunk, N)
        w = dequant(wq_bytes[c0:c1], ws_bits[c0:c1])
        y[:, c0:c1] = xf @ w.T
    return y
