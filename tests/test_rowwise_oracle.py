"""The per-row (G = K) quantizer mode of the numpy oracle, pinned on the CPU.

The per-row mode has no counterpart in the reference (which quantizes per (row,
128-group)), so nothing of the reference's can be compared with it.  It is the
reference's formula with one group per row, and two checks pin that restatement:
  * brute force on small inputs, element by element in plain Python
    (s = max|x| / D, q = round-half-even(x / s) clamped, s = 1 for a zero row);
  * on rows whose every 128-group reaches the row's max-abs, per-row and
    per-group quantization are the same computation, so their codes and scales
    must agree bit for bit with the per-group oracle that the reference pins.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import np_ref


def _brute(x, D, hi):
    rows, K = x.shape
    q = np.zeros((rows, K), np.int8)
    s = np.zeros(rows, np.float32)
    for m in range(rows):
        amax = np.float32(0)
        for k in range(K):
            amax = max(amax, np.float32(abs(x[m, k])))
        sm = np.float32(amax / np.float32(D)) if amax > 0 else np.float32(1)
        s[m] = sm
        for k in range(K):
            v = float(np.float32(x[m, k]) / sm)          # one fp32 rounding, as the kernel's quotient
            q[m, k] = max(-128, min(hi, int(np.rint(v))))
    return q, s


@pytest.mark.parametrize("rows,K", [(1, 128), (3, 256), (2, 640)])
def test_rowwise_brute_force(rows, K):
    rng = np.random.default_rng(rows * 1000 + K)
    x = (rng.standard_normal((rows, K)) * np.exp2(rng.integers(-6, 6, (rows, 1)))).astype(np.float32)
    x[0, : K // 2] = 0.0
    if rows > 2:
        x[2] = 0.0                                       # an all-zero row: s = 1, codes 0
    q, s, asu = np_ref.quant_act(x, G=K)
    qb, sb = _brute(x, 127, 127)
    assert np.array_equal(q, qb) and np.array_equal(s[:, 0], sb)
    assert np.array_equal(asu, q.reshape(rows, K // 128, 128).astype(np.int32).sum(axis=2))
    q8, s8 = np_ref.quant_rows_i8(x, G=K)
    q8b, s8b = _brute(x, 119, 119)
    assert np.array_equal(q8, q8b) and np.array_equal(s8[:, 0], s8b)


def test_rowwise_equals_per_group_when_every_group_reaches_the_row_max():
    rng = np.random.default_rng(5)
    rows, K = 4, 1024
    x = rng.standard_normal((rows, K)).astype(np.float32)
    top = np.abs(x).max(axis=1) * np.float32(1.5)
    for m in range(rows):
        for g in range(K // 128):
            x[m, 128 * g + rng.integers(0, 128)] = top[m] * (1 if g % 2 else -1)
    q_r, s_r, a_r = np_ref.quant_act(x, G=K)
    q_g, s_g, a_g = np_ref.quant_act(x)
    assert np.array_equal(q_r, q_g) and np.array_equal(a_r, a_g)
    assert np.array_equal(np.repeat(s_r, K // 128, axis=1), s_g)
    q8_r, s8_r = np_ref.quant_rows_i8(x, G=K)
    q8_g, s8_g = np_ref.quant_rows_i8(x)
    assert np.array_equal(q8_r, q8_g) and np.array_equal(np.repeat(s8_r, K // 128, axis=1), s8_g)
