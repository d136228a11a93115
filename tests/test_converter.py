"""The RT4 weight layout and weight quantizer against the reference's own writer.

The reference converter (tools/convert.c) is built from its source into
oracle/_ref/convert by oracle/Makefile (`make -C oracle ref`; it needs
/root/reference at build time).  These tests feed it a small BF16 safetensors
file and read its RT4 output through the manifest it writes
(tools/convert.c:546-560), which pins:
  * the nibble order of wq (docs/FORMAT.md:61-73) as the reader here decodes it
    (oracle rt4o_code, the layout every kernel of this library assumes);
  * the oracle's restatement of the converter's weight quantizer and of its own
    float->f16 rounding (rt4o_quant_weight_rows, rt4o_f32_to_f16_conv), bit for bit.
CPU only.
"""
from __future__ import annotations

import json
import struct
import subprocess

import numpy as np
import pytest

from conftest import REF_CONVERT

needs_convert = pytest.mark.skipif(not REF_CONVERT.exists(),
                                   reason="oracle/_ref/convert not built (needs /root/reference at build time)")

NAME = "model.layers.0.mlp.down_proj.weight"   # a 2-D BF16 tensor >= 1e6 elements -> int4 (convert.c:524-531)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def run_convert(tmp_path, w_bf16: np.ndarray):
    """Write one BF16 tensor as safetensors, run the reference converter, return
    (wq uint32 [N][K/8], ws uint16 [N][K/128]) read through its manifest."""
    N, K = w_bf16.shape
    data = np.ascontiguousarray(w_bf16, np.uint16).tobytes()
    header = json.dumps({NAME: {"dtype": "BF16", "shape": [N, K], "data_offsets": [0, len(data)]}}).encode()
    header += b" " * (-len(header) % 8)
    src = tmp_path / "in.safetensors"
    src.write_bytes(struct.pack("<Q", len(header)) + header + data)
    out = tmp_path / "out.rt4"
    subprocess.run([str(REF_CONVERT), str(src), str(out)], check=True, capture_output=True, timeout=120)
    man = json.loads((tmp_path / "out.rt4.json").read_text())
    (t,) = [t for t in man["tensors"] if t["name"] == NAME]
    assert t["kind"] == "i4" and t["shape"] == [N, K] and t["group"] == 128
    blob = out.read_bytes()
    q = np.frombuffer(blob, np.uint8, N * K // 2, t["q_off"]).copy().view(np.uint32).reshape(N, K // 8)
    s = np.frombuffer(blob, np.uint16, N * K // 128, t["s_off"]).reshape(N, K // 128)
    assert t["s_off"] % 256 == 0   # scales start 256-byte aligned (convert.c:368-371)
    return q, s


@needs_convert
def test_nibble_order_of_the_reference_writer(tmp_path, orc):
    """Weights that are exact multiples of 1/8 with a +-7 in every group quantize to
    known codes; the converter's packed bytes must decode to them."""
    rng = np.random.default_rng(1)
    N, K = 1024, 1024
    codes = rng.integers(-7, 8, size=(N, K))
    codes[:, ::128] = np.where(rng.random((N, K // 128)) < 0.5, 7, -7)   # amax = 7/8 per group
    w = to_bf16_bits(codes.astype(np.float32) / 8.0)
    q, s = run_convert(tmp_path, w)
    assert np.all(s == 0x3000)                         # f16(0.125)
    nib = (q[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF
    dec = np.where(nib >= 8, nib.astype(np.int64) - 16, nib.astype(np.int64)).reshape(N, K)
    np.testing.assert_array_equal(dec, codes)
    # the oracle's element reader agrees on a sample
    import ctypes
    L = orc.lib()
    L.rt4o_code.argtypes = [ctypes.c_void_p, ctypes.c_int]
    L.rt4o_code.restype = ctypes.c_int
    for n in (0, 17, 1023):
        row = np.ascontiguousarray(q[n])
        for k in (0, 1, 7, 8, 127, 128, 1023):
            assert L.rt4o_code(row.ctypes.data_as(ctypes.c_void_p), k) == codes[n, k]


@needs_convert
def test_oracle_weight_quantizer_matches_reference_converter(tmp_path, orc):
    rng = np.random.default_rng(2)
    N, K = 1024, 1152
    w = rng.standard_normal((N, K)).astype(np.float32) * 0.02
    w[3, 128:256] = 0.0                                  # an all-zero group -> s = 1, codes 0
    w[5, 7] = 0.9                                        # an outlier group
    w[9, :128] = np.linspace(-1, 1, 128)                 # many near-ties of roundf
    wb = to_bf16_bits(w)
    q_ref, s_ref = run_convert(tmp_path, wb)
    q, s = orc.quant_weight_rows(bf16_to_f32(wb).reshape(N, K))
    np.testing.assert_array_equal(s, s_ref)
    np.testing.assert_array_equal(q, q_ref)
    assert s[3, 1] == 0x3C00                             # f16(1.0)


def test_converter_f16_rounding(orc):
    """rt4o_f32_to_f16_conv: numpy's IEEE conversion wherever the discarded bits are not
    within one unit of a tie; exact ties round away from zero (convert.c:117)."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(20000) * 10.0 ** rng.uniform(-6, 4, 20000)).astype(np.float32)
    u = x.view(np.uint32)
    d = u & 0x1FFF
    normal = (np.abs(x) >= 2.0 ** -14) & (np.abs(x) < 65504)
    far = normal & (np.abs(d.astype(np.int64) - 0x1000) > 1)
    got = np.array([orc.f32_to_f16_conv(v) for v in x[far]], np.uint16)
    np.testing.assert_array_equal(got, x[far].astype(np.float16).view(np.uint16))
    # exact ties: 1 + 2^-11 lies halfway between f16 1.0 and 1.0009765625
    assert orc.f32_to_f16_conv(1.0 + 2.0 ** -11) == 0x3C01       # numpy (to even) gives 0x3C00
    assert orc.f32_to_f16_conv(-(1.0 + 2.0 ** -11)) == 0xBC01
    assert orc.f32_to_f16_conv(0.0) == 0 and orc.f32_to_f16_conv(1e9) == 0x7C00
