"""The RT4 file loader (include/rt4k.h "RT4 files", csrc/rt4file.hip) against the
files the reference converter writes (tools/convert.c, built from its source in
oracle/_ref) and against hand-made manifests for the error paths.  CPU only; the
device upload is in tests/test_gpu_rt4file.py."""
from __future__ import annotations

import json
import struct
import subprocess

import numpy as np
import pytest

from conftest import REF_CONVERT
from rt4_amd import layout
from test_converter import bf16_to_f32, to_bf16_bits  # noqa: F401

needs_convert = pytest.mark.skipif(not REF_CONVERT.exists(),
                                   reason="oracle/_ref/convert not built (needs /root/reference at build time)")


def write_safetensors(path, tensors: dict):
    """tensors: name -> (dtype string, shape, raw bytes)."""
    header, blob = {}, b""
    for name, (dt, shape, raw) in tensors.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [len(blob), len(blob) + len(raw)]}
        blob += raw
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    path.write_bytes(struct.pack("<Q", len(h)) + h + blob)


def convert(tmp_path, tensors):
    src = tmp_path / "in.safetensors"
    write_safetensors(src, tensors)
    out = tmp_path / "model.rt4"
    subprocess.run([str(REF_CONVERT), str(src), str(out)], check=True, capture_output=True, timeout=120)
    return out, tmp_path / "model.rt4.json"


@needs_convert
def test_loader_reads_the_reference_converter_output(tmp_path, orc):
    rng = np.random.default_rng(3)
    N1, K1 = 1024, 1024               # >= 1e6 elements: int4 (convert.c:524-531)
    N2, K2 = 2048, 640
    w1 = to_bf16_bits(rng.standard_normal((N1, K1)).astype(np.float32) * np.float32(0.02))
    w2 = to_bf16_bits(rng.standard_normal((N2, K2)).astype(np.float32) * np.float32(0.05))
    nrm = rng.standard_normal(K1).astype(np.float32)
    out, man = convert(tmp_path, {
        "model.language_model.layers.0.mlp.down_proj.weight": ("BF16", (N1, K1), w1.tobytes()),
        "model.language_model.layers.0.mlp.up_proj.weight": ("BF16", (N2, K2), w2.tobytes()),
        "model.language_model.norm.weight": ("F32", (K1,), nrm.tobytes()),
    })
    from rt4_amd.rt4file import RT4File
    manifest = json.loads(man.read_text())
    blob = out.read_bytes()
    with RT4File(str(man)) as f:
        assert len(f) == len(manifest["tensors"])
        assert f.names() == [t["name"] for t in manifest["tensors"]]
        assert f.size() == len(blob)
        for t in manifest["tensors"]:
            info = f.info(t["name"])
            assert info["kind"] == t["kind"] and info["shape"] == t["shape"] and info["q_off"] == t["q_off"]
            assert abs(info["relerr"] - t["relerr"]) < 1e-5
        for name, (N, K), w in (("model.language_model.layers.0.mlp.down_proj.weight", (N1, K1), w1),
                                ("model.language_model.layers.0.mlp.up_proj.weight", (N2, K2), w2)):
            info = f.info(name)
            assert info["kind"] == "i4" and info["group"] == 128 and info["s_off"] % 256 == 0
            q, s = f.host(name)
            assert q.shape == (N, K // 8) and s.shape == (N, K // 128)
            want_q = np.frombuffer(blob, np.uint8, N * K // 2, info["q_off"]).view(np.uint32).reshape(N, K // 8)
            want_s = np.frombuffer(blob, np.uint16, N * K // 128, info["s_off"]).reshape(N, K // 128)
            assert np.array_equal(q, want_q) and np.array_equal(s, want_s)
            # the oracle's restatement of the converter's quantizer yields the same bytes
            wq_o, ws_o = orc.quant_weight_rows(bf16_to_f32(w))
            assert np.array_equal(q, wq_o) and np.array_equal(s, ws_o)
        raw, none = f.host("model.language_model.norm.weight")
        assert none is None and np.array_equal(raw.view(np.float32), nrm)


def _manual(tmp_path, tensors, weight=b"", weight_name="w.bin", extra=None):
    (tmp_path / weight_name).write_bytes(weight)
    man = {"format": "RT4-v1", "group": 128, "weight_file": weight_name, "tensors": tensors}
    if extra:
        man.update(extra)
    p = tmp_path / "m.json"
    p.write_text(json.dumps(man))
    return p


def test_loader_resolves_relative_weight_file_and_reads_regions(tmp_path, monkeypatch):
    from rt4_amd.rt4file import RT4File
    rng = np.random.default_rng(4)
    N, K = 16, 256
    codes = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    q = layout.pack_rt4(codes).tobytes()
    s = (np.abs(rng.standard_normal((N, K // 128))) * 0.01 + 1e-3).astype(np.float16).view(np.uint16)
    pad = b"\0" * (-len(q) % 256)
    blob = q + pad + s.tobytes()
    p = _manual(tmp_path, [{"name": "w", "kind": "i4", "shape": [N, K], "group": 128, "q_off": 0,
                            "s_off": len(q) + len(pad), "nbytes": len(q), "relerr": 0.1, "src_rms": 0.02}], blob)
    monkeypatch.chdir("/")                       # "w.bin" is found next to the manifest
    with RT4File(str(p)) as f:
        qq, ss = f.host("w")
        assert np.array_equal(layout.unpack_rt4(qq), codes) and np.array_equal(ss, s)


@pytest.mark.parametrize("case,match", [
    ("outside", "outside"), ("misaligned", "256-byte"), ("bad_json", "not JSON"), ("no_weight", "cannot open weight"),
    ("bad_shape", "shape/group"), ("unknown_format", "unknown format")])
def test_loader_rejects_bad_files(tmp_path, rt4, case, match):
    from rt4_amd.rt4file import RT4File
    N, K = 16, 256
    ok = {"name": "w", "kind": "i4", "shape": [N, K], "group": 128, "q_off": 0, "s_off": 2048, "nbytes": 2048}
    blob = b"\0" * (2048 + N * 2 * 2)
    if case == "outside":
        p = _manual(tmp_path, [dict(ok, s_off=4096)], blob)
    elif case == "misaligned":
        p = _manual(tmp_path, [dict(ok, s_off=2048 + 16)], blob + b"\0" * 64)
    elif case == "bad_json":
        p = tmp_path / "m.json"
        p.write_text('{"tensors": [ {"name": "w", ')
    elif case == "no_weight":
        p = _manual(tmp_path, [ok], blob)
        (tmp_path / "w.bin").unlink()
    elif case == "bad_shape":
        p = _manual(tmp_path, [dict(ok, shape=[N, 200])], blob)
    else:
        p = _manual(tmp_path, [ok], blob, extra={"format": "RT5"})
    with pytest.raises(rt4.RT4Error, match=match):
        RT4File(str(p))
