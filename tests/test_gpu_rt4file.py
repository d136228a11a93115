"""Weights loaded from an RT4 file written by the reference converter, uploaded
per tensor and as a whole file, drive the GEMV to the oracle's result."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
from test_gpu_decode import TIGHT, dev, host
from test_rt4file import convert, needs_convert, to_bf16_bits

pytestmark = [pytest.mark.gpu, needs_convert]


def test_uploaded_rt4_weights_match_oracle(rt4, orc, torch_gpu, tmp_path):
    from rt4_amd.rt4file import RT4File
    torch = torch_gpu
    rng = np.random.default_rng(9)
    shapes = {"model.language_model.layers.0.mlp.gate_proj.weight": (2048, 1024),
              "model.language_model.layers.0.mlp.down_proj.weight": (1024, 2048)}
    tensors = {n: ("BF16", s, to_bf16_bits(rng.standard_normal(s).astype(np.float32) * np.float32(0.03)).tobytes())
               for n, s in shapes.items()}
    _, man = convert(tmp_path, tensors)
    with RT4File(str(man)) as f:
        buf = f.upload_all()
        for name, (N, K) in shapes.items():
            print(f"case rt4 file {name} N={N} K={K}", flush=True)
            wq, ws = f.upload(name)
            q_h, s_h = f.host(name)
            info = f.info(name)
            wq2 = buf[info["q_off"]:info["q_off"] + info["q_bytes"]].view(torch.int32).view(N, K // 8)
            ws2 = buf[info["s_off"]:info["s_off"] + info["s_bytes"]].view(torch.int16).view(N, K // 128)
            x = rng.standard_normal((4, K)).astype(np.float16).astype(np.float32)
            y = rt4.gemv_w4a8(wq, ws, dev(torch, x))
            y2 = rt4.gemv_w4a8(wq2, ws2, dev(torch, x))
            torch.cuda.synchronize()
            assert np.array_equal(host(wq).view(np.uint32), q_h) and np.array_equal(host(ws).view(np.uint16), s_h)
            assert np.array_equal(host(y), host(y2))
            err = rel_l2(host(y), orc.gemv_w4a8(q_h, s_h, x))
            print(f"  rel_l2 = {err:.3e}")
            assert err < TIGHT


def test_bench_runs_on_an_rt4_file(tmp_path):
    """bench.py --rt4: the decode step on converter-written layers (two layers of a
    small MLP), graph replay equal to the eager result."""
    import json
    import pathlib
    import subprocess
    import sys
    rng = np.random.default_rng(10)
    tensors = {}
    for il in range(2):
        for k, s in (("gate", (2048, 512)), ("up", (2048, 512)), ("down", (512, 2048))):
            w = to_bf16_bits(rng.standard_normal(s).astype(np.float32) * np.float32(0.03))
            tensors[f"model.language_model.layers.{il}.mlp.{k}_proj.weight"] = ("BF16", s, w.tobytes())
    _, man = convert(tmp_path, tensors)
    root = pathlib.Path(__file__).resolve().parents[1]
    print("case bench --rt4", flush=True)
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--rt4", str(man), "--steps", "5", "--warmup", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["data"].startswith("RT4 file") and out["config"]["graph_matches_eager"] is True
    assert out["config"]["gate_up_NK"] == [2048, 512] and out["config"]["layers_rotated"] == 2
    assert out["value"] > 0
