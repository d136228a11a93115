"""The measurement tooling on the CPU: the ceiling-probe library's exports and
argument checks (no device work), the counter summaries of rt4_amd.profiling on
synthetic rocprofv3 CSVs, and bench.py's one-GPU contract."""
from __future__ import annotations

import csv
import ctypes
import re
import subprocess
import sys

import pytest

from conftest import PKG_DIR, ROOT

PROBE_LIB = PKG_DIR / "rt4_amd" / "lib" / "librt4probe.so"


def _declared(header: str) -> set[str]:
    text = (ROOT / "include" / header).read_text()
    return set(re.findall(r"^int\s+(rt4p_\w+)\s*\(", text, flags=re.M))


def test_probe_library_exports_every_declared_symbol():
    from rt4_amd import probe
    assert PROBE_LIB.exists(), "built by __graft_entry__.build()"
    declared = _declared("rt4_probe.h")
    assert declared == set(probe.EXPORTS)
    L = ctypes.CDLL(str(PROBE_LIB))
    for name in declared:
        assert hasattr(L, name), name


def test_probe_argument_checks_return_before_any_launch():
    """Bad arguments return 1 without touching a device (none is present here)."""
    from rt4_amd import probe
    L = probe.lib()
    P = ctypes.c_void_p
    fake = P(0x10000)
    assert L.rt4p_read_burst(None, 4096, fake, 4, 256, 1, None) == 1          # null buffer
    assert L.rt4p_read_burst(fake, 4100, fake, 4, 256, 1, None) == 1          # not a multiple of 16
    assert L.rt4p_read_burst(fake, 4096, fake, 4, 96, 1, None) == 1           # threads not a multiple of 64
    assert L.rt4p_read_burst(fake, 4096, fake, 4, 2048, 1, None) == 1         # more than 1024 threads
    assert L.rt4p_read_burst(fake, 1 << 20, fake, 1, 64, 1, None) == 1        # 1024 loads per lane > 16
    assert L.rt4p_hbm_read(None, 4096, fake, 4, None) == 1
    assert L.rt4p_copy(fake, None, 4096, 4, None) == 1
    assert L.rt4p_mfma_i8(fake, 1, 0, 4, None) == 1
    assert L.rt4p_valu_fma(fake, 0, 4, None) == 1
    assert L.rt4p_mfma_f8_16x16(None, 4, 4, None) == 1
    assert L.rt4p_mfma_f8_16x16(fake, 0, 4, None) == 1


def _write_csv(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(("Kernel_Name", "Counter_Name", "Counter_Value"), r)))


def test_traffic_summary_scales_by_the_copy_calibration(tmp_path):
    from rt4_amd import profiling
    gemv = "void rt4::(anonymous namespace)::gemv_w4a8_tl_k<4, false>(...)"
    copy = "void (anonymous namespace)::copy_k(uint4*, uint4 const*, unsigned long)"
    kib = profiling.COPY_BYTES // 1024
    # the copy reads COPY_BYTES but FETCH_SIZE reports half of it: scale 2; WRITE_SIZE exact
    _write_csv(tmp_path / "f.csv", [(copy, "FETCH_SIZE", kib / 2), (copy, "FETCH_SIZE", kib / 2),
                                     (gemv, "FETCH_SIZE", 1000.0), (gemv, "FETCH_SIZE", 1200.0)])
    _write_csv(tmp_path / "w.csv", [(copy, "WRITE_SIZE", kib), (gemv, "WRITE_SIZE", 10.0)])
    res = profiling.summarize(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"))
    assert res["FETCH_SIZE_scale"] == pytest.approx(2.0)
    assert res["WRITE_SIZE_scale"] == pytest.approx(1.0)
    g = res["gemv_gate_up"]
    assert g["dispatches"] == 2
    assert g["fetch_bytes"] == 1100 * 1024 * 2 and g["write_bytes"] == 10 * 1024
    assert g["traffic_bytes"] == g["fetch_bytes"] + g["write_bytes"]


def test_traffic_and_sq_markdown_carry_the_json_numbers(tmp_path):
    """The markdown summaries are rendered from the same result dicts as the JSON."""
    from rt4_amd import profiling
    gemv = "void rt4::(anonymous namespace)::gemv_w4a8_tl_k<4, false>(...)"
    copy = "void (anonymous namespace)::copy_k(uint4*, uint4 const*, unsigned long)"
    kib = profiling.COPY_BYTES // 1024
    _write_csv(tmp_path / "f.csv", [(copy, "FETCH_SIZE", kib), (gemv, "FETCH_SIZE", 45_000.0)])
    _write_csv(tmp_path / "w.csv", [(copy, "WRITE_SIZE", kib), (gemv, "WRITE_SIZE", 300.0)])
    res = profiling.summarize(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"))
    md = profiling.traffic_md(res, "f.csv", "w.csv")
    g = res["gemv_gate_up"]
    assert g["algorithmic_bytes"] == 46_256_768
    assert f"{g['traffic_bytes']:,}" in md and f"{g['algorithmic_bytes']:,}" in md
    assert profiling.attention_bytes(1024, 33792, 24, 4)["total"] == 69_500_928
    rows = [(gemv, "SQ_WAVES", 100), (gemv, "SQ_INSTS_VALU", 100 * 50), (gemv, "SQ_INSTS_MFMA", 100 * 5)]
    _write_csv(tmp_path / "a.csv", rows)
    sq = profiling.summarize_sq([str(tmp_path / "a.csv")], 256)
    md = profiling.sq_md(sq, "a.csv", "b.csv")
    assert "| VALU per MFMA | 10.0 |" in md


def test_sq_summary_fractions(tmp_path):
    from rt4_amd import profiling
    gemm = "void rt4::(anonymous namespace)::gemm_w4a8_k<false>(...)"
    cus = 256                                   # 8 XCDs
    rows_a = [(gemm, "SQ_WAVES", 2048), (gemm, "SQ_INSTS_VALU", 2048 * 300), (gemm, "SQ_INSTS_MFMA", 2048 * 20)]
    rows_b = [(gemm, "GRBM_GUI_ACTIVE", 8 * 1000), (gemm, "SQ_VALU_MFMA_BUSY_CYCLES", cus * 4 * 1000 * 0.25),
              (gemm, "SQ_WAVE_CYCLES", 4000), (gemm, "SQ_WAIT_ANY", 1000), (gemm, "SQ_ACTIVE_INST_VALU", 2000)]
    _write_csv(tmp_path / "a.csv", rows_a)
    _write_csv(tmp_path / "b.csv", rows_b)
    d = profiling.summarize_sq([str(tmp_path / "a.csv"), str(tmp_path / "b.csv")], cus)["gemm_gate_up"]
    assert d["dispatch_cycles"] == 1000                       # GRBM_GUI_ACTIVE summed over the 8 XCDs
    assert d["mfma_busy_frac"] == pytest.approx(0.25)
    assert d["wait_any_frac"] == pytest.approx(0.25) and d["valu_active_frac"] == pytest.approx(0.5)
    assert d["per_wave_valu"] == 300 and d["per_wave_mfma"] == 20


def test_kernel_table_groups_by_kernel_and_grid(tmp_path):
    from rt4_amd import profiling
    cols = ["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Workgroup_Size_X", "Workgroup_Size_Y",
            "Grid_Size_X", "Grid_Size_Y"]
    gemv = "void rt4::(anonymous namespace)::gemv_w4a8_k<4, 2, 1, true, false, false, true>(unsigned int const*)"
    probe = "void (anonymous namespace)::read_burst_k<6, true>(uint4 const*, int)"
    other = "void at::native::vectorized_elementwise_kernel<4, at::native::float16_copy_kernel_cuda>(int)"
    rows = [(gemv, 0, 10_000, 256, 1, 1280 * 256, 1), (gemv, 0, 12_000, 256, 1, 1280 * 256, 1),
            (gemv, 0, 30_000, 1024, 1, 512 * 1024, 1),            # another launch grid: its own row
            (probe, 0, 8_000, 512, 1, 1024 * 512, 1), (other, 0, 99_000, 256, 1, 256, 1)]
    with open(tmp_path / "t.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(cols)
        for name, t0, t1, wg, wgy, gx, gy in rows:
            w.writerow(["KERNEL_DISPATCH", name, t0, t1, wg, wgy, gx, gy])
    tab = profiling.kernel_table(str(tmp_path / "t.csv"))
    assert [(r["kernel"], r["grid"], r["calls"]) for r in tab] == [
        ("rt4::gemv_w4a8_k<4, 2, 1, true, false, false, true>", "512 x 1024", 1),
        ("rt4::gemv_w4a8_k<4, 2, 1, true, false, false, true>", "1280 x 256", 2),
        ("read_burst_k<6, true>", "1024 x 512", 1)]          # torch's kernels are left out
    assert tab[1]["avg"] == pytest.approx(11.0) and tab[1]["min"] == pytest.approx(10.0)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
