"""HBM traffic and instruction mix per launch from rocprofv3 counter runs.

`bench.py --pmc-probe` launches the dominant kernels of the benchmark eagerly
next to a plain copy kernel (rt4p_copy) of known size.  Two counter runs of it,

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir> -o fetch -- python3 bench.py --pmc-probe
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d <dir> -o write -- python3 bench.py --pmc-probe

give per-dispatch kilobyte counts.  `python -m rt4_amd.profiling <fetch.csv>
<write.csv> <out.json>` scales each counter by what it reads for the copy
(the copy moves exactly COPY_BYTES in and out), averages it per kernel and
writes the bytes per launch that bench.py reports as roofline.traffic.

Two further runs collect the shader counters of the same launches (at most 8
SQ counters per run):

    rocprofv3 --pmc SQ_WAVES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_VMEM SQ_INSTS_LDS SQ_INSTS_SALU \
        SQ_INSTS_SMEM SQ_INSTS_BRANCH --output-format csv -d <dir> -o sqa -- python3 bench.py --pmc-probe
    rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_ANY \
        SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE --output-format csv -d <dir> -o sqb \
        -- python3 bench.py --pmc-probe

`python -m rt4_amd.profiling trace <kernel_trace.csv>` prints the per (kernel,
launch grid) duration table of a `rocprofv3 --kernel-trace` run, and
`python -m rt4_amd.profiling sq <sqa.csv> <sqb.csv> <out.json>` writes the
mean per dispatch of every counter for each kernel of KERNELS, with the derived
fractions: MFMA busy (SQ_VALU_MFMA_BUSY_CYCLES, summed over the SIMDs, per SIMD
per cycle of the dispatch; GRBM_GUI_ACTIVE is summed over the XCDs, 32 CUs
each, so cycles = GRBM_GUI_ACTIVE / XCDs), VALU-active and waiting shares of the
wave cycles (SQ_ACTIVE_INST_VALU, SQ_WAIT_ANY over SQ_WAVE_CYCLES, all in
quad-cycles) and instructions per wave.
"""
from __future__ import annotations

import csv
import json
import statistics
import sys

COPY_BYTES = 256 << 20            # bytes read and written by each probe copy launch
COPY_KERNEL = "copy_k("          # the probe library's plain copy kernel
KERNELS = {                       # report key -> substring of the rocprof kernel name
    "gemv_gate_up": "gemv_w4a8_tl_k<4",
    "gemm_gate_up": "gemm_w4a8_k<false>",
    "attention_c4": "fa_int4_k",
}
SIMDS_PER_CU = 4
CUS_PER_XCD = 32


def per_kernel(path: str, counter: str) -> dict[str, list[float]]:
    """Counter values (KiB) per dispatch, grouped by full kernel name."""
    out: dict[str, list[float]] = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            out.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
    return out


def pick(table: dict[str, list[float]], needle: str) -> list[float]:
    vals: list[float] = []
    for name, v in table.items():
        if needle in name:
            vals.extend(v)
    return vals


def summarize(fetch_csv: str, write_csv: str) -> dict:
    res: dict = {"copy_bytes": COPY_BYTES}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        t = per_kernel(path, counter)
        copy = pick(t, COPY_KERNEL)
        if not copy:
            raise SystemExit(f"{path}: no {COPY_KERNEL} dispatch with {counter}")
        kib = statistics.median(copy)
        factor = COPY_BYTES / (kib * 1024.0)          # bytes per counted KiB-unit
        res[f"{counter}_copy_KiB"] = kib
        res[f"{counter}_scale"] = round(factor, 5)
        for key, needle in KERNELS.items():
            v = pick(t, needle)
            if v:
                d = res.setdefault(key, {"dispatches": len(v)})
                d[f"{counter}_KiB_mean"] = round(statistics.mean(v), 1)
                d[f"{counter.split('_')[0].lower()}_bytes"] = round(statistics.mean(v) * 1024.0 * factor)
    for key in KERNELS:
        d = res.get(key)
        if d and "fetch_bytes" in d and "write_bytes" in d:
            d["traffic_bytes"] = d["fetch_bytes"] + d["write_bytes"]
    return res


def all_counters(path: str) -> dict[str, dict[str, list[float]]]:
    """{counter: {kernel name: [value per dispatch]}} of a counter-collection CSV."""
    out: dict[str, dict[str, list[float]]] = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            out.setdefault(row["Counter_Name"], {}).setdefault(row["Kernel_Name"], []).append(
                float(row["Counter_Value"]))
    return out


def summarize_sq(paths: list[str], cus: int) -> dict:
    res: dict = {"cus": cus}
    tables = {}
    for path in paths:
        tables.update(all_counters(path))
    for key, needle in KERNELS.items():
        d: dict = {}
        for counter, t in sorted(tables.items()):
            v = pick(t, needle)
            if v:
                d[counter] = round(statistics.mean(v), 1)
                d.setdefault("dispatches", len(v))
        if not d:
            continue
        wc = d.get("SQ_WAVE_CYCLES")
        if d.get("SQ_VALU_MFMA_BUSY_CYCLES") is not None and d.get("GRBM_GUI_ACTIVE"):
            cycles = d["GRBM_GUI_ACTIVE"] / max(1, cus // CUS_PER_XCD)
            d["dispatch_cycles"] = round(cycles)
            d["mfma_busy_frac"] = round(d["SQ_VALU_MFMA_BUSY_CYCLES"] / (cycles * cus * SIMDS_PER_CU), 4)
        if wc:
            for c, name in (("SQ_ACTIVE_INST_VALU", "valu_active_frac"), ("SQ_WAIT_ANY", "wait_any_frac"),
                            ("SQ_WAIT_INST_ANY", "wait_inst_frac"), ("SQ_ACTIVE_INST_ANY", "issue_any_frac")):
                if d.get(c) is not None:
                    d[name] = round(d[c] / wc, 4)
        if d.get("SQ_WAVES"):
            for c in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_VMEM", "SQ_INSTS_LDS", "SQ_INSTS_SALU"):
                if d.get(c) is not None:
                    d[c.replace("SQ_INSTS_", "per_wave_").lower()] = round(d[c] / d["SQ_WAVES"], 1)
        res[key] = d
    return res


def kernel_table(path: str, needles: tuple[str, ...] = ("rt4::", "read_burst_k", "mfma_i8_k", COPY_KERNEL)) -> list[dict]:
    """Per (kernel, launch grid) duration statistics in microseconds from a rocprofv3
    kernel trace (`--kernel-trace --output-format csv`), for the kernels whose name
    contains one of `needles` (this library, the probes), ordered by total time."""
    groups: dict[tuple, list[float]] = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            name = row["Kernel_Name"]
            if not any(n in name for n in needles):
                continue
            wg = int(row["Workgroup_Size_X"])
            gx, gy = int(row["Grid_Size_X"]) // wg, int(row["Grid_Size_Y"]) // max(1, int(row["Workgroup_Size_Y"]))
            short = name.replace("(anonymous namespace)::", "").split("(")[0]
            short = short[5:] if short.startswith("void ") else short
            us = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1000.0
            groups.setdefault((short, gx, wg, gy), []).append(us)
    rows = []
    for (short, gx, wg, gy), v in groups.items():
        rows.append({"kernel": short, "grid": f"{gx} x {wg}" + (f" (y {gy})" if gy > 1 else ""), "calls": len(v),
                     "avg": statistics.fmean(v), "median": statistics.median(v), "min": min(v), "max": max(v),
                     "total": sum(v)})
    rows.sort(key=lambda r: -r["total"])
    return rows


def main(argv: list[str]) -> int:
    if len(argv) == 3 and argv[1] == "trace":
        print("| kernel | grid | calls | avg us | median us | min us | max us |")
        print("|---|---|---|---|---|---|---|")
        for r in kernel_table(argv[2]):
            print(f"| `{r['kernel']}` | {r['grid']} | {r['calls']} | {r['avg']:.2f} | {r['median']:.2f} | "
                  f"{r['min']:.2f} | {r['max']:.2f} |")
        return 0
    if len(argv) >= 2 and argv[1] == "sq":
        if len(argv) != 5:
            print(__doc__, file=sys.stderr)
            return 2
        import os
        cus = int(os.environ.get("RT4_CUS", "256"))
        res = summarize_sq(argv[2:4], cus)
        with open(argv[4], "w") as f:
            json.dump(res, f, indent=1)
            f.write("\n")
        print(json.dumps(res))
        return 0
    if len(argv) != 4:
        print(__doc__, file=sys.stderr)
        return 2
    res = summarize(argv[1], argv[2])
    with open(argv[3], "w") as f:
        json.dump(res, f, indent=1)
        f.write("\n")
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
