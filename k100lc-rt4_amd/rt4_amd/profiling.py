"""HBM traffic, instruction mix and kernel durations from rocprofv3 runs, written
as the JSON and markdown summaries kept under profiles/.

`bench.py --pmc-probe` launches the kernels of KERNELS eagerly next to a plain
copy kernel (rt4p_copy) of known size.  Two counter runs of it,

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir> -o fetch -- python3 bench.py --pmc-probe
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d <dir> -o write -- python3 bench.py --pmc-probe

give per-dispatch kilobyte counts;

    python -m rt4_amd.profiling traffic <fetch.csv> <write.csv> <out.json> <out.md>

scales each counter by what it reads for the copy (which moves exactly
COPY_BYTES in and out), averages it per kernel and writes the bytes per launch
(bench.py reports the dominant kernel's as roofline.traffic) next to each
kernel's algorithmic bytes, both files from the same two runs.

Two further runs collect the shader counters of the same launches (at most 8
SQ counters per run):

    rocprofv3 --pmc SQ_WAVES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_VMEM SQ_INSTS_LDS SQ_INSTS_SALU \
        SQ_INSTS_SMEM SQ_INSTS_BRANCH --output-format csv -d <dir> -o sqa -- python3 bench.py --pmc-probe
    rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_ANY \
        SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE --output-format csv -d <dir> -o sqb \
        -- python3 bench.py --pmc-probe
    python -m rt4_amd.profiling sq <sqa.csv> <sqb.csv> <out.json> <out.md>

writes the mean per dispatch of every counter for each kernel of KERNELS, with
the derived fractions: MFMA busy (SQ_VALU_MFMA_BUSY_CYCLES, summed over the
SIMDs, per SIMD per cycle of the dispatch; GRBM_GUI_ACTIVE is summed over the
XCDs, 32 CUs each, so cycles = GRBM_GUI_ACTIVE / XCDs), VALU-active and waiting
shares of the wave cycles (SQ_ACTIVE_INST_VALU, SQ_WAIT_ANY over SQ_WAVE_CYCLES,
all in quad-cycles) and instructions per wave.

    python -m rt4_amd.profiling trace <kernel_trace.csv> [--last N] [<out.md> <title> <command>]

prints (or writes, under a title and the command that made the trace) the per
(kernel, launch grid) duration table of a `rocprofv3 --kernel-trace` run, with
--last N over the last N dispatches of each (kernel, grid) only.
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
    "gemv_c0": "gemv_w4a8_dot_k<2, 5",
    "gemm_gate_up": "gemm_w4a8_k<false>",
    "attention_c4": "fa_int4_k",
    "attention_c4_staging": "fa_expand_kv_k",
}
LABELS = {
    "gemv_gate_up": "gate/up GEMV (M=4, K=5120, N=17408)",
    "gemv_c0": "C0 GEMV (M=1, K=5120, N=5120)",
    "gemm_gate_up": "gate/up prefill GEMM (M=1024, K=5120, N=17408)",
    "attention_c4": "C4 attention (1024 queries over 33792 keys, 24/4 heads, D=256)",
    "attention_c4_staging": "C4 attention K/V staging pass (once per call)",
}


def gemv_bytes(M: int, N: int, K: int) -> int:
    """GEMV on quantized activations: int4 weights, fp16 scales, int8 activations
    and their fp32 group scales read once, fp32 output written once."""
    NG = K // 128
    return N * K // 2 + N * NG * 2 + M * K + M * NG * 4 + M * N * 4


def gemm_bytes(M: int, N: int, K: int) -> int:
    """Prefill GEMM (int8 entry): int8 activations, int4 weights, fp32 group-major
    weight scales and activation scales read once, fp32 C written once."""
    NG = K // 128
    return M * K + N * K // 2 + N * NG * 4 + M * NG * 4 + M * N * 4


def attention_bytes(n_q: int, n_kv: int, H: int, KVH: int, D: int = 256) -> dict:
    """int4-KV attention prefill: int8 Q codes and their per-(row, 128-group) scales,
    the int4 K and V caches with their scales (K per (token, 128 dims), V per (64-token
    tile, dim)), read once, and the fp32 output written once."""
    parts = {"q_codes": n_q * H * D, "q_scales": n_q * H * (D // 128) * 4,
             "k_codes": KVH * n_kv * D // 2, "k_scales": KVH * (D // 128) * n_kv * 4,
             "v_codes": KVH * n_kv * D // 2, "v_scales": KVH * (n_kv // 64) * D * 4,
             "output": n_q * H * D * 4}
    parts["total"] = sum(parts.values())
    return parts


def attention_staging_bytes(n_kv: int, KVH: int, D: int = 256) -> int:
    """The prefill's K/V staging pass: the int4 K and V codes read once and their
    staged operand bytes (16 KB per 64-key tile each for K and V) written once."""
    n_tile = (n_kv + 63) // 64
    return 2 * KVH * n_kv * D // 2 + 2 * KVH * n_tile * 16384


ALGO_BYTES = {
    "gemv_gate_up": gemv_bytes(4, 17408, 5120),
    "gemv_c0": gemv_bytes(1, 5120, 5120),
    "gemm_gate_up": gemm_bytes(1024, 17408, 5120),
    "attention_c4": attention_bytes(1024, 32768 + 1024, 24, 4)["total"],
    "attention_c4_staging": attention_staging_bytes(32768 + 1024, 4),
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
            d["algorithmic_bytes"] = ALGO_BYTES[key]
            d["traffic_over_algorithmic"] = round(d["traffic_bytes"] / ALGO_BYTES[key], 3)
    return res


def traffic_md(res: dict, fetch_csv: str, write_csv: str) -> str:
    """The markdown summary of summarize()'s result (the same numbers as the JSON)."""
    out = ["# HBM traffic per launch (rocprofv3 FETCH_SIZE / WRITE_SIZE)", "",
           "Commands (repository root, one MI355X), one counter per run, then this summary:", "", "```",
           "export TMPDIR=/tmp",
           "rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/pmcf -o fetch -- python3 bench.py --pmc-probe",
           "rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/pmcw -o write -- python3 bench.py --pmc-probe",
           "cd k100lc-rt4_amd && python3 -m rt4_amd.profiling traffic " + fetch_csv + " \\",
           "    " + write_csv + " ../profiles/traffic.json ../profiles/traffic.md", "```", "",
           "`bench.py --pmc-probe` launches, eagerly: the gate/up GEMV over 16 distinct weight sets twice, the",
           "C0 GEMV over 16 weight sets twice, the gate/up prefill GEMM 3 times, the C4 attention prefill 3",
           "times, and a plain copy of " + f"{COPY_BYTES:,}" + " bytes (`rt4p_copy`) 4 times.  Calibration: for the copy,",
           f"FETCH_SIZE reads {res['FETCH_SIZE_copy_KiB']:,.0f} KiB and WRITE_SIZE {res['WRITE_SIZE_copy_KiB']:,.0f} "
           f"KiB per dispatch against {COPY_BYTES // 1024:,} KiB moved each way, so",
           f"FETCH_SIZE is scaled by {res['FETCH_SIZE_scale']:.4f} and WRITE_SIZE by {res['WRITE_SIZE_scale']:.4f} "
           "(bytes per counted KiB / 1024).", "",
           "| kernel | dispatches | fetch bytes | write bytes | traffic | algorithmic bytes | traffic / algorithmic |",
           "|---|---|---|---|---|---|---|"]
    for key in KERNELS:
        d = res.get(key)
        if not d or "traffic_bytes" not in d:
            continue
        out.append(f"| {LABELS[key]} `{KERNELS[key]}...` | {d['dispatches']} | {d['fetch_bytes']:,} | "
                   f"{d['write_bytes']:,} | {d['traffic_bytes']:,} | {d['algorithmic_bytes']:,} | "
                   f"{d['traffic_over_algorithmic']:.3f} |")
    ab = attention_bytes(1024, 32768 + 1024, 24, 4)
    out += ["", "Algorithmic bytes are each operand read once and each output written once "
            "(`rt4_amd.profiling.gemv_bytes`, `gemm_bytes`, `attention_bytes`); for the attention: " +
            ", ".join(f"{k.replace('_', ' ')} {v:,}" for k, v in ab.items() if k != "total") + "."]
    return "\n".join(out) + "\n"


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


SQ_ROWS = (
    ("waves per dispatch", lambda x: f"{x['SQ_WAVES']:,.0f}"),
    ("dispatch cycles (GRBM_GUI_ACTIVE / XCDs)", lambda x: f"{x['dispatch_cycles']:,.0f}"),
    ("VALU instructions per wave", lambda x: f"{x['per_wave_valu']:,.1f}"),
    ("MFMA instructions per wave", lambda x: f"{x['per_wave_mfma']:,.1f}"),
    ("LDS instructions per wave", lambda x: f"{x['per_wave_lds']:,.1f}"),
    ("VMEM instructions per wave", lambda x: f"{x['per_wave_vmem']:,.1f}"),
    ("SALU instructions per wave", lambda x: f"{x['per_wave_salu']:,.1f}"),
    ("VALU per MFMA", lambda x: f"{x['per_wave_valu'] / x['per_wave_mfma']:.1f}" if x.get('per_wave_mfma') else "-"),
    ("MFMA busy (per SIMD, of dispatch cycles)", lambda x: f"{100 * x['mfma_busy_frac']:.1f}%"),
    ("VALU active (of wave cycles)", lambda x: f"{100 * x['valu_active_frac']:.1f}%"),
    ("any instruction issued (of wave cycles)", lambda x: f"{100 * x['issue_any_frac']:.1f}%"),
    ("waiting on anything (of wave cycles)", lambda x: f"{100 * x['wait_any_frac']:.1f}%"),
    ("waiting on an instruction dependency (of wave cycles)", lambda x: f"{100 * x['wait_inst_frac']:.1f}%"),
)


def sq_md(res: dict, sqa_csv: str, sqb_csv: str) -> str:
    """The markdown summary of summarize_sq()'s result (the same numbers as the JSON)."""
    keys = [k for k in KERNELS if k in res]
    out = ["# Shader (SQ) counters per launch", "",
           "Commands (repository root, one MI355X), at most 8 SQ counters per run, then this summary:", "", "```",
           "export TMPDIR=/tmp",
           "rocprofv3 --pmc SQ_WAVES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_VMEM SQ_INSTS_LDS SQ_INSTS_SALU SQ_INSTS_SMEM \\",
           "    SQ_INSTS_BRANCH --output-format csv -d gpurun_out/pmcsa -o sqa -- python3 bench.py --pmc-probe",
           "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_ANY SQ_WAVE_CYCLES \\",
           "    SQ_WAIT_ANY SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE --output-format csv -d gpurun_out/pmcsb -o sqb -- python3 bench.py --pmc-probe",
           "cd k100lc-rt4_amd && python3 -m rt4_amd.profiling sq " + sqa_csv + " \\",
           "    " + sqb_csv + " ../profiles/sq_counters.json ../profiles/sq_counters.md", "```", "",
           "Means per dispatch over the eager launches of `bench.py --pmc-probe` (dispatch counts: " +
           ", ".join(f"{LABELS[k].split(' (')[0]} {res[k].get('dispatches', 0)}" for k in keys) + ").",
           "Wave-cycle shares use SQ_WAVE_CYCLES, SQ_ACTIVE_INST_* and SQ_WAIT_* (quad-cycles summed over waves);",
           f"MFMA busy is SQ_VALU_MFMA_BUSY_CYCLES over {res['cus'] * SIMDS_PER_CU} SIMDs, per SIMD per dispatch cycle "
           "(an eager dispatch includes its start and drain).", "",
           "| | " + " | ".join(LABELS[k] for k in keys) + " |", "|---|" + "---|" * len(keys)]
    for name, fn in SQ_ROWS:
        cells = []
        for k in keys:
            try:
                cells.append(fn(res[k]))
            except (KeyError, ZeroDivisionError, TypeError):
                cells.append("-")
        out.append(f"| {name} | " + " | ".join(cells) + " |")
    return "\n".join(out) + "\n"


def trace_md(rows: list[dict]) -> str:
    out = ["| kernel | grid | calls | avg us | median us | min us | max us |", "|---|---|---|---|---|---|---|"]
    for r in rows:
        out.append(f"| `{r['kernel']}` | {r['grid']} | {r['calls']} | {r['avg']:.2f} | {r['median']:.2f} | "
                   f"{r['min']:.2f} | {r['max']:.2f} |")
    return "\n".join(out) + "\n"


def kernel_table(path: str, needles: tuple[str, ...] = ("rt4::", "read_burst_k", "mfma_i8_k", COPY_KERNEL),
                 last: int = 0) -> list[dict]:
    """Per (kernel, launch grid) duration statistics in microseconds from a rocprofv3
    kernel trace (`--kernel-trace --output-format csv`), for the kernels whose name
    contains one of `needles` (this library, the probes), ordered by total time; with
    `last` > 0 only the last `last` dispatches of each (kernel, grid) count."""
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
            groups.setdefault((short, gx, wg, gy), []).append((int(row["Start_Timestamp"]), us))
    rows = []
    for key, v in groups.items():          # dispatch order; with `last`, only the last dispatches
        v.sort()
        groups[key] = [us for _, us in (v[-last:] if last > 0 else v)]
    for (short, gx, wg, gy), v in groups.items():
        rows.append({"kernel": short, "grid": f"{gx} x {wg}" + (f" (y {gy})" if gy > 1 else ""), "calls": len(v),
                     "avg": statistics.fmean(v), "median": statistics.median(v), "min": min(v), "max": max(v),
                     "total": sum(v)})
    rows.sort(key=lambda r: -r["total"])
    return rows


def _dump(res: dict, path: str) -> None:
    with open(path, "w") as f:
        json.dump(res, f, indent=1)
        f.write("\n")


def main(argv: list[str]) -> int:
    if len(argv) >= 3 and argv[1] == "trace":
        args = argv[2:]
        last = 0
        if len(args) >= 3 and args[1] == "--last":
            last = int(args[2])
            args = args[:1] + args[3:]
        if len(args) not in (1, 4):
            print(__doc__, file=sys.stderr)
            return 2
        table = trace_md(kernel_table(args[0], last=last))
        if len(args) == 1:
            print(table, end="")
            return 0
        sel = f" --last {last}" if last else ""
        which = (f"the last {last} dispatches of each kernel and grid" if last else "every dispatch")
        with open(args[1], "w") as f:
            f.write(f"# {args[2]}\n\nCommand (repository root, one MI355X), then this summary:\n\n```\n"
                    f"export TMPDIR=/tmp\n{args[3]}\n"
                    f"cd k100lc-rt4_amd && python3 -m rt4_amd.profiling trace {args[0]}{sel} {args[1]} \\\n"
                    f"    '<the title above>' '<the rocprofv3 command above>'\n```\n\n"
                    f"Kernels of this library and of the ceiling probes, split by launch grid (workgroups x threads;\n"
                    f"y when the grid has one), ordered by total time, over {which}; durations in microseconds.\n\n"
                    f"{table}")
        return 0
    if len(argv) == 6 and argv[1] == "sq":
        import os
        cus = int(os.environ.get("RT4_CUS", "256"))
        res = summarize_sq(argv[2:4], cus)
        _dump(res, argv[4])
        with open(argv[5], "w") as f:
            f.write(sq_md(res, argv[2], argv[3]))
        print(json.dumps(res))
        return 0
    if len(argv) == 6 and argv[1] == "traffic":
        res = summarize(argv[2], argv[3])
        _dump(res, argv[4])
        with open(argv[5], "w") as f:
            f.write(traffic_md(res, argv[2], argv[3]))
        print(json.dumps(res))
        return 0
    print(__doc__, file=sys.stderr)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv))
