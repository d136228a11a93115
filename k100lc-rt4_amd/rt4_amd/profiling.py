"""HBM traffic per launch from rocprofv3 counter runs.

`bench.py --pmc-probe` launches the dominant kernels of the benchmark eagerly
next to a plain copy kernel (rt4p_copy) of known size.  Two counter runs of it,

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir> -o fetch -- python3 bench.py --pmc-probe
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d <dir> -o write -- python3 bench.py --pmc-probe

give per-dispatch kilobyte counts.  `python -m rt4_amd.profiling <fetch.csv>
<write.csv> <out.json>` scales each counter by what it reads for the copy
(the copy moves exactly COPY_BYTES in and out), averages it per kernel and
writes the bytes per launch that bench.py reports as roofline.traffic.
"""
from __future__ import annotations

import csv
import json
import statistics
import sys

COPY_BYTES = 256 << 20            # bytes read and written by each probe copy launch
COPY_KERNEL = "copy_k("          # the probe library's plain copy kernel
KERNELS = {                       # report key -> substring of the rocprof kernel name
    "gemv_gate_up": "gemv_w4a8_k<4",
    "gemm_gate_up": "gemm_w4a8_k<false>",
}


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


def main(argv: list[str]) -> int:
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
