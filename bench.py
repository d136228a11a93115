#!/usr/bin/env python3
"""bench.py -- the RT4 quantized-matmul hot path on one MI355X.

Workload (the configuration the metric is quoted on):
one decode MLP step at the MTP3 verify width M=4 on 27B layer shapes, i.e. the
three linears of one layer through the drop-in k_gemv_w4a8 entry (activation
quantize + W4A8 GEMV each): gate and up (K=5120, N=17408) and down (K=17408,
N=5120).  Consecutive steps walk through `--layers` distinct layers of random
RT4 weights (1.1 GB at the default 8), as the runtime walks its layers, so
weights stream from HBM rather than from the 256 MB MALL.  Inputs are resident
in HBM before timing; steps are replayed from a HIP graph (no host launch
overhead inside the timed region).

value = algorithmic bytes of a step / time per step (GB/s), where the bytes of
one linear are int4 weights + fp16 scales + fp32 activations + fp32 output
(46,317,568 B for gate/up, 46,222,336 B for down).

Also printed in the same JSON line:
  roofline      the dominant kernel (the gate/up GEMV launch), timed live with
                HIP events over a graph of back-to-back launches
  kernels       the same figure for the other kernels of the path
  cpu_baseline  the reference's CPU path (numpy RT4 dequant + matmul, restated
                in oracle/np_ref.py) on a bounded sample of the same workload
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import platform
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "k100lc-rt4_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X published HBM3E bandwidth
I8_PEAK_TOPS = 5000.0          # MI355X published dense int8 MFMA


def linear_bytes(M: int, N: int, K: int) -> int:
    """Algorithmic HBM bytes of one drop-in W4A8 linear: weights, their scales, the
    fp32 activations read once and the fp32 output written once."""
    NG = K // 128
    return N * K // 2 + N * NG * 2 + M * K * 4 + M * N * 4


def gemv_kernel_bytes(M: int, N: int, K: int) -> int:
    """Algorithmic HBM bytes of one GEMV launch on quantized activations: weights,
    their scales, int8 activations and their scales, fp32 output."""
    NG = K // 128
    return N * K // 2 + N * NG * 2 + M * K + M * NG * 4 + M * N * 4


# --only keys: (kernel, shape) pairs launched alone for per-shape profiler rows
ONLY = {
    "gemm_c2_gate_up": "int8 GEMM, M=1024 N=17408 K=5120",
    "gemm_c2_down": "int8 GEMM, M=1024 N=5120 K=17408",
    "gemm_ref_m2048": "int8 GEMM, M=2048 N=17408 K=5120",
    "gemm_dropin_c2_gate_up": "drop-in digit-plane GEMM entry, M=1024 N=17408 K=5120",
    "attn_c4": "FlashAttention prefill, 1024 queries over 32768 cached tokens",
    "attn_ref_131k": "FlashAttention prefill, 1024 queries over 131072 cached tokens",
    "gemv_gate_up_m4": "GEMV on quantized activations, M=4 N=17408 K=5120, 16 weight sets",
    "gemv_c0_m1": "GEMV on quantized activations, M=1 N=5120 K=5120, 16 weight sets",
}


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=8, help="distinct weight sets rotated through")
    ap.add_argument("--rt4", metavar="MANIFEST", default=None,
                    help="decode step on the MLP weights of an RT4 file (converter manifest) instead of "
                         "synthetic ones; the kernel table and CPU baseline are skipped")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the per-kernel table beyond the roofline")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="only launch the dominant kernels (gate/up and C0 GEMV, gate/up GEMM, C4 attention) and "
                         "a calibration copy, eagerly (for rocprofv3 --pmc)")
    ap.add_argument("--only", choices=sorted(ONLY), default=None,
                    help="only launch one kernel at one shape: --steps launches in a graph, replayed for 300 ms, "
                         "then timed once; prints their mean time (one rocprofv3 row per shape)")
    return ap.parse_args()


def timed_graph(torch, fn, reps: int = 5, warm_ms: float = 50.0) -> float:
    """Capture fn() in a HIP graph, replay it, return ms per replay (median of reps).
    Replays for at least warm_ms first: the GPU clock needs tens of milliseconds of
    load to settle, and a cold first measurement reads ~10% slow."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    t0 = time.perf_counter()
    while True:
        g.replay()
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= warm_ms:
            break
    times = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b))
    return statistics.median(times)


def cpu_info() -> dict:
    model = platform.processor()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    lscpu = None
    try:
        import subprocess
        r = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10)
        for line in r.stdout.splitlines():
            if line.startswith("Model name:"):
                lscpu = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    return {"cpu": model, "lscpu_model": lscpu, "os_cpu_count": os.cpu_count(),
            "affinity": len(os.sched_getaffinity(0))}


def cpu_baseline(step_bytes: int, seconds: float) -> dict:
    """The reference's CPU path (tools/rt4_io.py:40-52 dequant, then a float matmul,
    tools/ref_full.py:113-117) on the GPU box's host cores, output rows split over
    the cores with one BLAS thread each.  The decode MLP step is the reported value
    (dequant + matmul per call, as the tools do); `extra` adds the same step with
    the weights dequantised beforehand (matmul only), a row block of the C2 prefill
    GEMM and a row block of the C3 LM head, each the median of at least 5 timed
    repetitions after one warm-up."""
    import concurrent.futures as cf

    import numpy as np
    import threadpoolctl

    from oracle import np_ref

    rng = np.random.default_rng(0)
    threads = max(1, min(16, len(os.sched_getaffinity(0))))

    def mat(N, K):
        wq = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint32).view(np.uint8).reshape(N, K // 2)
        ws = (np.abs(rng.standard_normal((N, K // 128))) * 0.01 + 1e-3).astype(np.float16).view(np.uint16)
        return wq, ws

    def acts(M, K):
        x = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
        return np_ref.fake_quant_act(x)

    def split(pool, fn, N, *args):
        bounds = np.linspace(0, N, threads + 1).astype(int)
        futs = [pool.submit(fn, a, b, *args) for a, b in zip(bounds[:-1], bounds[1:]) if b > a]
        return [f.result() for f in futs]

    def dq_mm(a, b, wq, ws, xf):           # (i) dequant + matmul of output rows [a, b)
        return np_ref.cpu_linear(wq[a:b], ws[a:b], xf)

    def mm(a, b, w, xf):                    # (ii) matmul only
        return xf @ w[a:b].T

    def timed(fn, min_reps=5, budget=seconds):
        fn()                                # warm-up
        ts, t_start = [], time.perf_counter()
        while len(ts) < min_reps or (time.perf_counter() - t_start < budget and len(ts) < 20):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts), len(ts)

    M = 4
    shapes = [(17408, 5120), (17408, 5120), (5120, 17408)]
    mats = [mat(N, K) for N, K in shapes]
    xs = [acts(M, K) for _, K in shapes]
    out = {}
    with threadpoolctl.threadpool_limits(1), cf.ThreadPoolExecutor(threads) as pool:
        t_step, n_step = timed(lambda: [split(pool, dq_mm, wq.shape[0], wq, ws, xf)
                                        for (wq, ws), xf in zip(mats, xs)], budget=seconds)
        ws32 = [np_ref.dequant(wq, ws) for wq, ws in mats]
        t_mm, n_mm = timed(lambda: [split(pool, mm, w.shape[0], w, xf) for w, xf in zip(ws32, xs)], budget=2.0)
        out["decode_step_matmul_only"] = {"value": round(step_bytes / t_mm / 1e9, 3), "unit": "GB/s",
                                          "ms_per_step": round(t_mm * 1e3, 2), "reps": n_mm,
                                          "sample": "the same step, weights dequantised to fp32 beforehand"}
        del ws32
        # C2 prefill GEMM: M=1024 tokens, a block of 2048 of the 17408 gate/up rows
        Mp, Nb, Kp = 1024, 2048, 5120
        wq, ws = mat(Nb, Kp)
        xp = rng.standard_normal((Mp, Kp)).astype(np.float32)
        t_g, n_g = timed(lambda: split(pool, dq_mm, Nb, wq, ws, xp), budget=2.0)
        w32 = np_ref.dequant(wq, ws)
        t_gm, n_gm = timed(lambda: split(pool, mm, Nb, w32, xp), budget=2.0)
        ops = 2.0 * Mp * Nb * Kp
        out["prefill_gemm_c2_block"] = {
            "TOPS": round(ops / t_g / 1e12, 4), "TOPS_matmul_only": round(ops / t_gm / 1e12, 4),
            "us": round(t_g * 1e6, 1), "us_matmul_only": round(t_gm * 1e6, 1),
            "us_full_N_extrapolated": round(t_g * 1e6 * 17408 / Nb, 1), "reps": [n_g, n_gm],
            "sample": f"M={Mp}, K={Kp}, rows 0..{Nb} of N=17408 (dequant + matmul; and matmul only)"}
        del w32, xp
        # C3 LM head: M=4, K=5120, a block of 32768 of the 248320 rows, chunked by 8192
        Nl = 32768
        wq, ws = mat(Nl, 5120)
        xf = acts(M, 5120)
        t_l, n_l = timed(lambda: split(pool, dq_mm, Nl, wq, ws, xf), budget=2.0)
        lb = Nl * 5120 // 2 + Nl * 40 * 2 + M * 5120 * 4 + M * Nl * 4
        out["lm_head_c3_block"] = {"value": round(lb / t_l / 1e9, 3), "unit": "GB/s", "us": round(t_l * 1e6, 1),
                                   "us_full_N_extrapolated": round(t_l * 1e6 * 248320 / Nl, 1), "reps": n_l,
                                   "sample": f"M=4, K=5120, rows 0..{Nl} of N=248320 (dequant + matmul)"}
    try:
        blas = np.show_config(mode="dicts")["Build Dependencies"]["blas"]["name"]
    except Exception:  # noqa: BLE001
        blas = "unknown"
    return {"value": round(step_bytes / t_step / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "ms_per_step": round(t_step * 1e3, 2),
            "sample": f"{n_step} decode MLP steps (gate+up+down, M=4, 27B shapes), numpy RT4 dequant + "
                      f"matmul split over {threads} threads (1 BLAS thread each), median step",
            "blas": blas, **cpu_info(), "extra": out}


class GemmCase:
    """Device operands of one prefill GEMM shape: random RT4 weights in group-major
    scale order, outlier activations quantized for the int8 entry, the drop-in digit
    planes and the W4A4 codes."""

    def __init__(self, torch, rt4_amd, workload, gen, M, N, K):
        self.M, self.N, self.K = M, N, K
        self.wq, ws = workload.weights_torch(N, K, generator=gen)
        self.sb = rt4_amd.make_group_major(ws, K)
        self.x = x = workload.acts_torch(M, K, outliers=True, generator=gen)
        self.xq, self.sc = rt4_amd.quant_rows_i8(x)
        self.qh, self.ql, self.sc_, self.sc16 = rt4_amd.quant_rows_a8(x)
        self.aq4, self.sc4 = rt4_amd.quant_rows_a4(x)
        self.c = torch.empty((M, N), device="cuda")
        self.c2 = torch.empty((M, N), device="cuda")

    def int8(self, rt4_amd):
        rt4_amd.gemm_w4a8_i8(self.wq, self.sb, self.xq, self.sc, out=self.c)

    def dropin(self, rt4_amd):
        rt4_amd.gemm_w4a8(self.wq, self.sb, self.qh, self.ql, self.sc_, self.sc16, out=self.c, c2=self.c2)

    def w4a4(self, rt4_amd):
        rt4_amd.gemm_w4a4(self.wq, self.sb, self.aq4, self.sc4, out=self.c)

    def quant(self, rt4_amd):
        rt4_amd.quant_rows_a8(self.x)


def gemm_entry(torch, rt4_amd, g: GemmCase, w4a4: bool = True) -> dict:
    """int8-MFMA TOPS = 2*M*N*K / kernel time (GEMM launch only, graph-replayed), plus
    the whole drop-in k_gemm_i4_a8 call (digit recombination + GEMM) and the drop-in
    linear's activation quantizer k_quant_rows_a8 at this shape."""
    reps = 10
    runs = [("us", g.int8), ("dropin_us", g.dropin)] + ([("w4a4_dropin_us", g.w4a4)] if w4a4 else [])
    runs.append(("quant_rows_a8_us", g.quant))
    for _, f in runs:                                          # eager first calls: kernel attributes
        f(rt4_amd)
    torch.cuda.synchronize()
    res = {}
    for key, f in runs:
        res[key] = round(timed_graph(torch, lambda: [f(rt4_amd) for _ in range(reps)]) * 1e3 / reps, 2)
    ops = 2 * g.M * g.N * g.K
    res["TOPS"] = round(ops / res["us"] / 1e6, 1)
    res["frac_i8_peak"] = round(ops / res["us"] / 1e6 / I8_PEAK_TOPS, 4)
    return res


def gemm_table(torch, rt4_amd, workload, gen) -> dict:
    """Prefill GEMM: BASELINE configs[2] (M=1024 tokens, gate/up and down shapes) and
    the reference's own benchmark shape (M=2048 tokens, gate/up)."""
    out = {}
    shapes = [(f"gemm_{n}", s, True) for n, s in workload.GEMM_SHAPES.items()]
    shapes.append(("gemm_ref_m2048", workload.GEMM_REF_SHAPE, False))
    for key, (M, N, K), w4a4 in shapes:
        g = GemmCase(torch, rt4_amd, workload, gen, M, N, K)
        out[key] = gemm_entry(torch, rt4_amd, g, w4a4)
        if key == "gemm_ref_m2048":
            out[key]["shape"] = [M, N, K]
        del g
        torch.cuda.empty_cache()
    return out


def rt4_layers(rt4_amd, manifest: str, max_layers: int):
    """The MLP projections of up to max_layers layers of an RT4 file, uploaded for the
    kernels: ([{"gate", "up", "down"} -> (wq, ws)], (N, K) of gate/up, (N, K) of down)."""
    from rt4_amd.rt4file import RT4File
    f = RT4File(manifest)
    names = set(f.names())
    layers, shapes = [], None
    i = 0
    while len(layers) < max_layers:
        pre = next((p for p in (f"model.language_model.layers.{i}.mlp.", f"model.layers.{i}.mlp.")
                    if p + "gate_proj.weight" in names), None)
        if pre is None:
            if i > 4096:
                break
            i += 1
            continue
        lw = {k: f.upload(pre + f"{k}_proj.weight") for k in ("gate", "up", "down")}
        s = (tuple(f.info(pre + "gate_proj.weight")["shape"]), tuple(f.info(pre + "down_proj.weight")["shape"]))
        if shapes is None:
            shapes = s
        if s == shapes:
            layers.append(lw)
        i += 1
    f.close()
    if not layers:
        raise SystemExit(f"bench.py: no layer with mlp.gate_proj/up_proj/down_proj in {manifest}")
    return layers, shapes[0], shapes[1]


class AttnCase:
    """A filled int4 KV cache and quantized queries for one attention shape: n_q new
    queries at positions ctx..ctx+n_q-1 over n_kv = ctx + n_q cached tokens."""

    def __init__(self, torch, rt4_amd, workload, gen, cfg):
        n_q, ctx, H, KVH, D = cfg["n_q"], cfg["ctx"], cfg["H"], cfg["KVH"], cfg["D"]
        self.n_q, self.ctx, self.H, self.D, self.ratio = n_q, ctx, H, D, H // KVH
        self.n_kv = n_kv = ctx + n_q
        self.q, k, v = workload.attn_torch(n_q, n_kv, H, KVH, D, generator=gen)
        self.qq, self.qs = rt4_amd.attn_q_quant(self.q, n_q)
        self.kc = torch.zeros((KVH, n_kv, D // 8), dtype=torch.int32, device="cuda")
        self.ksc = torch.ones((KVH, D // 128, n_kv), device="cuda")
        self.vc = torch.zeros((KVH, n_kv // 8, D), dtype=torch.int32, device="cuda")
        self.vsc = torch.ones((KVH, n_kv // 64, D), device="cuda")
        self.stage = torch.zeros((KVH, 64, D), device="cuda")
        rt4_amd.kv_append_k(self.kc, self.ksc, k, 0)
        rt4_amd.kv_append_v(self.vc, self.vsc, self.stage, v, 0)
        self.k_new, self.v_new = k[ctx:].contiguous(), v[ctx:].contiguous()
        del k, v
        self.out = None

    def fa(self, rt4_amd):
        self.out = rt4_amd.attention_prefill(self.qq, self.qs, self.kc, self.ksc, self.vc, self.vsc, n_kv=self.n_kv,
                                             off=self.ctx, ratio=self.ratio, out=self.out)

    def feed(self, rt4_amd):
        rt4_amd.attn_q_quant(self.q, self.n_q, qq=self.qq, qs=self.qs)
        rt4_amd.kv_append_k(self.kc, self.ksc, self.k_new, self.ctx)
        rt4_amd.kv_append_v(self.vc, self.vsc, self.stage, self.v_new, self.ctx)

    def ops(self) -> int:
        """Two contractions of 2*D operations per visible (query, key) pair per head."""
        return sum(self.ctx + i + 1 for i in range(self.n_q)) * 2 * 2 * self.D * self.H


def attn_table(torch, rt4_amd, workload, gen) -> dict:
    """int4-KV FlashAttention prefill, 24 query heads over 4 KV heads, head dim 256,
    causal: BASELINE configs[4] (1024 new queries over a 32768-token cache) and the
    reference's own benchmark shape (over 131072 cached tokens).  Effective int8-MFMA
    TOPS counts the two contractions over the keys each query sees; at C4 also the Q
    quantizer and the K/V cache append of the 1024 new tokens."""
    res = {}
    for key, cfg, reps in (("attn_c4_prefill", workload.ATTN_C4, 3), ("attn_ref_131k_prefill", workload.ATTN_REF, 1)):
        a = AttnCase(torch, rt4_amd, workload, gen, cfg)
        a.fa(rt4_amd)
        torch.cuda.synchronize()
        us = timed_graph(torch, lambda: [a.fa(rt4_amd) for _ in range(reps)]) * 1e3 / reps
        ops = a.ops()
        res[key] = {"us": round(us, 1), "TOPS_effective": round(ops / us / 1e6, 1),
                    "frac_i8_peak": round(ops / us / 1e6 / I8_PEAK_TOPS, 4)}
        if key == "attn_c4_prefill":
            res[key]["feeders_us"] = round(timed_graph(torch, lambda: a.feed(rt4_amd)) * 1e3, 2)
        else:
            res[key]["n_q_ctx"] = [a.n_q, a.ctx]
        del a
        torch.cuda.empty_cache()
    return res


def pattern_entry(pat: dict, nbytes: int, kernel_us: float) -> dict:
    """The GEMV's own memory requests without its compute (rt4p_gemv_loads): time per
    launch, the rate at which it moves the GEMV's algorithmic bytes, and the GEMV's
    time over it (the share of the GEMV that its load pattern accounts for)."""
    return {"us": pat["us"], "GBs": round(nbytes / pat["us"] / 1e3, 1),
            "frac": round(pat["us"] / kernel_us, 4),
            "probe": ("rt4p_gemv_loads: the GEMV's grid and load form (" +
                      (f"one-row dot-product form, 2 rows per wave, {pat['waves']} waves per workgroup"
                       if pat["groups_per_wave"] == 0 else
                       f"{pat['groups_per_wave']} groups/wave, {pat['waves']} waves, {pat['k_splits']} K pieces per "
                       f"leftover tile") + "), weight/scale/activation loads only, same weight sets back to back in a "
                      "graph")}


def load_traffic(key: str):
    """Bytes per launch of `key` measured by the FETCH_SIZE / WRITE_SIZE counter runs
    (rt4_amd.profiling), or None when that summary is absent."""
    try:
        d = json.loads((ROOT / "profiles" / "traffic.json").read_text())[key]
        return int(d["traffic_bytes"])
    except (OSError, KeyError, ValueError, TypeError):
        return None


def pmc_probe(torch, rt4_amd, workload, gen) -> int:
    """Eager launches for counter collection: the gate/up GEMV over 16 distinct weight
    sets (twice), the C0 GEMV over 16 weight sets (twice), the gate/up prefill GEMM 3
    times, the C4 attention prefill 3 times, and 4 copies of COPY_BYTES."""
    import ctypes

    from rt4_amd import probe, profiling
    M, (N, K) = 4, (17408, 5120)
    mats = [workload.weights_torch(N, K, generator=gen) for _ in range(16)]
    x = workload.acts_torch(M, K, generator=gen)
    y = torch.empty((M, N), device="cuda")
    xq, sa = rt4_amd.quant_act_a8(x)
    for _ in range(2):
        for wq, ws in mats:
            rt4_amd.gemv_w4a8_q(wq, ws, xq, sa, out=y)
    # C0: one activation row over 5120 x 5120 slices of the same weight sets
    xq1, sa1 = rt4_amd.quant_act_a8(workload.acts_torch(1, K, generator=gen))
    y1 = torch.empty((1, 5120), device="cuda")
    for _ in range(2):
        for wq, ws in mats:
            rt4_amd.gemv_w4a8_q(wq[:5120], ws[:5120], xq1, sa1, out=y1)
    del mats
    g = GemmCase(torch, rt4_amd, workload, gen, *workload.GEMM_SHAPES["c2_gate_up"])
    for _ in range(3):
        g.int8(rt4_amd)
    del g
    a = AttnCase(torch, rt4_amd, workload, gen, workload.ATTN_C4)
    for _ in range(3):
        a.fa(rt4_amd)
    del a
    nb = profiling.COPY_BYTES
    src = torch.empty(nb // 4, dtype=torch.int32, device="cuda").random_()
    dst = torch.empty_like(src)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for _ in range(4):
        rc = probe.lib().rt4p_copy(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()), nb, cus * 8, st)
        if rc:
            raise RuntimeError(f"rt4p_copy failed ({rc})")
    torch.cuda.synchronize()
    print("pmc probe done", flush=True)
    return 0


def only_one(torch, rt4_amd, workload, gen, key: str, launches: int) -> int:
    """One kernel at one shape (--only), as bench.py times it: `launches` calls
    captured in a HIP graph, replayed for 300 ms (clocks settle), then replayed once
    more between two events; prints one JSON line.  In a kernel trace of this, the
    last `launches` dispatches are the counted ones."""
    if key.startswith("gemm_"):
        shape = {"gemm_c2_gate_up": workload.GEMM_SHAPES["c2_gate_up"], "gemm_c2_down": workload.GEMM_SHAPES["c2_down"],
                 "gemm_ref_m2048": workload.GEMM_REF_SHAPE,
                 "gemm_dropin_c2_gate_up": workload.GEMM_SHAPES["c2_gate_up"]}[key]
        c = GemmCase(torch, rt4_amd, workload, gen, *shape)
        one = (lambda i: c.dropin(rt4_amd)) if "dropin" in key else (lambda i: c.int8(rt4_amd))
    elif key.startswith("attn_"):
        c = AttnCase(torch, rt4_amd, workload, gen, workload.ATTN_C4 if key == "attn_c4" else workload.ATTN_REF)
        one = lambda i: c.fa(rt4_amd)  # noqa: E731
    else:
        M, N, K = (4, 17408, 5120) if key == "gemv_gate_up_m4" else (1, 5120, 5120)
        mats = [workload.weights_torch(N, K, generator=gen) for _ in range(16)]
        xq, sa = rt4_amd.quant_act_a8(workload.acts_torch(M, K, generator=gen))
        y = torch.empty((M, N), device="cuda")
        one = lambda i: rt4_amd.gemv_w4a8_q(*mats[i % 16], xq, sa, out=y)  # noqa: E731
    one(0)                                   # eager first call: kernel attributes, workspaces
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(launches):
            one(i)
    t_end = time.perf_counter() + 0.3
    while time.perf_counter() < t_end:
        g.replay()
        torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    g.replay()
    t1.record()
    torch.cuda.synchronize()
    print(json.dumps({"only": key, "what": ONLY[key], "launches": launches,
                      "us_per_launch": round(t0.elapsed_time(t1) * 1e3 / launches, 2)}), flush=True)
    return 0


def main() -> int:
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (--gpus 1); multi-GPU scaling is not part "
              "of it (the path would shard weight rows across GPUs with no exchange).", file=sys.stderr)
        return 2

    import torch

    import rt4_amd
    from rt4_amd import workload

    metric = json.loads((ROOT / "BASELINE.json").read_text())["metric"]
    torch.cuda.set_device(0)
    gen = torch.Generator(device="cuda").manual_seed(0)
    if args.pmc_probe:
        return pmc_probe(torch, rt4_amd, workload, gen)
    if args.only:
        return only_one(torch, rt4_amd, workload, gen, args.only, max(1, args.steps))
    M = 4
    (Ngu, Kgu), (Nd, Kd) = (17408, 5120), (5120, 17408)
    L = max(1, args.layers)
    layers = []
    rt4_source = None
    if args.rt4:
        layers, (Ngu, Kgu), (Nd, Kd) = rt4_layers(rt4_amd, args.rt4, L)
        L = len(layers)
        rt4_source = args.rt4
        args.no_extra = args.no_cpu = True
    for _ in range(L if not layers else 0):
        layers.append({k: workload.weights_torch(N, K, generator=gen)
                       for k, (N, K) in (("gate", (Ngu, Kgu)), ("up", (Ngu, Kgu)), ("down", (Nd, Kd)))})
    x_gu = workload.acts_torch(M, Kgu, generator=gen)
    x_d = workload.acts_torch(M, Kd, generator=gen)
    y_g = torch.empty((M, Ngu), device="cuda")
    y_u = torch.empty((M, Ngu), device="cuda")
    y_d = torch.empty((M, Nd), device="cuda")

    def step(i):
        lw = layers[i % L]
        rt4_amd.gemv_w4a8(*lw["gate"], x_gu, out=y_g)
        rt4_amd.gemv_w4a8(*lw["up"], x_gu, out=y_u)
        rt4_amd.gemv_w4a8(*lw["down"], x_d, out=y_d)

    for i in range(L):                 # eager pass: grows scratch, sets kernel attributes
        step(i)
    torch.cuda.synchronize()

    K_steps, W_steps = max(1, args.steps), max(0, args.warmup)
    g_timed = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_timed):
        for i in range(K_steps):
            step(i)
    if W_steps:
        g_warm = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_warm):
            for i in range(W_steps):
                step(i)
        g_warm.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    g_timed.replay()
    t1.record()
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / K_steps
    # the last timed step used layer (K-1) % L; the replay must reproduce the eager result
    graph_out = y_d.clone()
    step((K_steps - 1) % L)
    torch.cuda.synchronize()
    graph_ok = bool(torch.equal(graph_out, y_d))

    step_bytes = 2 * linear_bytes(M, Ngu, Kgu) + linear_bytes(M, Nd, Kd)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # ---- dominant kernel: the gate/up GEMV launch, back to back over all layers
    xq_gu, sa_gu = rt4_amd.quant_act_a8(x_gu)
    gu_mats = [lw[k] for lw in layers for k in ("gate", "up")]

    def gemv_gu():
        for wq, ws in gu_mats:
            rt4_amd.gemv_w4a8_q(wq, ws, xq_gu, sa_gu, out=y_g)

    gu_us = timed_graph(torch, gemv_gu) * 1e3 / len(gu_mats)
    gu_bytes = gemv_kernel_bytes(M, Ngu, Kgu)
    achieved = gu_bytes / (gu_us * 1e-6) / 1e9
    plan = rt4_amd.gemv_launch_plan(M, Ngu, Kgu)
    g_, w_, rb_ = plan["groups_per_wave"], plan["waves"], plan["row_blocks"]
    if g_ == 4 and rb_ == 1 and Kgu % 512 == 0 and w_ <= 8:
        kname = f"rt4::gemv_w4a8_tl_k<{M},false>"        # the row-transposed form
    else:
        # line-wise activation loads: one row block and their LDS slices within 64 KB (the launcher's rule)
        al = rb_ == 1 and w_ * 16 * g_ * 2 + w_ * M * 16 * 4 + w_ * M * g_ * 8 * 16 <= 65536
        # scales hoisted out of the chunk loop: 2 groups per wave, even K/128, 3-8 chunks per wave, <= 4 waves
        ng_gu = Kgu // 128
        per_wave = -(-(-(-ng_gu // g_)) // w_)
        hs = al and g_ == 2 and ng_gu % 2 == 0 and w_ <= 4 and 3 <= per_wave <= 8
        kname = f"rt4::gemv_w4a8_k<{M},{g_},{rb_},{str(al).lower()},false,false,{str(hs).lower()}>"
    # measured ceiling: the fastest single launch that reads the same byte count
    from rt4_amd import probe
    ceil_gu = probe.read_ceiling(torch, gu_bytes, timed_graph=timed_graph)
    roofline = {"kernel": f"{kname} (gate/up GEMV, M={M} K={Kgu} N={Ngu}, {g_} groups/wave, "
                          f"{plan['waves']} waves/tile, {plan['k_splits']} K pieces/leftover tile)",
                "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": load_traffic("gemv_gate_up"),
                "us_per_launch": round(gu_us, 3), "bytes_per_launch": gu_bytes,
                "weight_only_GBs": round((Ngu * Kgu // 2) / (gu_us * 1e-6) / 1e9, 1),
                "measured_peak": {"value": ceil_gu["GBs"], "unit": "GB/s", "us": ceil_gu["us"],
                                  "frac": round(achieved / ceil_gu["GBs"], 4),
                                  "probe": f"one-pass read of the same {gu_bytes} bytes (rt4p_read_burst, "
                                           f"{ceil_gu['blocks']}x{ceil_gu['threads']}, non-temporal), 16 buffers "
                                           f"back to back in a graph"}}
    pat_gu = probe.gemv_load_pattern(torch, rt4_amd, gu_mats, xq_gu, sa_gu, M, timed_graph)
    if pat_gu:
        roofline["load_pattern"] = pattern_entry(pat_gu, gu_bytes, gu_us)

    kernels = {}
    if not args.no_extra:
        d_mats = [lw["down"] for lw in layers]

        xq_d, sa_d = rt4_amd.quant_act_a8(x_d)
        aq_gu, sa4_gu = rt4_amd.quant_act_a4(x_gu)

        def gemv4_gu():
            for wq, ws in gu_mats:
                rt4_amd.gemv_w4a4_q(wq, ws, aq_gu, sa4_gu, out=y_g)

        g4_us = timed_graph(torch, gemv4_gu) * 1e3 / len(gu_mats)
        g4_bytes = Ngu * Kgu // 2 + Ngu * (Kgu // 128) * 2 + M * Kgu // 2 + M * (Kgu // 32) * 4 + M * Ngu * 4
        kernels["gemv_w4a4_gate_up_m4"] = {"us": round(g4_us, 3), "GBs": round(g4_bytes / g4_us / 1e3, 1)}

        def gemv_d():
            for wq, ws in d_mats:
                rt4_amd.gemv_w4a8_q(wq, ws, xq_d, sa_d, out=y_d)

        d_us = timed_graph(torch, gemv_d) * 1e3 / len(d_mats)
        d_bytes = gemv_kernel_bytes(M, Nd, Kd)
        ceil_d = probe.read_ceiling(torch, d_bytes, timed_graph=timed_graph)
        kernels["gemv_down_m4"] = {"us": round(d_us, 3), "GBs": round(d_bytes / d_us / 1e3, 1),
                                   "measured_peak_GBs": ceil_d["GBs"],
                                   "frac_measured": round(d_bytes / d_us / 1e3 / ceil_d["GBs"], 4)}
        pat_d = probe.gemv_load_pattern(torch, rt4_amd, d_mats, xq_d, sa_d, M, timed_graph)
        if pat_d:
            kernels["gemv_down_m4"]["load_pattern"] = pattern_entry(pat_d, d_bytes, d_us)

        def gemv_gu_fused():   # its own best measured config: 4 groups per wave, 8 waves
            for wq, ws in gu_mats:
                rt4_amd.gemv_w4a8(wq, ws, x_gu, out=y_g, groups_per_wave=4, waves=8)

        f_gu_us = timed_graph(torch, gemv_gu_fused) * 1e3 / len(gu_mats)
        kernels["gemv_gate_up_m4_fused_quant"] = {"us": round(f_gu_us, 3)}

        def quant_gu():
            for _ in range(16):
                rt4_amd.quant_act_a8(x_gu)

        q_us = timed_graph(torch, quant_gu) * 1e3 / 16
        kernels["quant_act_m4_k5120"] = {"us": round(q_us, 3)}
        # M=1 decode (C0 shape 5120x5120) over 16 rotated slices of the gate weights
        xq1, sa1 = rt4_amd.quant_act_a8(x_gu[:1].contiguous())
        c0_mats = [(wq[:5120], ws[:5120]) for wq, ws in gu_mats]
        y1 = torch.empty((1, 5120), device="cuda")

        def gemv_c0():
            for wq, ws in c0_mats:
                rt4_amd.gemv_w4a8_q(wq, ws, xq1, sa1, out=y1)

        c0_us = timed_graph(torch, gemv_c0) * 1e3 / len(c0_mats)
        c0_bytes = gemv_kernel_bytes(1, 5120, 5120)
        ceil_c0 = probe.read_ceiling(torch, c0_bytes, timed_graph=timed_graph)
        kernels["gemv_c0_m1"] = {"us": round(c0_us, 3), "GBs": round(c0_bytes / c0_us / 1e3, 1),
                                 "measured_peak_GBs": ceil_c0["GBs"], "measured_peak_us": ceil_c0["us"],
                                 "frac_measured": round(c0_bytes / c0_us / 1e3 / ceil_c0["GBs"], 4)}
        pat_c0 = probe.gemv_load_pattern(torch, rt4_amd, c0_mats, xq1, sa1, 1, timed_graph)
        if pat_c0:
            kernels["gemv_c0_m1"]["load_pattern"] = pattern_entry(pat_c0, c0_bytes, c0_us)
        kernels["ceilings"] = {"mfma_i32_16x16x64_i8_TOPS": probe.mfma_i8_rate(torch),
                               "mfma_i32_32x32x32_i8_TOPS": probe.mfma_i8_rate(torch, big=True),
                               "mfma_f32_16x16x128_fp8_TOPS": probe.mfma_f8_16x16_rate(torch),
                               **probe.mfma_f8f6f4_rates(torch),
                               "gemm_unit_skeleton": probe.gemm_unit_cycles(torch),
                               "graph_node_us": probe.launch_cost(torch, timed_graph),
                               "gemv_load_pattern_us": {k: v["load_pattern"]["us"] for k, v in
                                                        (("gemv_gate_up_m4", roofline), ("gemv_down_m4",
                                                         kernels["gemv_down_m4"]), ("gemv_c0_m1", kernels["gemv_c0_m1"]))
                                                        if "load_pattern" in v},
                               "published_i8_TOPS": I8_PEAK_TOPS, "published_hbm_GBs": HBM_PEAK_GBS}
        # LM head (C3): M=4, K=5120, N=248320, two 0.66 GB copies alternated
        del layers, gu_mats, d_mats, c0_mats
        torch.cuda.empty_cache()
        kernels.update(gemm_table(torch, rt4_amd, workload, gen))
        kernels.update(attn_table(torch, rt4_amd, workload, gen))
        # the same figures against the MFMA rate measured on this box for the instruction
        # each kernel runs (the GEMM int8 32x32x32, the attention FP8 16x16x128)
        for key, rate in (("gemm_c2_gate_up", "mfma_i32_32x32x32_i8_TOPS"),
                          ("gemm_c2_down", "mfma_i32_32x32x32_i8_TOPS"),
                          ("gemm_ref_m2048", "mfma_i32_32x32x32_i8_TOPS"),
                          ("attn_c4_prefill", "mfma_f32_16x16x128_fp8_TOPS"),
                          ("attn_ref_131k_prefill", "mfma_f32_16x16x128_fp8_TOPS")):
            tops = kernels[key].get("TOPS", kernels[key].get("TOPS_effective"))
            kernels[key]["frac_measured_issue"] = round(tops / kernels["ceilings"][rate], 4)
        lm = [workload.weights_torch(248320, 5120, generator=gen) for _ in range(2)]
        y_lm = torch.empty((M, 248320), device="cuda")

        def gemv_lm():
            for wq, ws in lm:
                rt4_amd.gemv_w4a8_q(wq, ws, xq_gu, sa_gu, out=y_lm)

        lm_us = timed_graph(torch, gemv_lm) * 1e3 / len(lm)
        lm_bytes = gemv_kernel_bytes(M, 248320, 5120)
        kernels["gemv_lm_head_m4"] = {"us": round(lm_us, 3), "GBs": round(lm_bytes / lm_us / 1e3, 1)}
        del lm
        torch.cuda.empty_cache()
        # its one-pass read ceiling: the same byte count through rt4p_hbm_read
        pk = probe.hbm_read_ceiling(torch, lm_bytes, timed_graph)
        kernels["gemv_lm_head_m4"].update({"measured_peak_us": pk["us"], "measured_peak_GBs": pk["GBs"],
                                           "frac_measured": round(pk["us"] / lm_us, 4)})

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(step_bytes, args.cpu_seconds)

    out = {
        "metric": metric, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": K_steps,
        "warmup": W_steps, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int4*int8->int32",
        "data": "synthetic" if rt4_source is None else f"RT4 file {rt4_source} (activations synthetic)",
        "config": {"workload": "decode MLP step, MTP3 verify width (BASELINE configs[1])", "M": M,
                   "gate_up_NK": [Ngu, Kgu], "down_NK": [Nd, Kd], "linears_per_step": 3,
                   "layers_rotated": L, "step_bytes": step_bytes, "graph_matches_eager": graph_ok,
                   "device": torch.cuda.get_device_name(0)},
        "roofline": roofline, "kernels": kernels, "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
