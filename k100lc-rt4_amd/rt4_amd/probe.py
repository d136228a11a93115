"""ctypes binding of librt4probe.so: gfx950 ceilings (HBM read, copy, int8 MFMA,
fp32 FMA issue rates) measured next to the published MI355X peaks."""
from __future__ import annotations

import ctypes
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().parent / "lib" / "librt4probe.so"
EXPORTS = ("rt4p_hbm_read", "rt4p_read_burst", "rt4p_copy", "rt4p_mfma_i8", "rt4p_valu_fma", "rt4p_gemv_loads",
           "rt4p_empty", "rt4p_mfma_f8f6f4", "rt4p_mfma_f8_16x16", "rt4p_gemm_unit")
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        try:
            import torch  # noqa: F401  (bind to the HIP runtime torch loaded, as rt4_amd.lib does)
        except ImportError:
            pass
        L = ctypes.CDLL(str(LIB_PATH))
        P, I, Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        sigs = {"rt4p_hbm_read": [P, Z, P, I, P], "rt4p_read_burst": [P, Z, P, I, I, I, P],
                "rt4p_copy": [P, P, Z, I, P],
                "rt4p_mfma_i8": [P, I, I, I, P], "rt4p_valu_fma": [P, I, I, P],
                "rt4p_gemv_loads": [P, P, P, P, P, I, I, I, I, I, I, I, P], "rt4p_empty": [I, I, P],
                "rt4p_mfma_f8f6f4": [P, I, I, I, P], "rt4p_mfma_f8_16x16": [P, I, I, P],
                "rt4p_gemm_unit": [P, I, I, I, P]}
        for name, args in sigs.items():
            getattr(L, name).argtypes = args
            getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def _timed(torch, launch, reps: int = 5) -> float:
    """Median milliseconds of `launch()` over reps, events on torch's current stream."""
    launch()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        launch()
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b))
    ts.sort()
    return ts[len(ts) // 2]


def measure(torch, gib: float = 2.0) -> dict:
    """Measured ceilings: HBM read and copy GB/s, int8 MFMA TOPS, fp32 FMA TFLOP/s."""
    L = lib()
    dev = torch.cuda.current_device()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nbytes = int(gib * 2**30) // 16 * 16
    buf = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").random_()
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    out = {"cus": cus}
    blocks = cus * 8
    ms = _timed(torch, lambda: L.rt4p_hbm_read(P(buf), nbytes, P(sink), blocks, st))
    out["hbm_read_GBs"] = round(nbytes / ms / 1e6, 1)
    half = nbytes // 2 // 16 * 16
    dst = buf.view(torch.uint8)[half:]
    ms = _timed(torch, lambda: L.rt4p_copy(P(dst), P(buf), half, blocks, st))
    out["copy_GBs"] = round(2 * half / ms / 1e6, 1)
    del buf, dst
    iters = 4096
    for big, name, macs in ((1, "mfma_i32_32x32x32_i8_TOPS", 32768), (0, "mfma_i32_16x16x64_i8_TOPS", 16384)):
        blocks = cus * 8          # 4 waves per block -> 8 waves per SIMD
        ms = _timed(torch, lambda: L.rt4p_mfma_i8(P(sink), big, iters, blocks, st))
        ops = 2.0 * macs * 4 * iters * blocks * 4
        out[name] = round(ops / ms / 1e9, 1)
    iters = 8192
    blocks = cus * 8
    ms = _timed(torch, lambda: L.rt4p_valu_fma(P(sink), iters, blocks, st))
    out["fp32_fma_TFLOPs"] = round(2.0 * 8 * iters * blocks * 256 / ms / 1e9, 2)
    return out


# Launch shapes tried for the one-pass read ceiling (workgroups, threads): the
# best of them on MI355X in a sweep of 256..4096 workgroups x 256..1024 threads.
READ_SHAPES = ((1024, 256), (1024, 512), (2048, 256), (2048, 512), (768, 512), (512, 512), (4096, 256))


def hbm_read_ceiling(torch, nbytes: int, timed_graph, copies: int = 2, mults=(2, 4, 8)) -> dict:
    """The fastest rt4p_hbm_read (grid-stride, 8 independent 16-byte loads per
    lane in flight) of `nbytes` over `copies` distinct buffers replayed back to back
    in a HIP graph, best over grids of cus * mult workgroups of 256 threads: the
    one-pass read ceiling for sizes beyond rt4p_read_burst's reach (the LM head).
    Returns {"us": per read, "GBs", "blocks"}."""
    L = lib()
    cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    nb = nbytes // 16 * 16
    bufs = [torch.empty(nb // 4, dtype=torch.int32, device="cuda").random_() for _ in range(copies)]
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    best = None
    for mult in mults:
        blocks = cus * mult

        def fn():
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for b in bufs:
                rc = L.rt4p_hbm_read(P(b), nb, P(sink), blocks, st)
                if rc:
                    raise RuntimeError(f"rt4p_hbm_read failed ({rc})")

        fn()
        torch.cuda.synchronize()
        us = timed_graph(torch, fn) * 1e3 / copies
        if best is None or us < best["us"]:
            best = {"us": round(us, 3), "GBs": round(nb / us / 1e3, 1), "blocks": blocks}
    del bufs
    torch.cuda.empty_cache()
    return best


def read_ceiling(torch, nbytes: int, copies: int = 16, timed_graph=None) -> dict:
    """The fastest single launch reading `nbytes` from HBM: rt4p_read_burst over
    `copies` distinct buffers replayed back to back in a HIP graph (so no buffer
    is cache-resident), best over READ_SHAPES with non-temporal loads.  Returns
    {"us": per launch, "GBs": nbytes / us, "blocks", "threads"}."""
    L = lib()
    nb = nbytes // 16 * 16
    bufs = [torch.empty(nb // 4, dtype=torch.int32, device="cuda").random_() for _ in range(copies)]
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    best = None
    for blocks, threads in READ_SHAPES:
        if (nb // 16 + blocks - 1) // blocks > 16 * threads:
            continue

        def fn():
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for b in bufs:
                rc = L.rt4p_read_burst(P(b), nb, P(sink), blocks, threads, 1, st)
                if rc:
                    raise RuntimeError(f"rt4p_read_burst failed ({rc})")

        fn()
        torch.cuda.synchronize()
        us = timed_graph(torch, fn) * 1e3 / copies
        if best is None or us < best["us"]:
            best = {"us": round(us, 3), "GBs": round(nb / us / 1e3, 1), "blocks": blocks, "threads": threads}
    del bufs
    torch.cuda.empty_cache()
    return best


def mfma_i8_rate(torch, big: bool = False, iters: int = 2048) -> float:
    """Measured dense int8 MFMA rate in TOPS (v_mfma_i32_16x16x64_i8, or 32x32x32
    when big): 8 waves per SIMD, 4 independent accumulator chains per wave (8 chains
    of the 16x16 form measured lower, 2.6-2.9 against 3.5 POP/s)."""
    L = lib()
    cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    blocks = cus * 8
    ms = _timed(torch, lambda: L.rt4p_mfma_i8(ctypes.c_void_p(sink.data_ptr()), 1 if big else 0, iters, blocks, st))
    macs = 32768 if big else 16384
    return round(2.0 * macs * 4 * iters * blocks * 4 / ms / 1e9, 1)


def gemv_load_pattern(torch, rt4_amd, mats, xq, sa, rows: int, timed_graph) -> dict | None:
    """The decode GEMV's memory requests alone (rt4p_gemv_loads) over the weight sets
    `mats` [(wq, ws)] with activations xq, back to back in a graph as the GEMV is
    timed: {"us": per launch, "groups_per_wave", "waves", "k_splits"}.  None when the
    shape's launch plan is not a one-row-block form the probe mirrors."""
    wq0, _ = mats[0]
    N, K = wq0.shape[0], wq0.shape[1] * 8
    for wq, ws in mats:
        if tuple(wq.shape) != (N, K // 8) or tuple(ws.shape) != (N, K // 128) or not (wq.is_contiguous()
                                                                                     and ws.is_contiguous()):
            raise ValueError("gemv_load_pattern: every weight set must be [N, K/8] codes and [N, K/128] scales")
    if tuple(xq.shape) != (rows, K) or xq.element_size() != 1 or not xq.is_contiguous():
        raise ValueError("gemv_load_pattern: xq must be int8 [rows, K]")
    plan = rt4_amd.gemv_launch_plan(rows, N, K)
    g = plan["groups_per_wave"]
    if g == 0:
        if rows != 1 or K % 256 or K > 8192:
            return None
    elif g not in (2, 4) or plan["row_blocks"] != 1 or K % (128 * g) or (g == 4 and plan["waves"] > 8):
        return None
    L = lib()
    cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    sink = torch.zeros(1 << 20, dtype=torch.int32, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def fn():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for wq, ws in mats:
            rc = L.rt4p_gemv_loads(P(wq), P(ws), P(xq), P(sa), P(sink), rows, N, K, g, plan["waves"],
                                   plan["k_splits"], cus, st)
            if rc:
                raise RuntimeError(f"rt4p_gemv_loads failed ({rc})")

    fn()
    torch.cuda.synchronize()
    us = timed_graph(torch, fn) * 1e3 / len(mats)
    return {"us": round(us, 3), "groups_per_wave": g, "waves": plan["waves"], "k_splits": plan["k_splits"]}


def launch_cost(torch, timed_graph, n: int = 64) -> float:
    """Microseconds per empty-kernel node in a graph of n back-to-back launches
    (one workgroup of 64 threads each)."""
    L = lib()

    def fn():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for _ in range(n):
            if L.rt4p_empty(1, 64, st):
                raise RuntimeError("rt4p_empty failed")

    fn()
    torch.cuda.synchronize()
    return round(timed_graph(torch, fn) * 1e3 / n, 3)


def mfma_f8_16x16_rate(torch, iters: int = 2048) -> float:
    """Measured dense rate (TOPS) of v_mfma_f32_16x16x128_f8f6f4 with FP8 operands and
    no block scale, as the attention kernel issues it: 2 waves per SIMD, 8
    independent accumulator chains per wave."""
    L = lib()
    cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    sink = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ms = _timed(torch, lambda: L.rt4p_mfma_f8_16x16(ctypes.c_void_p(sink.data_ptr()), iters, cus, st))
    return round(2.0 * 32768 * 8 * iters * 8 * cus / ms / 1e9, 1)


def mfma_f8f6f4_rates(torch, iters: int = 2048) -> dict:
    """Measured dense rate (TOPS) of v_mfma_scale_f32_32x32x64_f8f6f4 with FP8, FP6 and
    FP4 operands: 2 waves per SIMD, 4 independent accumulator chains per wave."""
    L = lib()
    cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    sink = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {}
    for fmt, name in ((0, "fp8"), (2, "fp6"), (4, "fp4")):
        ms = _timed(torch, lambda: L.rt4p_mfma_f8f6f4(ctypes.c_void_p(sink.data_ptr()), fmt, iters, cus, st))
        out[f"mfma_scale_32x32x64_{name}_TOPS"] = round(2.0 * 65536 * 4 * iters * 8 * cus / ms / 1e9, 1)
    return out


def gemm_unit_cycles(torch, units: int = 512) -> dict:
    """The prefill GEMM's unit skeleton (rt4p_gemm_unit, registers only, 8 waves per
    CU): nominal 2.4 GHz cycles per unit per SIMD (two waves' units), int8 form and
    FP8-digit form, and the corresponding C2 gate/up time (21,760 units over the CUs)."""
    L = lib()
    cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    sink = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {}
    units_c2 = (1024 // 128) * (17408 // 256) * (5120 // 128)
    for variant, name in ((0, "int8"), (1, "fp8_digits")):
        ms = _timed(torch, lambda: L.rt4p_gemm_unit(ctypes.c_void_p(sink.data_ptr()), variant, units, cus, st))
        cyc = ms * 1e-3 * 2.4e9 / units
        out[f"unit_{name}_cycles"] = round(cyc, 1)
        out[f"unit_{name}_c2_gate_up_us"] = round(cyc * units_c2 / cus / 2.4e3, 1)
    return out
