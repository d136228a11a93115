"""ctypes binding of librt4probe.so: gfx950 ceilings (HBM read, copy, int8 MFMA,
fp32 FMA issue rates) measured next to the published MI355X peaks."""
from __future__ import annotations

import ctypes
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().parent / "lib" / "librt4probe.so"
EXPORTS = ("rt4p_hbm_read", "rt4p_read_burst", "rt4p_copy", "rt4p_mfma_i8", "rt4p_valu_fma")
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
                "rt4p_mfma_i8": [P, I, I, I, P], "rt4p_valu_fma": [P, I, I, P]}
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
    when big): 8 waves per SIMD, 4 independent accumulator chains per wave."""
    L = lib()
    cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    blocks = cus * 8
    ms = _timed(torch, lambda: L.rt4p_mfma_i8(ctypes.c_void_p(sink.data_ptr()), 1 if big else 0, iters, blocks, st))
    macs = 32768 if big else 16384
    return round(2.0 * macs * 4 * iters * blocks * 4 / ms / 1e9, 1)
