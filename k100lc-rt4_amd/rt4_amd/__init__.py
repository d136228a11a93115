"""rt4_amd -- Python host side of the MI355X RT4 quantized-matmul library.

The compute lives in ``lib/librt4k.so`` (hand-written HIP for gfx950, C ABI in
``include/rt4k.h``).  This module binds that ABI with ctypes and offers thin
wrappers over torch device tensors (torch is used for device memory and streams
only).  There is no fallback: if the library is missing, every call raises.

Reference interface mirrored (src/kernels.h of K100LC-RT4):
    k_gemv_w4a8      -> gemv_w4a8            (src/kernels.h:27)
    k_quant_rows_a8  -> quant_rows_a8        (src/kernels.h:43)
    k_gemm_i4_a8     -> gemm_w4a8            (src/kernels.h:32)
    k_quant_rows     -> quant_rows_a4        (src/kernels.h:36)
    k_attn_q_quant   -> attn_q_quant         (src/kernels.h:40)
    k_kv_append_k/v  -> kv_append_k / _v     (src/kernels.h:50, :53)
    k_attention      -> attention_prefill    (src/kernels.h:81, prefill branch)
plus the pieces those wrappers launch internally (quant_act_a8, gemv_w4a8_q).
"""
from __future__ import annotations

import ctypes
import pathlib

from . import layout  # noqa: F401  (re-exported helpers)

LIB_PATH = pathlib.Path(__file__).resolve().parent / "lib" / "librt4k.so"
GROUP = 128

# Every symbol include/rt4k.h declares (checked by the CPU test suite).
C_EXPORTS = (
    "rt4_last_error", "rt4_abi_version", "rt4_release_scratch",
    "rt4_quant_act_a8", "rt4_quant_act_rowwise", "rt4_gemv_w4a8_q", "rt4_gemv_w4a8_q_cfg", "rt4_gemv_launch_plan",
    "rt4_gemv_w4a8_groupsums",
    "rt4_gemv_w4a8", "rt4_gemv_w4a8_noalloc", "rt4_gemv_w4a8_cfg", "rt4_quant_rows_a8", "rt4_quant_rows_i8", "rt4_digits_to_i8",
    "rt4_make_group_major", "rt4_quant_rows_a4", "rt4_quant_act_a4", "rt4_gemv_w4a4_q", "rt4_gemv_w4a4_q_cfg", "rt4_gemv_w4a4",
    "rt4_gemm_w4a4",
    "rt4_gemm_w4a8", "rt4_gemm_w4a8_i8", "rt4_gemm_w4a8_groupsums",
    "rt4_attn_q_quant", "rt4_kv_append_k", "rt4_kv_append_v", "rt4_attention_prefill",
    "rt4_attention_prefill_cfg",
    "rt4_file_open", "rt4_file_close", "rt4_file_count", "rt4_file_find", "rt4_file_info", "rt4_file_data",
    "rt4_file_size", "rt4_file_upload", "rt4_file_upload_tensor",
)
# The reference-compatible C++ entry points (include/rt4_kernels.h), mangled.
CXX_EXPORTS = (
    "_Z11k_gemv_w4a8PfPKjPKfS3_iii",
    "_Z15k_quant_rows_a8PjS_PfS0_PKfiiiii",
    "_Z12k_quant_rowsPjPfPKfiiiii",
    "_Z12k_gemm_i4_a8PfS_PKjPKfS1_S1_S3_S3_iii",
    "_Z14k_attn_q_quantPjPfPKfiiiii",
    "_Z13k_kv_append_kPjPfPKfiiiiii",
    "_Z13k_kv_append_vPjPfS0_PKfiiiiii",
    "_Z11k_attentionPfPKjPKfS1_S3_S1_S3_iiiiiiiiS_S_S_i",
    "_Z11k_gemv_w4a4PfPKjPKfS3_iii",
    "_Z9k_gemm_i4PfPKjPKfS1_S3_iii",
)


class RT4Error(RuntimeError):
    """A librt4k entry point returned an error status."""


_lib = None
_P = ctypes.c_void_p
_I = ctypes.c_int
_SIGS = {
    "rt4_quant_act_a8": [_P, _P, _P, _P, _I, _I, _P],
    "rt4_quant_act_rowwise": [_P, _P, _P, _P, _I, _I, _I, _P],
    "rt4_quant_act_a4": [_P, _P, _P, _I, _I, _P],
    "rt4_gemv_w4a4_q": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "rt4_gemv_w4a4_q_cfg": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    "rt4_gemv_w4a4": [_P, _P, _P, _P, _I, _I, _I, _P],
    "rt4_gemm_w4a4": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "rt4_gemv_w4a8_q": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "rt4_gemv_w4a8_q_cfg": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P],
    "rt4_gemv_launch_plan": [_I, _I, _I, _P, _P, _P, _P],
    "rt4_gemv_w4a8_groupsums": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "rt4_gemv_w4a8": [_P, _P, _P, _P, _I, _I, _I, _P],
    "rt4_gemv_w4a8_noalloc": [_P, _P, _P, _P, _I, _I, _I, _P],
    "rt4_gemv_w4a8_cfg": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P],
    "rt4_quant_rows_a8": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "rt4_quant_rows_i8": [_P, _P, _P, _I, _I, _I, _I, _P],
    "rt4_digits_to_i8": [_P, _P, _P, _I, _I, _P],
    "rt4_make_group_major": [_P, _P, _I, _I, _P],
    "rt4_quant_rows_a4": [_P, _P, _P, _I, _I, _I, _I, _I, _P],
    "rt4_gemm_w4a8": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "rt4_gemm_w4a8_i8": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "rt4_gemm_w4a8_groupsums": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "rt4_attn_q_quant": [_P, _P, _P, _I, _I, _I, _I, _I, _P],
    "rt4_kv_append_k": [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    "rt4_kv_append_v": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    "rt4_attention_prefill": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P],
    "rt4_attention_prefill_cfg": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P],
}


def lib() -> ctypes.CDLL:
    """Load librt4k.so once (no GPU work happens at load time).

    torch wheels bundle their own HIP runtime whose soname (libamdhip64.so.7)
    equals the system one librt4k.so links.  Importing torch first lets the
    dynamic linker bind librt4k.so to that already loaded runtime, so the
    process holds a single HIP/HSA runtime; loading librt4k.so first would pull
    in /opt/rocm's copy as well, and whichever of the two initialises second
    finds no device.
    """
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RT4Error(f"{LIB_PATH} is missing: build it with `make -C k100lc-rt4_amd` "
                           "or __graft_entry__.build()")
        try:
            import torch  # noqa: F401  (see the docstring: one HIP runtime per process)
        except ImportError:
            pass
        L = ctypes.CDLL(str(LIB_PATH))
        L.rt4_last_error.restype = ctypes.c_char_p
        L.rt4_last_error.argtypes = []
        L.rt4_abi_version.restype = ctypes.c_int
        L.rt4_release_scratch.restype = ctypes.c_int
        L.rt4_release_scratch.argtypes = []
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise RT4Error(lib().rt4_last_error().decode(errors="replace"))


def release_scratch() -> None:
    """Free the library scratch of the current device (see rt4_release_scratch in
    include/rt4k.h): waits for the device; graphs captured earlier must not be
    replayed afterwards."""
    _check(lib().rt4_release_scratch())


# ----------------------------------------------------------- torch helpers --
def _torch():
    import torch
    return torch


def _stream():
    return _P(_torch().cuda.current_stream().cuda_stream)


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise RT4Error("rt4_amd expects device tensors")
    if not t.is_contiguous():
        raise RT4Error("rt4_amd expects contiguous tensors")
    return _P(t.data_ptr())


def _empty(shape, dtype, device):
    return _torch().empty(shape, dtype=dtype, device=device)


# ---------------------------------------------------------------- decode ----
def quant_act_a8(x, want_sums: bool = False):
    """x f32 [rows, K] -> (xq int8 [rows, K] interleaved, sa f32 [rows, K/128][, asu])."""
    torch = _torch()
    rows, K = x.shape
    xq = _empty((rows, K), torch.int8, x.device)
    sa = _empty((rows, K // GROUP), torch.float32, x.device)
    asu = _empty((rows, K // GROUP), torch.int32, x.device) if want_sums else None
    _check(lib().rt4_quant_act_a8(_ptr(xq), _ptr(sa), _ptr(asu), _ptr(x), rows, K, _stream()))
    return (xq, sa, asu) if want_sums else (xq, sa)


def quant_act_rowwise(x, mode: int = 0, want_sums: bool = False):
    """Per-row quantizer (one scale per row; no counterpart in the reference).
    mode 0: (xq int8 [rows, K] interleaved, sa f32 [rows, K/128][, asu]) for
    gemv_w4a8_q; mode 1: (xq, sc f32 [K/128, rows]) for gemm_w4a8_i8.  The row's
    scale fills every group slot."""
    torch = _torch()
    rows, K = x.shape
    xq = _empty((rows, K), torch.int8, x.device)
    sa = _empty((rows, K // GROUP) if mode == 0 else (K // GROUP, rows), torch.float32, x.device)
    asu = _empty((rows, K // GROUP), torch.int32, x.device) if want_sums else None
    _check(lib().rt4_quant_act_rowwise(_ptr(xq), _ptr(sa), _ptr(asu), _ptr(x), rows, K, mode, _stream()))
    return (xq, sa, asu) if want_sums else (xq, sa)


def gemv_w4a8_q(wq, ws, xq, sa, out=None, groups_per_wave: int = 0, waves: int = 0, k_splits: int = 0,
                row_blocks: int = 0):
    """W4A8 GEMV on quantized activations.  wq int32/uint32 [N, K/8], ws int16/fp16 [N, K/128].

    groups_per_wave / waves / k_splits / row_blocks override the launch
    configuration (0 keeps the default; k_splits=1 keeps every tile whole;
    row_blocks 1 or 2 sixteen-row blocks per tile)."""
    torch = _torch()
    rows, K = xq.shape
    N = wq.shape[0]
    y = out if out is not None else _empty((rows, N), torch.float32, xq.device)
    _check(lib().rt4_gemv_w4a8_q_cfg(_ptr(y), _ptr(wq), _ptr(ws), _ptr(xq), _ptr(sa), rows, N, K,
                                     groups_per_wave, waves, k_splits, row_blocks, _stream()))
    return y


def gemv_launch_plan(rows: int, N: int, K: int) -> dict:
    """The default GEMV launch configuration for this shape on the current device."""
    g, w, s, r = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _check(lib().rt4_gemv_launch_plan(rows, N, K, ctypes.byref(g), ctypes.byref(w), ctypes.byref(s),
                                      ctypes.byref(r)))
    return {"groups_per_wave": g.value, "waves": w.value, "k_splits": s.value, "row_blocks": r.value}


def gemv_w4a8_groupsums(wq, ws, xq, sa):
    """Same kernel, returning (y, gsum int32 [rows, N, K/128])."""
    torch = _torch()
    rows, K = xq.shape
    N = wq.shape[0]
    y = _empty((rows, N), torch.float32, xq.device)
    gs = _empty((rows, N, K // GROUP), torch.int32, xq.device)
    _check(lib().rt4_gemv_w4a8_groupsums(_ptr(gs), _ptr(y), _ptr(wq), _ptr(ws), _ptr(xq), _ptr(sa),
                                         rows, N, K, _stream()))
    return y, gs


def gemv_w4a8(wq, ws, x, out=None, groups_per_wave: int = 0, waves: int = 0, k_splits: int = 0,
              row_blocks: int = 0):
    """Drop-in k_gemv_w4a8: quantize x f32 [rows, K] and multiply (rows <= 4).

    Two launches (quantizer, GEMV).  A launch configuration (see gemv_w4a8_q)
    selects rt4_gemv_w4a8_cfg instead: one launch that quantizes inside the GEMV
    (x 16-byte aligned), bit-identical output."""
    torch = _torch()
    rows, K = x.shape
    N = wq.shape[0]
    y = out if out is not None else _empty((rows, N), torch.float32, x.device)
    if groups_per_wave or waves or k_splits or row_blocks:
        _check(lib().rt4_gemv_w4a8_cfg(_ptr(y), _ptr(wq), _ptr(ws), _ptr(x), rows, N, K, groups_per_wave, waves,
                                       k_splits, row_blocks, _stream()))
    else:
        _check(lib().rt4_gemv_w4a8(_ptr(y), _ptr(wq), _ptr(ws), _ptr(x), rows, N, K, _stream()))
    return y


# --------------------------------------------------------------- prefill ----
def quant_rows_a8(x, rows: int | None = None, K: int | None = None, G: int = GROUP,
                  in_stride: int = 0, in_off: int = 0):
    """Drop-in k_quant_rows_a8 -> (qh, ql int32 [rows, K/8], sc, sc16 f32 [K/G, rows])."""
    torch = _torch()
    if rows is None or K is None:
        rows, K = x.shape
    qh = _empty((rows, K // 8), torch.int32, x.device)
    ql = _empty((rows, K // 8), torch.int32, x.device)
    sc = _empty((K // G, rows), torch.float32, x.device)
    sc16 = _empty((K // G, rows), torch.float32, x.device)
    _check(lib().rt4_quant_rows_a8(_ptr(qh), _ptr(ql), _ptr(sc), _ptr(sc16), _ptr(x), rows, K, G,
                                   in_stride, in_off, _stream()))
    return qh, ql, sc, sc16


def quant_rows_i8(x, rows: int | None = None, K: int | None = None, in_stride: int = 0,
                  in_off: int = 0):
    """Same quantizer -> (xq int8 [rows, K] interleaved, sc f32 [K/128, rows])."""
    torch = _torch()
    if rows is None or K is None:
        rows, K = x.shape
    xq = _empty((rows, K), torch.int8, x.device)
    sc = _empty((K // GROUP, rows), torch.float32, x.device)
    _check(lib().rt4_quant_rows_i8(_ptr(xq), _ptr(sc), _ptr(x), rows, K, in_stride, in_off, _stream()))
    return xq, sc


def digits_to_i8(qh, ql):
    torch = _torch()
    rows, KD = qh.shape
    xq = _empty((rows, KD * 8), torch.int8, qh.device)
    _check(lib().rt4_digits_to_i8(_ptr(xq), _ptr(qh), _ptr(ql), rows, KD * 8, _stream()))
    return xq


def make_group_major(ws, K: int):
    torch = _torch()
    N = ws.shape[0]
    out = _empty((K // GROUP, N), torch.float32, ws.device)
    _check(lib().rt4_make_group_major(_ptr(out), _ptr(ws), N, K, _stream()))
    return out


def quant_rows_a4(x, rows: int | None = None, K: int | None = None, G: int = GROUP,
                  in_stride: int = 0, in_off: int = 0):
    """Drop-in k_quant_rows -> (q int32 [rows, K/8], sc f32 [K/G, rows])."""
    torch = _torch()
    if rows is None or K is None:
        rows, K = x.shape
    q = _empty((rows, K // 8), torch.int32, x.device)
    sc = _empty((K // G, rows), torch.float32, x.device)
    _check(lib().rt4_quant_rows_a4(_ptr(q), _ptr(sc), _ptr(x), rows, K, G, in_stride, in_off,
                                   _stream()))
    return q, sc


def quant_act_a4(x):
    """Decode int4 quantizer of k_gemv_w4a4: x f32 [rows, K] -> (aq int32 [rows, K/8],
    sa f32 [rows, K/32])."""
    torch = _torch()
    rows, K = x.shape
    aq = _empty((rows, K // 8), torch.int32, x.device)
    sa = _empty((rows, K // 32), torch.float32, x.device)
    _check(lib().rt4_quant_act_a4(_ptr(aq), _ptr(sa), _ptr(x), rows, K, _stream()))
    return aq, sa


def gemv_w4a4_q(wq, ws, aq, sa, out=None, groups_per_wave: int = 0, waves: int = 0, k_splits: int = 0):
    """W4A4 GEMV on int4 activation codes aq int32 [rows, K/8], sa f32 [rows, K/32].

    groups_per_wave (2 or 4) / waves (1..16) / k_splits (1: tiles whole) override
    the launch configuration (0 keeps the default)."""
    torch = _torch()
    rows, KD = aq.shape
    N = wq.shape[0]
    y = out if out is not None else _empty((rows, N), torch.float32, aq.device)
    _check(lib().rt4_gemv_w4a4_q_cfg(_ptr(y), _ptr(wq), _ptr(ws), _ptr(aq), _ptr(sa), rows, N, KD * 8,
                                     groups_per_wave, waves, k_splits, _stream()))
    return y


def gemv_w4a4(wq, ws, x, out=None):
    """Drop-in k_gemv_w4a4: quantize x f32 [rows, K] to int4 per 32 and multiply (rows <= 4)."""
    torch = _torch()
    rows, K = x.shape
    N = wq.shape[0]
    y = out if out is not None else _empty((rows, N), torch.float32, x.device)
    _check(lib().rt4_gemv_w4a4(_ptr(y), _ptr(wq), _ptr(ws), _ptr(x), rows, N, K, _stream()))
    return y


def gemm_w4a4(wq, wsc_gm, aq, asc_gm, out=None):
    """Drop-in k_gemm_i4: aq int32 [M, K/8] (k_quant_rows codes), asc_gm f32 [K/128, M],
    wq int32 [N, K/8], wsc_gm f32 [K/128, N] -> c f32 [M, N]."""
    torch = _torch()
    M, KD = aq.shape
    N = wq.shape[0]
    c = out if out is not None else _empty((M, N), torch.float32, aq.device)
    _check(lib().rt4_gemm_w4a4(_ptr(c), _ptr(wq), _ptr(wsc_gm), _ptr(aq), _ptr(asc_gm), M, N, KD * 8, _stream()))
    return c


def gemm_w4a8_i8(wq, wsc_gm, xq, sc, out=None):
    """Prefill GEMM on int8 codes: xq int8 [M, K] interleaved, sc f32 [K/128, M],
    wq int32 [N, K/8], wsc_gm f32 [K/128, N] -> c f32 [M, N]."""
    torch = _torch()
    M, K = xq.shape
    N = wq.shape[0]
    c = out if out is not None else _empty((M, N), torch.float32, xq.device)
    _check(lib().rt4_gemm_w4a8_i8(_ptr(c), _ptr(wq), _ptr(wsc_gm), _ptr(xq), _ptr(sc), M, N, K, _stream()))
    return c


def gemm_w4a8_groupsums(wq, wsc_gm, xq, sc):
    """Same kernel, returning (c, gsum int32 [M, N, K/128]) -- small shapes only."""
    torch = _torch()
    M, K = xq.shape
    N = wq.shape[0]
    c = _empty((M, N), torch.float32, xq.device)
    gs = _empty((M, N, K // GROUP), torch.int32, xq.device)
    _check(lib().rt4_gemm_w4a8_groupsums(_ptr(gs), _ptr(c), _ptr(wq), _ptr(wsc_gm), _ptr(xq), _ptr(sc),
                                         M, N, K, _stream()))
    return c, gs


def gemm_w4a8(wq, wsc_gm, qh, ql, sc, sc16, out=None, c2=None):
    """Drop-in k_gemm_i4_a8 on the digit planes of quant_rows_a8 -> c f32 [M, N]."""
    torch = _torch()
    M, KD = qh.shape
    K = KD * 8
    N = wq.shape[0]
    c = out if out is not None else _empty((M, N), torch.float32, qh.device)
    c2 = c2 if c2 is not None else _empty((M, N), torch.float32, qh.device)
    _check(lib().rt4_gemm_w4a8(_ptr(c), _ptr(c2), _ptr(wq), _ptr(wsc_gm), _ptr(qh), _ptr(ql), _ptr(sc),
                               _ptr(sc16), M, N, K, _stream()))
    return c


# ------------------------------------------------------------- attention ----
HEAD_DIM = 256
KV_TILE = 64


def attn_q_quant(x, TP: int, G: int = GROUP, qq=None, qs=None):
    """k_attn_q_quant: x f32 [T, H, D] -> (qq int32 [H, TP, D/8], qs f32 [H, D/G, TP]).
    Rows >= T keep the buffers' contents (new buffers: zero codes, unit scales)."""
    torch = _torch()
    T, H, D = x.shape
    if qq is None:
        qq = torch.zeros((H, TP, D // 8), dtype=torch.int32, device=x.device)
    if qs is None:
        qs = torch.ones((H, D // G, TP), dtype=torch.float32, device=x.device)
    _check(lib().rt4_attn_q_quant(_ptr(qq), _ptr(qs), _ptr(x), T, H, D, G, TP, _stream()))
    return qq, qs


def kv_append_k(kc, ksc, kf, t0: int, G: int = GROUP):
    """k_kv_append_k, in place: kc int32 [H, kv_total, D/8], ksc f32 [H, D/G, kv_total]; kf f32 [T, H, D]."""
    T, H, D = kf.shape
    _check(lib().rt4_kv_append_k(_ptr(kc), _ptr(ksc), _ptr(kf), t0, T, H, D, G, kc.shape[1], _stream()))


def kv_append_v(vc, vsc, stage, vf, t0: int):
    """k_kv_append_v, in place: vc int32 [H, kv_total/8, D], vsc f32 [H, kv_total/BG, D],
    stage f32 [H, BG, D]; vf f32 [T, H, D]."""
    T, H, D = vf.shape
    BG = stage.shape[1]
    _check(lib().rt4_kv_append_v(_ptr(vc), _ptr(vsc), _ptr(stage), _ptr(vf), t0, T, H, D, BG,
                                 vc.shape[1] * 8, _stream()))


def attention_prefill(qq, qsc, kc, ksc, vc, vsc, n_kv: int, off: int, ratio: int,
                      n_tile: int | None = None, out=None, kv_splits: int = 0):
    """Prefill branch of k_attention -> out f32 [H, n_q, 256] (kv_splits 0 = automatic)."""
    torch = _torch()
    H, n_q, _ = qq.shape
    kv_cap = kc.shape[1]
    if n_tile is None:
        n_tile = (n_kv + KV_TILE - 1) // KV_TILE
    if out is None:
        out = torch.empty((H, n_q, HEAD_DIM), dtype=torch.float32, device=qq.device)
    _check(lib().rt4_attention_prefill_cfg(_ptr(out), _ptr(qq), _ptr(qsc), _ptr(kc), _ptr(ksc), _ptr(vc),
                                           _ptr(vsc), n_q, n_kv, off, n_tile, H, ratio, kv_cap, kv_splits, _stream()))
    return out
