"""ctypes front end of liboracle.so -- the C restatement in rt4_oracle.c.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Each wrapper names the
reference function it restates; the C file cites file:line for every step.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
GROUP = 128

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE), "oracle"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        P, I = ctypes.c_void_p, ctypes.c_int
        sig = {
            "rt4o_f16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
            "rt4o_dot8_i4": ([ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int32], ctypes.c_int32),
            "rt4o_quant_act": ([P, I, I, P, P, P], None),
            "rt4o_quant_rows_a8": ([P, I, I, I, I, I, P, P, P, P], None),
            "rt4o_quant_rows_i8": ([P, I, I, I, I, I, P, P], None),
            "rt4o_quant_rows_a4": ([P, I, I, I, I, I, P, P], None),
            "rt4o_make_group_major": ([P, I, I, P], None),
            "rt4o_f32_to_f16_conv": ([ctypes.c_float], ctypes.c_uint16),
            "rt4o_quant_weight_rows": ([P, I, I, P, P], None),
            "rt4o_attn_q_quant": ([P, P, P, I, I, I, I, I], None),
            "rt4o_kv_append_k": ([P, P, P, I, I, I, I, I, I], None),
            "rt4o_kv_append_v": ([P, P, P, P, I, I, I, I, I, I], None),
            "rt4o_fa_rows": ([P, P, P, P, P, P, I, I, I, I, I, I, P, I, I, P], None),
            "rt4o_gemv_groupsums": ([P, P, I, I, I, P], None),
            "rt4o_gemv_fold": ([P, P, P, I, I, I, P], None),
            "rt4o_gemv_w4a8": ([P, P, P, I, I, I, P], None),
            "rt4o_gemm_w4a8_points": ([P, P, P, P, P, P, I, I, I, P, P, I, P, P], None),
            "rt4o_gemm_w4a4_points": ([P, P, P, P, I, I, I, P, P, I, P, P], None),
            "rt4o_quant_act4": ([P, I, I, P, P], None),
            "rt4o_gemv_w4a4_sums": ([P, P, I, I, I, P], None),
            "rt4o_gemv_w4a4_fold": ([P, P, P, I, I, I, P], None),
            "rt4o_gemv_w4a4": ([P, P, P, I, I, I, P], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def f16_to_f32(h: int) -> float:
    return lib().rt4o_f16_to_f32(h)


def dot8_i4(a: int, b: int, acc: int = 0) -> int:
    """v_dot8_i32_i4 semantics (bench/bench_isa2.cpp:128-145)."""
    return lib().rt4o_dot8_i4(a & 0xFFFFFFFF, b & 0xFFFFFFFF, acc)


def quant_act(x: np.ndarray):
    """quant_act (kernels/gemv_w4a8_core.h:34-66) -> (q int8 [M,K] natural, sa [M,NG], asu [M,NG])."""
    x = _c(x, np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    sa = np.empty((M, K // GROUP), np.float32)
    asu = np.empty((M, K // GROUP), np.int32)
    lib().rt4o_quant_act(_p(x), M, K, _p(q), _p(sa), _p(asu))
    return q, sa, asu


def quant_rows_a8(x: np.ndarray, rows: int, K: int, G: int = GROUP, in_stride: int = 0,
                  in_off: int = 0):
    """quant_rows_a8_k (src/k_new.hip:268-301) -> (qh, ql uint32 [rows,K/8], sc, sc16 [K/G,rows])."""
    x = _c(x, np.float32)
    qh = np.empty((rows, K // 8), np.uint32)
    ql = np.empty((rows, K // 8), np.uint32)
    sc = np.empty((K // G, rows), np.float32)
    sc16 = np.empty((K // G, rows), np.float32)
    lib().rt4o_quant_rows_a8(_p(x), rows, K, G, in_stride, in_off, _p(qh), _p(ql), _p(sc), _p(sc16))
    return qh, ql, sc, sc16


def quant_rows_i8(x: np.ndarray, rows: int, K: int, G: int = GROUP, in_stride: int = 0,
                  in_off: int = 0):
    """The same quantizer's int8 code q8 = 16h + l (natural order) and sc."""
    x = _c(x, np.float32)
    q = np.empty((rows, K), np.int8)
    sc = np.empty((K // G, rows), np.float32)
    lib().rt4o_quant_rows_i8(_p(x), rows, K, G, in_stride, in_off, _p(q), _p(sc))
    return q, sc


def quant_rows_a4(x: np.ndarray, rows: int, K: int, G: int = GROUP, in_stride: int = 0,
                  in_off: int = 0):
    """quant_rows_k (src/k_new.hip:192-219) -> (q uint32 [rows,K/8], sc [K/G,rows])."""
    x = _c(x, np.float32)
    q = np.empty((rows, K // 8), np.uint32)
    sc = np.empty((K // G, rows), np.float32)
    lib().rt4o_quant_rows_a4(_p(x), rows, K, G, in_stride, in_off, _p(q), _p(sc))
    return q, sc


def f32_to_f16_conv(x: float) -> int:
    """The reference converter's float -> f16 bits (tools/convert.c:102-120)."""
    return int(lib().rt4o_f32_to_f16_conv(float(x)))


def quant_weight_rows(w: np.ndarray):
    """The reference converter's int4 weight quantizer (tools/convert.c:338-360):
    w f32 [N, K] -> (wq uint32 [N, K/8], ws uint16 [N, K/128])."""
    w = _c(w, np.float32)
    N, K = w.shape
    wq = np.empty((N, K // 8), np.uint32)
    ws = np.empty((N, K // GROUP), np.uint16)
    lib().rt4o_quant_weight_rows(_p(w), N, K, _p(wq), _p(ws))
    return wq, ws


def make_group_major(ws: np.ndarray) -> np.ndarray:
    """make_group_major (src/model.cpp:190-202): uint16 [N,NG] -> f32 [NG,N]."""
    ws = _c(ws, np.uint16)
    N, NG = ws.shape
    out = np.empty((NG, N), np.float32)
    lib().rt4o_make_group_major(_p(ws), N, NG, _p(out))
    return out


def gemv_groupsums(wq: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Exact I[m][n][g] = Σ code*q over each 128-group (q in natural order)."""
    wq = _c(wq, np.uint32)
    q = _c(q, np.int8)
    M, K = q.shape
    N = wq.shape[0]
    I = np.empty((M, N, K // GROUP), np.int32)
    lib().rt4o_gemv_groupsums(_p(wq), _p(q), M, N, K, _p(I))
    return I


def gemv_fold(I: np.ndarray, ws: np.ndarray, sa: np.ndarray) -> np.ndarray:
    """fp64 Σ_g f16(ws)*sa*I (kernels/gemv_w4a8_core.h:189-197)."""
    I = _c(I, np.int32)
    ws = _c(ws, np.uint16)
    sa = _c(sa, np.float32)
    M, N, NG = I.shape
    y = np.empty((M, N), np.float64)
    lib().rt4o_gemv_fold(_p(I), _p(ws), _p(sa), M, N, NG * GROUP, _p(y))
    return y


def gemv_w4a8(wq: np.ndarray, ws: np.ndarray, x: np.ndarray) -> np.ndarray:
    """k_gemv_w4a8 (src/k_gemv.hip:53-106) end to end, fp64 result."""
    wq = _c(wq, np.uint32)
    ws = _c(ws, np.uint16)
    x = _c(x, np.float32)
    M, K = x.shape
    N = wq.shape[0]
    y = np.empty((M, N), np.float64)
    lib().rt4o_gemv_w4a8(_p(wq), _p(ws), _p(x), M, N, K, _p(y))
    return y


SG = 32


def quant_act4(x: np.ndarray):
    """quant_act4 (kernels/gemv_w4a4_core.h:22-44): -> (aq uint32 [M, K/8], sa f32 [M, K/32])."""
    x = _c(x, np.float32)
    M, K = x.shape
    aq = np.empty((M, K // 8), np.uint32)
    sa = np.empty((M, K // SG), np.float32)
    lib().rt4o_quant_act4(_p(x), M, K, _p(aq), _p(sa))
    return aq, sa


def gemv_w4a4_sums(wq: np.ndarray, aq: np.ndarray) -> np.ndarray:
    """Exact I[m][n][j] over 32-element subgroups (int4 x int4)."""
    wq = _c(wq, np.uint32)
    aq = _c(aq, np.uint32)
    M, KD = aq.shape
    N = wq.shape[0]
    I = np.empty((M, N, KD * 8 // SG), np.int32)
    lib().rt4o_gemv_w4a4_sums(_p(wq), _p(aq), M, N, KD * 8, _p(I))
    return I


def gemv_w4a4_fold(I: np.ndarray, ws: np.ndarray, sa: np.ndarray) -> np.ndarray:
    """fp64 Σ_j f16(ws[n][j/4])*sa[m][j]*I[m][n][j]."""
    I = _c(I, np.int32)
    M, N, NS = I.shape
    y = np.empty((M, N), np.float64)
    lib().rt4o_gemv_w4a4_fold(_p(I), _p(_c(ws, np.uint16)), _p(_c(sa, np.float32)), M, N, NS * SG, _p(y))
    return y


def gemv_w4a4(wq: np.ndarray, ws: np.ndarray, x: np.ndarray) -> np.ndarray:
    """k_gemv_w4a4 (src/k_gemv.hip:14-42) end to end, fp64 result."""
    x = _c(x, np.float32)
    M, K = x.shape
    N = wq.shape[0]
    y = np.empty((M, N), np.float64)
    lib().rt4o_gemv_w4a4(_p(_c(wq, np.uint32)), _p(_c(ws, np.uint16)), _p(x), M, N, K, _p(y))
    return y


def gemm_w4a8_points(wq, sb, ah, al, sc, sc16, M, N, K, mi, ni):
    """k_gemm_i4_a8 (src/k_gemm.hip:22-34) at points (mi[p], ni[p]) -> (c fp64 [P], Ig int32 [P,NG])."""
    mi = _c(mi, np.int32)
    ni = _c(ni, np.int32)
    P = mi.size
    c = np.empty(P, np.float64)
    Ig = np.empty((P, K // GROUP), np.int32)
    lib().rt4o_gemm_w4a8_points(_p(_c(wq, np.uint32)), _p(_c(sb, np.float32)), _p(_c(ah, np.uint32)),
                                _p(_c(al, np.uint32)), _p(_c(sc, np.float32)), _p(_c(sc16, np.float32)),
                                M, N, K, _p(mi), _p(ni), P, _p(c), _p(Ig))
    return c, Ig


def gemm_w4a4_points(wq, sb, aq, sa, M, N, K, mi, ni):
    """k_gemm_i4 (src/k_gemm.hip:8-17) at points -> (c fp64 [P], Ig int32 [P,NG])."""
    mi = _c(mi, np.int32)
    ni = _c(ni, np.int32)
    P = mi.size
    c = np.empty(P, np.float64)
    Ig = np.empty((P, K // GROUP), np.int32)
    lib().rt4o_gemm_w4a4_points(_p(_c(wq, np.uint32)), _p(_c(sb, np.float32)), _p(_c(aq, np.uint32)),
                                _p(_c(sa, np.float32)), M, N, K, _p(mi), _p(ni), P, _p(c), _p(Ig))
    return c, Ig


# ------------------------------------------------------------ attention --
HD, BN = 256, 64


def attn_q_quant(x: np.ndarray, TP: int, G: int = GROUP, qq=None, qs=None):
    """attn_q_quant_k (src/k_new.hip:228-253): x f32 [T, H, D] -> (qq uint32 [H, TP, D/8],
    qs f32 [H, D/G, TP]); rows >= T keep the contents of the passed-in buffers (zeros/ones)."""
    x = _c(x, np.float32)
    T, H, D = x.shape
    if qq is None:
        qq = np.zeros((H, TP, D // 8), np.uint32)
    if qs is None:
        qs = np.ones((H, D // G, TP), np.float32)
    lib().rt4o_attn_q_quant(_p(qq), _p(qs), _p(x), T, H, D, G, TP)
    return qq, qs


def kv_append_k(kc: np.ndarray, ksc: np.ndarray, kf: np.ndarray, t0: int, G: int = GROUP):
    """kv_append_k_k (src/k_new.hip:327-347), in place: kc uint32 [H, kv_total, D/8],
    ksc f32 [H, D/G, kv_total]; kf f32 [T, H, D] written at keys t0..t0+T-1."""
    kf = _c(kf, np.float32)
    T, H, D = kf.shape
    lib().rt4o_kv_append_k(_p(kc), _p(ksc), _p(kf), t0, T, H, D, G, kc.shape[1])


def kv_append_v(vc: np.ndarray, vsc: np.ndarray, stage: np.ndarray, vf: np.ndarray, t0: int, kv_total: int):
    """kv_append_v_k (src/k_new.hip:351-392), in place: vc uint32 [H, kv_total/8, D],
    vsc f32 [H, kv_total/BG, D], stage f32 [H, BG, D]; vf f32 [T, H, D]."""
    vf = _c(vf, np.float32)
    T, H, D = vf.shape
    BG = stage.shape[1]
    lib().rt4o_kv_append_v(_p(vc), _p(vsc), _p(stage), _p(vf), t0, T, H, D, BG, kv_total)


def fa_rows(qq, qsc, kc, ksc, vc, vsc, n_q, n_kv, off, kv_cap, ratio, head, rows, mode):
    """fp64 attention outputs of query rows `rows` of q head `head`: mode 0 = exact softmax
    (ref_rows, kernels/flash_attn_int4.hip:146-170), mode 1 = the kernel's fixed-point
    algorithm (ref_alg, :175-217).  -> f64 [len(rows), 256]."""
    rows = _c(rows, np.int32)
    out = np.empty((rows.size, HD), np.float64)
    lib().rt4o_fa_rows(_p(_c(qq, np.uint32)), _p(_c(qsc, np.float32)), _p(_c(kc, np.uint32)),
                       _p(_c(ksc, np.float32)), _p(_c(vc, np.uint32)), _p(_c(vsc, np.float32)),
                       n_q, n_kv, off, kv_cap, ratio, head, _p(rows), rows.size, mode, _p(out))
    return out
