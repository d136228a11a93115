"""RT4 weight files (manifest JSON + weight file from the reference converter,
tools/convert.c) through librt4k's loader (include/rt4k.h, "RT4 files").

    f = RT4File("model.rt4.json")
    f.names()                                  # tensor names in manifest order
    f.info("lm_head.weight")                   # kind, shape, group, offsets, relerr
    q, s = f.host("model.language_model.layers.0.mlp.down_proj.weight")   # numpy views of the mapping
    wq, ws = f.upload("model.language_model.layers.0.mlp.down_proj.weight")  # torch device tensors
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _check, _stream, _torch, lib


class TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("kind", ctypes.c_char * 8), ("ndim", ctypes.c_int),
                ("shape", ctypes.c_int64 * 4), ("group", ctypes.c_int64), ("q_off", ctypes.c_int64),
                ("s_off", ctypes.c_int64), ("q_bytes", ctypes.c_int64), ("s_bytes", ctypes.c_int64),
                ("relerr", ctypes.c_double), ("src_rms", ctypes.c_double)]


_P = ctypes.c_void_p
_SIGS = {
    "rt4_file_open": [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)],
    "rt4_file_close": [_P],
    "rt4_file_count": [_P, ctypes.POINTER(ctypes.c_int)],
    "rt4_file_find": [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)],
    "rt4_file_info": [_P, ctypes.c_int, ctypes.POINTER(TensorInfo)],
    "rt4_file_data": [_P, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p)],
    "rt4_file_size": [_P, ctypes.POINTER(ctypes.c_int64)],
    "rt4_file_upload": [_P, _P, ctypes.c_int64, _P],
    "rt4_file_upload_tensor": [_P, ctypes.c_int, _P, _P, _P],
}


def _lib():
    L = lib()
    if not getattr(L, "_rt4file_sigs", False):
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        L._rt4file_sigs = True
    return L


class RT4File:
    def __init__(self, manifest: str, weight_file: str | None = None):
        h = ctypes.c_void_p()
        _check(_lib().rt4_file_open(str(manifest).encode(), None if weight_file is None else str(weight_file).encode(),
                                    ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if self._h:
            _lib().rt4_file_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass

    def __len__(self) -> int:
        n = ctypes.c_int()
        _check(_lib().rt4_file_count(self._h, ctypes.byref(n)))
        return n.value

    def index(self, name: str) -> int:
        i = ctypes.c_int()
        _check(_lib().rt4_file_find(self._h, name.encode(), ctypes.byref(i)))
        return i.value

    def _info(self, i: int) -> TensorInfo:
        t = TensorInfo()
        _check(_lib().rt4_file_info(self._h, i, ctypes.byref(t)))
        return t

    def names(self) -> list[str]:
        return [self._info(i).name.decode() for i in range(len(self))]

    def size(self) -> int:
        b = ctypes.c_int64()
        _check(_lib().rt4_file_size(self._h, ctypes.byref(b)))
        return b.value

    def info(self, name: str) -> dict:
        t = self._info(self.index(name))
        return {"name": t.name.decode(), "kind": t.kind.decode(), "shape": list(t.shape[:t.ndim]),
                "group": t.group, "q_off": t.q_off, "s_off": t.s_off, "q_bytes": t.q_bytes,
                "s_bytes": t.s_bytes, "relerr": t.relerr, "src_rms": t.src_rms}

    def host(self, name: str):
        """numpy views of the mapping: i4 -> (codes uint32 [N, K/8], scales uint16 [N, K/group]);
        i8 -> (int8 [N, K], uint16 scales); plain kinds -> (raw uint8 bytes, None)."""
        i = self.index(name)
        t = self._info(i)
        q, s = ctypes.c_void_p(), ctypes.c_void_p()
        _check(_lib().rt4_file_data(self._h, i, ctypes.byref(q), ctypes.byref(s)))
        qb = np.ctypeslib.as_array((ctypes.c_uint8 * t.q_bytes).from_address(q.value))
        kind = t.kind.decode()
        if kind not in ("i4", "i8"):
            return qb, None
        N, K = t.shape[0], t.shape[1]
        sb = np.ctypeslib.as_array((ctypes.c_uint16 * (t.s_bytes // 2)).from_address(s.value)).reshape(N, K // t.group)
        codes = qb.view(np.uint32).reshape(N, K // 8) if kind == "i4" else qb.view(np.int8).reshape(N, K)
        return codes, sb

    def upload(self, name: str, device: str = "cuda"):
        """An i4 tensor as the kernels take it: (wq int32 [N, K/8], ws int16 [N, K/128])."""
        torch = _torch()
        i = self.index(name)
        t = self._info(i)
        if t.kind.decode() != "i4" or t.group != 128:
            raise ValueError(f"{name}: kind {t.kind.decode()} group {t.group}; the kernels take i4 with group 128")
        N, K = t.shape[0], t.shape[1]
        wq = torch.empty((N, K // 8), dtype=torch.int32, device=device)
        ws = torch.empty((N, K // 128), dtype=torch.int16, device=device)
        _check(_lib().rt4_file_upload_tensor(self._h, i, ctypes.c_void_p(wq.data_ptr()),
                                             ctypes.c_void_p(ws.data_ptr()), _stream()))
        return wq, ws

    def upload_all(self, device: str = "cuda"):
        """The whole weight file in one device buffer (uint8), as the reference runtime keeps it."""
        torch = _torch()
        n = self.size()
        buf = torch.empty(n, dtype=torch.uint8, device=device)
        _check(_lib().rt4_file_upload(self._h, ctypes.c_void_p(buf.data_ptr()), n, _stream()))
        return buf
