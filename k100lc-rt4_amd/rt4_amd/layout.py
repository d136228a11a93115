"""Host-side (numpy) helpers for the RT4 layouts used by librt4k.

RT4 packed int4 (docs/FORMAT.md:61-73 of the reference): a uint32 dword d of a
row holds elements k = 8d..8d+7, element k in bits 4*(k%8) .. 4*(k%8)+3, two's
complement, low nibble first.  The byte view therefore has the even element in
the low nibble.

Interleaved int8 (this library's activation layout): for every 8-element block
b, bytes [a(8b+0) a(8b+2) a(8b+4) a(8b+6) a(8b+1) a(8b+3) a(8b+5) a(8b+7)] -- the
order in which the MFMA kernels unpack the even and odd nibbles of a dword.
"""
from __future__ import annotations

import numpy as np

_PERM = np.array([0, 2, 4, 6, 1, 3, 5, 7])
_INV = np.argsort(_PERM)


def pack_rt4(codes: np.ndarray) -> np.ndarray:
    """int codes in [-8, 7], shape [..., K] (K % 8 == 0) -> uint32 [..., K/8]."""
    c = np.asarray(codes)
    if c.size and (c.min() < -8 or c.max() > 7):
        raise ValueError("RT4 codes must lie in [-8, 7]")
    c8 = c.astype(np.int8, copy=False).reshape(-1, c.shape[-1] // 8, 8)
    out = np.empty(c8.shape[:2], np.uint32)
    step = max(1, (1 << 22) // max(1, c8.shape[1]))  # bounded temporaries for huge inputs
    for r0 in range(0, c8.shape[0], step):
        blk = c8[r0:r0 + step].view(np.uint8) & np.uint8(0xF)
        acc = np.zeros(blk.shape[:2], np.uint32)
        for e in range(8):
            acc |= blk[:, :, e].astype(np.uint32) << np.uint32(4 * e)
        out[r0:r0 + step] = acc
    return out.reshape(*c.shape[:-1], c.shape[-1] // 8)


def unpack_rt4(wq: np.ndarray) -> np.ndarray:
    """uint32 [..., K/8] -> int8 codes [..., K]."""
    w = np.asarray(wq).astype(np.uint32)
    shifts = (4 * np.arange(8, dtype=np.uint32))
    nib = ((w[..., None] >> shifts) & 0xF).astype(np.int16)
    nib = np.where(nib >= 8, nib - 16, nib).astype(np.int8)
    return nib.reshape(*w.shape[:-1], w.shape[-1] * 8)


def interleave(codes: np.ndarray) -> np.ndarray:
    """Natural-order int8 [..., K] -> interleaved int8 [..., K]."""
    c = np.asarray(codes)
    blk = c.reshape(*c.shape[:-1], c.shape[-1] // 8, 8)
    return np.ascontiguousarray(blk[..., _PERM]).reshape(c.shape)


def deinterleave(xq: np.ndarray) -> np.ndarray:
    """Interleaved int8 [..., K] -> natural order int8 [..., K]."""
    c = np.asarray(xq)
    blk = c.reshape(*c.shape[:-1], c.shape[-1] // 8, 8)
    return np.ascontiguousarray(blk[..., _INV]).reshape(c.shape)


def f16_bits(scales: np.ndarray) -> np.ndarray:
    """float values -> their IEEE binary16 bit patterns (uint16, round to nearest even)."""
    return np.asarray(scales, dtype=np.float16).view(np.uint16)
