"""Synthetic inputs of the RT4 matmul path (the benchmark configurations).

Distributions follow the benchmark spec: int4 weight codes uniform in [-8, 7],
packed RT4-style; one fp16 scale per 128-group, |N(0,1)|*0.01 + 1e-3; fp16
N(0,1) activations upcast to fp32; for the prefill GEMM, 1% of activation
entries multiplied by 20 (outliers).  numpy generators draw codes, then scales,
then activations from ``numpy.random.default_rng(seed)``.

The device generators (``*_torch``) draw the same distributions with torch on
the GPU (random 32-bit words are exactly eight uniform nibbles, i.e. codes
uniform in [-8, 7]); they are used where only the distribution matters
(benchmarks at full size), never for parity fixtures.
"""
from __future__ import annotations

import numpy as np

from .layout import pack_rt4

GROUP = 128

# (name, M, N, K) of the benchmark shapes (27B layer shapes).
GEMV_SHAPES = {
    "c0": (1, 5120, 5120),
    "c1_gate_up": (4, 17408, 5120),
    "c1_down": (4, 5120, 17408),
    "c3_lm_head": (4, 248320, 5120),
}
GEMM_SHAPES = {
    "c2_gate_up": (1024, 17408, 5120),
    "c2_down": (1024, 5120, 17408),
}
# The reference's own prefill GEMM benchmark shape (bench/int4_gemm2.cpp:4-9):
# 2048 tokens against the 27B gate/up projection.
GEMM_REF_SHAPE = (2048, 17408, 5120)


def weights_np(rng: np.random.Generator, N: int, K: int):
    """-> (wq uint32 [N, K/8], ws uint16 fp16-bits [N, K/128], codes int8 [N, K])."""
    codes = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    scales = (np.abs(rng.standard_normal((N, K // GROUP))) * 0.01 + 1e-3).astype(np.float16)
    return pack_rt4(codes), scales.view(np.uint16), codes


def acts_np(rng: np.random.Generator, M: int, K: int, outliers: bool = False) -> np.ndarray:
    x = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
    if outliers:
        mask = rng.random((M, K)) < 0.01
        x = np.where(mask, x * np.float32(20.0), x).astype(np.float32)
    return x


def gemv_case(seed: int, M: int, N: int, K: int) -> dict:
    rng = np.random.default_rng(seed)
    wq, ws, codes = weights_np(rng, N, K)
    x = acts_np(rng, M, K)
    return {"wq": wq, "ws": ws, "codes": codes, "x": x, "M": M, "N": N, "K": K}


def gemm_case(seed: int, M: int, N: int, K: int) -> dict:
    rng = np.random.default_rng(seed)
    wq, ws, codes = weights_np(rng, N, K)
    x = acts_np(rng, M, K, outliers=True)
    return {"wq": wq, "ws": ws, "codes": codes, "x": x, "M": M, "N": N, "K": K}


# ------------------------------------------------------------ device side --
def weights_torch(N: int, K: int, device="cuda", generator=None):
    """Random RT4 weights on the device: (wq int32 [N, K/8], ws int16 fp16-bits [N, K/128])."""
    import torch
    w = torch.randint(0, 2**32, (N, K // 8), dtype=torch.int64, device=device, generator=generator)
    wq = torch.where(w >= 2**31, w - 2**32, w).to(torch.int32)  # all 32-bit patterns, uniform
    s = torch.randn((N, K // GROUP), device=device, generator=generator).abs() * 0.01 + 1e-3
    ws = s.to(torch.float16).view(torch.int16)
    return wq, ws


def acts_torch(M: int, K: int, outliers: bool = False, device="cuda", generator=None):
    import torch
    x = torch.randn((M, K), device=device, generator=generator).to(torch.float16).to(torch.float32)
    if outliers:
        mask = torch.rand((M, K), device=device, generator=generator) < 0.01
        x = torch.where(mask, x * 20.0, x)
    return x.contiguous()


# ------------------------------------------------------------- attention --
# 24 query heads, 4 KV heads (GQA 6:1), head dim 256, 1024 new query
# rows over a 32768-token cache -> n_kv = 33792, query i at position 32768 + i.
ATTN_C4 = {"H": 24, "KVH": 4, "D": 256, "n_q": 1024, "ctx": 32768}
# The reference's own FlashAttention benchmark shape (docs/FLASH-ATTN.md:78-80): the
# same heads, 1024 new query rows over a 131072-token cache.
ATTN_REF = {"H": 24, "KVH": 4, "D": 256, "n_q": 1024, "ctx": 131072}


def attn_np(rng: np.random.Generator, T: int, n_kv: int, H: int, KVH: int, D: int = 256):
    """fp16 N(0,1) Q [T, H, D] (scaled by 1/sqrt(D), as src/model.cpp:1067 does before
    quantizing), K and V [n_kv, KVH, D], upcast to fp32."""
    q = rng.standard_normal((T, H, D)).astype(np.float16).astype(np.float32) * np.float32(1.0 / np.sqrt(D))
    k = rng.standard_normal((n_kv, KVH, D)).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((n_kv, KVH, D)).astype(np.float16).astype(np.float32)
    return q.astype(np.float32), k, v


def attn_torch(T: int, n_kv: int, H: int, KVH: int, D: int = 256, device="cuda", generator=None):
    import torch
    q = torch.randn((T, H, D), device=device, generator=generator).to(torch.float16).to(torch.float32) * (D ** -0.5)
    k = torch.randn((n_kv, KVH, D), device=device, generator=generator).to(torch.float16).to(torch.float32)
    v = torch.randn((n_kv, KVH, D), device=device, generator=generator).to(torch.float16).to(torch.float32)
    return q.contiguous(), k.contiguous(), v.contiguous()
