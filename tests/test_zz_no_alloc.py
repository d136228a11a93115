"""rt4_gemv_w4a8_noalloc: the drop-in decode linear with static device scratch.

Called through the C ABI (ctypes on librt4k.so) and compared bit for bit with
rt4_gemv_w4a8 (same launches, same split) on two calls in a row, the second
smaller, on shapes whose launch plan splits leftover tiles along K (so the
static partials and counters are exercised).  A fresh process also captures the
no-allocation call into a HIP graph as its very first library call, which
rt4_gemv_w4a8 refuses (its scratch would have to be allocated), and replays it.
"""
from __future__ import annotations

import ctypes
import subprocess
import sys
import textwrap

import pytest

from conftest import PKG_DIR, ROOT

pytestmark = pytest.mark.gpu


def _call(L, fn, y, wq, ws, x, rows, N, K, torch):
    P = ctypes.c_void_p
    st = P(torch.cuda.current_stream().cuda_stream)
    rc = getattr(L, fn)(P(y.data_ptr()), P(wq.data_ptr()), P(ws.data_ptr()), P(x.data_ptr()), rows, N, K, st)
    assert rc == 0, L.rt4_last_error().decode()


@pytest.mark.parametrize("calls", [[(4, 17408, 5120), (2, 3000, 2048)], [(4, 5120, 17408), (1, 5120, 5120)]])
def test_noalloc_matches_allocating_entry(rt4, torch_gpu, calls):
    torch = torch_gpu
    from rt4_amd import workload
    L = rt4.lib()
    gen = torch.Generator(device="cuda").manual_seed(11)
    for rows, N, K in calls:
        print(f"case noalloc rows={rows} N={N} K={K} plan={rt4.gemv_launch_plan(rows, N, K)}", flush=True)
        wq, ws = workload.weights_torch(N, K, generator=gen)
        x = workload.acts_torch(rows, K, generator=gen)
        y_ref = torch.full((rows, N), 7.0, device="cuda")
        y_na = torch.full((rows, N), -7.0, device="cuda")
        _call(L, "rt4_gemv_w4a8", y_ref, wq, ws, x, rows, N, K, torch)
        _call(L, "rt4_gemv_w4a8_noalloc", y_na, wq, ws, x, rows, N, K, torch)
        torch.cuda.synchronize()
        assert torch.equal(y_na.view(torch.int32), y_ref.view(torch.int32))


CHILD = textwrap.dedent(r"""
    import ctypes, sys
    sys.path[:0] = [{root!r}, {pkg!r}]
    import torch
    import rt4_amd
    from rt4_amd import workload
    torch.cuda.set_device(0)
    L = rt4_amd.lib()
    P = ctypes.c_void_p
    gen = torch.Generator(device="cuda").manual_seed(5)
    rows, N, K = 4, 17408, 5120
    wq, ws = workload.weights_torch(N, K, generator=gen)
    x = workload.acts_torch(rows, K, generator=gen)
    y = torch.empty((rows, N), device="cuda")
    torch.cuda.synchronize()
    args = lambda yy: (P(yy.data_ptr()), P(wq.data_ptr()), P(ws.data_ptr()), P(x.data_ptr()), rows, N, K,
                       P(torch.cuda.current_stream().cuda_stream))
    g = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(g):
        rcs.append(L.rt4_gemv_w4a8(*args(y)))
        rcs.append(L.rt4_gemv_w4a8_noalloc(*args(y)))
    print("first-call capture status: allocating", rcs[0], "no-alloc", rcs[1], flush=True)
    assert rcs[0] == 4 and rcs[1] == 0, rcs
    want = torch.empty_like(y)
    assert L.rt4_gemv_w4a8(*args(want)) == 0
    torch.cuda.synchronize()
    for _ in range(3):
        y.fill_(3.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), want.view(torch.int32))
    print("NOALLOC-CAPTURE-OK", flush=True)
""")


def test_noalloc_captured_as_first_call():
    print("case noalloc capture in a fresh process", flush=True)
    r = subprocess.run([sys.executable, "-u", "-c", CHILD.format(root=str(ROOT), pkg=str(PKG_DIR))],
                       capture_output=True, text=True, timeout=300)
    print(r.stdout[-3000:])
    print(r.stderr[-3000:])
    assert r.returncode == 0 and "NOALLOC-CAPTURE-OK" in r.stdout
