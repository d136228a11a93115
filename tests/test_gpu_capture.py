"""HIP graph capture of calls whose library scratch does not exist yet.

Nothing may be allocated while a stream is being captured.  In a fresh process
(library scratch empty) the test captures:

* the prefill GEMM: its split-tile workspace would have to be allocated, so the
  call fails with RT4_E_CAPTURE and nothing is recorded; after one eager call at
  the shape the same capture succeeds and every replay equals the eager result;
* the drop-in decode linear (quantizer scratch): the same;
* the attention prefill with an automatic split count: it falls back to one
  split (no workspace) and every replay equals the eager one-split result.

Then it frees the library scratch (rt4_release_scratch): the GEMM capture fails
again until an eager call re-allocates it, and the re-run calls are bit-identical.

Each replay is preceded by eager work and a synchronisation, and checked bit for
bit.  The child process runs the whole sequence and prints one line per check.
"""
from __future__ import annotations

import subprocess
import sys
import textwrap

import pytest

from conftest import PKG_DIR, ROOT

pytestmark = pytest.mark.gpu

CHILD = textwrap.dedent(r"""
    import sys
    sys.path[:0] = [{root!r}, {pkg!r}]
    import torch
    import rt4_amd
    from rt4_amd import workload

    torch.cuda.set_device(0)
    gen = torch.Generator(device="cuda").manual_seed(3)

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        err = None
        with torch.cuda.graph(g):
            try:
                fn()
            except rt4_amd.RT4Error as e:
                err = str(e)
        return g, err

    def replays_equal(g, out, want):
        for _ in range(3):
            out.fill_(7.0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            if not torch.equal(out.view(torch.int32), want.view(torch.int32)):
                return False
        return True

    # ---- prefill GEMM
    M, N, K = 512, 2304, 1024
    wq, ws = workload.weights_torch(N, K, generator=gen)
    sb = rt4_amd.make_group_major(ws, K)
    x = workload.acts_torch(M, K, outliers=True, generator=gen)
    xq, sc = rt4_amd.quant_rows_i8(x)
    c = torch.empty((M, N), device="cuda")
    torch.cuda.synchronize()
    g, err = capture(lambda: rt4_amd.gemm_w4a8_i8(wq, sb, xq, sc, out=c))
    print("gemm first capture:", err, flush=True)
    assert err is not None and "captur" in err, err
    want = rt4_amd.gemm_w4a8_i8(wq, sb, xq, sc).clone()
    torch.cuda.synchronize()
    g, err = capture(lambda: rt4_amd.gemm_w4a8_i8(wq, sb, xq, sc, out=c))
    assert err is None, err
    assert replays_equal(g, c, want)
    print("gemm replays equal eager", flush=True)

    # ---- drop-in decode linear (quantizer scratch)
    Nd, Kd = 4096, 5120
    wq2, ws2 = workload.weights_torch(Nd, Kd, generator=gen)
    xa = workload.acts_torch(4, Kd, generator=gen)
    y = torch.empty((4, Nd), device="cuda")
    g, err = capture(lambda: rt4_amd.gemv_w4a8(wq2, ws2, xa, out=y))
    print("gemv first capture:", err, flush=True)
    assert err is not None and "captur" in err, err
    wantv = rt4_amd.gemv_w4a8(wq2, ws2, xa).clone()
    torch.cuda.synchronize()
    g, err = capture(lambda: rt4_amd.gemv_w4a8(wq2, ws2, xa, out=y))
    assert err is None, err
    assert replays_equal(g, y, wantv)
    print("gemv replays equal eager", flush=True)

    # ---- attention prefill, automatic split count, no workspace yet
    H, KVH, n_q, n_kv = 8, 2, 128, 4096
    q, k, v = workload.attn_torch(n_q, n_kv, H, KVH, generator=gen)
    qq, qs = rt4_amd.attn_q_quant(q, n_q)
    kc = torch.zeros((KVH, n_kv, 32), dtype=torch.int32, device="cuda")
    ksc = torch.ones((KVH, 2, n_kv), device="cuda")
    vc = torch.zeros((KVH, n_kv // 8, 256), dtype=torch.int32, device="cuda")
    vsc = torch.ones((KVH, n_kv // 64, 256), device="cuda")
    st = torch.zeros((KVH, 64, 256), device="cuda")
    rt4_amd.kv_append_k(kc, ksc, k, 0)
    rt4_amd.kv_append_v(vc, vsc, st, v, 0)
    out = torch.empty((H, n_q, 256), device="cuda")
    kw = dict(n_kv=n_kv, off=n_kv - n_q, ratio=H // KVH)
    torch.cuda.synchronize()
    g, err = capture(lambda: rt4_amd.attention_prefill(qq, qs, kc, ksc, vc, vsc, out=out, **kw))
    assert err is None, err
    want1 = rt4_amd.attention_prefill(qq, qs, kc, ksc, vc, vsc, kv_splits=1, **kw).clone()
    auto = rt4_amd.attention_prefill(qq, qs, kc, ksc, vc, vsc, **kw).clone()
    torch.cuda.synchronize()
    assert replays_equal(g, out, want1)
    rel = float((auto - want1).norm() / want1.norm())
    print(f"attention captured without workspace = one split; eager automatic split vs one split {{rel:.2e}}",
          flush=True)
    assert rel < 1e-5

    # ---- release the scratch: capture needs an eager call again, results unchanged
    del g
    rt4_amd.release_scratch()
    g, err = capture(lambda: rt4_amd.gemm_w4a8_i8(wq, sb, xq, sc, out=c))
    print("gemm capture after release:", err, flush=True)
    assert err is not None and "captur" in err, err
    again = rt4_amd.gemm_w4a8_i8(wq, sb, xq, sc).clone()
    againv = rt4_amd.gemv_w4a8(wq2, ws2, xa).clone()
    againa = rt4_amd.attention_prefill(qq, qs, kc, ksc, vc, vsc, **kw).clone()
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int32), want.view(torch.int32))
    assert torch.equal(againv.view(torch.int32), wantv.view(torch.int32))
    assert torch.equal(againa.view(torch.int32), auto.view(torch.int32))
    rt4_amd.release_scratch()
    rt4_amd.release_scratch()   # nothing left to free: still fine
    print("release: re-allocated scratch gives bit-identical GEMM, GEMV and attention", flush=True)

    print("CAPTURE-OK", flush=True)
""")


def test_capture_before_any_eager_call():
    print("case capture in a fresh process (GEMM, drop-in GEMV, attention)", flush=True)
    code = CHILD.format(root=str(ROOT), pkg=str(PKG_DIR))
    r = subprocess.run([sys.executable, "-u", "-c", code], capture_output=True, text=True, timeout=300)
    print(r.stdout[-4000:])
    print(r.stderr[-4000:])
    assert r.returncode == 0 and "CAPTURE-OK" in r.stdout
