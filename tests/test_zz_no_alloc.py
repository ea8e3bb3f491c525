"""mc_rmsnorm_bwd_noalloc (the allocation-free variant of mc_rmsnorm_bwd, for
callers that cannot allocate device memory) against mc_rmsnorm_bwd, both
called through the C ABI with ctypes.

Both entry points run the same kernels with the same row partition; only
the home of the dw partials differs (the caller's workspace, or the
library's static device scratch). dx and dw must therefore agree bit for bit.
Two calls in a row, the second on a smaller input, check that the second
call does not depend on what the first left in the scratch. The oracle
checks the no-alloc outputs to the fp32 / bf16 tolerance as well.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def _vp(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _inputs(dev, rows, dim, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, dim, generator=g).to(dtype)
    w = (torch.randn(dim, generator=g) * 0.1 + 1.0).to(dtype)
    dy = (torch.randn(rows, dim, generator=g) * 1e-2).to(dtype)
    return x.to(dev), w.to(dev), dy.to(dev)


def _both(mc, dev, rows, dim, dtype, seed, eps=1e-6):
    """(dx, dw) from mc_rmsnorm_bwd and from mc_rmsnorm_bwd_noalloc."""
    L = mc._lib.lib()
    code = mc._lib.MC_F32 if dtype == torch.float32 else mc._lib.MC_BF16
    x, w, dy = _inputs(dev, rows, dim, dtype, seed)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    need = L.mc_rmsnorm_bwd_workspace_size(rows, dim)
    assert 0 < need <= SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    dx_ref, dw_ref = torch.empty_like(x), torch.empty(dim, dtype=torch.float32, device=dev)
    mc._lib.check(L.mc_rmsnorm_bwd(rows, dim, eps, code, _vp(x), _vp(w), None, _vp(dy), _vp(dx_ref),
                                   _vp(dw_ref), _vp(ws), need, stream))
    dx, dw = torch.full_like(x, float("nan")), torch.full((dim,), float("nan"), device=dev)
    mc._lib.check(L.mc_rmsnorm_bwd_noalloc(rows, dim, eps, code, _vp(x), _vp(w), None, _vp(dy), _vp(dx),
                                           _vp(dw), stream))
    torch.cuda.synchronize()
    return (x, w, dy), (dx_ref, dw_ref), (dx, dw)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_no_alloc_matches_workspace_entry(mc, dev, dtype):
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    # second call smaller than the first (fewer rows and a narrower dim)
    for rows, dim, seed in ((4096, 1536, 1), (300, 896, 2)):
        (x, w, dy), (dx_ref, dw_ref), (dx, dw) = _both(mc, dev, rows, dim, dtype, seed)
        print(f"no-alloc rmsnorm bwd {dtype} rows={rows} dim={dim}", flush=True)
        assert torch.equal(dx, dx_ref), "dx differs from mc_rmsnorm_bwd"
        assert torch.equal(dw, dw_ref), "dw differs from mc_rmsnorm_bwd"
        xo, wo, dyo = (t.float().cpu().numpy() for t in (x, w, dy))
        dx_o, dw_o = oracle.rmsnorm_bwd(xo, dyo, 1e-6, w=wo)
        assert rel_err(dx, dx_o) <= tol
        assert rel_err(dw, dw_o) <= 1e-4


def test_no_alloc_rejects_oversize(mc, dev):
    """Partials beyond the static scratch are rejected on the host with
    MC_ERR_SHAPE before anything is enqueued; dw = NULL needs no scratch."""
    L = mc._lib.lib()
    rows, dim = 1 << 16, 16384  # 512 partial rows x 16384 x 4 B = 32 MiB
    assert L.mc_rmsnorm_bwd_workspace_size(rows, dim) > SCRATCH_BYTES
    fake = ctypes.c_void_p(256)
    st = L.mc_rmsnorm_bwd_noalloc(rows, dim, 1e-6, 1, fake, None, None, fake, fake, fake, None)
    assert st == mc._lib.MC_ERR_SHAPE
    assert "static scratch" in mc._lib.last_error()
    # without dw the scratch is not used, so any size runs
    x, w, dy = _inputs(dev, 64, 16384, torch.bfloat16, 3)
    dx = torch.empty_like(x)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    mc._lib.check(L.mc_rmsnorm_bwd_noalloc(64, 16384, 1e-6, 1, _vp(x), _vp(w), None, _vp(dy), _vp(dx), None,
                                           stream))
    torch.cuda.synchronize()
    dx_o, _ = oracle.rmsnorm_bwd(x.float().cpu().numpy(), dy.float().cpu().numpy(), 1e-6,
                                 w=w.float().cpu().numpy())
    assert rel_err(dx, dx_o) <= 2e-2


def _noalloc_call(mc, L, x, w, dy, dx, dw, code, stream):
    rows, dim = x.shape
    mc._lib.check(L.mc_rmsnorm_bwd_noalloc(rows, dim, 1e-6, code, _vp(x), _vp(w), None, _vp(dy), _vp(dx), _vp(dw),
                                           stream))


def test_no_alloc_under_graph_capture(mc, dev):
    """Captured in a HIP graph (torch.cuda.CUDAGraph on the current stream),
    the entry point records only kernel launches: replays, with eager calls
    of it on another shape in between (which overwrite the shared scratch),
    give dx and dw bitwise equal to the eager call on every replay."""
    L = mc._lib.lib()
    code = mc._lib.MC_BF16
    x, w, dy = _inputs(dev, 2048, 1536, torch.bfloat16, 11)
    xo, wo, dyo = _inputs(dev, 512, 896, torch.bfloat16, 12)
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)  # noqa: E731
    dx_e, dw_e = torch.empty_like(x), torch.empty(1536, dtype=torch.float32, device=dev)
    _noalloc_call(mc, L, x, w, dy, dx_e, dw_e, code, cur())
    torch.cuda.synchronize()
    dx, dw = torch.full_like(x, float("nan")), torch.full((1536,), float("nan"), device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _noalloc_call(mc, L, x, w, dy, dx, dw, code, cur())
    torch.cuda.synchronize()
    dx_o, dw_o = torch.empty_like(xo), torch.empty(896, dtype=torch.float32, device=dev)
    for rep in range(3):
        _noalloc_call(mc, L, xo, wo, dyo, dx_o, dw_o, code, cur())  # other contents in the scratch
        torch.cuda.synchronize()
        dx.fill_(float("nan"))
        dw.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        print(f"no-alloc graph replay {rep}", flush=True)
        assert torch.equal(dx, dx_e) and torch.equal(dw, dw_e), f"replay {rep} differs from the eager call"


_FIRST_CALL_IN_CAPTURE = r"""
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[1])
import __graft_entry__ as ge
mc = ge.load_package()
L = mc._lib.lib()
dev = torch.device("cuda:0")
g = torch.Generator().manual_seed(13)
x = torch.randn(1024, 1536, generator=g).to(torch.bfloat16).to(dev)
w = (torch.randn(1536, generator=g) * 0.1 + 1).to(torch.bfloat16).to(dev)
dy = (torch.randn(1024, 1536, generator=g) * 1e-2).to(torch.bfloat16).to(dev)
vp = lambda t: ctypes.c_void_p(t.data_ptr())
dx, dw = torch.empty_like(x), torch.empty(1536, dtype=torch.float32, device=dev)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):  # the process's first call of the entry point
    st = L.mc_rmsnorm_bwd_noalloc(1024, 1536, 1e-6, 1, vp(x), vp(w), None, vp(dy), vp(dx), vp(dw),
                                  ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
torch.cuda.synchronize()
assert st == 0, (st, mc._lib.last_error())
graph.replay()
torch.cuda.synchronize()
ws_n = L.mc_rmsnorm_bwd_workspace_size(1024, 1536)
ws = torch.empty(ws_n, dtype=torch.uint8, device=dev)
dx_r, dw_r = torch.empty_like(x), torch.empty(1536, dtype=torch.float32, device=dev)
mc._lib.check(L.mc_rmsnorm_bwd(1024, 1536, 1e-6, 1, vp(x), vp(w), None, vp(dy), vp(dx_r), vp(dw_r), vp(ws), ws_n,
                               ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
torch.cuda.synchronize()
assert torch.equal(dx, dx_r) and torch.equal(dw, dw_r), "first-call capture differs from mc_rmsnorm_bwd"
print("FIRST_CALL_IN_CAPTURE_OK", flush=True)
"""


def test_no_alloc_first_call_during_capture():
    """A process whose first call of the entry point happens under graph
    capture (the per-device scratch address is looked up during the capture)
    gets a graph whose replay equals mc_rmsnorm_bwd bit for bit. Run in a
    fresh process, since any earlier call in this one has already looked the
    address up."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("no-alloc first call under capture (subprocess)", flush=True)
    p = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE, root], capture_output=True, text=True,
                       timeout=180)
    assert p.returncode == 0 and "FIRST_CALL_IN_CAPTURE_OK" in p.stdout, (p.stdout + p.stderr)[-3000:]
