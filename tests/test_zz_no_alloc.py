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
