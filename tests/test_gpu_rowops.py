"""GPU parity of RMSNorm and softmax (fwd + bwd) against the CPU oracle.

Shapes: the reference's own fused-vs-candle test shapes
(tests/rmsnorm_correctness.rs:40-265, tests/softmax_correctness.rs:30-243),
their known answers (src/backend/tensor.rs:126-420, tests/executor_direct.rs:
480-495), and BASELINE.json's configs at full size, where the oracle runs on a
seeded sample of rows (rows are independent) and size-independent properties
(rows of P sum to 1, rows of dS sum to 0, exact zeros under the mask) are
checked on every row. Tolerance: max|out-ref|/max|ref| <= 1e-5 (fp32),
<= 2e-2 (bf16).
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err, to_np

pytestmark = pytest.mark.gpu

F32_TOL, BF16_TOL = 1e-5, 2e-2
REF_SHAPES = [(4, 1024), (2, 128, 512), (1, 512), (16, 256), (1, 128, 768), (4, 64, 1024)]


def _tol(dtype):
    return F32_TOL if dtype == torch.float32 else BF16_TOL


# ------------------------------------------------------------------ RMSNorm
@pytest.mark.parametrize("shape", REF_SHAPES + [(3, 5), (2, 7, 3), (1, 1), (5, 2), (8192, 896), (37, 4100),
                                   (5, 16384), (3, 32768), (2, 32772), (4, 4098)])
@pytest.mark.parametrize("weighted", [False, True])
def test_rmsnorm_fwd_f32(mc, dev, shape, weighted):
    g = torch.Generator().manual_seed(hash((shape, weighted)) % 2**31)
    x = torch.randn(*shape, generator=g)
    w = torch.randn(shape[-1], generator=g) * 0.1 + 1.0 if weighted else None
    y, rstd = mc.rms_norm_forward(x.to(dev), 1e-6, None if w is None else w.to(dev))
    y_ref, r_ref = oracle.rmsnorm_fwd(x.numpy(), 1e-6, None if w is None else w.numpy())
    assert rel_err(y, y_ref) <= F32_TOL
    assert rel_err(rstd, r_ref) <= F32_TOL


def test_rmsnorm_known_answers(mc, dev):
    # executor_direct.rs:480-495: [3, 4], eps 0 -> [0.8485, 1.1314]
    y, _ = mc.rms_norm_forward(torch.tensor([3.0, 4.0], device=dev), 0.0)
    assert np.allclose(to_np(y), [0.8485, 1.1314], atol=1e-3)
    assert rel_err(y, [3 / np.sqrt(12.5), 4 / np.sqrt(12.5)]) <= F32_TOL
    # tensor.rs:382-397: [2, 4, 6] keeps ratios 2, 3
    y, _ = mc.rms_norm_forward(torch.tensor([[2.0, 4.0, 6.0]], device=dev), 1e-6)
    v = to_np(y)[0]
    assert abs(v[1] / v[0] - 2) < 1e-4 and abs(v[2] / v[0] - 3) < 1e-4
    # tensor.rs:400-420: single value -> 1
    y, _ = mc.rms_norm_forward(torch.tensor([[5.0]], device=dev), 1e-6)
    assert abs(to_np(y)[0, 0] - 1) < 1e-5
    # rmsnorm_correctness.rs:205-265: constant rows 100 / 0.01 at eps 1e-5 (closed form c/sqrt(c^2+eps))
    for c in (100.0, 0.01):
        y, _ = mc.rms_norm_forward(torch.full((2, 256), c, device=dev), 1e-5)
        assert rel_err(y, np.full((2, 256), c / np.sqrt(c * c + 1e-5))) <= F32_TOL


@pytest.mark.parametrize("shape", [(16384, 1536), (64, 3584), (4, 1024), (2, 24), (16, 8200), (4, 16384), (8, 65536),
                                   (2, 65544)])
def test_rmsnorm_fwd_bf16(mc, dev, shape):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(*shape, generator=g).to(torch.bfloat16)
    w = (torch.randn(shape[-1], generator=g) * 0.1 + 1.0).to(torch.bfloat16)
    y, _ = mc.rms_norm_forward(x.to(dev), 1e-6, w.to(dev))
    y_ref, _ = oracle.rmsnorm_fwd(x.float().numpy(), 1e-6, w.float().numpy())
    assert rel_err(y, y_ref) <= BF16_TOL


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(8192, 896), (4, 64, 1024), (3, 5), (1, 1), (300, 8), (16, 8200), (600, 5120),
                                   (4097, 5120), (64, 8192), (3, 16384), (2, 16392), (256, 3584), (40, 2056)])
@pytest.mark.parametrize("use_rstd", [False, True])
def test_rmsnorm_bwd(mc, dev, dtype, shape, use_rstd):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(*shape, generator=g).to(dtype)
    w = (torch.randn(shape[-1], generator=g) * 0.1 + 1.0).to(dtype)
    dy = torch.randn(*shape, generator=g).to(dtype)
    xd, wd, dyd = x.to(dev), w.to(dev), dy.to(dev)
    _, rstd = mc.rms_norm_forward(xd, 1e-6, wd)
    dx, dw = mc.rms_norm_backward(xd, dyd, 1e-6, wd, rstd if use_rstd else None)
    dx_ref, dw_ref = oracle.rmsnorm_bwd(x.float().numpy(), dy.float().numpy(), 1e-6, w.float().numpy())
    tol = _tol(dtype)
    # dx = r*g - x*r^3*mean(g*x) cancels to ~eps for dim = 1; measure the error
    # against the size of its terms (r*g) where that exceeds the result
    _, r_ref = oracle.rmsnorm_fwd(x.float().numpy(), 1e-6, w.float().numpy())
    terms = np.abs(dy.float().numpy() * w.float().numpy() * r_ref.reshape(x.shape[:-1] + (1,))).max()
    err = np.abs(to_np(dx).astype(np.float64) - dx_ref).max() / max(np.abs(dx_ref).max(), terms)
    assert err <= tol
    assert rel_err(dw, dw_ref) <= (1e-5 if dtype == torch.float32 else 1e-4)  # dw accumulates in fp32
    # fixed-order split reduction: bitwise reproducible
    dx2, dw2 = mc.rms_norm_backward(xd, dyd, 1e-6, wd, rstd if use_rstd else None)
    assert torch.equal(dw, dw2) and torch.equal(dx, dx2)


def test_rmsnorm_bwd_unweighted_no_dw(mc, dev):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(128, 768, generator=g)
    dy = torch.randn(128, 768, generator=g)
    dx, dw = mc.rms_norm_backward(x.to(dev), dy.to(dev), 1e-5, None, None, need_dw=False)
    assert dw is None
    dx_ref, _ = oracle.rmsnorm_bwd(x.numpy(), dy.numpy(), 1e-5)
    assert rel_err(dx, dx_ref) <= F32_TOL


# ------------------------------------------------------------------ softmax
@pytest.mark.parametrize("shape", REF_SHAPES + [(1, 3), (2, 5), (3, 1), (7, 4100), (2, 4096)])
def test_softmax_fwd_f32(mc, dev, shape):
    g = torch.Generator().manual_seed(5)
    s = torch.randn(*shape, generator=g) * 3
    p = mc.softmax_forward(s.to(dev))
    assert rel_err(p, oracle.softmax_fwd(s.numpy())) <= F32_TOL
    assert np.allclose(to_np(p).sum(-1), 1.0, atol=1e-5)


def test_softmax_known_answers(mc, dev):
    # tensor.rs:262-276: zeros -> 1/3
    p = mc.softmax_forward(torch.zeros(1, 3, device=dev))
    assert np.allclose(to_np(p), 1 / 3, atol=1e-6)
    # tensor.rs:146-162: [100, 200, 300] stays finite, sums to 1
    p = to_np(mc.softmax_forward(torch.tensor([[100.0, 200.0, 300.0]], device=dev)))
    assert np.isfinite(p).all() and abs(p.sum() - 1) < 1e-6 and abs(p[0, 2] - 1) < 1e-6
    # softmax_correctness.rs:200-243: constant +-100 rows -> uniform
    for c in (100.0, -100.0):
        p = mc.softmax_forward(torch.full((2, 256), c, device=dev))
        assert np.allclose(to_np(p), 1 / 256, rtol=1e-6)
    # tensor.rs:400-420: single value -> 1
    assert abs(to_np(mc.softmax_forward(torch.tensor([[5.0]], device=dev)))[0, 0] - 1) < 1e-6
    # shift invariance
    g = torch.Generator().manual_seed(1)
    s = torch.randn(4, 1024, generator=g)
    assert rel_err(mc.softmax_forward((s + 17.0).to(dev)), to_np(mc.softmax_forward(s.to(dev)))) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,dim,causal", [(64, 64, 64), (2 * 100, 100, 100), (3 * 8, 24, 8), (16, 1024, 16),
                                             (5, 7, 5), (4 * 48, 4096, 48)])
def test_softmax_causal(mc, dev, dtype, rows, dim, causal):
    g = torch.Generator().manual_seed(9)
    s = (torch.randn(rows, dim, generator=g) * 3).to(dtype)
    dp = (torch.randn(rows, dim, generator=g) * 1e-2).to(dtype)
    p = mc.softmax_forward(s.to(dev), causal_rows=causal)
    p_ref = oracle.softmax_fwd(s.float().numpy(), causal_rows=causal)
    assert rel_err(p, p_ref) <= _tol(dtype)
    pn = to_np(p)
    masked = p_ref == 0
    assert (pn[masked] == 0).all()  # exact zeros under the mask
    ds = mc.softmax_backward(p, dp.to(dev), causal_rows=causal)
    ds_ref = oracle.softmax_bwd(pn, dp.float().numpy(), causal_rows=causal)
    assert rel_err(ds, ds_ref) <= _tol(dtype)
    assert (to_np(ds)[masked] == 0).all()


@pytest.mark.parametrize("shape", REF_SHAPES + [(1, 3), (7, 4100)])
def test_softmax_bwd_f32(mc, dev, shape):
    g = torch.Generator().manual_seed(13)
    s = torch.randn(*shape, generator=g) * 3
    dp = torch.randn(*shape, generator=g) * 1e-2
    p = mc.softmax_forward(s.to(dev))
    ds = mc.softmax_backward(p, dp.to(dev))
    ds_ref = oracle.softmax_bwd(to_np(p), dp.numpy())
    assert rel_err(ds, ds_ref) <= F32_TOL
    assert np.abs(to_np(ds).sum(-1)).max() <= 1e-6  # rows of dS sum to 0


# Rows past the one-wave paths (8 vectors per lane: fp32 2048, bf16 4096
# columns): a workgroup per row with the row in the registers of up to 1024
# threads (fp32 to 32768, bf16 to 65536 columns; the bf16 backward to 32768),
# two streaming passes past that, and the scalar kernels for rows that are
# not whole 16-byte vectors (4098 fp32 columns).
@pytest.mark.parametrize("dtype,rows,dim,causal", [
    (torch.float32, 3, 4100, 0), (torch.float32, 3, 16384, 0), (torch.float32, 2, 32768, 0),
    (torch.float32, 2, 40000, 0), (torch.float32, 3, 4098, 0), (torch.float32, 40, 40000, 40),
    (torch.bfloat16, 5, 6144, 0), (torch.bfloat16, 64, 8192, 64), (torch.float32, 6, 3000, 0),
    (torch.bfloat16, 3, 8200, 0), (torch.bfloat16, 2, 40000, 0), (torch.bfloat16, 2, 65536, 0),
    (torch.bfloat16, 2, 70000, 0), (torch.bfloat16, 64, 20000, 20000), (torch.bfloat16, 64, 70000, 70000)])
def test_softmax_long_rows(mc, dev, dtype, rows, dim, causal):
    g = torch.Generator().manual_seed(rows * 7 + dim)
    s = (torch.randn(rows, dim, generator=g) * 3).to(dtype)
    dp = (torch.randn(rows, dim, generator=g) * 1e-2).to(dtype)
    p = mc.softmax_forward(s.to(dev), causal_rows=causal)
    p_ref = oracle.softmax_fwd(s.float().numpy(), causal_rows=causal)
    assert rel_err(p, p_ref) <= _tol(dtype)
    pn = to_np(p)
    cols = np.arange(dim)[None, :]
    lim = (np.arange(rows) % causal + (dim - causal))[:, None] if causal else np.full((rows, 1), dim - 1)
    masked = cols > lim
    assert (pn[masked] == 0).all()
    assert np.abs(pn.astype(np.float64).sum(-1) - 1).max() <= (1e-5 if dtype == torch.float32 else 2e-2)
    ds = mc.softmax_backward(p, dp.to(dev), causal_rows=causal)
    ds_ref = oracle.softmax_bwd(pn, dp.float().numpy(), causal_rows=causal)
    assert rel_err(ds, ds_ref) <= _tol(dtype)
    assert (to_np(ds)[masked] == 0).all()


def _sampled_rows(n_rows, k, seed):
    return np.sort(np.random.default_rng(seed).choice(n_rows, size=min(k, n_rows), replace=False))


@pytest.mark.parametrize("dtype,shape", [(torch.float32, (8, 14, 1024, 1024)), (torch.bfloat16, (8, 12, 2048, 2048)),
                                         (torch.bfloat16, (1, 1, 16384, 16384)), (torch.float32, (1, 1, 16384, 16384))])
def test_softmax_config_full_size(mc, dev, dtype, shape):
    """BASELINE.json c2 (fp32) and the c4 attention softmax (bf16), causal, fwd + bwd; and a 16384-token causal
    score matrix, whose rows take the workgroup-per-row kernels."""
    S = shape[-1]
    gen = torch.Generator(device=dev).manual_seed(2024)
    s = (torch.randn(*shape, generator=gen, device=dev) * 3).to(dtype)
    dp = (torch.randn(*shape, generator=gen, device=dev) * 1e-2).to(dtype)
    p = mc.softmax_forward(s, causal_rows=S)
    ds = mc.softmax_backward(p, dp, causal_rows=S)
    torch.cuda.synchronize()
    rows = s.numel() // S
    idx = torch.from_numpy(_sampled_rows(rows, 512, 1)).to(dev)
    s2, p2, dp2, ds2 = (t.reshape(rows, S).index_select(0, idx) for t in (s, p, dp, ds))
    ids = idx.cpu().numpy()
    p_ref = oracle.softmax_fwd(to_np(s2), causal_rows=S, row_ids=ids)
    assert rel_err(p2, p_ref) <= _tol(dtype)
    ds_ref = oracle.softmax_bwd(to_np(p2), to_np(dp2), causal_rows=S, row_ids=ids)
    assert rel_err(ds2, ds_ref) <= _tol(dtype)
    # properties on every row
    pf = p.reshape(rows, S).float()
    assert torch.allclose(pf.sum(-1), torch.ones(rows, device=dev), atol=1e-5 if dtype == torch.float32 else 2e-2)
    cols = torch.arange(S, device=dev)
    qpos = torch.arange(S, device=dev)[:, None]
    mask = (cols[None, :] > qpos)
    assert (p.reshape(-1, S, S)[:, mask] == 0).all()
    assert (ds.reshape(-1, S, S)[:, mask] == 0).all()


@pytest.mark.parametrize("dim", [4, 3])
def test_softmax_rows_past_one_launch(mc, dev, dim):
    """2^26 + 37 short rows: more than one launch's 2^32 - 1 work-items at one
    wave per row, so the forward (4 rows per 256 threads) and the backward (one
    row per 64 threads) split the rows over two launches; dim 3 takes the
    scalar kernels. Causal over 3 columns, so each row's mask depends on its
    global index across the launch boundary. Rows next to the boundaries and a
    seeded sample are checked against the oracle; P's row sums on every row."""
    rows, S = (1 << 26) + 37, 3
    gen = torch.Generator(device=dev).manual_seed(7)
    s = torch.randn(rows, dim, generator=gen, device=dev) * 3
    dp = torch.randn(rows, dim, generator=gen, device=dev)
    p = mc.softmax_forward(s, causal_rows=S)
    ds = mc.softmax_backward(p, dp, causal_rows=S)
    torch.cuda.synchronize()
    fwd_cap, bwd_cap = ((2**32 - 1) // 256) * 4, (2**32 - 1) // 64
    edge = [0, 1, 2, 3, rows - 3, rows - 2, rows - 1]
    for c in (fwd_cap, bwd_cap):
        edge += list(range(c - 3, c + 3))
    ids = np.unique(np.concatenate([np.array(edge), _sampled_rows(rows, 256, 3)]))
    idx = torch.from_numpy(ids).to(dev)
    s2, p2, dp2, ds2 = (t.index_select(0, idx) for t in (s, p, dp, ds))
    p_ref = oracle.softmax_fwd(to_np(s2), causal_rows=S, row_ids=ids)
    assert rel_err(p2, p_ref) <= F32_TOL
    ds_ref = oracle.softmax_bwd(to_np(p2), to_np(dp2), causal_rows=S, row_ids=ids)
    assert rel_err(ds2, ds_ref) <= F32_TOL
    assert torch.allclose(p.sum(-1), torch.ones(rows, device=dev), atol=1e-5)


def test_norm_bwd_many_calls_and_streams(mc, dev):
    """The fixed-order dw (and LayerNorm's db) reductions over 8, 38 and 512
    row blocks: 300 calls in a row over three shapes, and calls on two
    streams in flight together, must all give the bits of the first call of
    their shape."""
    g = torch.Generator().manual_seed(21)
    shapes = [(64, 896), (300, 1536), (8192, 896)]  # 8, 38 and 512 row blocks
    cases = []
    for rows, dim in shapes:
        x = torch.randn(rows, dim, generator=g).to(torch.bfloat16).to(dev)
        w = (torch.randn(dim, generator=g) * 0.1 + 1).to(torch.bfloat16).to(dev)
        dy = torch.randn(rows, dim, generator=g).to(torch.bfloat16).to(dev)
        ref = mc.rms_norm_backward(x, dy, 1e-6, w)
        lref = mc.layer_norm_backward(x, dy, 1e-5, w)
        cases.append((x, w, dy, ref, lref))
    torch.cuda.synchronize()
    print("norm bwd: 300 sequential calls", flush=True)
    for i in range(300):
        x, w, dy, ref, lref = cases[i % 3]
        dx, dw = mc.rms_norm_backward(x, dy, 1e-6, w)
        if i % 10 == 0:
            _, ldw, ldb = mc.layer_norm_backward(x, dy, 1e-5, w)
            torch.cuda.synchronize()
            assert torch.equal(ldw, lref[1]) and torch.equal(ldb, lref[2]), f"LayerNorm call {i}"
        torch.cuda.synchronize()
        assert torch.equal(dw, ref[1]) and torch.equal(dx, ref[0]), f"RMSNorm call {i}"
    print("norm bwd: two streams", flush=True)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs = []
    for rep in range(20):
        for s, k in ((s1, 2), (s2, 1)):
            with torch.cuda.stream(s):
                x, w, dy, _, _ = cases[k]
                outs.append((k, mc.rms_norm_backward(x, dy, 1e-6, w)))
    torch.cuda.synchronize()
    for k, (dx, dw) in outs:
        assert torch.equal(dw, cases[k][3][1]) and torch.equal(dx, cases[k][3][0])
