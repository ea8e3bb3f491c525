"""GPU parity of LayerNorm, log-softmax and cross-entropy (fwd + bwd) against
the CPU oracle (pinned in tests/test_oracle_rowops.py).

Cases: the reference's own tests (layer_norm, tensor.rs:165-300;
cross_entropy_loss and label smoothing, loss.rs:247-380), BERT-like
LayerNorm rows with weight and bias (the embeddings' MetalLayerNorm), a
Qwen-sized hidden (16384 x 1536, bf16) and vocabulary (151936), rows that take
the scalar paths (length not a multiple of the vector width), ignore_index
with label smoothing, a scaled loss gradient, and the reference's error cases
(every row ignored, a target past the vocabulary), which give NaN here.
Tolerance max|out-ref|/max|ref|: 1e-5 (fp32), 2e-2 (bf16); the scalar loss
is compared relative to itself.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err, to_np

pytestmark = pytest.mark.gpu

F32_TOL, BF16_TOL = 1e-5, 2e-2


def tol(dtype):
    return F32_TOL if dtype == torch.float32 else BF16_TOL


def rnd(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


# ---------------------------------------------------------------- LayerNorm
def test_layernorm_reference_tests(mc, dev):
    x = torch.tensor([[1.0, 2, 3, 4], [5, 6, 7, 8]], device=dev)
    y, mean, rstd = mc.layer_norm_forward(x, 1e-5)
    assert float(to_np(y).mean(axis=1).__abs__().max()) < 1e-4          # test_layer_norm
    ref, _, _ = oracle.layernorm_fwd(to_np(x), 1e-5)
    assert rel_err(y, ref) <= F32_TOL
    z, _, _ = mc.layer_norm_forward(torch.zeros(1, 3, device=dev), 1e-5)
    assert torch.equal(z, torch.zeros(1, 3, device=dev))               # test_layer_norm_with_zeros
    x3 = rnd((3, 5, 7), 1).to(dev)                                       # test_layer_norm_preserves_shape
    y3, _, _ = mc.layer_norm_forward(x3, 1e-5)
    assert y3.shape == x3.shape
    assert rel_err(y3, oracle.layernorm_fwd(to_np(x3), 1e-5)[0]) <= F32_TOL


@pytest.mark.parametrize("rows,D,dtype,affine", [
    (64, 384, torch.float32, True), (33, 768, torch.bfloat16, True), (17, 1024, torch.float32, False),
    (16384, 1536, torch.bfloat16, True), (9, 5000, torch.float32, True), (5, 13, torch.bfloat16, True),
    (8, 4096, torch.bfloat16, False), (1024, 3584, torch.bfloat16, True), (300, 2048, torch.float32, True),
    # rows past the one-wave paths: workgroup-per-row forward, row-block backward (bf16 to 8192, fp32 to 8192
    # columns), scalar backward past that; 4097 rows leave the last row blocks empty
    (600, 5120, torch.bfloat16, True), (4097, 4104, torch.bfloat16, True), (40, 8192, torch.float32, False),
    (3, 16384, torch.bfloat16, True), (2, 40000, torch.float32, True),
])
def test_layernorm_fwd_bwd(mc, dev, rows, D, dtype, affine):
    x = (rnd((rows, D), rows + D, 2.0) + 0.3).to(dtype)
    w = (rnd((D,), 3, 0.1) + 1.0).to(dtype) if affine else None
    b = rnd((D,), 4, 0.1).to(dtype) if affine else None
    dy = rnd((rows, D), 5, 1.0, dtype)
    xd, wd, bd, dyd = x.to(dev), None if w is None else w.to(dev), None if b is None else b.to(dev), dy.to(dev)
    y, mean, rstd = mc.layer_norm_forward(xd, 1e-5, wd, bd)
    yr, mr, rr = oracle.layernorm_fwd(x.float().numpy(), 1e-5, None if w is None else w.float().numpy(),
                                      None if b is None else b.float().numpy())
    assert rel_err(y, yr) <= tol(dtype)
    assert rel_err(mean, mr) <= F32_TOL * 10 and rel_err(rstd, rr) <= F32_TOL * 10
    dxr, dwr, dbr = oracle.layernorm_bwd(x.float().numpy(), dy.float().numpy(), 1e-5,
                                         None if w is None else w.float().numpy())
    for saved in (True, False):
        dx, dw, db = mc.layer_norm_backward(xd, dyd, 1e-5, wd, mean if saved else None, rstd if saved else None)
        assert rel_err(dx, dxr) <= tol(dtype)
        assert rel_err(dw, dwr) <= tol(dtype) and rel_err(db, dbr) <= tol(dtype)
    # fixed-order reductions: the same call twice gives the same bits
    dx1, dw1, db1 = mc.layer_norm_backward(xd, dyd, 1e-5, wd, mean, rstd)
    dx2, dw2, db2 = mc.layer_norm_backward(xd, dyd, 1e-5, wd, mean, rstd)
    assert torch.equal(dx1, dx2) and torch.equal(dw1, dw2) and torch.equal(db1, db2)
    dx3, n1, n2 = mc.layer_norm_backward(xd, dyd, 1e-5, wd, mean, rstd, need_dw=False, need_db=False)
    assert n1 is None and n2 is None and rel_err(dx3, dxr) <= tol(dtype)


# -------------------------------------------------------------- log-softmax
@pytest.mark.parametrize("rows,D,dtype", [(7, 33, torch.float32), (4, 1000, torch.float32),
                                          (16, 50257, torch.bfloat16), (3, 151936, torch.bfloat16),
                                          (64, 2048, torch.bfloat16)])
def test_log_softmax(mc, dev, rows, D, dtype):
    x = rnd((rows, D), D, 3.0, dtype)
    y = mc.log_softmax_forward(x.to(dev))
    yr = oracle.log_softmax_fwd(x.float().numpy())
    assert rel_err(y, yr) <= tol(dtype)
    dy = rnd((rows, D), D + 1, 1.0, dtype)
    dx = mc.log_softmax_backward(y, dy.to(dev))
    dxr = oracle.log_softmax_bwd(to_np(y), dy.float().numpy())
    assert rel_err(dx, dxr) <= tol(dtype)


# ------------------------------------------------------------ cross entropy
def run_xent(mc, dev, logits, targets, ignore=None, smoothing=0.0, dloss=1.0):
    ld = logits.to(dev)
    td = torch.from_numpy(np.asarray(targets, np.uint32).astype(np.int32)).to(dev)  # uint32 bytes
    loss, stats = mc.cross_entropy_forward(ld, td, ignore, smoothing)
    g = mc.cross_entropy_backward(ld, td, stats, torch.full((1,), dloss, device=dev), ignore, smoothing)
    torch.cuda.synchronize()
    return float(loss.cpu()), stats.cpu().numpy(), g


def test_cross_entropy_reference_tests(mc, dev):
    lg = torch.tensor([[10.0, 0.0, 0.0]])
    assert run_xent(mc, dev, lg, [0])[0] < 0.1                           # test_cross_entropy_loss_basic
    assert run_xent(mc, dev, lg, [2])[0] > 5.0                           # _wrong_prediction
    row = torch.tensor([1.0, 2.0, 3.0])
    l, st, _ = run_xent(mc, dev, row.repeat(4, 1), [2, 0, 2, 0], ignore=0)  # _with_ignore
    assert st[-1] == 2.0
    assert abs(l - oracle.cross_entropy_fwd(row.repeat(4, 1).numpy(), [2, 0, 2, 0], 0)[0]) < 1e-6
    assert run_xent(mc, dev, row[None], [2], smoothing=0.0)[0] == run_xent(mc, dev, row[None], [2])[0]
    a = run_xent(mc, dev, lg, [0])[0]
    b = run_xent(mc, dev, lg, [0], smoothing=0.1)[0]                     # test_label_smoothing_effect
    assert b > a and abs(b - oracle.cross_entropy_fwd(lg.numpy(), [0], smoothing=0.1)[0]) < 1e-5 * b


def test_cross_entropy_error_cases_are_nan(mc, dev):
    row = torch.tensor([1.0, 2.0, 3.0])
    assert np.isnan(run_xent(mc, dev, row.repeat(2, 1), [0, 0], ignore=0)[0])   # every row ignored
    assert np.isnan(run_xent(mc, dev, row[None], [3])[0])                       # target past the vocabulary


@pytest.mark.parametrize("rows,V,dtype,ignore,smoothing,dloss", [
    (64, 1000, torch.float32, None, 0.0, 1.0), (64, 1000, torch.float32, 7, 0.0, 1.0),
    (48, 999, torch.float32, 7, 0.1, 2.5), (128, 32000, torch.bfloat16, None, 0.1, 1.0),
    (256, 151936, torch.bfloat16, 151643, 0.0, 1.0), (37, 77, torch.bfloat16, 3, 0.2, 0.5),
])
def test_cross_entropy(mc, dev, rows, V, dtype, ignore, smoothing, dloss):
    logits = rnd((rows, V), rows + V, 2.0, dtype)
    t = np.random.default_rng(V).integers(0, V, rows).astype(np.uint32)
    if ignore is not None:
        t[::5] = ignore
    loss, stats, g = run_xent(mc, dev, logits, t, ignore, smoothing, dloss)
    lr, lser, cnt = oracle.cross_entropy_fwd(logits.float().numpy(), t, -1 if ignore is None else ignore, smoothing)
    assert abs(loss - lr) <= (1e-5 if dtype == torch.float32 else 1e-4) * abs(lr)
    assert rel_err(stats[:-1], lser) <= 1e-5 and stats[-1] == cnt
    gr = oracle.cross_entropy_bwd(logits.float().numpy(), t, -1 if ignore is None else ignore, smoothing, dloss)
    assert rel_err(g, gr) <= tol(dtype)
    # determinism of the loss reduction
    loss2, _, _ = run_xent(mc, dev, logits, t, ignore, smoothing, dloss)
    assert loss2 == loss
