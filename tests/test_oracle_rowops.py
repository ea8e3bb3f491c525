"""Pins the LayerNorm, log-softmax and cross-entropy oracles before they are
trusted as checkers (no GPU):
  * the reference's own tests: layer_norm (src/backend/tensor.rs:165-300:
    row means ~0 on [[1..4],[5..8]], zeros in -> zeros out, eps changes the
    result), cross_entropy_loss and its label smoothing (src/training/
    loss.rs:247-380), each with its closed form;
  * torch (fp64, CPU) as a library cross-check: layer_norm,
    log_softmax, cross_entropy (ignore_index; label smoothing where torch's
    definition coincides with the reference's, i.e. no ignored rows) and their
    autograd;
  * central finite differences for the backward where torch's definition
    differs (smoothing together with ignored rows).
"""
import numpy as np
import pytest
import torch

import oracle


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


def rand(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


# ---------------------------------------------------------------- LayerNorm
def test_layernorm_reference_tests():
    x = np.array([[1, 2, 3, 4], [5, 6, 7, 8]], np.float32)
    y, mean, rstd = oracle.layernorm_fwd(x, 1e-5)
    assert np.abs(y.mean(axis=1)).max() < 1e-4                       # test_layer_norm
    s = 1 / np.sqrt(1.25 + 1e-5)
    assert np.allclose(y[0], [-1.5 * s, -0.5 * s, 0.5 * s, 1.5 * s], atol=1e-6)
    assert np.allclose(mean, [2.5, 6.5]) and np.allclose(rstd, s)
    z, _, _ = oracle.layernorm_fwd(np.zeros((1, 3), np.float32), 1e-5)
    assert np.array_equal(z, np.zeros((1, 3), np.float32))            # test_layer_norm_with_zeros
    a, _, _ = oracle.layernorm_fwd(np.array([[1, 2, 3]], np.float32), 1e-5)
    b, _, _ = oracle.layernorm_fwd(np.array([[1, 2, 3]], np.float32), 1e-3)
    assert a.shape == b.shape and not np.array_equal(a, b)            # test_layer_norm_with_different_eps


@pytest.mark.parametrize("rows,D,affine", [(6, 64, False), (5, 96, True), (3, 7, True)])
def test_layernorm_matches_torch(rows, D, affine):
    x = rand((rows, D), 1, 2.0) + 0.5
    w = rand(D, 2) if affine else None
    b = rand(D, 3) if affine else None
    y, _, _ = oracle.layernorm_fwd(x, 1e-5, w, b)
    tx = torch.from_numpy(x.astype(np.float64)).requires_grad_()
    tw = torch.from_numpy(w.astype(np.float64)).requires_grad_() if affine else None
    tb = torch.from_numpy(b.astype(np.float64)).requires_grad_() if affine else None
    ty = torch.nn.functional.layer_norm(tx, (D,), tw, tb, eps=1e-5)
    assert rel(y, ty.detach().numpy()) < 1e-6
    dy = rand((rows, D), 4)
    ty.backward(torch.from_numpy(dy.astype(np.float64)))
    dx, dw, db = oracle.layernorm_bwd(x, dy, 1e-5, w)
    assert rel(dx, tx.grad.numpy()) < 1e-6
    if affine:
        assert rel(dw, tw.grad.numpy()) < 1e-6 and rel(db, tb.grad.numpy()) < 1e-6
    else:
        assert rel(dw, (dy * ((x - x.mean(1, keepdims=True)) / np.sqrt(x.var(1, keepdims=True) + 1e-5))).sum(0)) < 1e-5
        assert rel(db, dy.sum(0)) < 1e-6


def test_layernorm_backward_finite_differences():
    x, w, dy = rand((3, 10), 5), rand(10, 6), rand((3, 10), 7)
    dx, dw, db = oracle.layernorm_bwd(x, dy, 1e-5, w)

    def f(x_, w_):
        y, _, _ = oracle.layernorm_fwd(x_, 1e-5, w_, None)
        return float((y.astype(np.float64) * dy).sum())

    eps = 1e-3
    for idx in [(0, 0), (1, 5), (2, 9)]:
        xp, xm = x.copy(), x.copy()
        xp[idx] += eps
        xm[idx] -= eps
        assert abs((f(xp, w) - f(xm, w)) / (2 * eps) - dx[idx]) < 5e-3 * max(1, abs(dx[idx]))
    for j in (0, 4, 9):
        wp, wm = w.copy(), w.copy()
        wp[j] += eps
        wm[j] -= eps
        assert abs((f(x, wp) - f(x, wm)) / (2 * eps) - dw[j]) < 5e-3 * max(1, abs(dw[j]))


# -------------------------------------------------------------- log-softmax
def test_log_softmax_matches_torch():
    x = rand((7, 33), 8, 3.0)
    y = oracle.log_softmax_fwd(x)
    tx = torch.from_numpy(x.astype(np.float64)).requires_grad_()
    ty = torch.log_softmax(tx, dim=-1)
    assert rel(y, ty.detach().numpy()) < 1e-6
    assert np.allclose(np.exp(y.astype(np.float64)).sum(1), 1.0, atol=1e-6)
    assert np.allclose(oracle.log_softmax_fwd(x + 100.0), y, atol=1e-4)   # shift invariance
    dy = rand((7, 33), 9)
    ty.backward(torch.from_numpy(dy.astype(np.float64)))
    assert rel(oracle.log_softmax_bwd(y, dy), tx.grad.numpy()) < 1e-5


# ------------------------------------------------------------ cross entropy
def test_cross_entropy_reference_tests():
    # test_cross_entropy_loss_basic / _wrong_prediction: logits [10, 0, 0]
    lg = np.array([[10.0, 0.0, 0.0]], np.float32)
    lse = 10 + np.log1p(2 * np.exp(-10.0))
    loss, _, _ = oracle.cross_entropy_fwd(lg, [0])
    assert loss < 0.1 and abs(loss - (lse - 10)) < 1e-9
    loss, _, _ = oracle.cross_entropy_fwd(lg, [2])
    assert loss > 5.0 and abs(loss - lse) < 1e-6
    # test_cross_entropy_loss_with_ignore: [[2, 0], [2, 0]] with ignore 0 -> two counted rows
    row = np.array([1.0, 2.0, 3.0], np.float32)
    lg = np.tile(row, (4, 1))
    loss, _, cnt = oracle.cross_entropy_fwd(lg, [2, 0, 2, 0], ignore_index=0)
    want = np.log(np.exp(row.astype(np.float64)).sum()) - 3.0
    assert cnt == 2 and abs(loss - want) < 1e-9
    # test_label_smoothing_zero: smoothing 0 equals the plain loss
    lg = row[None, :]
    assert oracle.cross_entropy_fwd(lg, [2], smoothing=0.0)[0] == oracle.cross_entropy_fwd(lg, [2])[0]
    # test_label_smoothing_effect: [10, 0, 0], target 0, s = 0.1 raises the loss
    lg = np.array([[10.0, 0.0, 0.0]], np.float32)
    a = oracle.cross_entropy_fwd(lg, [0])[0]
    b = oracle.cross_entropy_fwd(lg, [0], smoothing=0.1)[0]
    lp = np.array([10.0, 0.0, 0.0]) - lse
    assert b > a and abs(b - (0.9 * a + 0.1 * (-lp.mean()))) < 1e-7  # s enters as fp32 0.1
    # errors of the reference become NaN: every row ignored, target out of range
    assert np.isnan(oracle.cross_entropy_fwd(np.tile(row, (2, 1)), [0, 0], ignore_index=0)[0])
    assert np.isnan(oracle.cross_entropy_fwd(row[None, :], [3])[0])


@pytest.mark.parametrize("ignore,smoothing", [(-1, 0.0), (5, 0.0), (-1, 0.2)])
def test_cross_entropy_matches_torch(ignore, smoothing):
    rows, V = 24, 37
    x = rand((rows, V), 10, 2.0)
    t = np.random.default_rng(11).integers(0, V, rows).astype(np.uint32)
    t[[1, 7, 8]] = 5
    loss, lse, _ = oracle.cross_entropy_fwd(x, t, ignore_index=ignore, smoothing=smoothing)
    tx = torch.from_numpy(x.astype(np.float64)).requires_grad_()
    tl = torch.nn.functional.cross_entropy(tx, torch.from_numpy(t.astype(np.int64)),
                                           ignore_index=ignore if ignore >= 0 else -100, label_smoothing=smoothing)
    assert abs(loss - float(tl.detach())) < 1e-9 * max(1.0, abs(float(tl.detach())))
    assert rel(lse, torch.logsumexp(tx, 1).detach().numpy()) < 1e-6
    tl.backward()
    assert rel(oracle.cross_entropy_bwd(x, t, ignore, smoothing), tx.grad.numpy()) < 1e-6


def test_cross_entropy_smoothing_with_ignored_rows():
    """The reference's smoothing term is the mean over every row, ignored ones
    included (log_probs.mean_all(), loss.rs:236-237); torch averages it over
    counted rows only, so this case is pinned by the closed form and by
    finite differences."""
    rows, V, s = 6, 9, 0.3
    x = rand((rows, V), 12)
    t = np.array([1, 0, 4, 0, 8, 2], np.uint32)
    loss, _, cnt = oracle.cross_entropy_fwd(x, t, ignore_index=0, smoothing=s)
    lp = torch.log_softmax(torch.from_numpy(x.astype(np.float64)), 1).numpy()
    keep = t != 0
    want = (1 - s) * (-lp[keep, t[keep]].mean()) + s * (-lp.mean())
    assert cnt == 4 and abs(loss - want) < 1e-7 * abs(want)  # s enters as fp32
    g = oracle.cross_entropy_bwd(x, t, 0, s)
    eps = 1e-3
    for idx in [(0, 1), (1, 3), (5, 8), (3, 0)]:
        xp, xm = x.copy(), x.copy()
        xp[idx] += eps
        xm[idx] -= eps
        fd = (oracle.cross_entropy_fwd(xp, t, 0, s)[0] - oracle.cross_entropy_fwd(xm, t, 0, s)[0]) / (2 * eps)
        assert abs(fd - g[idx]) < 1e-4
