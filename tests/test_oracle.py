"""Pins the CPU oracle before it is trusted as the checker (no GPU).

Each oracle function is checked against something a plausible mistake (a
dropped term, a wrong sign / index, a transposed operand) would fail:
  * the reference's known answers (executor_direct.rs:345-367, 480-495;
    tensor.rs:126-420; rmsnorm_correctness.rs:205-265;
    softmax_correctness.rs:200-243),
  * committed fp64 numpy fixtures (tests/golden/golden_small.json, written
    by tests/golden/make_golden.py in whole-matrix form),
  * central finite differences of the oracle's own forward for every
    backward (the LoRA output is linear in x, A and B separately, so its
    differences are exact up to rounding),
  * invariants: B = 0 => delta = 0, shift invariance, rows of P sum to 1 and
    of dS to 0, exact zeros under the causal mask,
  * Philox4x32-10 known-answer vectors of Random123 (Salmon et al., SC'11).
"""
import json
import os

import numpy as np
import pytest

import oracle

GOLD = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_small.json")))


def arr(v):
    return None if v is None else np.asarray(v, dtype=np.float32)


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


# ---------------------------------------------------------------- Philox
@pytest.mark.parametrize("ctr,key,out", [
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
])
def test_philox_known_answers(ctr, key, out):
    assert list(oracle.philox4x32_10(ctr, key)) == out


def test_dropout_mask_statistics():
    m = oracle.dropout_mask(1234, 0.1, 16384, 64)
    assert m.dtype == np.uint8 and set(np.unique(m)) <= {0, 1}
    assert abs(m.mean() - 0.9) < 0.003
    assert not np.array_equal(m, oracle.dropout_mask(1235, 0.1, 16384, 64))
    # element i depends only on (seed, i): a prefix of a larger mask is the smaller mask
    assert np.array_equal(oracle.dropout_mask(7, 0.3, 10, 8).ravel(), oracle.dropout_mask(7, 0.3, 20, 8).ravel()[:80])
    assert oracle.dropout_mask(1, 0.0, 4, 4).all()


# ------------------------------------------------------------------ LoRA
def test_lora_executor_known_answer():
    ka = GOLD["known_answers"]["lora_executor"]
    y = oracle.lora_fwd(arr(ka["x"]), arr(ka["A"]), arr(ka["B"]), ka["scale"])
    assert rel(y, ka["y"]) < 1e-6


@pytest.mark.parametrize("i", range(len(GOLD["lora"])))
def test_lora_golden(i):
    c = GOLD["lora"][i]
    mask = None if c["mask"] is None else np.asarray(c["mask"], np.uint8)
    y, hd = oracle.lora_fwd(arr(c["x"]), arr(c["A"]), arr(c["B"]), c["scale"], W=arr(c["W"]), bias=arr(c["bias"]),
                            mask=mask, p=c["p"], return_hidden=True)
    assert rel(y, c["y"]) < 1e-6
    assert rel(hd, c["hd"]) < 1e-7
    dx, dA, dB = oracle.lora_bwd(arr(c["x"]), arr(c["A"]), arr(c["B"]), arr(c["dy"]), c["scale"], W=arr(c["W"]),
                                 mask=mask, p=c["p"])
    assert dx.shape == arr(c["x"]).shape and dA.shape == arr(c["A"]).shape and dB.shape == arr(c["B"]).shape
    assert rel(dx, c["dx"]) < 1e-6 and rel(dA, c["dA"]) < 1e-6 and rel(dB, c["dB"]) < 1e-6


def _loss(x, A, B, W, dy, s, mask, p):
    y = oracle.lora_fwd(x, A, B, s, W=W, mask=mask, p=p).astype(np.float64)
    return float((y * dy).sum())


@pytest.mark.parametrize("with_w,p", [(True, 0.0), (False, 0.0), (True, 0.3)])
def test_lora_backward_finite_differences(with_w, p):
    rng = np.random.default_rng(11)
    T, K, N, r, s = 5, 6, 7, 3, 2.0
    f = lambda *sh: rng.standard_normal(sh).astype(np.float32)  # noqa: E731
    x, A, B, dy = f(T, K), f(K, r), f(r, N), f(T, N)
    W = f(N, K) if with_w else None
    mask = (rng.random((T, r)) >= p).astype(np.uint8) if p > 0 else None
    dx, dA, dB = oracle.lora_bwd(x, A, B, dy, s, W=W, mask=mask, p=p)
    h = 0.5  # y is linear in each of x, A, B: central differences are exact up to rounding
    for name, ref, grad in (("x", x, dx), ("A", A, dA), ("B", B, dB)):
        fd = np.zeros(ref.shape)
        for idx in np.ndindex(ref.shape):
            plus, minus = ref.copy(), ref.copy()
            plus[idx] += h
            minus[idx] -= h
            args = {"x": x, "A": A, "B": B}
            args[name] = plus
            lp = _loss(args["x"], args["A"], args["B"], W, dy, s, mask, p)
            args[name] = minus
            lm = _loss(args["x"], args["A"], args["B"], W, dy, s, mask, p)
            fd[idx] = (lp - lm) / (2 * h)
        assert rel(grad, fd) < 1e-4, name


def test_lora_zero_B_and_linearity():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((8, 16)).astype(np.float32)
    A = rng.standard_normal((16, 4)).astype(np.float32)
    W = rng.standard_normal((12, 16)).astype(np.float32)
    B0 = np.zeros((4, 12), np.float32)
    base = oracle.lora_fwd(x, A, B0, 2.0, W=W)
    assert rel(base, x.astype(np.float64) @ W.T.astype(np.float64)) < 1e-6  # B = 0 => delta = 0
    assert np.abs(oracle.lora_fwd(x, A, B0, 2.0)).max() == 0.0
    B = rng.standard_normal((4, 12)).astype(np.float32)
    # the delta scales linearly with the LoRA scale
    d1 = oracle.lora_fwd(x, A, B, 1.0)
    d2 = oracle.lora_fwd(x, A, B, 2.0)
    assert rel(d2, 2 * d1.astype(np.float64)) < 1e-6


# --------------------------------------------------------------- RMSNorm
def test_rmsnorm_known_answers():
    ka = GOLD["known_answers"]["rmsnorm_3_4"]
    y, _ = oracle.rmsnorm_fwd(arr([ka["x"]]), ka["eps"])
    assert rel(y[0], ka["y"]) < 1e-6 and abs(y[0, 0] - 0.8485) < 1e-3 and abs(y[0, 1] - 1.1314) < 1e-3
    y, _ = oracle.rmsnorm_fwd(arr([[2, 4, 6]]), 1e-6)
    assert abs(y[0, 1] / y[0, 0] - 2) < 1e-5 and abs(y[0, 2] / y[0, 0] - 3) < 1e-5
    assert abs(oracle.rmsnorm_fwd(arr([[5.0]]), 1e-6)[0][0, 0] - 1) < 1e-5
    assert abs(oracle.rmsnorm_fwd(arr([[1.0, 1, 1, 1]]), 1e-6)[0] - 1).max() < 1e-5
    for c in (100.0, 0.01):  # closed form c / sqrt(c^2 + eps)
        y, _ = oracle.rmsnorm_fwd(np.full((2, 256), c, np.float32), 1e-5)
        assert rel(y, np.full((2, 256), c / np.sqrt(c * c + 1e-5))) < 1e-6
    assert abs(0.01 / np.sqrt(1e-4 + 1e-5) - 0.95346) < 1e-5
    # output RMS ~ 1 (rmsnorm_correctness.rs:117-146)
    x = np.random.default_rng(0).standard_normal((64, 512)).astype(np.float32) * 7
    y, _ = oracle.rmsnorm_fwd(x, 1e-6)
    assert np.abs(np.sqrt((y.astype(np.float64) ** 2).mean(-1)) - 1).max() < 1e-2


@pytest.mark.parametrize("i", range(len(GOLD["rmsnorm"])))
def test_rmsnorm_golden(i):
    c = GOLD["rmsnorm"][i]
    y, rstd = oracle.rmsnorm_fwd(arr(c["x"]), c["eps"], arr(c["w"]))
    assert rel(y, c["y"]) < 1e-6 and rel(rstd, c["rstd"]) < 1e-6
    dx, dw = oracle.rmsnorm_bwd(arr(c["x"]), arr(c["dy"]), c["eps"], arr(c["w"]))
    # dim 1 with eps 0: dx = r*g - x*r^3*g*x is 0 up to the rounding of its
    # terms, so the error is measured against the terms' size r*|g|
    w = np.ones(c["D"]) if c["w"] is None else np.asarray(c["w"])
    terms = np.abs(np.asarray(c["dy"]) * w * np.asarray(c["rstd"])[:, None]).max()
    assert np.abs(dx - np.asarray(c["dx"])).max() / max(np.abs(np.asarray(c["dx"])).max(), terms) < 1e-6
    assert rel(dw, c["dw"]) < 1e-6


def test_rmsnorm_backward_finite_differences():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 6)).astype(np.float32)
    w = (rng.standard_normal(6) * 0.3 + 1).astype(np.float32)
    dy = rng.standard_normal((3, 6)).astype(np.float32)
    eps = 1e-3
    dx, dw = oracle.rmsnorm_bwd(x, dy, eps, w)
    loss = lambda xx, ww: float((oracle.rmsnorm_fwd(xx, eps, ww)[0].astype(np.float64) * dy).sum())  # noqa: E731
    h = 1e-2
    fdx = np.zeros(x.shape)
    for idx in np.ndindex(x.shape):
        p_, m_ = x.copy(), x.copy()
        p_[idx] += h
        m_[idx] -= h
        fdx[idx] = (loss(p_, w) - loss(m_, w)) / (2 * h)
    fdw = np.zeros(w.shape)
    for j in range(w.size):
        p_, m_ = w.copy(), w.copy()
        p_[j] += h
        m_[j] -= h
        fdw[j] = (loss(x, p_) - loss(x, m_)) / (2 * h)
    assert rel(dx, fdx) < 2e-3
    assert rel(dw, fdw) < 1e-4  # y is linear in w


# --------------------------------------------------------------- softmax
def test_softmax_known_answers():
    ka = GOLD["known_answers"]["softmax_zeros"]
    assert rel(oracle.softmax_fwd(arr(ka["s"])), ka["p"]) < 1e-6
    p = oracle.softmax_fwd(arr([[100.0, 200.0, 300.0]]))
    assert np.isfinite(p).all() and abs(p.sum() - 1) < 1e-6
    for c in (100.0, -100.0):
        assert np.abs(oracle.softmax_fwd(np.full((2, 256), c, np.float32)) - 1 / 256).max() < 1e-9
    assert oracle.softmax_fwd(arr([[5.0]]))[0, 0] == 1.0
    s = np.random.default_rng(1).standard_normal((4, 64)).astype(np.float32)
    assert rel(oracle.softmax_fwd(s + 5.0), oracle.softmax_fwd(s)) < 1e-6


@pytest.mark.parametrize("i", range(len(GOLD["softmax"])))
def test_softmax_golden(i):
    c = GOLD["softmax"][i]
    p = oracle.softmax_fwd(arr(c["s"]), causal_rows=c["causal_rows"])
    assert rel(p, c["p"]) < 1e-6
    assert np.array_equal(p == 0, np.asarray(c["p"]) == 0)
    ds = oracle.softmax_bwd(p, arr(c["dp"]), causal_rows=c["causal_rows"])
    assert rel(ds, c["ds_given_p32"]) < 1e-6
    # the row-indexed variant agrees on a shuffled sample of rows
    ids = np.random.default_rng(0).permutation(c["rows"])[: max(1, c["rows"] // 2)]
    ps = oracle.softmax_fwd(arr(c["s"])[ids], causal_rows=c["causal_rows"], row_ids=ids)
    assert np.array_equal(ps, p[ids])


@pytest.mark.parametrize("causal", [0, 5])
def test_softmax_backward_finite_differences(causal):
    rng = np.random.default_rng(6)
    rows, D = 5, 7
    s = (rng.standard_normal((rows, D)) * 2).astype(np.float32)
    dp = rng.standard_normal((rows, D)).astype(np.float32)
    p = oracle.softmax_fwd(s, causal_rows=causal)
    ds = oracle.softmax_bwd(p, dp, causal_rows=causal)
    loss = lambda ss: float((oracle.softmax_fwd(ss, causal_rows=causal).astype(np.float64) * dp).sum())  # noqa
    h = 1e-2
    fd = np.zeros(s.shape)
    for idx in np.ndindex(s.shape):
        a, b = s.copy(), s.copy()
        a[idx] += h
        b[idx] -= h
        fd[idx] = (loss(a) - loss(b)) / (2 * h)
    assert rel(ds, fd) < 2e-3
    assert np.abs(ds.astype(np.float64).sum(-1)).max() < 1e-6
    if causal:
        masked = p == 0
        assert masked.any() and (ds[masked] == 0).all()


def test_round_bf16():
    v = np.array([1.0, 1.00390625, 1.005859375, -2.5, 3.0e38, np.inf], np.float32)
    r = oracle.round_bf16(v)
    assert r[0] == 1.0 and r[1] == 1.0 and r[2] == np.float32(1.0078125) and r[3] == -2.5
    assert np.isinf(r[5])
