"""GPU parity of the fused LoRA linear (fwd + bwd) against the CPU oracle.

Cases: the executor known answer (tests/executor_direct.rs:345-367), the
reference's fused-vs-candle LoRA shapes (tests/custom_ops_correctness.rs:
15-170: [2,64,512] r8 s2, batches 1/4/8 at [b,32,256], ranks 4..32),
BASELINE.json config 1 (fp32, 1e-5) and the bf16 projection shapes of configs 3-5
(2e-2), with dropout masks from the shared host generator, bias, delta-only
(W absent, as FusedLoRAOp) and ragged sizes. At full token counts the
O(T.K.N) outputs y and dX are checked on a seeded sample of token rows (rows
are independent), dA / dB (reductions over all tokens) in full.
Tolerance: max|out-ref|/max|ref|.
"""
import zlib

import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err
from inputs import lora_case, np32

pytestmark = pytest.mark.gpu

F32_TOL, BF16_TOL = 1e-5, 2e-2


def _run(mc, dev, c, scale, mask=None, p=0.0):
    g = lambda t: None if t is None else t.to(dev)  # noqa: E731
    md = None if mask is None else torch.from_numpy(mask).to(dev)
    y, h = mc.lora_forward(g(c["x"]), g(c["A"]), g(c["B"]), scale, W=g(c["W"]), bias=g(c["bias"]), mask=md,
                           dropout_p=p)
    dX, dA, dB = mc.lora_backward(g(c["x"]), g(c["A"]), g(c["B"]), g(c["dy"]), scale, W=g(c["W"]), mask=md,
                                  dropout_p=p, h_save=h)
    torch.cuda.synchronize()
    return y, h, dX, dA, dB


def _check(mc, dev, c, scale, tol, mask=None, p=0.0, sample_rows=None):
    y, h, dX, dA, dB = _run(mc, dev, c, scale, mask, p)
    x, W, A, B, dy, bias = (np32(c[k]) for k in ("x", "W", "A", "B", "dy", "bias"))
    T = x.shape[0]
    rows = np.arange(T) if sample_rows is None else np.sort(
        np.random.default_rng(0).choice(T, size=min(sample_rows, T), replace=False))
    m = None if mask is None else mask[rows]
    y_ref, hd_ref = oracle.lora_fwd(x[rows], A, B, scale, W=W, bias=bias, mask=m, p=p, return_hidden=True)
    dx_ref, _, _ = oracle.lora_bwd(x[rows], A, B, dy[rows], scale, W=W, mask=m, p=p, need_dA=False, need_dB=False)
    _, dA_ref, dB_ref = oracle.lora_bwd(x, A, B, dy, scale, W=W, mask=mask, p=p, need_dx=False)
    ri = torch.from_numpy(rows).to(dev)
    errs = {
        "y": rel_err(y.index_select(0, ri), y_ref),
        "h": rel_err(h.index_select(1, ri).t(), hd_ref),
        "dX": rel_err(dX.index_select(0, ri), dx_ref),
        "dA": rel_err(dA, dA_ref),
        "dB": rel_err(dB, dB_ref),
    }
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, f"rel-err above {tol}: {errs}"
    return y, h, dX, dA, dB


def test_executor_known_answer(mc, dev):
    """executor_direct.rs:345-367 inputs; y derived by hand from them (x·A·B·scale)."""
    x = torch.tensor([[1.0, 2, 3, 4], [5, 6, 7, 8]], device=dev)
    A = torch.tensor([[0.1, 0.2], [0.3, 0.4], [0.5, 0.6], [0.7, 0.8]], device=dev)
    B = torch.tensor([[1.0, 2, 3, 4], [5, 6, 7, 8]], device=dev)
    y, _ = mc.lora_forward(x, A, B, 0.5)
    expect = np.array([[17.5, 23, 28.5, 34], [40.7, 53.4, 66.1, 78.8]])
    assert rel_err(y, expect) <= F32_TOL


def test_config1_fp32(mc, dev):
    """BASELINE.json c1: x [4,128,768] fp32, W 768x768, r8 a16, no dropout, seed 0."""
    c = lora_case(0, 4 * 128, 768, 768, 8, dtype=torch.float32)
    _check(mc, dev, c, 2.0, F32_TOL)


@pytest.mark.parametrize("T,K,N,r", [(128, 512, 512, 8), (32, 256, 256, 4), (4 * 32, 256, 256, 16),
                                     (8 * 32, 256, 256, 32), (100, 40, 24, 3), (1, 8, 8, 1), (65, 72, 136, 17),
                                     # ranks past 64 (eight 16-rank MFMA tiles, 32-row projection blocks)
                                     (300, 264, 200, 100), (64, 128, 128, 128),
                                     # past 128 ranks: rank passes of 128 in the row projections
                                     (200, 264, 136, 150)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_shapes(mc, dev, T, K, N, r, dtype):
    c = lora_case(T * 7 + r, T, K, N, r, dtype=dtype, bias=True)
    _check(mc, dev, c, 2.0, F32_TOL if dtype == torch.float32 else BF16_TOL)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_delta_only(mc, dev, dtype):
    """W absent: exactly FusedLoRAOp's delta (custom_ops.rs:53-66)."""
    c = lora_case(5, 2 * 64, 512, 512, 8, dtype=dtype, w=False, x_std=1.0)
    c["B"] = c["B"] * 50  # make the delta O(1)
    _check(mc, dev, c, 2.0, F32_TOL if dtype == torch.float32 else BF16_TOL)


@pytest.mark.parametrize("name,T,K,N,r,p,bias,w", [
    # bf16 K or N not a multiple of 8 (the reference takes any shape,
    # custom_ops.rs:118-148): the single-projection calls run on copies
    # zero-padded to multiples of 8
    ("K 37 N 45, bias, dropout", 300, 37, 45, 8, 0.1, True, True),
    ("K 40 N 45", 257, 40, 45, 16, 0.0, False, True),
    ("K 1001 N 8", 1000, 1001, 8, 4, 0.0, True, True),
    ("K 37 N 45 delta only", 130, 37, 45, 8, 0.0, False, False),
    ("K 3 N 5 rank 70", 64, 3, 5, 70, 0.2, True, True),
])
def test_bf16_features_not_multiple_of_8(mc, dev, name, T, K, N, r, p, bias, w):
    c = lora_case(zlib.crc32(name.encode()), T, K, N, r, bias=bias, w=w)
    if not w:
        c["B"] = c["B"] * 50  # make the delta O(1)
    mask = mc.dropout_mask(zlib.crc32(name.encode()), p, T, r).numpy() if p > 0 else None
    y, h, dX, dA, dB = _check(mc, dev, c, 2.0, BF16_TOL, mask=mask, p=p)
    assert y.shape == (T, N) and dX.shape == (T, K) and dA.shape == (K, r) and dB.shape == (r, N)


def test_zero_B_gives_base(mc, dev):
    """B = 0 => delta = 0 (lora.rs:244, lora.rs:656-659): y equals the base linear."""
    c = lora_case(6, 256, 256, 384, 8)
    c["B"] = torch.zeros_like(c["B"])
    y, _, _, _, _ = _run(mc, dev, c, 2.0)
    y0, _, _, _, _ = _run(mc, dev, dict(c, A=torch.zeros_like(c["A"])), 2.0)
    assert torch.equal(y, y0)


@pytest.mark.parametrize("name,T,K,N,r", [("c3 q_proj", 8192, 896, 896, 8), ("c3 v_proj", 8192, 896, 128, 8),
                                          ("c4 q_proj", 16384, 1536, 1536, 16), ("c4 k_proj", 16384, 1536, 256, 16),
                                          ("c4 v_proj", 16384, 1536, 256, 16), ("c4 o_proj", 16384, 1536, 1536, 16),
                                          ("c4 gate_proj", 16384, 1536, 8960, 16),
                                          ("c4 up_proj", 16384, 1536, 8960, 16),
                                          ("c4 down_proj", 16384, 8960, 1536, 16),
                                          # ragged sizes on each GEMM plan (one tile shape of 256x256, 256x192,
                                          # 256x128 or 128x128, or 256x256 tiles over most columns and a
                                          # 256x128 / 256x192 tail, chosen by shape; rows / columns past M, N
                                          # are masked)
                                          ("ragged split 256x256 + 256x128 fwd, 256x256 dX", 16400, 1544, 9000, 16),
                                          ("ragged 256x256", 16400, 1544, 1544, 32),
                                          ("ragged split, 256x128 tail", 16300, 1536, 1536, 16),
                                          ("ragged split, 320-column tail", 16300, 1536, 1344, 16),
                                          ("ragged 256x192", 16300, 1536, 768, 16),
                                          ("ragged split, 256x192 tail", 16300, 1536, 8960, 16),
                                          ("ragged 128x128", 4000, 1000, 264, 8)])
def test_config_projections_bf16(mc, dev, name, T, K, N, r):
    c = lora_case(zlib.crc32(name.encode()), T, K, N, r)
    _check(mc, dev, c, 2.0, BF16_TOL, sample_rows=256)


@pytest.mark.parametrize("name,T,K,N,r,p", [
    # dY of >= 2^26 elements at rank <= 32 takes the fused dY pass (G and the
    # dB partials from one read of dY): odd T (scalar Hd^T loads, a last
    # split past T), 17-32 ranks (two 16-rank tiles), dropout, a ragged last
    # 512-column group
    ("fused dY pass, odd T, r24, dropout", 16383, 1024, 8200, 24, 0.1),
    ("fused dY pass, r16, no dropout", 8192, 512, 8192, 16, 0.0),
])
def test_fused_dy_pass(mc, dev, name, T, K, N, r, p):
    c = lora_case(zlib.crc32(name.encode()), T, K, N, r)
    mask = mc.dropout_mask(zlib.crc32(name.encode()), p, T, r).numpy() if p > 0 else None
    _check(mc, dev, c, 2.0, BF16_TOL, mask=mask, p=p, sample_rows=256)


@pytest.mark.parametrize("name,T,K,N,r,p", [
    # more than 128 ranks: the row projections take the ranks in passes of
    # at most 128 (a ragged last pass, mask columns at a stride of r), the
    # column reductions in groups of 64
    ("rank 200, dropout", 3000, 512, 384, 200, 0.1),
    ("rank 257, no dropout", 2048, 256, 520, 257, 0.0),
    # more than 64 groups of 64 ranks in one column-reduction bin (a full
    # bin is launched before the rest are queued)
    ("rank 4200, dropout", 264, 64, 72, 4200, 0.1),
])
def test_rank_above_128(mc, dev, name, T, K, N, r, p):
    c = lora_case(zlib.crc32(name.encode()), T, K, N, r)
    mask = mc.dropout_mask(zlib.crc32(name.encode()), p, T, r).numpy() if p > 0 else None
    _check(mc, dev, c, 2.0, BF16_TOL, mask=mask, p=p, sample_rows=256)


def test_config5_dropout_bf16(mc, dev):
    """c5-style: rank 64, alpha 128, dropout 0.1 with the seed-1234 host mask."""
    T, K, N, r = 2048, 3584, 512, 64
    c = lora_case(1234, T, K, N, r)
    mask = mc.dropout_mask(1234, 0.1, T, r).numpy()
    assert np.array_equal(mask, oracle.dropout_mask(1234, 0.1, T, r))
    _check(mc, dev, c, 2.0, BF16_TOL, mask=mask, p=0.1, sample_rows=256)


@pytest.mark.parametrize("name,T,K,N,r,p", [
    # projections of 33-64 ranks take the split row projection (256-row
    # workgroups, column splits, a finishing pass) both ways (fp32 B in the
    # backward), and in the forward so do those of >= 4096 columns: ragged T
    # and last split, 33 and 40 ranks (zero rows in the last 16-rank tile),
    # rank 8 over 4608 columns, more splits than columns (empty splits)
    ("rank 40, ragged T and split, dropout", 3000, 1000, 264, 40, 0.1),
    ("rank 33, 4104 columns", 517, 4104, 96, 33, 0.0),
    ("rank 8, 4608 columns, dropout", 700, 4608, 4160, 8, 0.2),
    ("rank 64, dY of 4104 columns", 1100, 520, 4104, 64, 0.0),
    # 42 column-reduction splits of 416 tokens: the last two are empty and
    # must still write their (zero) partials
    ("rank 64, empty trailing splits", 16384, 2568, 264, 64, 0.0),
])
def test_split_row_projection(mc, dev, name, T, K, N, r, p):
    c = lora_case(zlib.crc32(name.encode()), T, K, N, r)
    mask = mc.dropout_mask(zlib.crc32(name.encode()), p, T, r).numpy() if p > 0 else None
    _check(mc, dev, c, 2.0, BF16_TOL, mask=mask, p=p, sample_rows=256)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dropout_mask_semantics(mc, dev, dtype):
    """Masked hidden entries are exactly zero; kept ones scaled by 1/(1-p)."""
    T, K, N, r, p = 96, 64, 64, 8, 0.5
    c = lora_case(3, T, K, N, r, dtype=dtype)
    mask = oracle.dropout_mask(77, p, T, r)
    _, h, _, _, _ = _check(mc, dev, c, 2.0, F32_TOL if dtype == torch.float32 else BF16_TOL, mask=mask, p=p)
    hn = h.t().cpu().numpy()
    assert (hn[mask == 0] == 0).all()


def test_backward_deterministic(mc, dev):
    c = lora_case(21, 4096, 1536, 256, 16)
    a = _run(mc, dev, c, 2.0)
    b = _run(mc, dev, c, 2.0)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_partial_outputs(mc, dev):
    """dX / dA / dB individually optional (NULL outputs are skipped)."""
    c = lora_case(8, 256, 128, 64, 8)
    g = lambda t: t.to(dev)  # noqa: E731
    y, h = mc.lora_forward(g(c["x"]), g(c["A"]), g(c["B"]), 2.0, W=g(c["W"]))
    full = mc.lora_backward(g(c["x"]), g(c["A"]), g(c["B"]), g(c["dy"]), 2.0, W=g(c["W"]), h_save=h)
    only_b = mc.lora_backward(None, g(c["A"]), g(c["B"]), g(c["dy"]), 2.0, W=g(c["W"]), h_save=h,
                              need_dx=False, need_dA=False)
    only_x = mc.lora_backward(None, g(c["A"]), g(c["B"]), g(c["dy"]), 2.0, W=g(c["W"]), need_dA=False,
                              need_dB=False)
    only_a = mc.lora_backward(g(c["x"]), g(c["A"]), g(c["B"]), g(c["dy"]), 2.0, W=g(c["W"]), need_dx=False,
                              need_dB=False)
    assert only_b[0] is None and only_b[1] is None and torch.equal(only_b[2], full[2])
    assert torch.equal(only_x[0], full[0])
    assert only_a[0] is None and only_a[2] is None and torch.equal(only_a[1], full[1])


def test_wide_dB_split_bound(mc, dev):
    """dB over a 196608-wide dY (a vocabulary-sized output): T x N x 2 bytes
    exceeds 2^31, so the token reduction must split into chunks whose rows
    stay inside one buffer resource. Reference: scale * h_save @ dY in fp32
    (torch on the GPU)."""
    T, N, r, s = 6144, 196608, 16, 2.0
    g = torch.Generator(device=dev).manual_seed(5)
    dy = (torch.randn(T, N, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    h = torch.randn(r, T, generator=g, device=dev)
    A = torch.zeros(64, r, device=dev)
    B = torch.randn(r, N, generator=g, device=dev) * 0.02
    _, _, dB = mc.lora_backward(None, A, B, dy, s, h_save=h, need_dx=False, need_dA=False)
    ref = s * (h @ dy.float())
    torch.cuda.synchronize()
    assert rel_err(dB, ref.cpu().numpy()) <= 1e-4


def test_random_shapes_gemm_plans(mc, dev):
    """Seeded random shapes across the GEMM plans (one tile shape, or a
    256x256 split with a 256x128 / 256x192 tail; ragged M, N and K, K past
    the full k-tiles): the forward base product with bias and the dX product,
    against torch fp32 on the GPU, bf16 tolerance."""
    import random
    rng = random.Random(7)
    for it in range(16):
        M = rng.choice([rng.randint(1, 600), rng.randint(3000, 17000)])
        N = rng.choice([384 * rng.randint(1, 10) + rng.choice([0, 8, -8, 64, 136]), rng.randint(1, 300) * 8])
        N = max(8, N - N % 8)
        K = max(8, rng.randint(1, 600) * 8)
        r = rng.choice([4, 8, 16, 33, 64])
        g = torch.Generator(device=dev).manual_seed(it)
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        W = (torch.randn(N, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
        bias = (torch.randn(N, generator=g, device=dev) * 0.1).to(torch.bfloat16)
        A = torch.randn(K, r, generator=g, device=dev) * 0.01
        B = torch.zeros(r, N, device=dev)  # the base product alone
        y, h = mc.lora_forward(x, A, B, 2.0, W=W, bias=bias)
        dy = (torch.randn(M, N, generator=g, device=dev) * 0.01).to(torch.bfloat16)
        dX, _, _ = mc.lora_backward(x, A, B, dy, 2.0, W=W, h_save=h, need_dA=False, need_dB=False)
        ref_y = x.float() @ W.float().t() + bias.float()
        ref_dx = dy.float() @ W.float()
        torch.cuda.synchronize()
        for name, out, ref in (("y", y, ref_y), ("dX", dX, ref_dx)):
            err = ((out.float() - ref).abs().max() / ref.abs().max()).item()
            assert err <= BF16_TOL, f"{name} M={M} N={N} K={K} r={r}: rel-err {err:.3e}"


def test_random_shapes_lora(mc, dev):
    """Seeded random shapes, ranks 1-128 and dropout rates through the whole
    bf16 LoRA forward and backward, against a torch fp32 composite of the
    same maths on the GPU (Hd = (x.A) * M/(1-p), y = x.W^T + s Hd.B,
    Gd = s (dY.B^T) * M/(1-p), dX = dY.W + Gd.A^T, dA = x^T.Gd,
    dB = s Hd^T.dY). y and dX to the bf16 tolerance; dA and dB (fp32 outputs
    of bf16 inputs with hi/lo-split fp32 factors) to 1e-4."""
    import random
    rng = random.Random(11)
    for it in range(12):
        M = rng.choice([rng.randint(1, 700), rng.randint(2000, 8000)])
        K, N = max(8, rng.randint(1, 300) * 8), max(8, rng.randint(1, 400) * 8)
        r, p, s = rng.randint(1, 128), rng.choice([0.0, 0.1, 0.3]), 2.0
        g = torch.Generator(device=dev).manual_seed(100 + it)
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        W = (torch.randn(N, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
        A = torch.randn(K, r, generator=g, device=dev) * 0.05
        B = torch.randn(r, N, generator=g, device=dev) * 0.05
        dy = (torch.randn(M, N, generator=g, device=dev) * 0.01).to(torch.bfloat16)
        mask = mc.dropout_mask(it, p, M, r).to(dev) if p > 0 else None
        y, h = mc.lora_forward(x, A, B, s, W=W, mask=mask, dropout_p=p)
        dX, dA, dB = mc.lora_backward(x, A, B, dy, s, W=W, mask=mask, dropout_p=p, h_save=h)
        xf, Wf, dyf = x.float(), W.float(), dy.float()
        mf = mask.float() / (1.0 - p) if mask is not None else torch.ones(M, r, device=dev)
        Hd = (xf @ A) * mf
        Gd = s * (dyf @ B.t()) * mf
        refs = {"y": xf @ Wf.t() + s * (Hd @ B), "dX": dyf @ Wf + Gd @ A.t(), "dA": xf.t() @ Gd,
                "dB": s * (Hd.t() @ dyf)}
        outs = {"y": y, "dX": dX, "dA": dA, "dB": dB}
        torch.cuda.synchronize()
        for name, ref in refs.items():
            err = ((outs[name].float() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
            tol = 1e-4 if name in ("dA", "dB") else BF16_TOL
            assert err <= tol, f"{name} M={M} K={K} N={N} r={r} p={p}: rel-err {err:.3e}"
