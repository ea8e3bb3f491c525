"""GPU parity of the grouped LoRA entry points (mc_lora_group_fwd / _bwd):
the projections of one input, as q / k / v on the attention's normalised
input and gate / up on the MLP's (src/models/transformer.rs:241-243,
389-395).

* y_g, h_save_g, dA_g and dB_g must equal the per-projection entry points'
  (mc_lora_fwd / mc_lora_bwd) bit for bit: the same kernels reduce each
  output element in the same order.
* dX is the sum of the projections' input gradients, one GEMM over the
  concatenated reduction: checked against the CPU oracle (the sum of its
  per-projection dx in fp64) on sampled rows, bf16 tolerance 2e-2, and
  against the fp32 sum of the per-projection dX.
Shapes: c4's q/k/v (1536 -> 1536, 256, 256, r16, bias) and gate/up
(1536 -> 8960 x2), c5's q/k/v with dropout 0.1 (r64: one projection per
row-projection pass), ragged ranks and sizes (r17: padded extension
columns), a delta-only member (W absent) and four projections.
"""
import zlib

import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err, to_np

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _group_case(dev, T, K, Ns, r, p, seed, bias=True, no_w=()):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(T, K, generator=g, device=dev).to(torch.bfloat16)
    projs, dys = [], []
    for i, N in enumerate(Ns):
        pr = dict(
            W=None if i in no_w else (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16),
            A=(torch.rand(K, r, generator=g, device=dev) * 2 - 1) / K ** 0.5,
            B=torch.randn(r, N, generator=g, device=dev) * 0.02,
        )
        pr["bias"] = ((torch.randn(N, generator=g, device=dev) * 0.02).to(torch.bfloat16)
                      if bias and pr["W"] is not None else None)
        pr["mask"] = None
        projs.append(pr)
        dys.append((torch.randn(T, N, generator=g, device=dev) * 1e-2).to(torch.bfloat16))
    return x, projs, dys


def _masks(mc, dev, projs, T, r, p, seed):
    if p > 0:
        for i, pr in enumerate(projs):
            pr["mask"] = mc.dropout_mask(seed + i, p, T, r).to(dev)


def _check_group(mc, dev, T, K, Ns, r, p, seed, scale=2.0, bias=True, no_w=(), sample_rows=256):
    print(f"group T={T} K={K} Ns={Ns} r={r} p={p} no_w={no_w}", flush=True)
    x, projs, dys = _group_case(dev, T, K, Ns, r, p, seed, bias, no_w)
    _masks(mc, dev, projs, T, r, p, 1234 + seed)
    ys, hs = mc.lora_group_forward(x, projs, scale, dropout_p=p)
    dX, dAs, dBs = mc.lora_group_backward(x, projs, dys, scale, dropout_p=p, h_saves=hs)
    singles = []
    for pr, dy in zip(projs, dys):
        y1, h1 = mc.lora_forward(x, pr["A"], pr["B"], scale, W=pr["W"], bias=pr["bias"], mask=pr["mask"], dropout_p=p)
        d1 = mc.lora_backward(x, pr["A"], pr["B"], dy, scale, W=pr["W"], mask=pr["mask"], dropout_p=p, h_save=h1)
        singles.append((y1, h1) + d1)
    torch.cuda.synchronize()
    for g, (y1, h1, dx1, dA1, dB1) in enumerate(singles):
        assert torch.equal(ys[g], y1), f"y[{g}] differs from mc_lora_fwd"
        assert torch.equal(hs[g], h1), f"h_save[{g}] differs from mc_lora_fwd"
        assert torch.equal(dAs[g], dA1), f"dA[{g}] differs from mc_lora_bwd"
        assert torch.equal(dBs[g], dB1), f"dB[{g}] differs from mc_lora_bwd"
    # dX: against the fp32 sum of the per-projection dX and the oracle's sum
    dx_sum = sum(s[2].float() for s in singles)
    assert rel_err(dX, to_np(dx_sum)) <= BF16_TOL
    rows = np.sort(np.random.default_rng(seed).choice(T, size=min(sample_rows, T), replace=False))
    ri = torch.from_numpy(rows).to(dev)
    xs = to_np(x.index_select(0, ri))
    ref = np.zeros((len(rows), K), dtype=np.float64)
    for pr, dy in zip(projs, dys):
        m = None if pr["mask"] is None else pr["mask"].cpu().numpy()[rows]
        dx_o, _, _ = oracle.lora_bwd(xs, to_np(pr["A"]), to_np(pr["B"]), to_np(dy.index_select(0, ri)), scale,
                                     W=None if pr["W"] is None else to_np(pr["W"]), mask=m, p=p,
                                     need_dA=False, need_dB=False)
        ref += dx_o
    err = rel_err(dX.index_select(0, ri), ref)
    print(f"  dX rel-err vs oracle sum {err:.2e}", flush=True)
    assert err <= BF16_TOL


@pytest.mark.parametrize("name,T,K,Ns,r,p", [
    ("c4 q/k/v", 16384, 1536, [1536, 256, 256], 16, 0.0),
    ("c4 gate/up", 16384, 1536, [8960, 8960], 16, 0.0),
    ("c5 q/k/v dropout", 16384, 3584, [3584, 512, 512], 64, 0.1),
    ("ragged r17 dropout", 3000, 1000, [264, 136], 17, 0.1),
    ("four projections r8", 4096, 512, [512, 128, 384, 64], 8, 0.0),
    ("r32 pair", 2048, 896, [896, 128], 32, 0.2),
    ("r150 pair dropout (rank passes of 128 + 22)", 2048, 512, [512, 136], 150, 0.1),
    # split row projection (K >= 4096) over passes of 48 + 24 ranks (one
    # launch, the second pass's operand 32 rows), ragged T, dropout
    ("r24 three projections, passes of 48 + 24", 2000, 4104, [136, 264, 72], 24, 0.1),
    # dA over the group's 3 x 1500 ranks in one column reduction: more than
    # 64 groups of 64 ranks, so a full bin launches before the rest queue
    ("r1500 three projections", 264, 64, [72, 64, 80], 1500, 0.0),
])
def test_group_matches_single_calls(mc, dev, name, T, K, Ns, r, p):
    _check_group(mc, dev, T, K, Ns, r, p, zlib.crc32(name.encode()) % 1000)


def test_group_delta_only_member(mc, dev):
    """A projection without W (delta only, FusedLoRAOp) beside two with W."""
    _check_group(mc, dev, 1024, 256, [256, 64, 128], 16, 0.0, 41, no_w=(1,))


@pytest.mark.parametrize("T,K,Ns,r", [(2048, 512, [512, 256], 16),
                                      (8192, 512, [8192, 8200], 16),  # the fused dY pass (dY of >= 2^26 elements)
                                      # 33-64 ranks: split row projection and the column reductions over bf16
                                      # planes (dB only: Hd^T planes without a finishing launch)
                                      (2048, 520, [512, 264], 48)])
def test_group_partial_outputs(mc, dev, T, K, Ns, r):
    """dX only, dA / dB only, dB only: the same values as the full call."""
    x, projs, dys = _group_case(dev, T, K, Ns, r, 0.0, 7)
    ys, hs = mc.lora_group_forward(x, projs, 2.0)
    full = mc.lora_group_backward(x, projs, dys, 2.0, h_saves=hs)
    only_dx = mc.lora_group_backward(x, projs, dys, 2.0, need_dA=False, need_dB=False)
    only_ab = mc.lora_group_backward(x, projs, dys, 2.0, h_saves=hs, need_dx=False)
    only_b = mc.lora_group_backward(x, projs, dys, 2.0, h_saves=hs, need_dx=False, need_dA=False)
    # without x (dA not requested): shapes from dY and A, as lora_backward
    no_x = mc.lora_group_backward(None, projs, dys, 2.0, h_saves=hs, need_dA=False)
    torch.cuda.synchronize()
    assert torch.equal(only_dx[0], full[0]) and only_dx[1][0] is None
    assert only_ab[0] is None and only_b[0] is None and only_b[1][0] is None
    assert torch.equal(no_x[0], full[0]) and no_x[1][0] is None
    for g in range(2):
        assert torch.equal(only_ab[1][g], full[1][g]) and torch.equal(only_ab[2][g], full[2][g])
        assert torch.equal(only_b[2][g], full[2][g])
        assert torch.equal(no_x[2][g], full[2][g])


def test_group_with_caller_wt(mc, dev):
    """Projections carrying a caller-built W^T (transpose_weight, built once
    for a frozen W): the backward reads it in place of its own transposed
    copy, so dX, dA and dB equal the call without Wt bit for bit; W^T itself
    equals torch's transpose."""
    x, projs, dys = _group_case(dev, 4096, 1536, [1536, 256, 256], 16, 0.0, 11)
    for pr in projs:
        pr["Wt"] = mc.transpose_weight(pr["W"])
        assert torch.equal(pr["Wt"], pr["W"].t().contiguous())
    ys, hs = mc.lora_group_forward(x, projs, 2.0)
    with_wt = mc.lora_group_backward(x, projs, dys, 2.0, h_saves=hs)
    plain = [dict(pr, Wt=None) for pr in projs]
    without = mc.lora_group_backward(x, plain, dys, 2.0, h_saves=hs)
    torch.cuda.synchronize()
    assert torch.equal(with_wt[0], without[0])
    for g in range(3):
        assert torch.equal(with_wt[1][g], without[1][g]) and torch.equal(with_wt[2][g], without[2][g])


@pytest.mark.parametrize("rows,cols", [(8, 8), (200, 72), (8960, 1536), (1536, 8960)])
def test_transpose_weight(mc, dev, rows, cols):
    W = torch.randn(rows, cols, device=dev).to(torch.bfloat16)
    Wt = mc.transpose_weight(W)
    torch.cuda.synchronize()
    assert Wt.shape == (cols, rows) and torch.equal(Wt, W.t().contiguous())
