"""BASELINE.json config c5 at its own workload on the GPU, against the CPU oracle.

c5 is a Qwen2.5-7B-shaped decoder layer: hidden 3584, intermediate 18944,
28 q heads / 4 kv heads of 128, LoRA rank 64, alpha 128 (scale 2), tokens
4 x 4096, LoRA dropout 0.1 on the rank-r hidden with host-generated masks
(seed 1234 + the projection's index, as bench.py draws them), causal softmax
over [4, 28, 4096, 4096] scores ~N(0, 3).

Reference call sites: the LoRA composite with dropout on the hidden
(src/training/lora.rs:320-339), the projections of the layer
(src/models/transformer.rs:189-192, 241-243, 285, 389-395), the weighted
RMSNorm (src/models/qwen.rs:314-325) and the masked score softmax
(src/models/transformer.rs:264-278).

Every projection runs at T = 16384 with its real K and N: y, the saved
hidden and dX are checked on 256 seeded sample rows (rows are independent),
dA and dB (reductions over all tokens) in full. RMSNorm [16384, 3584] is
checked fwd + bwd on every row, as is the c4 RMSNorm backward at
[16384, 1536]. The softmax is checked against the oracle on sampled rows
(the first and last query of a head among them) and, on every row, through
properties: rows of P sum to 1, masked P and dS are exactly 0, rows of dS
sum to 0. Tolerance: max|out-ref|/max|ref| <= 2e-2 (bf16 outputs); dA, dB
and dw (fp32 accumulations of bf16 inputs) <= 1e-4.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err, to_np

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
T, HIDDEN, INTER, RANK, ALPHA, P_DROP = 4 * 4096, 3584, 18944, 64, 128, 0.1
KV = 4 * 128
# name, K, N, bias (q / k / v carry a bias in Qwen2.5)
PROJECTIONS = [("q", HIDDEN, HIDDEN, True), ("k", HIDDEN, KV, True), ("v", HIDDEN, KV, True),
               ("o", HIDDEN, HIDDEN, False), ("gate", HIDDEN, INTER, False), ("up", HIDDEN, INTER, False),
               ("down", INTER, HIDDEN, False)]


def _sample(n, k, seed):
    rows = np.random.default_rng(seed).choice(n, size=min(k, n), replace=False)
    return np.unique(np.concatenate([rows, [0, n - 1]]))


@pytest.mark.parametrize("idx", range(len(PROJECTIONS)), ids=[p[0] for p in PROJECTIONS])
def test_c5_projection(mc, dev, idx):
    name, K, N, has_bias = PROJECTIONS[idx]
    scale = ALPHA / RANK
    print(f"c5 {name}_proj: T={T} K={K} N={N} r={RANK} p={P_DROP}", flush=True)
    g = torch.Generator(device=dev).manual_seed(500 + idx)
    x = torch.randn(T, K, generator=g, device=dev).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g, device=dev) * 0.02).to(torch.bfloat16) if has_bias else None
    A = (torch.rand(K, RANK, generator=g, device=dev) * 2 - 1) / K ** 0.5
    B = torch.randn(RANK, N, generator=g, device=dev) * 0.02
    dy = (torch.randn(T, N, generator=g, device=dev) * 1e-2).to(torch.bfloat16)
    mask = mc.dropout_mask(1234 + idx, P_DROP, T, RANK)
    mask_np = mask.numpy()
    assert np.array_equal(mask_np, oracle.dropout_mask(1234 + idx, P_DROP, T, RANK))  # byte-identical masks
    md = mask.to(dev)

    y, h = mc.lora_forward(x, A, B, scale, W=W, bias=bias, mask=md, dropout_p=P_DROP)
    dX, dA, dB = mc.lora_backward(x, A, B, dy, scale, W=W, mask=md, dropout_p=P_DROP, h_save=h)
    torch.cuda.synchronize()

    rows = _sample(T, 256, 77 + idx)
    ri = torch.from_numpy(rows).to(dev)
    xs, dys = to_np(x.index_select(0, ri)), to_np(dy.index_select(0, ri))
    Wn, An, Bn = to_np(W), to_np(A), to_np(B)
    bn = None if bias is None else to_np(bias)
    y_ref, hd_ref = oracle.lora_fwd(xs, An, Bn, scale, W=Wn, bias=bn, mask=mask_np[rows], p=P_DROP,
                                    return_hidden=True)
    dx_ref, _, _ = oracle.lora_bwd(xs, An, Bn, dys, scale, W=Wn, mask=mask_np[rows], p=P_DROP, need_dA=False,
                                   need_dB=False)
    _, dA_ref, dB_ref = oracle.lora_bwd(to_np(x), An, Bn, to_np(dy), scale, W=Wn, mask=mask_np, p=P_DROP,
                                        need_dx=False)
    errs = {
        "y": rel_err(y.index_select(0, ri), y_ref),
        "h": rel_err(h.index_select(1, ri).t(), hd_ref),
        "dX": rel_err(dX.index_select(0, ri), dx_ref),
        "dA": rel_err(dA, dA_ref),
        "dB": rel_err(dB, dB_ref),
    }
    tol = {"y": BF16_TOL, "h": BF16_TOL, "dX": BF16_TOL, "dA": 1e-4, "dB": 1e-4}
    print(f"  rel-err {({k: f'{v:.2e}' for k, v in errs.items()})}", flush=True)
    bad = {k: v for k, v in errs.items() if not v <= tol[k]}
    assert not bad, f"c5 {name}_proj rel-err above tolerance: {errs}"
    # dropped hidden entries are exactly zero on every token
    hn = h.t().cpu().numpy()
    assert (hn[mask_np == 0] == 0).all()


@pytest.mark.parametrize("rows,dim", [(T, HIDDEN), (16384, 1536)], ids=["c5 [16384,3584]", "c4 [16384,1536]"])
def test_c5_c4_rmsnorm_full(mc, dev, rows, dim):
    """Weighted RMSNorm (qwen.rs:314-325) fwd + bwd in bf16 on every row."""
    print(f"rmsnorm bf16 [{rows},{dim}] fwd+bwd", flush=True)
    g = torch.Generator(device=dev).manual_seed(dim)
    x = torch.randn(rows, dim, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(dim, generator=g, device=dev) * 0.1 + 1.0).to(torch.bfloat16)
    dy = (torch.randn(rows, dim, generator=g, device=dev) * 1e-2).to(torch.bfloat16)
    y, rstd = mc.rms_norm_forward(x, 1e-6, w)
    dx, dw = mc.rms_norm_backward(x, dy, 1e-6, w, rstd)
    torch.cuda.synchronize()
    xn, wn, dyn = to_np(x), to_np(w), to_np(dy)
    y_ref, r_ref = oracle.rmsnorm_fwd(xn, 1e-6, wn)
    dx_ref, dw_ref = oracle.rmsnorm_bwd(xn, dyn, 1e-6, wn)
    errs = {"y": rel_err(y, y_ref), "rstd": rel_err(rstd, r_ref), "dx": rel_err(dx, dx_ref), "dw": rel_err(dw, dw_ref)}
    print(f"  rel-err {({k: f'{v:.2e}' for k, v in errs.items()})}", flush=True)
    assert errs["y"] <= BF16_TOL and errs["dx"] <= BF16_TOL
    assert errs["rstd"] <= 1e-5 and errs["dw"] <= 1e-4


def test_c5_softmax_full(mc, dev):
    """Causal softmax over [4, 28, 4096, 4096] bf16 scores ~N(0, 3), fwd + bwd
    (transformer.rs:264-278: -inf above the diagonal, softmax_stable)."""
    Bt, H, S = 4, 28, 4096
    print(f"softmax bf16 [{Bt},{H},{S},{S}] causal fwd+bwd", flush=True)
    g = torch.Generator(device=dev).manual_seed(4096)
    s = (torch.randn(Bt, H, S, S, generator=g, device=dev) * 3).to(torch.bfloat16)
    dp = (torch.randn(Bt, H, S, S, generator=g, device=dev) * 1e-2).to(torch.bfloat16)
    p = mc.softmax_forward(s, causal_rows=S)
    ds = mc.softmax_backward(p, dp, causal_rows=S)
    torch.cuda.synchronize()
    rows = Bt * H * S
    ids = np.unique(np.concatenate([_sample(rows, 512, 5), [S - 1, S, 2 * S - 1, rows - S]]))
    idx = torch.from_numpy(ids).to(dev)
    s2, p2, dp2, ds2 = (t.reshape(rows, S).index_select(0, idx) for t in (s, p, dp, ds))
    p_ref = oracle.softmax_fwd(to_np(s2), causal_rows=S, row_ids=ids)
    ds_ref = oracle.softmax_bwd(p_ref, to_np(dp2), causal_rows=S, row_ids=ids)
    errs = {"P": rel_err(p2, p_ref), "dS": rel_err(ds2, ds_ref)}
    print(f"  sampled rows rel-err {({k: f'{v:.2e}' for k, v in errs.items()})}", flush=True)
    assert errs["P"] <= BF16_TOL and errs["dS"] <= BF16_TOL
    # every row, one batch at a time (bounded temporaries)
    masked = torch.ones(S, S, dtype=torch.bool, device=dev).triu(1)
    for b in range(Bt):
        pb, dpb, dsb = p[b].float(), dp[b].float(), ds[b].float()
        sums = pb.sum(-1)
        assert (sums - 1).abs().max().item() <= 1e-2, f"batch {b}: rows of P do not sum to 1"
        assert (p[b][:, masked] == 0).all(), f"batch {b}: masked P not exactly 0"
        assert (ds[b][:, masked] == 0).all(), f"batch {b}: masked dS not exactly 0"
        # sum_j dS_j = dot (1 - sum_j P_j) with dot = sum_j dP_j P_j, for the
        # P the backward read: it is 0 for exact probabilities, and the
        # bf16-rounded P sums to 1 only within its rounding. Bound: the bf16
        # rounding of the dS entries plus the fp32 rounding of dot.
        pdp = pb * dpb
        dot = pdp.sum(-1)
        lhs = (dsb.sum(-1) - dot * (1.0 - sums)).abs()
        bound = 4e-3 * dsb.abs().sum(-1) + 1e-5 * pdp.abs().sum(-1)
        assert (lhs <= bound).all(), f"batch {b}: rows of dS break sum_j dS_j = dot (1 - sum_j P_j)"
        del pb, dpb, dsb, sums, pdp, dot, lhs, bound
