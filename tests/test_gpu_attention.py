"""GPU parity of the attention core (mc_attention_fwd / mc_attention_bwd)
against the CPU oracle (oracle_attention_fwd / _bwd, pinned in
tests/test_oracle_attention.py).

Cases: the reference's attention test geometries (src/models/transformer.rs:
443-480: H = 4 with 2 or 4 K/V heads, S = 8, D = 32, fp32, zero mask),
sequence lengths around the 64-key / 128-query block edges for both head dims
of the MFMA kernel (64, 128), GQA ratios 1, 2 and 6, causal / additive mask /
both, -inf mask entries and a fully masked row, the workspace-free kernel
(fp32, other bf16 head dims), and BASELINE.json c4's attention [8, 12, 2048, 128]
with 2 K/V heads: there the oracle checks two whole K/V groups (6 heads, every
query) and every output row is checked to lie within the range of the v rows
it averages. Tolerance max|out-ref|/max|ref|: 1e-5 (fp32), 2e-2 (bf16); the
log-sum-exp, computed from fp32 scores: 1e-4 (bf16), 1e-5 (fp32).
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err, to_np
from inputs import gen

pytestmark = pytest.mark.gpu

F32_TOL, BF16_TOL = 1e-5, 2e-2


def case(seed, B, H, Hkv, S, D, dtype, masked=False):
    g = gen(seed)
    q = torch.randn(B, H, S, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, S, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, S, D, generator=g).to(dtype)
    mask = torch.randn(S, S, generator=g) if masked else None
    return q, k, v, mask


def run(mc, dev, q, k, v, mask, causal, scale=None):
    o, lse = mc.attention_forward(q.to(dev), k.to(dev), v.to(dev), causal=causal, scale=scale,
                                  mask=None if mask is None else mask.to(dev))
    torch.cuda.synchronize()
    return o, lse


def ref(q, k, v, mask, causal, scale=None):
    D = q.shape[-1]
    return oracle.attention_fwd(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                D ** -0.5 if scale is None else scale, causal=causal,
                                mask=None if mask is None else mask.numpy())


def check(o, lse, o_ref, lse_ref, dtype):
    tol = F32_TOL if dtype == torch.float32 else BF16_TOL
    assert rel_err(o, o_ref) <= tol
    assert rel_err(lse, lse_ref) <= (F32_TOL if dtype == torch.float32 else 1e-4)


@pytest.mark.parametrize("B,H,Hkv,S,D,causal,masked", [
    (1, 4, 2, 8, 32, False, False),   # test_attention_forward (transformer.rs:456-466)
    (1, 4, 4, 8, 32, False, True),    # test_attention_with_mask (transformer.rs:469-480)
    (2, 6, 2, 37, 16, True, False),
    (1, 4, 1, 64, 128, True, True),
    (2, 2, 2, 130, 64, False, False),
    (1, 3, 3, 5, 200, True, False),
])
def test_attention_fwd_f32(mc, dev, B, H, Hkv, S, D, causal, masked):
    q, k, v, mask = case(B * 1000 + S, B, H, Hkv, S, D, torch.float32, masked)
    o, lse = run(mc, dev, q, k, v, mask, causal)
    o_ref, lse_ref = ref(q, k, v, mask, causal)
    check(o, lse, o_ref, lse_ref, torch.float32)


def test_attention_reference_zero_mask_f32(mc, dev):
    # test_attention_with_mask passes a [1, 1, 8, 8] zero mask: same result as none
    q, k, v, _ = case(1, 1, 4, 4, 8, 32, torch.float32)
    a, la = run(mc, dev, q, k, v, None, False)
    b, lb = run(mc, dev, q, k, v, torch.zeros(8, 8), False)
    assert torch.equal(a, b) and torch.equal(la, lb)


MFMA_CASES = [
    # B, H, Hkv, S, D, causal
    (1, 4, 4, 1, 64, False), (1, 4, 4, 1, 128, True),
    (1, 4, 2, 7, 128, True), (2, 4, 2, 63, 64, True),
    (1, 4, 2, 64, 128, False), (1, 4, 2, 64, 128, True),
    (1, 2, 1, 65, 64, True), (2, 12, 2, 127, 128, True),
    (1, 12, 2, 128, 128, True), (1, 12, 2, 129, 128, False),
    (1, 12, 2, 129, 64, True), (2, 6, 6, 200, 128, True),
    (1, 4, 2, 256, 64, False), (1, 12, 2, 333, 128, True),
    (1, 14, 2, 300, 64, True), (2, 28, 4, 192, 128, True),
]


@pytest.mark.parametrize("B,H,Hkv,S,D,causal", MFMA_CASES)
def test_attention_fwd_bf16(mc, dev, B, H, Hkv, S, D, causal):
    q, k, v, _ = case(7 * S + D + H, B, H, Hkv, S, D, torch.bfloat16)
    o, lse = run(mc, dev, q, k, v, None, causal)
    o_ref, lse_ref = ref(q, k, v, None, causal)
    check(o, lse, o_ref, lse_ref, torch.bfloat16)


@pytest.mark.parametrize("profile", ["rising", "falling", "spike"])
@pytest.mark.parametrize("D,causal", [(128, True), (128, False), (64, True)])
def test_attention_fwd_bf16_score_range(mc, dev, profile, D, causal):
    """Score rows whose max moves by more and by less than the forward's slack
    before it moves its softmax reference point (8 in log2 units): keys along
    one direction u with weights rising steadily to ~60 log2 units (the
    reference moves every few blocks), falling (it never moves after the first
    block), or one key 10^3 above the rest (a one-hot row). Against the oracle's
    fp64 softmax; lse included."""
    B, H, Hkv, S = 1, 2, 1, 1024
    g = gen(41)
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    w = torch.linspace(0.0, 40.0, S) if profile == "rising" else torch.linspace(40.0, 0.0, S)
    if profile == "spike":
        w = torch.zeros(S)
        w[700] = 1000.0 / D ** 0.5
    q = (u * D ** 0.5).expand(B, H, S, D).clone() + 0.05 * torch.randn(B, H, S, D, generator=g)
    k = w[None, None, :, None] * u + 0.05 * torch.randn(B, Hkv, S, D, generator=g)
    v = torch.randn(B, Hkv, S, D, generator=g)
    q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    o, lse = run(mc, dev, q, k, v, None, causal)
    o_ref, lse_ref = ref(q, k, v, None, causal)
    check(o, lse, o_ref, lse_ref, torch.bfloat16)


@pytest.mark.parametrize("S,D,causal", [(100, 128, False), (256, 128, True), (77, 64, True), (130, 64, False)])
def test_attention_fwd_bf16_mask(mc, dev, S, D, causal):
    q, k, v, mask = case(S + D, 2, 4, 2, S, D, torch.bfloat16, masked=True)
    mask[:, S - 3:] = float("-inf")  # padded keys, as an attention_mask would mark them
    o, lse = run(mc, dev, q, k, v, mask, causal)
    o_ref, lse_ref = ref(q, k, v, mask, causal)
    check(o, lse, o_ref, lse_ref, torch.bfloat16)


@pytest.mark.parametrize("D", [32, 96, 8])
def test_attention_fwd_bf16_generic_head_dims(mc, dev, D):
    q, k, v, mask = case(D, 2, 4, 2, 45, D, torch.bfloat16, masked=True)
    o, lse = run(mc, dev, q, k, v, mask, True)
    o_ref, lse_ref = ref(q, k, v, mask, True)
    check(o, lse, o_ref, lse_ref, torch.bfloat16)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.bfloat16, 64), (torch.float32, 32)])
def test_attention_fully_masked_row_is_nan(mc, dev, dtype, D):
    q, k, v, _ = case(3, 1, 2, 1, 70, D, dtype)
    mask = torch.zeros(70, 70)
    mask[5, :] = float("-inf")
    o, lse = run(mc, dev, q, k, v, mask, False)
    o = to_np(o)
    assert np.isnan(o[0, 5]).all()
    assert np.isfinite(np.delete(o[0], 5, axis=0)).all()
    assert to_np(lse)[0, :, 5].tolist() == [float("-inf")] * 2


def test_attention_scale_argument(mc, dev):
    q, k, v, _ = case(11, 1, 4, 2, 96, 128, torch.bfloat16)
    o, lse = run(mc, dev, q, k, v, None, True, scale=0.05)
    o_ref, lse_ref = ref(q, k, v, None, True, scale=0.05)
    check(o, lse, o_ref, lse_ref, torch.bfloat16)


def test_attention_deterministic(mc, dev):
    q, k, v, _ = case(12, 2, 12, 2, 300, 128, torch.bfloat16)
    a, la = run(mc, dev, q, k, v, None, True)
    b, lb = run(mc, dev, q, k, v, None, True)
    assert torch.equal(a, b) and torch.equal(la, lb)


def test_attention_c4_shape(mc, dev):
    """BASELINE.json c4's attention: [8, 12, 2048, 128], 2 K/V heads, causal."""
    B, H, Hkv, S, D = 8, 12, 2, 2048, 128
    g = gen(2048)
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o, lse = mc.attention_forward(qd, kd, vd, causal=True)
    torch.cuda.synchronize()
    # two whole K/V groups against the oracle (all 6 heads, every query)
    rep = H // Hkv
    for b, hk in ((0, 0), (7, 1)):
        hs = slice(hk * rep, (hk + 1) * rep)
        o_ref, lse_ref = oracle.attention_fwd(q[b:b + 1, hs].float().numpy(), k[b:b + 1, hk:hk + 1].float().numpy(),
                                              v[b:b + 1, hk:hk + 1].float().numpy(), D ** -0.5, causal=True)
        assert rel_err(o[b:b + 1, :, hs.start * D:hs.stop * D], o_ref) <= BF16_TOL
        assert rel_err(lse[b:b + 1, hs], lse_ref) <= 1e-4
    # every row: a convex combination of the v rows of its causal prefix
    vf = vd.float()
    lo = torch.cummin(vf, dim=2).values.repeat_interleave(rep, dim=1)  # [B, H, S, D]
    hi = torch.cummax(vf, dim=2).values.repeat_interleave(rep, dim=1)
    of = o.float().view(B, S, H, D).transpose(1, 2)
    assert torch.isfinite(of).all()
    slack = 1e-2 * (hi - lo).abs() + 1e-2
    assert bool(((of >= lo - slack) & (of <= hi + slack)).all())
    assert torch.isfinite(lse).all()


# ------------------------------------------------------------------ backward
def run_bwd(mc, dev, q, k, v, mask, causal, dout, scale=None):
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    md = None if mask is None else mask.to(dev)
    o, lse = mc.attention_forward(qd, kd, vd, causal=causal, scale=scale, mask=md)
    grads = mc.attention_backward(qd, kd, vd, o, lse, dout.to(dev), causal=causal, scale=scale, mask=md)
    torch.cuda.synchronize()
    return grads


def ref_bwd(q, k, v, mask, causal, dout, scale=None):
    D = q.shape[-1]
    return oracle.attention_bwd(q.float().numpy(), k.float().numpy(), v.float().numpy(), dout.float().numpy(),
                                D ** -0.5 if scale is None else scale, causal=causal,
                                mask=None if mask is None else mask.numpy())


def check_bwd(got, want, dtype):
    tol = F32_TOL if dtype == torch.float32 else BF16_TOL
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        assert rel_err(g, w) <= tol, name


@pytest.mark.parametrize("B,H,Hkv,S,D,causal,masked", [
    (1, 4, 2, 8, 32, False, False),   # test_attention_forward's geometry
    (1, 4, 4, 8, 32, False, True),    # test_attention_with_mask's geometry
    (2, 6, 2, 37, 16, True, False),
    (1, 4, 1, 64, 128, True, True),
    (1, 3, 3, 21, 200, False, False),
])
def test_attention_bwd_f32(mc, dev, B, H, Hkv, S, D, causal, masked):
    q, k, v, mask = case(B * 77 + S, B, H, Hkv, S, D, torch.float32, masked)
    dout = torch.randn(B, S, H * D, generator=gen(S))
    got = run_bwd(mc, dev, q, k, v, mask, causal, dout)
    check_bwd(got, ref_bwd(q, k, v, mask, causal, dout), torch.float32)


BWD_CASES = [
    # B, H, Hkv, S, D, causal
    (1, 4, 4, 1, 64, False), (1, 4, 4, 1, 128, True),
    (1, 4, 2, 7, 128, True), (2, 4, 2, 63, 64, True),
    (1, 4, 4, 64, 128, False), (1, 4, 2, 64, 128, True),
    (1, 2, 1, 65, 64, True), (2, 12, 2, 127, 128, True),
    (1, 12, 2, 129, 128, False), (1, 6, 6, 200, 128, True),
    (1, 4, 2, 256, 64, False), (1, 12, 2, 333, 128, True),
    (1, 14, 2, 300, 64, True),
]


@pytest.mark.parametrize("B,H,Hkv,S,D,causal", BWD_CASES)
def test_attention_bwd_bf16(mc, dev, B, H, Hkv, S, D, causal):
    q, k, v, _ = case(5 * S + D + H, B, H, Hkv, S, D, torch.bfloat16)
    dout = torch.randn(B, S, H * D, generator=gen(S + 1)).to(torch.bfloat16)
    got = run_bwd(mc, dev, q, k, v, None, causal, dout)
    check_bwd(got, ref_bwd(q, k, v, None, causal, dout), torch.bfloat16)


@pytest.mark.parametrize("S,D,causal", [(100, 128, False), (200, 128, True), (77, 64, True)])
def test_attention_bwd_bf16_mask(mc, dev, S, D, causal):
    q, k, v, mask = case(S * 3 + D, 2, 4, 2, S, D, torch.bfloat16, masked=True)
    mask[:, S - 3:] = float("-inf")
    dout = torch.randn(2, S, 4 * D, generator=gen(S + 2)).to(torch.bfloat16)
    got = run_bwd(mc, dev, q, k, v, mask, causal, dout)
    check_bwd(got, ref_bwd(q, k, v, mask, causal, dout), torch.bfloat16)


@pytest.mark.parametrize("D", [32, 96])
def test_attention_bwd_bf16_generic_head_dims(mc, dev, D):
    q, k, v, mask = case(D + 5, 1, 4, 2, 40, D, torch.bfloat16, masked=True)
    dout = torch.randn(1, 40, 4 * D, generator=gen(D)).to(torch.bfloat16)
    got = run_bwd(mc, dev, q, k, v, mask, True, dout)
    check_bwd(got, ref_bwd(q, k, v, mask, True, dout), torch.bfloat16)


def test_attention_bwd_deterministic(mc, dev):
    q, k, v, _ = case(13, 2, 12, 2, 300, 128, torch.bfloat16)
    dout = torch.randn(2, 300, 12 * 128, generator=gen(14)).to(torch.bfloat16)
    a = run_bwd(mc, dev, q, k, v, None, True, dout)
    b = run_bwd(mc, dev, q, k, v, None, True, dout)
    assert all(torch.equal(x, y) for x, y in zip(a, b))


@pytest.mark.parametrize("B,H,Hkv,S,causal,masked", [(16, 4, 2, 2048, True, False), (8, 8, 4, 1024, False, False),
                                                      (32, 4, 2, 1024, True, True)])
def test_attention_bwd_whole_kv_group(mc, dev, B, H, Hkv, S, causal, masked):
    """Shapes whose dK/dV workgroups take all H/Hkv query heads of a K/V head
    (no partials, no summing launch; the workspace test pins the choice):
    one K/V group of two batches against the oracle, every head's dK summing
    to ~0 over the keys (rows of dS sum to 0), and bitwise equal reruns."""
    D = 128
    g = gen(B * S + H)
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    dout = torch.randn(B, S, H * D, generator=g).to(torch.bfloat16)
    mask = None
    if masked:  # additive mask with padded keys, shared by every head
        mask = torch.randn(S, S, generator=g)
        mask[:, S - 5:] = float("-inf")
    dq, dk, dv = run_bwd(mc, dev, q, k, v, mask, causal, dout)
    rep = H // Hkv
    for b, hk in ((0, 0), (B - 1, Hkv - 1)):
        hs = slice(hk * rep, (hk + 1) * rep)
        rq, rk, rv = oracle.attention_bwd(q[b:b + 1, hs].float().numpy(), k[b:b + 1, hk:hk + 1].float().numpy(),
                                          v[b:b + 1, hk:hk + 1].float().numpy(),
                                          dout[b:b + 1].view(1, S, H, D)[:, :, hs].reshape(1, S, rep * D).float().numpy(),
                                          D ** -0.5, causal=causal, mask=None if mask is None else mask.numpy())
        assert rel_err(dq[b:b + 1, hs], rq) <= BF16_TOL
        assert rel_err(dk[b:b + 1, hk:hk + 1], rk) <= BF16_TOL
        assert rel_err(dv[b:b + 1, hk:hk + 1], rv) <= BF16_TOL
    ksum = dk.float().sum(dim=2)
    assert float(ksum.abs().max()) <= 2e-2 * float(dk.float().abs().max()) * 8
    again = run_bwd(mc, dev, q, k, v, mask, causal, dout)
    assert all(torch.equal(x, y) for x, y in zip((dq, dk, dv), again))


def test_attention_bwd_long_sequence(mc, dev):
    """S = 32800: a head's stored dS^T (S x 32896 bf16) passes 2^31 bytes, so
    dQ takes the kernel that recomputes S and dP. Causal: the gradients of the
    last 64 queries and of the last 64 keys involve only the last 64 query
    rows of P and dS, which an fp32 torch composite computes on the GPU from
    the inputs (softmax over all 32800 keys, O = P.V, Delta = rowsum(dO * O));
    the first 2048 queries' dQ matches a 2048-long problem over the same
    prefix (dQ_i depends on keys <= i only), which runs the dS^T path."""
    B, H, Hkv, S, D = 1, 2, 1, 32800, 64
    assert S * ((S + 127) // 128 * 128) * 2 >= 2 ** 31
    g = torch.Generator(device=dev).manual_seed(32800)
    q = torch.randn(B, H, S, D, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g, device=dev).to(torch.bfloat16)
    do = torch.randn(B, S, H * D, generator=g, device=dev).to(torch.bfloat16)
    o, lse = mc.attention_forward(q, k, v, causal=True)
    dq, dk, dv = mc.attention_backward(q, k, v, o, lse, do, causal=True)
    torch.cuda.synchronize()
    for t in (dq, dk, dv):
        assert torch.isfinite(t).all()
    scale, R = D ** -0.5, 64
    r0 = S - R
    kf, vf = k[0, 0].float(), v[0, 0].float()
    dk_ref, dv_ref = torch.zeros(R, D, device=dev), torch.zeros(R, D, device=dev)
    for h in range(H):
        qr = q[0, h, r0:].float()
        dor = do[0, r0:].view(R, H, D)[:, h].float()
        s = (qr @ kf.t()) * scale
        s = s.masked_fill(torch.arange(S, device=dev)[None, :] > torch.arange(r0, S, device=dev)[:, None],
                          float("-inf"))
        p = torch.softmax(s, -1)
        delta = (dor * (p @ vf)).sum(-1, keepdim=True)
        ds = p * (dor @ vf.t() - delta)
        assert rel_err(dq[0, h, r0:], (scale * ds @ kf).cpu().numpy()) <= BF16_TOL
        dk_ref += scale * ds[:, r0:].t() @ qr
        dv_ref += p[:, r0:].t() @ dor
    assert rel_err(dk[0, 0, r0:], dk_ref.cpu().numpy()) <= BF16_TOL
    assert rel_err(dv[0, 0, r0:], dv_ref.cpu().numpy()) <= BF16_TOL
    P = 2048
    qp, kp, vp = q[:, :, :P].contiguous(), k[:, :, :P].contiguous(), v[:, :, :P].contiguous()
    dop = do[:, :P].contiguous()
    op, lsep = mc.attention_forward(qp, kp, vp, causal=True)
    dqp, _, _ = mc.attention_backward(qp, kp, vp, op, lsep, dop, causal=True)
    torch.cuda.synchronize()
    assert rel_err(dq[:, :, :P], dqp.float().cpu().numpy()) <= BF16_TOL


def test_attention_bwd_c4_shape(mc, dev):
    """Backward at BASELINE.json c4's attention shape: one whole K/V group (6 query
    heads, every query and key) against the oracle; on every head, the rows
    of dS sum to 0, so sum_j dK_j = scale sum_i (sum_j dS_ij) q_i = 0."""
    B, H, Hkv, S, D = 8, 12, 2, 2048, 128
    g = gen(4096)
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    dout = torch.randn(B, S, H * D, generator=g).to(torch.bfloat16)
    dq, dk, dv = run_bwd(mc, dev, q, k, v, None, True, dout)
    rep = H // Hkv
    b, hk = 3, 1
    hs = slice(hk * rep, (hk + 1) * rep)
    rq, rk, rv = oracle.attention_bwd(q[b:b + 1, hs].float().numpy(), k[b:b + 1, hk:hk + 1].float().numpy(),
                                      v[b:b + 1, hk:hk + 1].float().numpy(),
                                      dout[b:b + 1].view(1, S, H, D)[:, :, hs].reshape(1, S, rep * D).float().numpy(),
                                      D ** -0.5, causal=True)
    assert rel_err(dq[b:b + 1, hs], rq) <= BF16_TOL
    assert rel_err(dk[b:b + 1, hk:hk + 1], rk) <= BF16_TOL
    assert rel_err(dv[b:b + 1, hk:hk + 1], rv) <= BF16_TOL
    # rows of dS sum to 0, so the keys' gradients sum to 0 over the keys of each head
    ksum = dk.float().sum(dim=2)
    assert float(ksum.abs().max()) <= 2e-2 * float(dk.float().abs().max()) * 8
    for t in (dq, dk, dv):
        assert torch.isfinite(t).all()


def test_random_shapes_attention(mc, dev):
    """Seeded random shapes (batch, grouped K/V heads, ragged S, causal,
    additive mask; bf16 D = 64 / 128 through the MFMA kernels, fp32 through
    the generic ones) through the forward and backward, against an fp32 torch
    composite of the same maths (K/V heads repeated, scores scaled, mask
    added, causal entries -inf, softmax, .V) and its autograd on the GPU."""
    import random
    rng = random.Random(5)
    for it in range(12):
        dt = torch.bfloat16 if it % 4 else torch.float32
        D = rng.choice([64, 128]) if dt == torch.bfloat16 else rng.choice([32, 64, 80])
        Hkv, rep = rng.choice([1, 2, 4]), rng.choice([1, 2, 3])
        H, B = Hkv * rep, rng.randint(1, 3)
        S = rng.randint(1, 700 if dt == torch.bfloat16 else 200)
        causal, use_mask = rng.random() < 0.6, rng.random() < 0.25
        g = torch.Generator(device=dev).manual_seed(it)
        q = torch.randn(B, H, S, D, generator=g, device=dev).to(dt)
        k = torch.randn(B, Hkv, S, D, generator=g, device=dev).to(dt)
        v = torch.randn(B, Hkv, S, D, generator=g, device=dev).to(dt)
        mask = (torch.randn(S, S, generator=g, device=dev) * 2) if use_mask else None
        o, lse = mc.attention_forward(q, k, v, causal=causal, mask=mask)
        do = (torch.randn(B, S, H * D, generator=g, device=dev) * 0.1).to(dt)
        dq, dk, dv = mc.attention_backward(q, k, v, o, lse, do, causal=causal, mask=mask)
        qf, kf, vf = (t.float().requires_grad_(True) for t in (q, k, v))
        s = (qf @ kf.repeat_interleave(rep, dim=1).transpose(-1, -2).contiguous()) * D ** -0.5
        if mask is not None:
            s = s + mask
        if causal:
            s = s.masked_fill(torch.ones(S, S, dtype=torch.bool, device=dev).triu(1), float("-inf"))
        of = (torch.softmax(s, -1) @ vf.repeat_interleave(rep, dim=1)).transpose(1, 2).reshape(B, S, H * D)
        of.backward(do.float())
        torch.cuda.synchronize()
        # the reference itself is fp32 (not the fp64 oracle): 1e-4 for the fp32 kernels
        tol = 1e-4 if dt == torch.float32 else BF16_TOL
        for name, out, ref in (("o", o, of.detach()), ("dq", dq, qf.grad), ("dk", dk, kf.grad), ("dv", dv, vf.grad)):
            err = ((out.float() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
            assert err <= tol, f"{name} {dt} B={B} H={H} Hkv={Hkv} S={S} D={D} causal={causal} mask={use_mask}: {err:.3e}"
