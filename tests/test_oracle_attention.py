"""Pins the attention oracle (oracle_attention_fwd / _bwd) before it is trusted
as the checker of the attention kernels (no GPU).

The reference's own attention tests (src/models/transformer.rs:443-480) only
assert shapes (zero weights give zero activations), so the oracle is pinned by:
  * closed forms: q = 0 makes every score equal, so a row of o is the mean of
    the v rows it sees (all of them, or the causal prefix); S = 1 gives o = v;
    one key with a dominant score gives that key's v row;
  * an all-zero [1, 1, S, S] mask equal to no mask (transformer.rs:469-480);
  * torch.nn.functional.scaled_dot_product_attention on the CPU in fp64 as a
    library cross-check (K/V repeated with repeat_interleave, the order
    repeat_kv builds at transformer.rs:300-318), for o and the log-sum-exp;
  * grouped K/V heads equal to explicitly repeated heads;
  * the backward against torch autograd of the fp64 composite and against
    central finite differences of the oracle's own forward.
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


def torch_attention(q, k, v, scale, causal, mask):
    """fp64 CPU composite: q.k^T * scale + mask (+ causal -inf), softmax, .v."""
    q, k, v = (torch.from_numpy(np.asarray(a, np.float64)) for a in (q, k, v))
    B, H, S, D = q.shape
    rep = H // k.shape[1]
    k = k.repeat_interleave(rep, dim=1)
    v = v.repeat_interleave(rep, dim=1)
    add = torch.zeros(S, S, dtype=torch.float64)
    if mask is not None:
        add = add + torch.from_numpy(np.asarray(mask, np.float64))
    if causal:
        add = add.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=add, scale=scale)
    scores = q @ k.transpose(-1, -2) * scale + add
    lse = torch.logsumexp(scores, dim=-1)
    return o.transpose(1, 2).reshape(B, S, H * D).numpy(), lse.numpy()


def test_uniform_scores_give_mean_of_v():
    B, H, Hkv, S, D = 2, 4, 2, 9, 16
    q = np.zeros((B, H, S, D), np.float32)
    k, v = rand((B, Hkv, S, D), 1), rand((B, Hkv, S, D), 2)
    o, lse = oracle.attention_fwd(q, k, v, 0.25, causal=False)
    oc, lsec = oracle.attention_fwd(q, k, v, 0.25, causal=True)
    for b in range(B):
        for h in range(H):
            vh = v[b, h // 2].astype(np.float64)
            full = o[b, :, h * D:(h + 1) * D]
            assert np.allclose(full, vh.mean(axis=0)[None, :], atol=1e-6)
            prefix = np.cumsum(vh, axis=0) / np.arange(1, S + 1)[:, None]
            assert np.allclose(oc[b, :, h * D:(h + 1) * D], prefix, atol=1e-6)
    assert np.allclose(lse, np.log(S), atol=1e-6)
    assert np.allclose(lsec, np.log(np.arange(1, S + 1))[None, None, :], atol=1e-6)


def test_single_key_gives_v():
    q, k, v = rand((2, 3, 1, 8), 3), rand((2, 3, 1, 8), 4), rand((2, 3, 1, 8), 5)
    for causal in (False, True):
        o, lse = oracle.attention_fwd(q, k, v, 0.3, causal=causal)
        assert np.array_equal(o.reshape(2, 1, 3, 8), v.transpose(0, 2, 1, 3))
        s = (q * k).sum(-1, dtype=np.float64) * np.float32(0.3)
        assert np.allclose(lse, s, atol=1e-6)


def test_dominant_key_selects_its_value():
    S, D = 12, 8
    k = rand((1, 1, S, D), 6)
    v = rand((1, 1, S, D), 7)
    q = (k[:, :, 5:6, :] * 50.0).repeat(S, axis=2)  # score of key 5 dominates every row
    o, _ = oracle.attention_fwd(q, k, v, 1.0, causal=False)
    assert np.allclose(o[0], np.repeat(v[0, 0, 5:6, :], S, axis=0), atol=1e-5)


def test_zero_mask_equals_no_mask():
    # test_attention_with_mask: 4 heads, no GQA, [1, 1, 8, 8] zero mask
    q, k, v = rand((1, 4, 8, 32), 8), rand((1, 4, 8, 32), 9), rand((1, 4, 8, 32), 10)
    a, la = oracle.attention_fwd(q, k, v, 32 ** -0.5)
    b, lb = oracle.attention_fwd(q, k, v, 32 ** -0.5, mask=np.zeros((8, 8), np.float32))
    assert np.array_equal(a, b) and np.array_equal(la, lb)


@pytest.mark.parametrize("B,H,Hkv,S,D,causal,masked", [
    (1, 4, 2, 8, 32, False, False),    # test_attention_forward's geometry (transformer.rs:456-466)
    (1, 4, 4, 8, 32, False, True),     # test_attention_with_mask's geometry
    (2, 6, 2, 37, 16, True, False),
    (1, 12, 2, 64, 128, True, True),
    (2, 3, 1, 50, 64, False, True),
])
def test_matches_torch_sdpa(B, H, Hkv, S, D, causal, masked):
    q, k, v = rand((B, H, S, D), 11), rand((B, Hkv, S, D), 12), rand((B, Hkv, S, D), 13)
    mask = rand((S, S), 14) if masked else None
    scale = D ** -0.5
    o, lse = oracle.attention_fwd(q, k, v, scale, causal=causal, mask=mask)
    ro, rl = torch_attention(q, k, v, scale, causal, mask)
    assert rel(o, ro) < 1e-6
    assert rel(lse, rl) < 1e-6


def test_grouped_heads_equal_repeated_heads():
    B, H, Hkv, S, D = 2, 6, 2, 20, 16
    q, k, v = rand((B, H, S, D), 15), rand((B, Hkv, S, D), 16), rand((B, Hkv, S, D), 17)
    rep = H // Hkv
    a, la = oracle.attention_fwd(q, k, v, 0.2, causal=True)
    b, lb = oracle.attention_fwd(q, np.repeat(k, rep, axis=1), np.repeat(v, rep, axis=1), 0.2, causal=True)
    assert np.array_equal(a, b) and np.array_equal(la, lb)


def test_fully_masked_row_is_nan():
    q, k, v = rand((1, 1, 4, 8), 18), rand((1, 1, 4, 8), 19), rand((1, 1, 4, 8), 20)
    mask = np.zeros((4, 4), np.float32)
    mask[2, :] = -np.inf
    o, lse = oracle.attention_fwd(q, k, v, 0.5, mask=mask)
    assert np.isnan(o[0, 2]).all() and np.isfinite(np.delete(o[0], 2, axis=0)).all()


@pytest.mark.parametrize("B,H,Hkv,S,D,causal,masked", [
    (1, 2, 1, 7, 8, True, False),
    (2, 4, 2, 11, 16, False, True),
    (1, 3, 3, 16, 32, True, True),
])
def test_backward_matches_torch_autograd(B, H, Hkv, S, D, causal, masked):
    q, k, v = rand((B, H, S, D), 21), rand((B, Hkv, S, D), 22), rand((B, Hkv, S, D), 23)
    do = rand((B, S, H * D), 24)
    mask = rand((S, S), 25) if masked else None
    scale = D ** -0.5
    dq, dk, dv = oracle.attention_bwd(q, k, v, do, scale, causal=causal, mask=mask)
    tq, tk, tv = (torch.from_numpy(a.astype(np.float64)).requires_grad_() for a in (q, k, v))
    rep = H // Hkv
    add = torch.zeros(S, S, dtype=torch.float64)
    if mask is not None:
        add = add + torch.from_numpy(mask.astype(np.float64))
    if causal:
        add = add.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    p = torch.softmax(tq @ tk.repeat_interleave(rep, 1).transpose(-1, -2) * scale + add, dim=-1)
    o = (p @ tv.repeat_interleave(rep, 1)).transpose(1, 2).reshape(B, S, H * D)
    o.backward(torch.from_numpy(do.astype(np.float64)))
    assert rel(dq, tq.grad.numpy()) < 1e-6
    assert rel(dk, tk.grad.numpy()) < 1e-6
    assert rel(dv, tv.grad.numpy()) < 1e-6


def test_backward_finite_differences():
    B, H, Hkv, S, D = 1, 2, 1, 6, 4
    q, k, v = rand((B, H, S, D), 26), rand((B, Hkv, S, D), 27), rand((B, Hkv, S, D), 28)
    do = rand((B, S, H * D), 29)
    scale = 0.7
    dq, dk, dv = oracle.attention_bwd(q, k, v, do, scale, causal=True)

    def loss(q_, k_, v_):
        o, _ = oracle.attention_fwd(q_, k_, v_, scale, causal=True)
        return float((o.astype(np.float64) * do).sum())

    eps = 1e-2
    for name, x, g in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
        for idx in [(0, 0, 0, 0), (0, 0, 3, 2), (0, x.shape[1] - 1, S - 1, D - 1), (0, 0, 1, 3)]:
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = {"q": (xp, k, v), "k": (q, xp, v), "v": (q, k, xp)}[name]
            args_m = {"q": (xm, k, v), "k": (q, xm, v), "v": (q, k, xm)}[name]
            fd = (loss(*args_p) - loss(*args_m)) / (2 * eps)
            assert abs(fd - g[idx]) < 2e-3 * max(1.0, abs(fd)), (name, idx, fd, g[idx])
