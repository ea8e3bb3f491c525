"""Pins the AdamW oracle (oracle_adamw_step) before it is trusted as the
checker of the AdamW kernel (no GPU):
  * the reference's own AdamW tests (src/training/optimizer.rs:395-509): one
    step at lr 0.1 from ones with gradient ones changes the parameter (the
    closed form gives 1 - 0.1 - 0.1 * 0.01 = 0.899), five default steps lower
    the sum below 9, the step count drives the bias correction;
  * the constant-gradient closed form: with g_t = c for every t the bias
    corrections give m_hat = c and v_hat = c^2 exactly in real arithmetic, so
    p_t = p_{t-1} - lr c / (|c| + eps) - lr wd p_{t-1};
  * torch.optim.AdamW (decoupled weight decay) on the CPU as a library
    cross-check over several steps with fresh gradients.
"""
import numpy as np
import pytest
import torch

import oracle


def test_reference_single_step_known_answer():
    # test_adamw_step (optimizer.rs:417-445): ones (5, 5), gradient ones, lr 0.1
    p, m, v = oracle.adamw_step(np.ones(25, np.float32), np.ones(25, np.float32), np.zeros(25, np.float32),
                                np.zeros(25, np.float32), 1, lr=0.1)
    assert np.allclose(p, 0.899, atol=1e-6)
    assert abs(p.sum() - 25.0) > 1e-6
    assert np.allclose(m, 0.1, rtol=1e-6) and np.allclose(v, 0.001, rtol=1e-5)


def test_reference_multiple_steps_lower_the_sum():
    # test_adamw_multiple_steps (optimizer.rs:448-470): 5 default steps, ones, gradient ones
    p = np.ones(9, np.float32)
    m = np.zeros(9, np.float32)
    v = np.zeros(9, np.float32)
    for t in range(1, 6):
        p, m, v = oracle.adamw_step(p, np.ones(9, np.float32), m, v, t)
    assert p.sum() < 9.0
    # each step moves by lr * (1 / (1 + eps) + wd * p) in the closed form
    ref = 1.0
    for _ in range(5):
        ref = ref - 1e-4 * (1.0 / (1.0 + 1e-8)) - 1e-4 * 0.01 * ref
    assert np.allclose(p, ref, rtol=1e-6)


@pytest.mark.parametrize("c", [0.3, -2.0, 1e-3, 7.5])
def test_constant_gradient_closed_form(c):
    lr, wd, eps = 1e-2, 0.05, 1e-8
    rng = np.random.default_rng(1)
    p = rng.standard_normal(64).astype(np.float32)
    m = np.zeros(64, np.float32)
    v = np.zeros(64, np.float32)
    ref = p.astype(np.float64)
    g = np.full(64, c, np.float32)
    for t in range(1, 11):
        p, m, v = oracle.adamw_step(p, g, m, v, t, lr=lr, weight_decay=wd, eps=eps)
        ref = ref - lr * float(np.float32(c)) / (abs(float(np.float32(c))) + eps) - lr * wd * ref
    assert np.abs(p - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


def test_matches_torch_adamw():
    rng = np.random.default_rng(2)
    shape = (40, 16)
    p0 = rng.standard_normal(shape).astype(np.float32)
    lr, b1, b2, eps, wd = 3e-3, 0.85, 0.99, 1e-6, 0.1
    tp = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.AdamW([tp], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    p, m, v = p0.copy(), np.zeros(shape, np.float32), np.zeros(shape, np.float32)
    for t in range(1, 7):
        g = rng.standard_normal(shape).astype(np.float32)
        tp.grad = torch.from_numpy(g.copy())
        opt.step()
        p, m, v = oracle.adamw_step(p, g, m, v, t, lr=lr, beta1=b1, beta2=b2, eps=eps, weight_decay=wd)
    st = opt.state[tp]
    assert np.abs(p - tp.detach().numpy()).max() <= 1e-6 * np.abs(p).max()
    assert np.abs(m - st["exp_avg"].numpy()).max() <= 1e-6 * np.abs(m).max()
    assert np.abs(v - st["exp_avg_sq"].numpy()).max() <= 1e-6 * np.abs(v).max()


def test_inputs_not_modified_and_zero_gradient():
    p = np.linspace(-1, 1, 10).astype(np.float32)
    g = np.zeros(10, np.float32)
    m = np.zeros(10, np.float32)
    v = np.zeros(10, np.float32)
    out, m1, v1 = oracle.adamw_step(p, g, m, v, 1, lr=0.5, weight_decay=0.2)
    assert not m.any() and not v.any()
    # g = 0: the moments stay 0, only the decoupled decay acts: p (1 - lr wd), with lr wd rounded to fp32
    assert np.array_equal(m1, np.zeros(10, np.float32))
    assert np.allclose(out, p - p * np.float32(0.5 * np.float32(0.2)), atol=1e-7)
