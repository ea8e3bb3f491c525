"""GPU parity of the AdamW kernel (mc_adamw_step) against the CPU oracle
(oracle_adamw_step, pinned in tests/test_oracle_adamw.py).

The kernel evaluates the reference's fp32 op sequence (optimizer.rs:242-275)
with no fused multiply-add and correctly rounded division and square root,
so the bar is bit-exact: parameters and both moments are compared with
array_equal over several steps. Cases: the reference's test shapes (5x5,
3x3), ragged element counts around the kernel's vector width and block size,
more tensors than one launch's table holds, in-place and out-of-place
updates, per-tensor step counts (the reference's optimizer counts one step
per AdamW::step call), the c4 LoRA parameter set (A and B of the 7
projections), and non-finite gradients.
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def draw(g, n):
    return torch.randn(n, generator=g)


def run_case(mc, dev, sizes, steps, cfg, in_place=True, seed=0, grads=None):
    g = torch.Generator().manual_seed(seed)
    ps = [draw(g, n) for n in sizes]
    ms = [torch.zeros(n) for n in sizes]
    vs = [torch.zeros(n) for n in sizes]
    dp = [t.to(dev) for t in ps]
    dm = [t.to(dev) for t in ms]
    dv = [t.to(dev) for t in vs]
    ref = [(p.numpy().copy(), m.numpy().copy(), v.numpy().copy()) for p, m, v in zip(ps, ms, vs)]
    for it, step in enumerate(steps):
        gs = grads(it) if grads else [draw(g, n) for n in sizes]
        dg = [t.to(dev) for t in gs]
        step_list = step if isinstance(step, list) else [step] * len(sizes)
        if in_place:
            mc.adamw_step(dp, dg, dm, dv, step_list, **cfg)
        else:
            outs = [torch.empty_like(t) for t in dp]
            mc.adamw_step(dp, dg, dm, dv, step_list, outs=outs, **cfg)
            dp = outs
        ref = [oracle.adamw_step(p, gg.numpy(), m, v, s, **cfg) for (p, m, v), gg, s in zip(ref, gs, step_list)]
    torch.cuda.synchronize()
    for (p, m, v), a, b, c in zip(ref, dp, dm, dv):
        for got, want in ((a, p), (b, m), (c, v)):
            got = got.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)) or \
                np.array_equal(got, want, equal_nan=True)


DEFAULT = dict(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01)


def test_reference_shapes(mc, dev):
    # optimizer.rs:417-470: ones (5, 5) at lr 0.1; ones (3, 3) for five steps
    p = [torch.ones(25, device=dev)]
    mc.adamw_step(p, [torch.ones(25, device=dev)], [torch.zeros(25, device=dev)], [torch.zeros(25, device=dev)], 1,
                  lr=0.1)
    torch.cuda.synchronize()
    want, _, _ = oracle.adamw_step(np.ones(25, np.float32), np.ones(25, np.float32), np.zeros(25, np.float32),
                                   np.zeros(25, np.float32), 1, lr=0.1)
    assert np.array_equal(p[0].cpu().numpy(), want)
    run_case(mc, dev, [9], [1, 2, 3, 4, 5], DEFAULT, grads=lambda it: [torch.ones(9)])


@pytest.mark.parametrize("in_place", [True, False])
def test_ragged_sizes(mc, dev, in_place):
    sizes = [1, 3, 4, 5, 7, 8, 1023, 1024, 2047, 2048, 2049, 4096, 4099, 24576, 100003]
    run_case(mc, dev, sizes, [1, 2, 3], dict(lr=3e-3, beta1=0.85, beta2=0.99, eps=1e-6, weight_decay=0.1),
             in_place=in_place, seed=1)


def test_more_tensors_than_one_launch(mc, dev):
    sizes = [(i * 37) % 500 + 1 for i in range(37)] + [0, 0]
    run_case(mc, dev, sizes, [1, 2], DEFAULT, seed=2)


def test_per_tensor_steps(mc, dev):
    # the reference's optimizer counts one step per AdamW::step call, so the
    # tensors of one training step see different t (optimizer.rs:235-237)
    sizes = [100, 200, 300, 400]
    run_case(mc, dev, sizes, [[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]], DEFAULT, seed=3)


def test_c4_lora_parameters(mc, dev):
    shapes = [(1536, 16), (16, 1536), (1536, 16), (16, 256), (1536, 16), (16, 256), (1536, 16), (16, 1536),
              (1536, 16), (16, 8960), (1536, 16), (16, 8960), (8960, 16), (16, 1536)]
    sizes = [a * b for a, b in shapes]
    run_case(mc, dev, sizes, list(range(1, 15)), dict(lr=2e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01),
             seed=4)


def test_large_step_counts(mc, dev):
    run_case(mc, dev, [513, 4097], [1000, 2 ** 20, 2 ** 31 - 1], DEFAULT, seed=5)


def test_non_finite_gradients(mc, dev):
    def grads(it):
        g = torch.randn(64, generator=torch.Generator().manual_seed(it))
        g[3] = float("nan")
        g[5] = float("inf")
        g[7] = -float("inf")
        return [g]
    run_case(mc, dev, [64], [1, 2], DEFAULT, seed=6, grads=grads)
