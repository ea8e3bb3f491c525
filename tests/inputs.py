"""Seeded synthetic inputs in the distributions BASELINE.json's configs name.

N(mu, sigma) is mean / standard deviation; kaiming-uniform A is U(-1/sqrt(K),
1/sqrt(K)) (torch kaiming_uniform_ with a = sqrt(5), fan_in = K). bf16
tensors are rounded from the fp32 draw, and the oracle is fed the rounded
values, so both paths see the same bytes.
"""
import numpy as np
import torch


def gen(seed):
    return torch.Generator().manual_seed(seed)


def normal(g, shape, std=1.0, mean=0.0):
    return torch.randn(*shape, generator=g) * std + mean


def kaiming_uniform(g, K, r):
    b = 1.0 / np.sqrt(K)
    return (torch.rand(K, r, generator=g) * 2 - 1) * b


def lora_case(seed, T, K, N, r, dtype=torch.bfloat16, bias=False, w=True, dy_std=1e-2, x_std=1.0):
    g = gen(seed)
    c = {
        "x": normal(g, (T, K), x_std).to(dtype),
        "W": normal(g, (N, K), 0.02).to(dtype) if w else None,
        "A": kaiming_uniform(g, K, r),
        "B": normal(g, (r, N), 0.02),
        "dy": normal(g, (T, N), dy_std).to(dtype),
    }
    c["bias"] = normal(g, (N,), 0.02).to(dtype) if bias else None
    return c


def np32(t):
    return None if t is None else t.float().numpy()
