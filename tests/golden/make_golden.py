"""Writes tests/golden/golden_small.json: fp64 numpy evaluations of the six
hot-path functions on tiny seeded inputs, plus the known answers of the
reference's own tests. The numpy forms here (whole-matrix products, closed
form gradients) are written independently of oracle.c's loops, so the
fixtures catch index / transposition / dropped-term mistakes in the oracle.

Reference known answers recorded:
  LoRA executor test      tests/executor_direct.rs:345-367 (inputs; output
                          hand-derived: (x.A).B * 0.5)
  RMSNorm [3, 4], eps 0   tests/executor_direct.rs:480-495
  softmax zeros -> 1/3    src/backend/tensor.rs:262-276

Run: python tests/golden/make_golden.py
"""
import json
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_small.json")


def keep_mask(rng, T, r, p):
    return (rng.random((T, r)) >= p).astype(np.uint8)


def lora_case(seed, T, K, N, r, scale, p, with_w, with_bias):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    x, A, B, dy = f(T, K), f(K, r), f(r, N), f(T, N)
    W = f(N, K) if with_w else None
    b = f(N) if with_bias else None
    mask = keep_mask(rng, T, r, p) if p > 0 else None
    x64, A64, B64, dy64 = (a.astype(np.float64) for a in (x, A, B, dy))
    ks = np.float64(np.float32(1.0) / (np.float32(1.0) - np.float32(p))) if mask is not None else 1.0
    H = (x64 @ A64).astype(np.float32).astype(np.float64)  # candle stores x.A in fp32
    M = mask.astype(np.float64) * ks if mask is not None else 1.0
    Hd = (H * M).astype(np.float32).astype(np.float64)
    y = scale * (Hd @ B64)
    if W is not None:
        y = y + x64 @ W.astype(np.float64).T
        if b is not None:
            y = y + b.astype(np.float64)
    G = scale * (dy64 @ B64.T)
    Gd = G * M
    dx = Gd @ A64.T
    if W is not None:
        dx = dx + dy64 @ W.astype(np.float64)
    dA = x64.T @ Gd
    dB = scale * (Hd.T @ dy64)
    enc = lambda a: None if a is None else np.asarray(a).tolist()  # noqa: E731
    return {
        "seed": seed, "T": T, "K": K, "N": N, "r": r, "scale": scale, "p": p,
        "x": enc(x), "W": enc(W), "bias": enc(b), "A": enc(A), "B": enc(B), "dy": enc(dy), "mask": enc(mask),
        "y": enc(y), "hd": enc(Hd), "dx": enc(dx), "dA": enc(dA), "dB": enc(dB),
    }


def rmsnorm_case(seed, rows, D, eps, weighted):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, D)).astype(np.float32)
    w = (rng.standard_normal(D) * 0.1 + 1).astype(np.float32) if weighted else None
    dy = rng.standard_normal((rows, D)).astype(np.float32)
    x64 = x.astype(np.float64)
    w64 = w.astype(np.float64) if weighted else np.ones(D)
    rms = np.sqrt((x64 ** 2).mean(-1, keepdims=True) + eps)
    y = x64 / rms * w64
    r = 1 / rms
    g = dy.astype(np.float64) * w64
    dx = r * g - x64 * r ** 3 * (g * x64).mean(-1, keepdims=True)
    dw = (dy.astype(np.float64) * x64 * r).sum(0)
    return {"seed": seed, "rows": rows, "D": D, "eps": eps, "x": x.tolist(), "w": None if w is None else w.tolist(),
            "dy": dy.tolist(), "y": y.tolist(), "rstd": r[:, 0].tolist(), "dx": dx.tolist(), "dw": dw.tolist()}


def softmax_case(seed, rows, D, causal_rows):
    rng = np.random.default_rng(seed)
    s = (rng.standard_normal((rows, D)) * 3).astype(np.float32)
    dp = rng.standard_normal((rows, D)).astype(np.float32)
    z = s.astype(np.float64).copy()
    if causal_rows:
        q = np.arange(rows)[:, None] % causal_rows
        z[np.arange(D)[None, :] > q + (D - causal_rows)] = -np.inf
    e = np.exp(z - z.max(-1, keepdims=True))
    P = e / e.sum(-1, keepdims=True)
    P32 = P.astype(np.float32).astype(np.float64)
    ds = P32 * (dp.astype(np.float64) - (P32 * dp).sum(-1, keepdims=True))
    return {"seed": seed, "rows": rows, "D": D, "causal_rows": causal_rows, "s": s.tolist(), "dp": dp.tolist(),
            "p": P.tolist(), "ds_given_p32": ds.tolist()}


def main():
    data = {
        "lora": [
            lora_case(1, 4, 8, 6, 2, 2.0, 0.0, True, True),
            lora_case(2, 4, 8, 6, 2, 2.0, 0.25, True, False),
            lora_case(3, 5, 3, 7, 3, 0.5, 0.0, False, False),
            lora_case(4, 6, 16, 8, 4, 1.5, 0.5, False, False),
        ],
        "rmsnorm": [rmsnorm_case(5, 3, 5, 1e-6, True), rmsnorm_case(6, 4, 8, 1e-5, False),
                    rmsnorm_case(7, 2, 1, 0.0, True)],
        "softmax": [softmax_case(8, 4, 6, 0), softmax_case(9, 8, 6, 4), softmax_case(10, 3, 3, 3)],
        "known_answers": {
            "lora_executor": {"x": [[1, 2, 3, 4], [5, 6, 7, 8]],
                              "A": [[0.1, 0.2], [0.3, 0.4], [0.5, 0.6], [0.7, 0.8]],
                              "B": [[1, 2, 3, 4], [5, 6, 7, 8]], "scale": 0.5,
                              "y": [[17.5, 23.0, 28.5, 34.0], [40.7, 53.4, 66.1, 78.8]]},
            "rmsnorm_3_4": {"x": [3.0, 4.0], "eps": 0.0, "y": [3 / np.sqrt(12.5), 4 / np.sqrt(12.5)]},
            "softmax_zeros": {"s": [[0.0, 0.0, 0.0]], "p": [[1 / 3, 1 / 3, 1 / 3]]},
        },
    }
    with open(OUT, "w") as fh:
        json.dump(data, fh, indent=None, separators=(",", ":"))
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
