"""Benchmark of the fused LoRA / RMSNorm / softmax hot path on one MI355X.

A step is one forward + backward pass of the custom ops of one decoder layer
(BASELINE.json config 4 by default: a Qwen2.5-1.5B-shaped layer, bf16,
tokens 8 x 2048, hidden 1536, intermediate 8960, 12 q / 2 kv heads of 128,
LoRA rank 16 / alpha 32 on all 7 projections, preceded by RMSNorm):

  forward   RMSNorm(input_layernorm) -> LoRA q, k, v (with bias)
            causal softmax over the [8, 12, 2048, 2048] attention scores
            LoRA o_proj ; RMSNorm(post_attention_layernorm)
            LoRA gate, up ; LoRA down
  backward  the same ops in reverse (dX, dA, dB for every projection with W
            frozen; dx, dw for both norms; dS for the softmax)

The attention matmuls and the SiLU are not custom ops of the reference and
are not part of the step; their outputs are synthetic tensors of the right
shape. Inputs are synthetic (seeded normal / kaiming-uniform draws) and
resident in HBM before timing starts.

value = tokens / second of the timed steps (plain eager calls; with --graph
the step is captured once into a HIP graph, torch.cuda.CUDAGraph, and the
timed steps are replays: the entry points allocate nothing, never
synchronise and record no memset, so they capture). The roofline object is
for the dominant kernel, the MFMA GEMM (base x.W^T / dY.W with the rank-r
columns folded in), timed per launch with hipEvents on its stream by the
library's profiling hook in a separate pass after the timed steps (the
hook's events are not in the timed region); achieved counts the
base-product FLOPs only.

The attention core next to the softmax (mc_attention_fwd / _bwd, flash
kernels, the materialised score matrix never reaches HBM) is measured in the
same run at the layer's attention shape, outside the step and outside value:
the "attention" object gives its per-call times and MFMA rate (FLOPs of the
score and P.V products over the causal lower triangle; the backward counts
its four algorithmic products, not the recomputation). The "adamw" object
times one AdamW step (mc_adamw_step) over the layer's LoRA parameters, and
"row_ops" the LayerNorm and cross-entropy row kernels (cross entropy over a
Qwen2.5-sized vocabulary of 151936), also outside the step.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# HBM bytes per base-GEMM launch (gemm_bf16_kernel / gemm_bf16_split, average
# over a step's launches),
# measured with two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE)
# scaled by the same counters on a 256 MiB copy (--copy-calibration); the
# summary and commands are in profiles/gemm_bf16_c4_hbm_traffic.md.
# Re-measured whenever the GEMM's tiling changes; None for unmeasured configs.
GEMM_TRAFFIC_BYTES = {"c4": 468.3e6}
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3

CONFIGS = {
    # name: tokens, hidden, intermediate, q heads, kv heads, head_dim, rank, alpha, dropout, batch, seq, dtype
    "c3": dict(batch=16, seq=512, hidden=896, inter=None, heads=14, kv_heads=2, head_dim=64, rank=8, alpha=16,
               dropout=0.0, projections=("q", "v"), norm=False, softmax=False, dtype="bf16",
               workload="LoRA fwd+bwd, Qwen2.5-0.5B-shaped q_proj 896->896 + v_proj 896->128, r8, T=16x512"),
    "c4": dict(batch=8, seq=2048, hidden=1536, inter=8960, heads=12, kv_heads=2, head_dim=128, rank=16, alpha=32,
               dropout=0.0, projections=("q", "k", "v", "o", "gate", "up", "down"), norm=True, softmax=True,
               dtype="bf16",
               workload="Qwen2.5-1.5B-shaped decoder layer custom ops fwd+bwd: RMSNorm x2, LoRA r16 on 7 "
                        "projections, causal softmax [8,12,2048,2048]; T=8x2048"),
    "c5": dict(batch=4, seq=4096, hidden=3584, inter=18944, heads=28, kv_heads=4, head_dim=128, rank=64, alpha=128,
               dropout=0.1, projections=("q", "k", "v", "o", "gate", "up", "down"), norm=True, softmax=True,
               dtype="bf16",
               workload="Qwen2.5-7B-shaped decoder layer custom ops fwd+bwd: RMSNorm x2, LoRA r64 p=0.1 on 7 "
                        "projections, causal softmax [4,28,4096,4096]; T=4x4096"),
}


def proj_shapes(c):
    h, kv = c["hidden"], c["kv_heads"] * c["head_dim"]
    inter = c["inter"]
    table = {
        "q": (h, c["heads"] * c["head_dim"], True),
        "k": (h, kv, True),
        "v": (h, kv, True),
        "o": (c["heads"] * c["head_dim"], h, False),
        "gate": (h, inter, False),
        "up": (h, inter, False),
        "down": (inter, h, False),
    }
    return {p: table[p] for p in c["projections"]}


class Layer:
    """Device-resident tensors of one layer's custom ops."""

    def __init__(self, mc, c, dev, seed=0):
        import torch

        self.mc, self.c, self.dev = mc, c, dev
        self.T = c["batch"] * c["seq"]
        dt = torch.bfloat16 if c["dtype"] == "bf16" else torch.float32
        g = torch.Generator(device=dev).manual_seed(seed)
        rn = lambda *s, std=1.0: (torch.randn(*s, generator=g, device=dev) * std)  # noqa: E731
        T, H = self.T, c["hidden"]
        self.scale = c["alpha"] / c["rank"]
        self.p = c["dropout"]
        self.proj = {}
        for name, (K, N, bias) in proj_shapes(c).items():
            b = 1.0 / K ** 0.5
            self.proj[name] = dict(
                K=K, N=N,
                W=rn(N, K, std=0.02).to(dt),
                bias=rn(N, std=0.02).to(dt) if bias else None,
                A=(torch.rand(K, c["rank"], generator=g, device=dev) * 2 - 1) * b,
                B=rn(c["rank"], N, std=0.02),
                dy=rn(T, N, std=1e-2).to(dt),
                mask=(mc.dropout_mask(1234 + len(self.proj), self.p, T, c["rank"]).to(dev) if self.p > 0 else None),
            )
        self.h_in = rn(T, H).to(dt)
        self.h_mid = rn(T, H).to(dt)
        self.attn = rn(T, c["heads"] * c["head_dim"]).to(dt)
        self.act = rn(T, c["inter"]).to(dt) if c["inter"] else None
        self.ln1 = (rn(H, std=0.1) + 1.0).to(dt)
        self.ln2 = (rn(H, std=0.1) + 1.0).to(dt)
        self.dy_ln = rn(T, H, std=1e-2).to(dt)
        if c["softmax"]:
            shape = (c["batch"], c["heads"], c["seq"], c["seq"])
            self.scores = (rn(*shape, std=3.0)).to(dt)
            self.dP = (rn(*shape, std=1e-2)).to(dt)
        self.xn1 = rn(T, H).to(dt)
        self.xn2 = rn(T, H).to(dt)

    def _input_of(self, name):
        if name in ("q", "k", "v"):
            return self.xn1
        if name == "o":
            return self.attn
        if name in ("gate", "up"):
            return self.xn2
        return self.act

    def step(self):
        mc, c = self.mc, self.c
        saved = {}
        if c["norm"]:
            self.xn1, r1 = mc.rms_norm_forward(self.h_in, 1e-6, self.ln1)
        order_f = [p for p in ("q", "k", "v") if p in self.proj]
        for name in order_f:
            saved[name] = self._lora_f(name)
        P = mc.softmax_forward(self.scores, causal_rows=c["seq"]) if c["softmax"] else None
        if "o" in self.proj:
            saved["o"] = self._lora_f("o")
        if c["norm"]:
            self.xn2, r2 = mc.rms_norm_forward(self.h_mid, 1e-6, self.ln2)
        for name in ("gate", "up", "down"):
            if name in self.proj:
                saved[name] = self._lora_f(name)
        # backward
        for name in ("down", "up", "gate"):
            if name in self.proj:
                self._lora_b(name, saved[name])
        if c["norm"]:
            mc.rms_norm_backward(self.h_mid, self.dy_ln, 1e-6, self.ln2, r2)
        if "o" in self.proj:
            self._lora_b("o", saved["o"])
        if c["softmax"]:
            mc.softmax_backward(P, self.dP, causal_rows=c["seq"])
        for name in ("v", "k", "q"):
            if name in self.proj:
                self._lora_b(name, saved[name])
        if c["norm"]:
            mc.rms_norm_backward(self.h_in, self.dy_ln, 1e-6, self.ln1, r1)

    def _lora_f(self, name):
        pr = self.proj[name]
        _, h = self.mc.lora_forward(self._input_of(name), pr["A"], pr["B"], self.scale, W=pr["W"],
                                    bias=pr["bias"], mask=pr["mask"], dropout_p=self.p)
        return h

    def _lora_b(self, name, h):
        pr = self.proj[name]
        self.mc.lora_backward(self._input_of(name), pr["A"], pr["B"], pr["dy"], self.scale, W=pr["W"],
                              mask=pr["mask"], dropout_p=self.p, h_save=h)

    def flops_per_step(self):
        base = sum(4.0 * self.T * p["K"] * p["N"] for p in self.proj.values())
        low = sum(6.0 * self.T * self.c["rank"] * (p["K"] + p["N"]) for p in self.proj.values())
        return base, low


def cpu_baseline(c, tokens, threads):
    """The oracle (C, fp64 accumulation, OpenMP) on a token sample of the
    same layer: LoRA fwd+bwd of every projection, both RMSNorms fwd+bwd and
    the softmax rows of the sampled tokens. Returns tokens / second."""
    import numpy as np

    import oracle

    rng = np.random.default_rng(0)
    T = tokens
    f32 = lambda *s, std=1.0: (rng.standard_normal(s) * std).astype(np.float32)  # noqa: E731
    work = []
    for name, (K, N, bias) in proj_shapes(c).items():
        b = 1.0 / K ** 0.5
        work.append(dict(x=f32(T, K), W=f32(N, K, std=0.02), bias=f32(N, std=0.02) if bias else None,
                         A=((rng.random((K, c["rank"])) * 2 - 1) * b).astype(np.float32),
                         B=f32(c["rank"], N, std=0.02), dy=f32(T, N, std=1e-2),
                         mask=oracle.dropout_mask(1234, c["dropout"], T, c["rank"]) if c["dropout"] > 0 else None))
    H = c["hidden"]
    xs, dys, w = f32(T, H), f32(T, H, std=1e-2), f32(H, std=0.1) + 1
    S = c["seq"]
    srows = T * c["heads"] if c["softmax"] else 0
    scores = f32(srows, S, std=3.0) if srows else None
    dP = f32(srows, S, std=1e-2) if srows else None
    ids = (np.arange(srows) % S).astype(np.int64) if srows else None
    s = c["alpha"] / c["rank"]
    t0 = time.perf_counter()
    for wk in work:
        oracle.lora_fwd(wk["x"], wk["A"], wk["B"], s, W=wk["W"], bias=wk["bias"], mask=wk["mask"],
                        p=c["dropout"], threads=threads)
        oracle.lora_bwd(wk["x"], wk["A"], wk["B"], wk["dy"], s, W=wk["W"], mask=wk["mask"], p=c["dropout"],
                        threads=threads)
    if c["norm"]:
        for _ in range(2):
            oracle.rmsnorm_fwd(xs, 1e-6, w, threads=threads)
            oracle.rmsnorm_bwd(xs, dys, 1e-6, w, threads=threads)
    if srows:
        P = oracle.softmax_fwd(scores, causal_rows=S, threads=threads, row_ids=ids)
        oracle.softmax_bwd(P, dP, causal_rows=S, threads=threads, row_ids=ids)
    dt = time.perf_counter() - t0
    return T / dt, dt


def queue_ahead(torch):
    """Occupy the GPU for a few ms before a loop of short calls, so the host
    has enqueued them all before the first runs: the profiling hook's events
    then bracket each call's kernels rather than the host's launch gaps."""
    torch.cuda._sleep(5_000_000)  # ~2 ms: ample for the host to enqueue a loop of calls


def attention_core(mc, c, dev, iters):
    """fwd / bwd of the attention core at the layer's shape, timed per call by
    the library's profiling hook (hipEvents on the launch stream)."""
    import torch

    B, H, Hkv, S, D = c["batch"], c["heads"], c["kv_heads"], c["seq"], c["head_dim"]
    g = torch.Generator(device=dev).manual_seed(7)
    q = torch.randn(B, H, S, D, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, device=dev, generator=g).to(torch.bfloat16)
    dout = torch.randn(B, S, H * D, device=dev, generator=g).to(torch.bfloat16)
    o, lse = mc.attention_forward(q, k, v, causal=True)
    mc.attention_backward(q, k, v, o, lse, dout, causal=True)
    torch.cuda.synchronize()
    out = {"shape": {"batch": B, "heads": H, "kv_heads": Hkv, "seq": S, "head_dim": D, "causal": True},
           "iters": iters}
    for name, fn in (("fwd", lambda: mc.attention_forward(q, k, v, causal=True)),
                     ("bwd", lambda: mc.attention_backward(q, k, v, o, lse, dout, causal=True))):
        mc._lib.check(mc._lib.lib().mc_profile_reset())
        mc._lib.check(mc._lib.lib().mc_profile_enable(1))
        queue_ahead(torch)
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
        mc._lib.check(mc._lib.lib().mc_profile_enable(0))
        mc._lib.check(mc._lib.lib().mc_profile_collect())
        ms, n, fl, by = mc._lib.profile_read("attention")
        tf = fl / (ms * 1e-3) / 1e12
        out[name] = {"us_per_call": ms * 1e3 / n, "TFLOP_s": tf, "mfma_frac": tf / BF16_PEAK_TFLOPS,
                     "GB_s": by / (ms * 1e-3) / 1e9}
    return out


def adamw_update(mc, c, dev, iters):
    """One AdamW step over the layer's LoRA parameters (A [K, r] and B [r, N]
    of every projection) per call, timed by the library's profiling hook."""
    import torch

    g = torch.Generator(device=dev).manual_seed(11)
    shapes = []
    for name in c["projections"]:
        K, N, _ = proj_shapes(c)[name]
        shapes += [(K, c["rank"]), (c["rank"], N)]
    ps = [torch.randn(*s, device=dev, generator=g) for s in shapes]
    gs = [torch.randn(*s, device=dev, generator=g) for s in shapes]
    ms = [torch.zeros(*s, device=dev) for s in shapes]
    vs = [torch.zeros(*s, device=dev) for s in shapes]
    n = sum(p.numel() for p in ps)
    steps = list(range(1, len(ps) + 1))
    mc.adamw_step(ps, gs, ms, vs, steps)
    torch.cuda.synchronize()
    mc._lib.check(mc._lib.lib().mc_profile_reset())
    mc._lib.check(mc._lib.lib().mc_profile_enable(1))
    queue_ahead(torch)
    for _ in range(iters):
        mc.adamw_step(ps, gs, ms, vs, steps)
    torch.cuda.synchronize()
    mc._lib.check(mc._lib.lib().mc_profile_enable(0))
    mc._lib.check(mc._lib.lib().mc_profile_collect())
    ms_, calls, _, by = mc._lib.profile_read("adamw")
    return {"tensors": len(ps), "elements": n, "iters": iters, "us_per_call": ms_ * 1e3 / calls,
            "GB_s": by / (ms_ * 1e-3) / 1e9, "hbm_frac": by / (ms_ * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "bytes_per_call": by / calls}


QWEN_VOCAB = 151936  # Qwen2.5 vocabulary: the LM head's logits row


def row_ops(mc, c, dev, iters):
    """LayerNorm fwd / bwd at the layer's [tokens, hidden] (with weight and
    bias, as the embeddings' MetalLayerNorm) and the cross-entropy loss fwd /
    bwd over [tokens, vocabulary] logits, each timed per call by the library's
    profiling hook; GB/s from the algorithmic bytes of each call."""
    import torch

    T, D = c["batch"] * c["seq"], c["hidden"]
    g = torch.Generator(device=dev).manual_seed(13)
    x = torch.randn(T, D, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(D, device=dev, generator=g) * 0.1 + 1).to(torch.bfloat16)
    b = (torch.randn(D, device=dev, generator=g) * 0.1).to(torch.bfloat16)
    dy = torch.randn(T, D, device=dev, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, QWEN_VOCAB, device=dev, generator=g).to(torch.bfloat16)
    targets = torch.randint(0, QWEN_VOCAB, (T,), device=dev, generator=g, dtype=torch.int32)
    y, mean, rstd = mc.layer_norm_forward(x, 1e-5, w, b)
    loss, stats = mc.cross_entropy_forward(logits, targets)
    calls = {
        "layernorm_fwd": lambda: mc.layer_norm_forward(x, 1e-5, w, b),
        "layernorm_bwd": lambda: mc.layer_norm_backward(x, dy, 1e-5, w, mean, rstd),
        "cross_entropy_fwd": lambda: mc.cross_entropy_forward(logits, targets),
        "cross_entropy_bwd": lambda: mc.cross_entropy_backward(logits, targets, stats),
    }
    out = {"layernorm_shape": [T, D], "cross_entropy_shape": [T, QWEN_VOCAB], "dtype": "bf16", "iters": iters}
    for name, fn in calls.items():
        fn()
        torch.cuda.synchronize()
        mc._lib.check(mc._lib.lib().mc_profile_reset())
        mc._lib.check(mc._lib.lib().mc_profile_enable(1))
        queue_ahead(torch)
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
        mc._lib.check(mc._lib.lib().mc_profile_enable(0))
        mc._lib.check(mc._lib.lib().mc_profile_collect())
        ms, n, _, by = mc._lib.profile_read("rowops")
        out[name] = {"us_per_call": ms * 1e3 / n, "GB_s": by / (ms * 1e-3) / 1e9,
                     "hbm_frac": by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    del logits
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-tokens", type=int, default=2048, help="token sample of the CPU-oracle baseline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true", help="time HIP graph replays of one captured step")
    ap.add_argument("--attention-iters", type=int, default=5,
                    help="calls of the attention core fwd / bwd timed after the step (0: skip)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="run one plain device copy of BYTES before the steps (a kernel of known HBM traffic "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (every box in this setup has one); --gpus {args.gpus} "
              "is not supported", file=sys.stderr)
        sys.exit(2)

    import torch

    import __graft_entry__

    mc = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    c = CONFIGS[args.config]
    layer = Layer(mc, c, dev)
    if args.copy_calibration > 0:
        src = torch.empty(args.copy_calibration // 2, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    for _ in range(args.warmup):
        layer.step()
    torch.cuda.synchronize()

    if args.graph:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            layer.step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            layer.step()
        torch.cuda.synchronize()
        graph.replay()  # one untimed replay
        run = graph.replay
    else:
        run = layer.step
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # per-kernel event timing of eager steps (the library's profiling hook),
    # after and outside the timed region
    prof_steps = max(1, min(args.steps, 20))
    mc._lib.check(mc._lib.lib().mc_profile_reset())
    mc._lib.check(mc._lib.lib().mc_profile_enable(1))
    for _ in range(prof_steps):
        layer.step()
    torch.cuda.synchronize()
    mc._lib.check(mc._lib.lib().mc_profile_enable(0))
    mc._lib.check(mc._lib.lib().mc_profile_collect())

    ms_step = elapsed * 1e3 / args.steps
    tokens_s = layer.T / (elapsed / args.steps)
    kernels = {}
    for kind in ("gemm", "lowrank", "rmsnorm", "softmax"):
        ms, n, fl, by = mc._lib.profile_read(kind)
        if n == 0:
            continue
        kernels[kind] = {
            "launches_per_step": n / prof_steps,
            "ms_per_step": ms / prof_steps,
            "avg_launch_us": ms * 1e3 / n,
            "TFLOP_s": fl / (ms * 1e-3) / 1e12 if fl else None,
            "GB_s": by / (ms * 1e-3) / 1e9,
            "hbm_frac": by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        }

    gemm_ms, gemm_n, gemm_fl, _ = mc._lib.profile_read("gemm")
    achieved = gemm_fl / gemm_n / (gemm_ms / gemm_n * 1e-3) / 1e12
    base_fl, low_fl = layer.flops_per_step()
    line = {
        "metric": "LoRA fwd+bwd tokens/s + MFMA util @1.5B shapes; RMSNorm/softmax HBM GB/s",
        "value": tokens_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": c["dtype"],
        "data": "synthetic (seeded normal / kaiming-uniform, resident in HBM)",
        "config": {"workload": c["workload"], "config": args.config, "tokens": layer.T, "rank": c["rank"],
                   "alpha": c["alpha"], "dropout": c["dropout"]},
        "roofline": {
            "kernel": "gemm_bf16_kernel / gemm_bf16_split (base GEMMs x.W^T and dY.W with the rank-r columns folded in)",
            "bound": "mfma",
            "achieved": achieved,
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / BF16_PEAK_TFLOPS,
            "traffic": GEMM_TRAFFIC_BYTES.get(args.config),
        },
        "layer_TFLOP_s": (base_fl + low_fl) / (ms_step * 1e-3) / 1e12,
        "launch": "hip_graph" if args.graph else "eager",
        "kernels": kernels,
    }
    if args.attention_iters > 0 and c["softmax"]:
        line["attention"] = attention_core(mc, c, dev, args.attention_iters)
    if args.attention_iters > 0:
        line["adamw"] = adamw_update(mc, c, dev, 20)
        line["row_ops"] = row_ops(mc, c, dev, args.attention_iters)
    if not args.no_cpu_baseline:
        threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
        v, dt = cpu_baseline(c, args.cpu_tokens, threads)
        line["cpu_baseline"] = {
            "value": v, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{args.cpu_tokens} tokens of the same layer (LoRA fwd+bwd x{len(c['projections'])}, "
                      f"RMSNorm fwd+bwd x2, softmax rows of those tokens) through the C oracle, {dt:.1f} s",
        }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
