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
Qwen2.5-sized vocabulary of 151936), also outside the step. "c2_row_ops_f32"
and "c1_lora_f32" time BASELINE.json's two fp32 configs (RMSNorm / causal
softmax at c2's shapes; c1's single LoRA linear fwd and bwd against the fp32
peak).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# HBM bytes per base-GEMM launch (average over a step's launches), measured
# with two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE) scaled by the
# same counters on a 256 MiB copy (--copy-calibration). The committed summary
# profiles/gemm_bf16_<config>_hbm_traffic.md holds the figure on a line
# "traffic_bytes_per_launch: <bytes> (source: <commit or build>)", re-measured
# whenever the GEMM changes; read_gemm_traffic() takes it from there.
def read_gemm_traffic(config):
    path = os.path.join(ROOT, "profiles", f"gemm_bf16_{config}_hbm_traffic.md")
    try:
        with open(path) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_launch:"):
                    rest = ln.split(":", 1)[1].strip()
                    value = float(rest.split()[0])
                    src = rest[rest.find("(") + 1:rest.rfind(")")] if "(" in rest else ""
                    return value, f"profiles/gemm_bf16_{config}_hbm_traffic.md ({src})"
    except (OSError, ValueError):
        pass
    return None, None

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

    def __init__(self, mc, c, dev, seed=0, group=True, cached_wt=True):
        import torch

        self.mc, self.c, self.dev = mc, c, dev
        self.group = group and c["dtype"] == "bf16"
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
        if self.group and cached_wt:
            # W is frozen: its transpose for the backward's dX product is a
            # load-time layout, built once here (mc_transpose_bf16), not per step
            for pr in self.proj.values():
                pr["Wt"] = mc.transpose_weight(pr["W"])
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
        """One forward + backward of the layer's custom ops. The projections
        that read the same input (q / k / v, gate / up) run as one grouped
        call each (mc_lora_group_fwd / _bwd: one pass over the input per
        rank-r pass, one GEMM launch, dX summed over the group), o and down as
        groups of one, each with its load-time W^T, unless the layer was built
        with group=False (per-projection mc_lora_fwd / _bwd, which transpose W
        in every backward)."""
        mc, c = self.mc, self.c
        saved = {}
        if c["norm"]:
            self.xn1, r1 = mc.rms_norm_forward(self.h_in, 1e-6, self.ln1)
        attn_in = [p for p in ("q", "k", "v") if p in self.proj]
        mlp_in = [p for p in ("gate", "up") if p in self.proj]
        self._fwd(attn_in, saved)
        P = mc.softmax_forward(self.scores, causal_rows=c["seq"]) if c["softmax"] else None
        self._fwd([p for p in ("o",) if p in self.proj], saved)
        if c["norm"]:
            self.xn2, r2 = mc.rms_norm_forward(self.h_mid, 1e-6, self.ln2)
        self._fwd(mlp_in, saved)
        self._fwd([p for p in ("down",) if p in self.proj], saved)
        # backward
        self._bwd([p for p in ("down",) if p in self.proj], saved)
        self._bwd(mlp_in, saved)
        if c["norm"]:
            mc.rms_norm_backward(self.h_mid, self.dy_ln, 1e-6, self.ln2, r2)
        self._bwd([p for p in ("o",) if p in self.proj], saved)
        if c["softmax"]:
            mc.softmax_backward(P, self.dP, causal_rows=c["seq"])
        self._bwd(attn_in, saved)
        if c["norm"]:
            mc.rms_norm_backward(self.h_in, self.dy_ln, 1e-6, self.ln1, r1)

    def _fwd(self, names, saved):
        if not names:
            return
        if not self.group:
            for name in names:
                saved[name] = self._lora_f(name)
            return
        _, hs = self.mc.lora_group_forward(self._input_of(names[0]), [self.proj[n] for n in names], self.scale,
                                           dropout_p=self.p)
        for name, h in zip(names, hs):
            saved[name] = h

    def _bwd(self, names, saved):
        if not names:
            return
        if not self.group:
            for name in names:
                self._lora_b(name, saved[name])
            return
        self.mc.lora_group_backward(self._input_of(names[0]), [self.proj[n] for n in names],
                                    [self.proj[n]["dy"] for n in names], self.scale, dropout_p=self.p,
                                    h_saves=[saved[n] for n in names])

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


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(mc, c, tokens, threads, iters):
    """The reference's CPU path for the same layer on a token sample, restated
    with torch CPU fp32 ops in the candle composite's op order:
      LoRA  H = x.A, Hd = dropout(H), y = x.W^T + b + (Hd.B).s
            (src/training/lora.rs:320-339; candle_nn::Linear), and its
            autograd: G = s dY.B^T (.) M/(1-p), dX = dY.W + G.A^T,
            dA = x^T.G, dB = s Hd^T.dY (W frozen)
      RMSNorm x / sqrt(mean(x^2) + eps) * w (src/backend/tensor.rs:111-117,
            src/models/qwen.rs:314-325) and its closed-form gradient
      softmax max, sub, exp, sum, div over the masked scores
            (src/backend/tensor.rs:91-98, src/models/transformer.rs:264-275)
            for the sampled tokens' rows, and dS = P (.) (dP - sum dP P).
    The GEMMs run in torch's CPU BLAS (MKL / oneDNN), the elementwise ops
    vectorised, on `threads` threads. Inputs are bf16-rounded values held in
    fp32, as the GPU path sees them. Two warmup passes, then the median of
    `iters` timed passes. Returns (tokens / second, median seconds)."""
    import statistics

    import torch

    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    T, S, H = tokens, c["seq"], c["hidden"]
    rb = lambda *shape, std=1.0: (torch.randn(*shape, generator=g) * std).bfloat16().float()  # noqa: E731
    s, p = c["alpha"] / c["rank"], c["dropout"]
    work = []
    for i, (name, (K, N, bias)) in enumerate(proj_shapes(c).items()):
        b = 1.0 / K ** 0.5
        # the same host-generated keep-masks as the GPU step (seed 1234 + index)
        mask = mc.dropout_mask(1234 + i, p, T, c["rank"]).float() / (1.0 - p) if p > 0 else None
        work.append(dict(x=rb(T, K), W=rb(N, K, std=0.02), bias=rb(N, std=0.02) if bias else None,
                         A=(torch.rand(K, c["rank"], generator=g) * 2 - 1) * b, B=rb(c["rank"], N, std=0.02),
                         dy=rb(T, N, std=1e-2), mask=mask))
    xs, dys, w = rb(T, H), rb(T, H, std=1e-2), rb(H, std=0.1) + 1.0
    srows = T * c["heads"] if c["softmax"] else 0
    if srows:
        scores, dP = rb(c["heads"], T, S, std=3.0), rb(c["heads"], T, S, std=1e-2)
        q = torch.arange(T)[:, None] % S
        neg = torch.zeros(T, S).masked_fill(torch.arange(S)[None, :] > q, float("-inf"))

    def one_pass():
        for wk in work:
            x, W, A, B, dy, m = wk["x"], wk["W"], wk["A"], wk["B"], wk["dy"], wk["mask"]
            hd = x @ A
            if m is not None:
                hd = hd * m
            y = torch.addmm(wk["bias"], x, W.t()) if wk["bias"] is not None else x @ W.t()
            y += (hd @ B) * s
            gd = (dy @ B.t()) * s
            if m is not None:
                gd = gd * m
            dx = dy @ W + gd @ A.t()
            dA = x.t() @ gd
            dB = (hd.t() @ dy) * s
            del y, dx, dA, dB
        if c["norm"]:
            for _ in range(2):
                r = torch.rsqrt((xs * xs).mean(-1, keepdim=True) + 1e-6)
                y = xs * r * w
                gw = dys * w
                dx = r * gw - xs * (r ** 3) * (gw * xs).mean(-1, keepdim=True)
                dw = (dys * xs * r).sum(0)
                del y, dx, dw
        if srows:
            z = scores + neg
            z = z - z.amax(-1, keepdim=True)
            e = z.exp()
            P = e / e.sum(-1, keepdim=True)
            dS = P * (dP - (dP * P).sum(-1, keepdim=True))
            del P, dS

    for _ in range(2):
        one_pass()
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return T / med, med


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


def c2_row_ops(mc, dev, iters):
    """BASELINE config c2 (fp32): RMSNorm over [8192, 896] (weight ~N(1, 0.1),
    eps 1e-6) and the causal softmax over [8, 14, 1024, 1024] scores ~N(0, 3),
    fwd and bwd, each timed per call by the library's profiling hook. GB/s
    counts the algorithmic bytes (RMSNorm fwd: read x, write y, rstd; bwd:
    read x, dy, write dx; softmax: the unmasked part read, every row written;
    bwd reads P and dP over the unmasked part)."""
    import torch

    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn(8192, 896, device=dev, generator=g)
    w = torch.randn(896, device=dev, generator=g) * 0.1 + 1.0
    dy = torch.randn(8192, 896, device=dev, generator=g)
    sc = torch.randn(8, 14, 1024, 1024, device=dev, generator=g) * 3.0
    dP = torch.randn(8, 14, 1024, 1024, device=dev, generator=g) * 1e-2
    _, rstd = mc.rms_norm_forward(x, 1e-6, w)
    P = mc.softmax_forward(sc, causal_rows=1024)
    calls = {
        "rmsnorm_fwd": ("rmsnorm", lambda: mc.rms_norm_forward(x, 1e-6, w)),
        "rmsnorm_bwd": ("rmsnorm", lambda: mc.rms_norm_backward(x, dy, 1e-6, w, rstd)),
        "softmax_fwd": ("softmax", lambda: mc.softmax_forward(sc, causal_rows=1024)),
        "softmax_bwd": ("softmax", lambda: mc.softmax_backward(P, dP, causal_rows=1024)),
    }
    out = {"rmsnorm_shape": [8192, 896], "softmax_shape": [8, 14, 1024, 1024], "dtype": "f32", "iters": iters}
    for name, (kind, fn) in calls.items():
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
        ms, n, _, by = mc._lib.profile_read(kind)
        out[name] = {"us_per_call": ms * 1e3 / n, "GB_s": by / (ms * 1e-3) / 1e9,
                     "hbm_frac": by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    del sc, dP, P
    return out


def c1_lora_f32(mc, dev, iters):
    """BASELINE config c1 (fp32, the reference's own fused-kernel dtype): one
    LoRA linear, x [4, 128, 768] ~N(0, 1), frozen W [768, 768] ~N(0, 0.02),
    A [768, 8] kaiming-uniform, B [8, 768] ~N(0, 0.02), rank 8, alpha 16, no
    dropout; forward y and backward (dX, dA, dB) with dY ~N(0, 1e-2). Each
    call is timed whole (every launch of it) with events on the stream,
    median of `iters` timed repetitions of 20 calls queued behind a GPU spin. FLOPs count the
    algorithmic products: forward 2TKN + 2TKr + 2TrN, backward 2TNK + 2TrK (dX),
    2TNr (G), 2TKr (dA), 2TrN (dB); the roofline is the fp32 peak (vector
    and matrix fp32 are both 157.3 TFLOP/s on MI355X)."""
    import statistics
    import torch

    T, K, N, r, s = 4 * 128, 768, 768, 8, 2.0
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(T, K, device=dev, generator=g)
    W = torch.randn(N, K, device=dev, generator=g) * 0.02
    bound = 1.0 / K ** 0.5
    A = (torch.rand(K, r, device=dev, generator=g) * 2 - 1) * bound
    B = torch.randn(r, N, device=dev, generator=g) * 0.02
    dy = torch.randn(T, N, device=dev, generator=g) * 1e-2
    fwd = lambda: mc.lora_forward(x, A, B, s, W=W)  # noqa: E731
    _, h = fwd()
    bwd = lambda: mc.lora_backward(x, A, B, dy, s, W=W, h_save=h)  # noqa: E731
    flops = {"fwd": 2.0 * T * K * N + 2.0 * T * K * r + 2.0 * T * r * N,
             "bwd": 2.0 * T * N * K + 2.0 * T * r * K + 2.0 * T * N * r + 2.0 * T * K * r + 2.0 * T * r * N}
    out = {"shape": {"tokens": T, "in": K, "out": N, "rank": r}, "dtype": "f32", "iters": iters,
           "gflop_fwd_bwd": (flops["fwd"] + flops["bwd"]) / 1e9}
    for name, fn in (("fwd", fwd), ("bwd", bwd)):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        times = []
        for _ in range(iters):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            queue_ahead(torch)  # the 20 calls run back to back after the spin, not at the host's launch rate
            e0.record()
            for _ in range(20):
                fn()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / 20 * 1e3)
        us = statistics.median(times)
        tf = flops[name] / (us * 1e-6) / 1e12
        out[name] = {"us_per_call": us, "TFLOP_s": tf, "fp32_frac": tf / FP32_PEAK_TFLOPS}
    out["fwd_bwd_us"] = out["fwd"]["us_per_call"] + out["bwd"]["us_per_call"]
    out["tokens_per_s"] = T / (out["fwd_bwd_us"] * 1e-6)
    return out


# Row widths past the one-wave RMSNorm / softmax / LayerNorm paths: (op,
# dtype, rows, dim, causal_rows). c5's 3584 and 5120 (14B/32B hidden) take the
# workgroup-per-row backward; 8192-16384 the wide kernels; 131072 the
# streaming softmax.
ROW_SWEEP = [
    ("rmsnorm", "bf16", 16384, 3584, 0), ("rmsnorm", "bf16", 16384, 5120, 0), ("rmsnorm", "bf16", 16384, 8192, 0),
    ("rmsnorm", "f32", 16384, 8192, 0), ("rmsnorm", "bf16", 8192, 16384, 0),
    ("softmax", "bf16", 8192, 6144, 0), ("softmax", "bf16", 8192, 8192, 0), ("softmax", "f32", 8192, 4096, 0),
    ("softmax", "bf16", 4096, 16384, 0), ("softmax", "bf16", 16384, 16384, 16384), ("softmax", "bf16", 1024, 131072, 0),
    ("layernorm", "bf16", 16384, 5120, 0), ("layernorm", "bf16", 16384, 8192, 0), ("layernorm", "f32", 8192, 8192, 0),
]


def row_sweep(mc, dev, iters):
    """RMSNorm and softmax fwd / bwd over the row widths of ROW_SWEEP, each
    call after a 1 GiB read-only pass (so its input comes from HBM, with no
    dirty lines left to write back), timed with events on the launch stream;
    the median of ITERS calls. GB/s counts the algorithmic bytes (RMSNorm fwd:
    x in, y and rstd out; bwd: x, dy in, dx out, w and dw amortised; LayerNorm
    likewise with mean and rstd; softmax: the unmasked part read, every row
    written, P and dP read by the bwd)."""
    import torch

    flush = torch.empty(1 << 28, device=dev)
    g = torch.Generator(device=dev).manual_seed(5)

    def timed(fn):
        ts = []
        for _ in range(iters):
            flush.sum()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b) * 1e3)
        return sorted(ts)[len(ts) // 2]

    out = []
    for op, dt, rows, dim, causal in ROW_SWEEP:
        tdt = torch.bfloat16 if dt == "bf16" else torch.float32
        es = 2 if dt == "bf16" else 4
        x = torch.randn(rows, dim, device=dev, generator=g).to(tdt)
        if op == "layernorm":
            x2 = torch.randn(rows, dim, device=dev, generator=g).to(tdt)
            w = (torch.randn(dim, device=dev, generator=g) * 0.1 + 1).to(tdt)
            bb = (torch.randn(dim, device=dev, generator=g) * 0.1).to(tdt)
            _, mu, r = mc.layer_norm_forward(x, 1e-5, w, bb)
            us_f = timed(lambda: mc.layer_norm_forward(x, 1e-5, w, bb))
            us_b = timed(lambda: mc.layer_norm_backward(x, x2, 1e-5, w, mu, r))
            by_f, by_b = rows * (2 * dim * es + 8), rows * (3 * dim * es + 8)
        elif op == "rmsnorm":
            x2 = torch.randn(rows, dim, device=dev, generator=g).to(tdt)
            w = (torch.randn(dim, device=dev, generator=g) * 0.1 + 1).to(tdt)
            _, r = mc.rms_norm_forward(x, 1e-6, w)
            us_f = timed(lambda: mc.rms_norm_forward(x, 1e-6, w))
            us_b = timed(lambda: mc.rms_norm_backward(x, x2, 1e-6, w, r))
            by_f, by_b = rows * (2 * dim * es + 4), rows * (3 * dim * es + 4)
        else:
            x = x * 3
            x2 = (torch.randn(rows, dim, device=dev, generator=g) * 1e-2).to(tdt)
            p = mc.softmax_forward(x, causal_rows=causal)
            un = rows * dim if not causal else (rows // causal) * sum(r + dim - causal + 1 for r in range(causal))
            us_f = timed(lambda: mc.softmax_forward(x, causal_rows=causal))
            us_b = timed(lambda: mc.softmax_backward(p, x2, causal_rows=causal))
            by_f, by_b = es * (un + rows * dim), es * (2 * un + rows * dim)
            del p
        out.append({"op": op, "dtype": dt, "shape": [rows, dim], "causal_rows": causal,
                    "fwd_us": us_f, "fwd_GB_s": by_f / us_f / 1e3, "bwd_us": us_b, "bwd_GB_s": by_b / us_b / 1e3})
        del x, x2
    del flush
    return {"iters": iters, "method": "median of per-call events, each call after a 1 GiB read-only pass",
            "rows": out}


def blas_reference(c, dev, iters):
    """The vendor library on the layer's forward GEMM shapes: torch.matmul
    (hipBLASLt on ROCm) of x [T, K] bf16 by W^T for each projection's
    [N, K] W, warm back-to-back calls, as a reference point for the base
    GEMM's MFMA fraction (no LoRA columns, no bias)."""
    import torch

    T = c["batch"] * c["seq"]
    out = {"library": "hipBLASLt via torch.matmul (x @ W.t(), bf16)", "iters": iters, "shapes": []}
    seen = set()
    for name, (K, N, _) in proj_shapes(c).items():
        if (K, N) in seen:
            continue
        seen.add((K, N))
        x = torch.randn(T, K, device=dev).to(torch.bfloat16)
        w = torch.randn(N, K, device=dev).to(torch.bfloat16)
        for _ in range(3):
            torch.matmul(x, w.t())
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            torch.matmul(x, w.t())
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / iters
        tf = 2.0 * T * N * K / (us * 1e-6) / 1e12
        out["shapes"].append({"projection": name, "M": T, "N": N, "K": K, "us": us, "TFLOP_s": tf,
                              "frac": tf / BF16_PEAK_TFLOPS})
        del x, w
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-tokens", type=int, default=2048, help="token sample of the CPU baseline")
    ap.add_argument("--cpu-iters", type=int, default=10, help="timed passes of the CPU baseline (median)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true", help="time HIP graph replays of one captured step")
    ap.add_argument("--no-group", action="store_true",
                    help="run q/k/v and gate/up as separate per-projection calls instead of grouped calls")
    ap.add_argument("--no-cached-wt", action="store_true",
                    help="grouped calls without the load-time W^T: every backward transposes W into its workspace")
    ap.add_argument("--attention-iters", type=int, default=5,
                    help="calls of the attention core fwd / bwd timed after the step (0: skip)")
    ap.add_argument("--blas-reference", type=int, default=0, metavar="ITERS",
                    help="also time the vendor library (hipBLASLt via torch.matmul) on the layer's forward GEMM "
                         "shapes, ITERS calls each")
    ap.add_argument("--row-sweep", type=int, default=0, metavar="ITERS",
                    help="also time RMSNorm, softmax and LayerNorm fwd / bwd over row widths past the one-wave paths "
                         "(ROW_SWEEP), ITERS calls each from cold caches")
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
    layer = Layer(mc, c, dev, group=not args.no_group, cached_wt=not args.no_cached_wt)
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
            "traffic": read_gemm_traffic(args.config)[0],
            "traffic_source": read_gemm_traffic(args.config)[1],
        },
        "layer_TFLOP_s": (base_fl + low_fl) / (ms_step * 1e-3) / 1e12,
        "launch": "hip_graph" if args.graph else "eager",
        "projections": "per-projection calls" if args.no_group else "grouped calls for q/k/v and gate/up",
        "weights": ("W^T transposed in every backward" if args.no_group or args.no_cached_wt
                    else "frozen W with its W^T built once at load (mc_transpose_bf16)"),
        "kernels": kernels,
    }
    if args.attention_iters > 0 and c["softmax"]:
        line["attention"] = attention_core(mc, c, dev, args.attention_iters)
    if args.attention_iters > 0:
        line["adamw"] = adamw_update(mc, c, dev, 20)
        line["row_ops"] = row_ops(mc, c, dev, args.attention_iters)
    line["c2_row_ops_f32"] = c2_row_ops(mc, dev, 5)
    line["c1_lora_f32"] = c1_lora_f32(mc, dev, 5)
    if args.blas_reference > 0:
        line["blas_reference"] = blas_reference(c, dev, args.blas_reference)
    if args.row_sweep > 0:
        line["row_sweep"] = row_sweep(mc, dev, args.row_sweep)
    if not args.no_cpu_baseline:
        threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
        v, dt = cpu_baseline(mc, c, args.cpu_tokens, threads, args.cpu_iters)
        line["cpu_baseline"] = {
            "value": v, "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu": cpu_model(),
            "sample": f"{args.cpu_tokens} tokens of the same layer (LoRA fwd+bwd x{len(c['projections'])}, "
                      f"RMSNorm fwd+bwd x2, causal softmax fwd+bwd of those tokens' score rows), torch CPU fp32 "
                      f"composite in the reference's op order (BLAS GEMMs), median of {args.cpu_iters} passes "
                      f"after 2 warmup passes: {dt * 1e3:.1f} ms per pass",
        }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
