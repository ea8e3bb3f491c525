"""The entry points under HIP graph capture: a LoRA fwd + bwd, RMSNorm fwd + bwd
and causal softmax fwd + bwd sequence captured once (torch.cuda.CUDAGraph on
the current stream) and replayed several times, with eager calls of the same
ops in between, must give bitwise the eager results on every replay. The
entry points allocate nothing, never synchronise and record no memset, so
they can be captured; the kernels are deterministic, so replays are
bit-identical."""
import pytest
import torch

from inputs import lora_case

pytestmark = pytest.mark.gpu


def _sequence(mc, dev, t):
    y, h = mc.lora_forward(t["x"], t["A"], t["B"], 2.0, W=t["W"], bias=t["bias"])
    dX, dA, dB = mc.lora_backward(t["x"], t["A"], t["B"], t["dy"], 2.0, W=t["W"], h_save=h)
    yn, rstd = mc.rms_norm_forward(t["xn"], 1e-6, t["wn"])
    dxn, dwn = mc.rms_norm_backward(t["xn"], t["dyn"], 1e-6, t["wn"], rstd)
    p = mc.softmax_forward(t["s"], causal_rows=t["s"].shape[-2])
    ds = mc.softmax_backward(p, t["dp"], causal_rows=t["s"].shape[-2])
    return [y, h, dX, dA, dB, yn, rstd, dxn, dwn, p, ds]


def test_graph_replay_matches_eager(mc, dev):
    c = lora_case(99, 1024, 512, 768, 16, bias=True)
    g = torch.Generator().manual_seed(5)
    t = {k: c[k].to(dev) for k in ("x", "W", "bias", "A", "B", "dy")}
    t["xn"] = torch.randn(512, 1536, generator=g).to(torch.bfloat16).to(dev)
    t["wn"] = (torch.randn(1536, generator=g) * 0.1 + 1).to(torch.bfloat16).to(dev)
    t["dyn"] = (torch.randn(512, 1536, generator=g) * 1e-2).to(torch.bfloat16).to(dev)
    t["s"] = (torch.randn(2, 4, 256, 256, generator=g) * 3).to(torch.bfloat16).to(dev)
    t["dp"] = (torch.randn(2, 4, 256, 256, generator=g) * 1e-2).to(torch.bfloat16).to(dev)

    eager = [o.clone() for o in _sequence(mc, dev, t)]
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _sequence(mc, dev, t)  # warm the allocator on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _sequence(mc, dev, t)
    torch.cuda.synchronize()

    for rep in range(3):
        between = _sequence(mc, dev, t)  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a, b), f"replay {rep}: output {i} differs from eager"
        for i, (a, b) in enumerate(zip(between, eager)):
            assert torch.equal(a, b), f"eager call between replays: output {i} differs"
