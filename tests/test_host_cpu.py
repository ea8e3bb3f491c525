"""C++ host interface (metal-candle_amd/host/mc_candle.hpp): the cases that
need no GPU — LoRAConfig / LoRALayer validation, FusedLoRAOp::new checks, op
names, the CPU-forward errors, AsyncExecutor input-count errors, Operation
shapes, the dropout-mask generator and AdamWConfig / AdamW state handling —
with the reference's messages."""
import host_runner


def test_host_interface_cpu_cases():
    out = host_runner.run("--cpu", timeout=120)
    assert "0 failed" in out
