"""C++ host interface on the GPU: the reference's op / layer / executor tests
(custom_ops_correctness, rmsnorm_correctness, softmax_correctness,
executor_direct, lora_dropout, gradient_verification, lora_lazy /
rmsnorm_lazy / softmax_lazy through the lazy graph, and the AdamW tests of
src/training/optimizer.rs) run through
libmc_candle.so -> libmc_hip.so and are checked against the CPU oracle."""
import pytest

import host_runner


@pytest.mark.gpu
def test_host_interface_all_cases():
    out = host_runner.run("--gpu", timeout=110)
    assert "0 failed" in out
