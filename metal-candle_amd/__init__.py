"""metal-candle's fused LoRA / RMSNorm / softmax custom ops and the attention
core on MI355X (gfx950).

The arithmetic lives in libmc_hip.so (HIP kernels behind the C ABI of
include/mc_hip.h); this package is the Python host side over that ABI.
The directory name is not an identifier: load it with
__graft_entry__.load_package(), which registers it as `metal_candle_amd`.
"""
from . import _lib, ops  # noqa: F401
from ._lib import McError  # noqa: F401
from .ops import (  # noqa: F401
    adamw_step,
    attention_backward,
    attention_forward,
    cross_entropy_backward,
    cross_entropy_forward,
    dropout_mask,
    layer_norm_backward,
    layer_norm_forward,
    log_softmax_backward,
    log_softmax_forward,
    lora_backward,
    lora_forward,
    lora_group_backward,
    lora_group_forward,
    rms_norm_backward,
    rms_norm_forward,
    softmax_backward,
    softmax_forward,
    transpose_weight,
)
