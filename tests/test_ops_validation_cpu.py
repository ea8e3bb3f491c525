"""The torch front end (metal-candle_amd/ops.py) rejects wrongly shaped,
typed or placed tensors before the C ABI is called, so no kernel is ever
handed a buffer smaller than its shape arguments imply. CPU tensors suffice:
every error here is raised before anything touches a device. Messages follow
FusedLoRAOp::new / compute_output_shape (src/backend/custom_ops.rs:118-174)
where the reference has one."""
import pytest
import torch


def _lora(T=16, K=32, N=24, r=4, dtype=torch.bfloat16):
    return dict(x=torch.zeros(T, K, dtype=dtype), W=torch.zeros(N, K, dtype=dtype),
                bias=torch.zeros(N, dtype=dtype), A=torch.zeros(K, r), B=torch.zeros(r, N),
                dy=torch.zeros(T, N, dtype=dtype), mask=torch.ones(T, r, dtype=torch.uint8),
                h=torch.zeros(r, T))


def _raises(mc, code, text, fn, *a, **k):
    with pytest.raises(mc.McError) as e:
        fn(*a, **k)
    assert e.value.code == code, e.value
    assert text in str(e.value), e.value


def test_lora_forward_shape_errors(mc):
    L, c = mc._lib, _lora()
    f = mc.lora_forward
    _raises(mc, L.MC_ERR_SHAPE, "LoRA matrices must be 2D", f, c["x"], c["A"].reshape(-1), c["B"], 2.0)
    _raises(mc, L.MC_ERR_SHAPE, "Incompatible LoRA matrix dimensions: 32×4 and 5×24", f, c["x"], c["A"],
            torch.zeros(5, 24), 2.0)
    _raises(mc, L.MC_ERR_SHAPE, "Input feature dimension mismatch: expected 32, got 31", f,
            torch.zeros(16, 31, dtype=torch.bfloat16), c["A"], c["B"], 2.0)
    _raises(mc, L.MC_ERR_SHAPE, "W has shape (24, 16)", f, c["x"], c["A"], c["B"], 2.0,
            W=torch.zeros(24, 16, dtype=torch.bfloat16))
    _raises(mc, L.MC_ERR_SHAPE, "bias has shape (23,)", f, c["x"], c["A"], c["B"], 2.0, W=c["W"],
            bias=torch.zeros(23, dtype=torch.bfloat16))
    _raises(mc, L.MC_ERR_SHAPE, "mask has shape (16, 3)", f, c["x"], c["A"], c["B"], 2.0,
            mask=torch.ones(16, 3, dtype=torch.uint8), dropout_p=0.1)


def test_lora_forward_dtype_layout_errors(mc):
    L, c = mc._lib, _lora()
    f = mc.lora_forward
    _raises(mc, L.MC_ERR_DTYPE, "A has dtype torch.bfloat16", f, c["x"], c["A"].bfloat16(), c["B"], 2.0)
    _raises(mc, L.MC_ERR_DTYPE, "W has dtype torch.float32", f, c["x"], c["A"], c["B"], 2.0, W=c["W"].float())
    _raises(mc, L.MC_ERR_DTYPE, "mask has dtype torch.bool", f, c["x"], c["A"], c["B"], 2.0,
            mask=c["mask"].bool(), dropout_p=0.1)
    _raises(mc, L.MC_ERR_DTYPE, "unsupported dtype torch.float16", f, c["x"].half(), c["A"], c["B"], 2.0)
    _raises(mc, L.MC_ERR_LAYOUT, "x must be contiguous", f, torch.zeros(32, 16, dtype=torch.bfloat16).t(),
            torch.zeros(16, 4), c["B"], 2.0)
    _raises(mc, L.MC_ERR_LAYOUT, "W must be contiguous", f, c["x"], c["A"], c["B"], 2.0,
            W=torch.zeros(32, 24, dtype=torch.bfloat16).t())


def test_lora_backward_shape_errors(mc):
    L, c = mc._lib, _lora()
    b = mc.lora_backward
    _raises(mc, L.MC_ERR_SHAPE, "dY feature dimension mismatch: expected 24, got 23", b, c["x"], c["A"], c["B"],
            torch.zeros(16, 23, dtype=torch.bfloat16), 2.0)
    _raises(mc, L.MC_ERR_SHAPE, "x has shape (15, 32)", b, torch.zeros(15, 32, dtype=torch.bfloat16), c["A"],
            c["B"], c["dy"], 2.0, h_save=c["h"])
    _raises(mc, L.MC_ERR_SHAPE, "h_save has shape (4, 15)", b, c["x"], c["A"], c["B"], c["dy"], 2.0,
            h_save=torch.zeros(4, 15))
    _raises(mc, L.MC_ERR_DTYPE, "h_save has dtype torch.bfloat16", b, c["x"], c["A"], c["B"], c["dy"], 2.0,
            h_save=c["h"].bfloat16())
    _raises(mc, L.MC_ERR_DTYPE, "x has dtype torch.float32", b, c["x"].float(), c["A"], c["B"], c["dy"], 2.0,
            h_save=c["h"])
    _raises(mc, L.MC_ERR_SHAPE, "mask has shape (16, 5)", b, c["x"], c["A"], c["B"], c["dy"], 2.0,
            mask=torch.ones(16, 5, dtype=torch.uint8), dropout_p=0.1, h_save=c["h"])
    _raises(mc, L.MC_ERR_LAYOUT, "dY must be contiguous", b, c["x"], c["A"], c["B"],
            torch.zeros(24, 16, dtype=torch.bfloat16).t(), 2.0)


def test_row_op_errors(mc):
    L = mc._lib
    x = torch.zeros(8, 64, dtype=torch.bfloat16)
    _raises(mc, L.MC_ERR_LAYOUT, "x must be contiguous", mc.rms_norm_forward, torch.zeros(64, 8).t(), 1e-6)
    _raises(mc, L.MC_ERR_SHAPE, "w has shape (63,)", mc.rms_norm_forward, x, 1e-6,
            torch.zeros(63, dtype=torch.bfloat16))
    _raises(mc, L.MC_ERR_DTYPE, "w has dtype torch.float32", mc.rms_norm_forward, x, 1e-6, torch.zeros(64))
    _raises(mc, L.MC_ERR_SHAPE, "dy has shape (8, 32)", mc.rms_norm_backward, x,
            torch.zeros(8, 32, dtype=torch.bfloat16), 1e-6)
    _raises(mc, L.MC_ERR_SHAPE, "rstd has shape (7,)", mc.rms_norm_backward, x, x, 1e-6, None, torch.zeros(7))
    _raises(mc, L.MC_ERR_LAYOUT, "s must be contiguous", mc.softmax_forward, torch.zeros(64, 8).t())
    _raises(mc, L.MC_ERR_DTYPE, "dp has dtype torch.float32", mc.softmax_backward, x, torch.zeros(8, 64))
    _raises(mc, L.MC_ERR_SHAPE, "Input must have at least 1 dimension", mc.softmax_forward, torch.tensor(1.0))


def test_attention_and_loss_errors(mc):
    L = mc._lib
    q = torch.zeros(1, 4, 16, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 16, 64, dtype=torch.bfloat16)
    _raises(mc, L.MC_ERR_SHAPE, "v has shape (1, 2, 15, 64)", mc.attention_forward, q, k,
            torch.zeros(1, 2, 15, 64, dtype=torch.bfloat16))
    _raises(mc, L.MC_ERR_SHAPE, "k has shape (1, 2, 16, 32)", mc.attention_forward, q,
            torch.zeros(1, 2, 16, 32, dtype=torch.bfloat16), k)
    _raises(mc, L.MC_ERR_DTYPE, "k has dtype torch.float32", mc.attention_forward, q, k.float(), k)
    _raises(mc, L.MC_ERR_SHAPE, "mask has shape (16, 15)", mc.attention_forward, q, k, k, mask=torch.zeros(16, 15))
    _raises(mc, L.MC_ERR_SHAPE, "lse has shape (1, 4, 15)", mc.attention_backward, q, k, k,
            torch.zeros(1, 16, 256, dtype=torch.bfloat16), torch.zeros(1, 4, 15),
            torch.zeros(1, 16, 256, dtype=torch.bfloat16))
    logits = torch.zeros(6, 32, dtype=torch.bfloat16)
    _raises(mc, L.MC_ERR_DTYPE, "targets have dtype torch.float32", mc.cross_entropy_forward, logits,
            torch.zeros(6))
    _raises(mc, L.MC_ERR_SHAPE, "targets have 5 entries, expected 6", mc.cross_entropy_forward, logits,
            torch.zeros(5, dtype=torch.int32))
    _raises(mc, L.MC_ERR_SHAPE, "stats has shape (6,)", mc.cross_entropy_backward, logits,
            torch.zeros(6, dtype=torch.int32), torch.zeros(6))
    _raises(mc, L.MC_ERR_SHAPE, "w has shape (31,)", mc.layer_norm_forward, logits, 1e-5,
            torch.zeros(31, dtype=torch.bfloat16))
    _raises(mc, L.MC_ERR_SHAPE, "dy has shape (6, 31)", mc.log_softmax_backward, logits,
            torch.zeros(6, 31, dtype=torch.bfloat16))


def test_group_backward_without_x(mc):
    """lora_group_backward takes x = None when dA is not requested, as
    lora_backward and mc_lora_group_bwd do: the leading dims come from dY,
    K from A. Asking for dA without x is a null-argument error."""
    L, c = mc._lib, _lora()
    proj = dict(W=c["W"], bias=None, A=c["A"], B=c["B"])
    gb = mc.lora_group_backward
    _raises(mc, L.MC_ERR_NULL, "dA requires x", gb, None, [proj], [c["dy"]], 2.0)
    _raises(mc, L.MC_ERR_SHAPE, "dY[1] has shape (15, 24)", gb, None, [proj, proj],
            [c["dy"], torch.zeros(15, 24, dtype=torch.bfloat16)], 2.0, need_dA=False)
    _raises(mc, L.MC_ERR_DTYPE, "grouped projections run in bfloat16 only", gb, None, [proj], [c["dy"].float()],
            2.0, need_dA=False)
    _raises(mc, L.MC_ERR_SHAPE, "h_save[0] has shape (4, 15)", gb, None, [proj], [c["dy"]], 2.0,
            h_saves=[torch.zeros(4, 15)], need_dA=False)
    _raises(mc, L.MC_ERR_SHAPE, "mask has shape (16, 3)", gb, None,
            [dict(proj, mask=torch.ones(16, 3, dtype=torch.uint8))], [c["dy"]], 2.0, dropout_p=0.1, need_dA=False)
    # with x given, the same shapes are checked against x
    _raises(mc, L.MC_ERR_SHAPE, "dY[0] has shape (16, 24)", gb, torch.zeros(15, 32, dtype=torch.bfloat16), [proj],
            [c["dy"]], 2.0)
