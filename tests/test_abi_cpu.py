"""C ABI checks that need no GPU: libmc_hip.so loads, exports every function
include/mc_hip.h declares, and rejects bad arguments on the host with the
reference's error conventions (validation runs before anything is enqueued,
so these calls never touch a device)."""
import ctypes

import numpy as np
import pytest


def test_library_loads_and_exports_header(mc):
    L = mc._lib.lib()
    names = mc._lib.header_symbols()
    assert len(names) >= 16
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert b"gfx950" in L.mc_version()


def _desc(mc, T=16, K=16, N=16, r=4, scale=2.0, p=0.0, dtype=1):
    return mc._lib.LoraDesc(T, K, N, r, scale, p, dtype)


@pytest.mark.parametrize("field,value,code,msg", [
    ("rank", 0, 2, "LoRA rank must be greater than 0"),        # lora.rs:99-104
    ("dropout_p", 1.0, 5, "LoRA dropout must be in [0, 1)"),    # lora.rs:113-118
    ("dropout_p", -0.1, 5, "LoRA dropout must be in [0, 1)"),
    ("rank", 8193, 2, "exceeds the supported maximum 8192"),
    ("tokens", 0, 2, "must be >= 1"),
    ("act_dtype", 7, 3, "unsupported act_dtype"),
    ("out_features", 1 << 22, 2, "must be below 2^22"),   # 32-bit buffer offsets of the bf16 kernels
    ("tokens", 1 << 24, 2, "must be below 2^24"),
])
def test_lora_desc_validation(mc, field, value, code, msg):
    L = mc._lib.lib()
    d = _desc(mc)
    setattr(d, field, value)
    assert L.mc_lora_fwd_workspace_size(ctypes.byref(d)) == 0
    fake = ctypes.c_void_p(256)
    st = L.mc_lora_fwd(ctypes.byref(d), fake, None, None, fake, fake, None, fake, None, None, 0, None)
    assert st == code
    assert msg in mc._lib.last_error()


def test_lora_null_and_workspace_errors(mc):
    L = mc._lib.lib()
    d = _desc(mc)
    fake = ctypes.c_void_p(256)
    assert L.mc_lora_fwd(ctypes.byref(d), None, None, None, fake, fake, None, fake, None, None, 0, None) == 1
    assert L.mc_lora_fwd(None, fake, None, None, fake, fake, None, fake, None, None, 0, None) == 1
    # workspace too small
    need = L.mc_lora_fwd_workspace_size(ctypes.byref(d))
    assert need > 0
    assert L.mc_lora_fwd(ctypes.byref(d), fake, None, None, fake, fake, None, fake, None, fake, need - 1,
                         None) == 6
    assert "workspace" in mc._lib.last_error()
    # misaligned activations
    assert L.mc_lora_fwd(ctypes.byref(d), ctypes.c_void_p(258), None, None, fake, fake, None, fake, None, fake,
                         need, None) == 4
    # dropout without a mask
    d.dropout_p = 0.1
    assert L.mc_lora_fwd(ctypes.byref(d), fake, None, None, fake, fake, None, fake, None, fake, need, None) == 1
    assert "requires a mask" in mc._lib.last_error()
    # backward: dB without the saved hidden
    d.dropout_p = 0.0
    nb = L.mc_lora_bwd_workspace_size(ctypes.byref(d))
    assert L.mc_lora_bwd(ctypes.byref(d), fake, None, fake, fake, None, None, fake, None, None, fake, fake, nb,
                         None) == 1
    assert "h_save" in mc._lib.last_error()


def test_rowop_validation(mc):
    L = mc._lib.lib()
    fake = ctypes.c_void_p(256)
    assert L.mc_rmsnorm_fwd(0, 8, 1e-6, 0, fake, None, fake, None, None) == 2
    assert L.mc_rmsnorm_fwd(4, 8, -1.0, 0, fake, None, fake, None, None) == 5
    assert L.mc_rmsnorm_fwd(4, 8, 1e-6, 2, fake, None, fake, None, None) == 3
    assert L.mc_rmsnorm_bwd(4, 8, 1e-6, 0, fake, None, None, fake, fake, fake, None, 0, None) == 6
    assert L.mc_softmax_fwd(4, 8, 9, 0, fake, fake, None) == 2
    assert "causal_rows" in mc._lib.last_error()
    assert L.mc_softmax_bwd(4, 8, 0, 0, None, fake, fake, None) == 1
    assert L.mc_profile_read(9, None, None, None, None) == 5


def test_rowop_row_limits(mc):
    """One launch holds at most 2^32 - 1 work-items: the wave-per-row forward
    kernels (4 rows per 256 threads) stop at 67108860 rows, the
    workgroup-per-row kernels at 16777215; softmax splits its launches."""
    L = mc._lib.lib()
    fake = ctypes.c_void_p(256)
    wave_max, block_max = ((2**32 - 1) // 256) * 4, (2**32 - 1) // 256
    assert L.mc_rmsnorm_fwd(wave_max + 1, 8, 1e-6, 0, fake, None, fake, None, None) == 2
    assert "rows must be <= 67108860" in mc._lib.last_error()
    assert L.mc_layernorm_fwd(wave_max + 1, 8, 1e-6, 0, fake, None, None, fake, None, None, None) == 2
    assert L.mc_log_softmax_fwd(block_max + 1, 8, 0, fake, fake, None) == 2
    assert "rows must be <= 16777215" in mc._lib.last_error()
    assert L.mc_log_softmax_bwd(block_max + 1, 8, 0, fake, fake, fake, None) == 2
    d = mc._lib.XentDesc(block_max + 1, 8, -100, 0.0, 0)
    assert L.mc_cross_entropy_fwd(ctypes.byref(d), fake, fake, fake, None, None, 0, None) == 2
    # below the bound the shape passes and the next check (NULL output) answers
    assert L.mc_rmsnorm_fwd(wave_max, 8, 1e-6, 0, fake, None, None, None, None) == 1
    assert L.mc_log_softmax_fwd(block_max, 8, 0, fake, None, None) == 1
    # softmax has no row bound: a NULL output is the first error at any row count
    assert L.mc_softmax_fwd(2**40, 8, 0, 0, fake, None, None) == 1


def test_dropout_mask_matches_oracle(mc):
    import oracle

    for seed, p, rows, rank in [(1234, 0.1, 257, 64), (0, 0.5, 3, 5), (2**40 + 7, 0.25, 100, 8)]:
        got = mc.dropout_mask(seed, p, rows, rank).numpy()
        assert np.array_equal(got, oracle.dropout_mask(seed, p, rows, rank))
    m = mc.dropout_mask(1234, 0.1, 16384, 64).numpy()
    assert abs(m.mean() - 0.9) < 0.005
    assert mc._lib.lib().mc_dropout_mask(1, 1.0, 4, 4, ctypes.c_void_p(256)) == 5


def _attn(mc, B=1, S=64, H=4, Hkv=2, D=64, causal=1, scale=0.125, dtype=1):
    return mc._lib.AttnDesc(B, S, H, Hkv, D, causal, scale, dtype)


@pytest.mark.parametrize("field,value,code,msg", [
    ("kv_heads", 3, 2, "must be a multiple of kv_heads"),   # repeat_kv, transformer.rs:258-259
    ("heads", 0, 2, "must be >= 1"),
    ("seq", 0, 2, "must be >= 1"),
    ("head_dim", 257, 2, "head_dim must be in [1, 256]"),
    ("head_dim", 36, 2, "multiple of 8"),
    ("causal", 2, 5, "causal must be 0 or 1"),
    ("scale", float("nan"), 5, "scale must be finite"),
    ("dtype", 9, 3, "unsupported dtype"),
])
def test_attention_desc_validation(mc, field, value, code, msg):
    L = mc._lib.lib()
    d = _attn(mc)
    setattr(d, field, value)
    assert L.mc_attention_fwd_workspace_size(ctypes.byref(d)) == 0
    fake = ctypes.c_void_p(256)
    st = L.mc_attention_fwd(ctypes.byref(d), fake, fake, fake, None, fake, None, fake, 1 << 30, None)
    assert st == code
    assert msg in mc._lib.last_error()


def test_attention_null_workspace_and_layout_errors(mc):
    L = mc._lib.lib()
    d = _attn(mc)
    fake = ctypes.c_void_p(256)
    need = L.mc_attention_fwd_workspace_size(ctypes.byref(d))
    assert need == 1 * 2 * 64 * 64 * 2  # V^T [B, Hkv, D, Sp] bf16
    assert L.mc_attention_fwd(ctypes.byref(d), None, fake, fake, None, fake, None, fake, need, None) == 1
    assert L.mc_attention_fwd(ctypes.byref(d), fake, fake, fake, None, fake, None, fake, need - 1, None) == 6
    assert L.mc_attention_fwd(ctypes.byref(d), fake, ctypes.c_void_p(264), fake, None, fake, None, fake, need,
                              None) == 4
    # a mask of S * S fp32 beyond 2^31 bytes
    big = _attn(mc, S=30000)
    st = L.mc_attention_fwd(ctypes.byref(big), fake, fake, fake, fake, fake, None, fake, 1 << 40, None)
    assert st == 2 and "explicit mask" in mc._lib.last_error()
    # fp32 and other bf16 head dims take the workspace-free kernel
    assert L.mc_attention_fwd_workspace_size(ctypes.byref(_attn(mc, dtype=0))) == 0
    assert L.mc_attention_fwd_workspace_size(ctypes.byref(_attn(mc, D=32))) == 0


@pytest.mark.parametrize("field,value,msg", [
    ("learning_rate", 0.0, "learning rate must be positive"),          # optimizer.rs:68-73
    ("learning_rate", -1.0, "learning rate must be positive"),
    ("beta1", 1.5, "beta1 must be in [0, 1), got 1.5"),               # optimizer.rs:75-80
    ("beta2", -0.1, "beta2 must be in [0, 1), got -0.1"),             # optimizer.rs:82-87
    ("epsilon", 0.0, "epsilon must be positive"),                      # optimizer.rs:89-94
    ("weight_decay", -0.01, "weight decay must be non-negative"),      # optimizer.rs:96-101
])
def test_adamw_config_validation(mc, field, value, msg):
    L = mc._lib.lib()
    cfg = mc._lib.AdamWConfig(1e-4, 0.9, 0.999, 1e-8, 0.01)
    setattr(cfg, field, value)
    assert L.mc_adamw_step(ctypes.byref(cfg), None, 0, None) == 5
    assert mc._lib.last_error() == msg


def test_adamw_table_errors(mc):
    L = mc._lib.lib()
    cfg = mc._lib.AdamWConfig(1e-4, 0.9, 0.999, 1e-8, 0.01)
    assert L.mc_adamw_step(ctypes.byref(cfg), None, 0, None) == 0   # nothing to do
    assert L.mc_adamw_step(None, None, 0, None) == 1
    assert L.mc_adamw_step(ctypes.byref(cfg), None, 2, None) == 1
    t = (mc._lib.AdamWTensor * 1)()
    t[0] = mc._lib.AdamWTensor(256, 256, 256, 256, 256, 10, 0)
    assert L.mc_adamw_step(ctypes.byref(cfg), t, 1, None) == 5 and "step" in mc._lib.last_error()
    t[0] = mc._lib.AdamWTensor(256, 256, None, 256, 256, 10, 1)
    assert L.mc_adamw_step(ctypes.byref(cfg), t, 1, None) == 1
    t[0] = mc._lib.AdamWTensor(256, 260, 256, 256, 256, 10, 1)
    assert L.mc_adamw_step(ctypes.byref(cfg), t, 1, None) == 4
    t[0] = mc._lib.AdamWTensor(None, None, None, None, None, 0, 1)   # empty tensors need no pointers
    assert L.mc_adamw_step(ctypes.byref(cfg), t, 1, None) == 0


def test_lora_group_validation(mc):
    """Grouped entry points: the shared descriptor is checked as for one
    projection, every projection's N and pointers on their own, before any
    launch."""
    L = mc._lib.lib()
    d = _desc(mc, T=16, K=16, N=0, r=4)
    fake = 256
    projs = (mc._lib.LoraProj * 2)(mc._lib.LoraProj(16, fake, None, fake, fake, None),
                                   mc._lib.LoraProj(24, fake, None, fake, fake, None))
    need_f = L.mc_lora_group_fwd_workspace_size(ctypes.byref(d), projs, 2)
    need_b = L.mc_lora_group_bwd_workspace_size(ctypes.byref(d), projs, 2)
    assert need_f > 0 and need_b > 0
    ys = (ctypes.c_void_p * 2)(fake, fake)
    hs = (ctypes.c_void_p * 2)(fake, fake)
    w = ctypes.c_void_p(fake)
    # count out of range
    assert L.mc_lora_group_fwd(ctypes.byref(d), w, projs, 0, ys, hs, w, need_f, None) == 2
    assert L.mc_lora_group_fwd(ctypes.byref(d), w, projs, 5, ys, hs, w, need_f, None) == 2
    # fp32 is per-projection only
    d32 = _desc(mc, T=16, K=16, N=0, r=4, dtype=0)
    assert L.mc_lora_group_fwd(ctypes.byref(d32), w, projs, 2, ys, hs, w, need_f, None) == 3
    assert "bf16 only" in mc._lib.last_error()
    # a projection's N, or K, not a multiple of 8 (single calls pad; groups do not)
    projs[1].out_features = 20
    assert L.mc_lora_group_fwd_workspace_size(ctypes.byref(d), projs, 2) == 0
    assert L.mc_lora_group_fwd(ctypes.byref(d), w, projs, 2, ys, hs, w, need_f, None) == 2
    assert "multiples of 8" in mc._lib.last_error()
    projs[1].out_features = 24
    d.in_features = 20
    assert L.mc_lora_group_fwd(ctypes.byref(d), w, projs, 2, ys, hs, w, need_f, None) == 2
    d.in_features = 16
    # missing B, bias without W, dropout without a mask
    projs[0].B = None
    assert L.mc_lora_group_fwd(ctypes.byref(d), w, projs, 2, ys, hs, w, need_f, None) == 1
    projs[0].B = fake
    projs[1].W, projs[1].bias = None, fake
    assert L.mc_lora_group_fwd(ctypes.byref(d), w, projs, 2, ys, hs, w, need_f, None) == 1
    assert "bias given without W" in mc._lib.last_error()
    projs[1].W, projs[1].bias = fake, None
    d.dropout_p = 0.1
    assert L.mc_lora_group_fwd(ctypes.byref(d), w, projs, 2, ys, hs, w, need_f, None) == 1
    assert "requires a mask" in mc._lib.last_error()
    d.dropout_p = 0.0
    # workspace too small, misaligned output
    assert L.mc_lora_group_fwd(ctypes.byref(d), w, projs, 2, ys, hs, w, need_f - 1, None) == 6
    ys[1] = 264
    assert L.mc_lora_group_fwd(ctypes.byref(d), w, projs, 2, ys, hs, w, need_f, None) == 4
    # backward: dB without h_save
    dys = (ctypes.c_void_p * 2)(fake, fake)
    dbs = (ctypes.c_void_p * 2)(fake, None)
    assert L.mc_lora_group_bwd(ctypes.byref(d), w, projs, 2, None, dys, None, None, dbs, w, need_b, None) == 1
    assert "requires h_save" in mc._lib.last_error()
    # nothing requested: no work, OK
    assert L.mc_lora_group_bwd(ctypes.byref(d), w, projs, 2, None, dys, None, None, None, w, need_b, None) == 0
    # a caller's W^T: needs W and 16-byte alignment; the backward's workspace
    # then holds no transposed copy of that W (16 x 16 bf16, 256-byte aligned)
    projs[0].Wt = fake
    assert L.mc_lora_group_bwd_workspace_size(ctypes.byref(d), projs, 2) == need_b - 512
    projs[0].Wt = 264
    assert L.mc_lora_group_bwd(ctypes.byref(d), w, projs, 2, None, dys, None, None, None, w, need_b, None) == 4
    assert "Wt must be 16-byte aligned" in mc._lib.last_error()
    projs[0].W, projs[0].Wt = None, fake
    assert L.mc_lora_group_bwd(ctypes.byref(d), w, projs, 2, None, dys, None, None, None, w, need_b, None) == 1
    assert "Wt given without W" in mc._lib.last_error()


def test_transpose_validation(mc):
    """mc_transpose_bf16: sizes multiples of 8, pointers present and aligned."""
    L = mc._lib.lib()
    fake = 256
    assert L.mc_transpose_bf16(0, 8, fake, fake, None) == 2
    assert L.mc_transpose_bf16(12, 8, fake, fake, None) == 2
    assert "multiples of 8" in mc._lib.last_error()
    assert L.mc_transpose_bf16(8, 8, None, fake, None) == 1
    assert L.mc_transpose_bf16(8, 8, fake, 264, None) == 4


def _a256(n):
    return (n + 255) // 256 * 256


@pytest.mark.parametrize("B,S,H,Hkv,causal,groups", [
    (8, 2048, 12, 2, 1, 2),    # c4: 3 query heads per dK/dV workgroup, two partials per K/V head
    (4, 4096, 28, 4, 1, 1),    # c5: all 7 heads of a K/V head in one workgroup, no partials
    (16, 2048, 4, 2, 1, 1),
    (8, 1024, 8, 4, 0, 1),
    (1, 64, 4, 2, 1, 2),       # small grids keep one query head per workgroup
    (2, 300, 12, 12, 1, 1),
])
def test_attention_bwd_workspace_groups(mc, B, S, H, Hkv, causal, groups):
    """The bf16 backward's workspace: lse/Delta blocks, the dK/dV partials of
    the query-head groups (none when a group holds all H/Hkv heads of a K/V
    head), and dS^T [B, H, S, S rounded up to 128] for the dQ pass."""
    L = mc._lib.lib()
    D = 128
    d = _attn(mc, B=B, S=S, H=H, Hkv=Hkv, D=D, causal=causal)
    Sp = (S + 63) // 64 * 64
    want = _a256(B * H * (Sp // 64) * 128 * 4)
    if groups > 1:
        want += 2 * _a256(B * Hkv * groups * S * D * 4)
    want += _a256(B * H * S * ((S + 127) // 128 * 128) * 2)
    assert L.mc_attention_bwd_workspace_size(ctypes.byref(d)) == want


def test_lora_odd_features_padded_workspace(mc):
    """bf16 K or N not a multiple of 8: the single-projection calls accept the
    shape and run on zero-padded copies, whose buffers extend the padded
    shape's workspace."""
    L = mc._lib.lib()
    T, r = 300, 8
    for K, N in ((37, 45), (40, 45), (37, 48)):
        d = _desc(mc, T=T, K=K, N=N, r=r)
        Kp, Np = (K + 7) // 8 * 8, (N + 7) // 8 * 8
        dp = _desc(mc, T=T, K=Kp, N=Np, r=r)
        inner_f = L.mc_lora_fwd_workspace_size(ctypes.byref(dp))
        inner_b = L.mc_lora_bwd_workspace_size(ctypes.byref(dp))
        bufs = _a256(T * Kp * 2) + _a256(Np * Kp * 2) + _a256(Np * 2) + _a256(Kp * r * 4) + _a256(r * Np * 4)
        assert L.mc_lora_fwd_workspace_size(ctypes.byref(d)) == _a256(inner_f) + bufs + _a256(T * Np * 2)
        assert L.mc_lora_bwd_workspace_size(ctypes.byref(d)) == (_a256(inner_b) + bufs + _a256(T * Np * 2) +
                                                                 _a256(T * Kp * 2) + _a256(Kp * r * 4) +
                                                                 _a256(r * Np * 4))
