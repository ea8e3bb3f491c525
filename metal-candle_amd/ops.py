"""torch-tensor front end of the C ABI (device memory and streams come from
torch; all arithmetic runs in libmc_hip.so's HIP kernels).

Shapes follow the reference: x [..., K], W [N, K], A [K, r], B [r, N]; the
leading dims of x are folded into T tokens as FusedLoRAOp::extract_dimensions
does (src/backend/custom_ops.rs:254-270). Activations are float32 or bfloat16;
A, B and their gradients are float32. Every call enqueues on torch's current
stream of the tensors' device and does not synchronise.
"""
import ctypes

import torch

from . import _lib
from ._lib import AdamWConfig, AdamWTensor, AttnDesc, LoraDesc, LoraProj, McError, XentDesc, check, lib

_DTYPES = {torch.float32: _lib.MC_F32, torch.bfloat16: _lib.MC_BF16}


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _dtype_code(t):
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise McError(_lib.MC_ERR_DTYPE, f"unsupported dtype {t.dtype} (float32 or bfloat16)")


def _contig(t, name):
    if t is None:
        return None
    if not t.is_contiguous():
        raise McError(_lib.MC_ERR_LAYOUT, f"{name} must be contiguous")
    return t


def _expect(t, name, shape=None, dtype=None, device=None):
    """Raise McError unless t is contiguous with the given shape, dtype and
    device. These checks run before the C ABI is called: the kernels read
    each buffer over the extent its shape arguments give, so a tensor of the
    wrong size must never reach them."""
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        raise McError(_lib.MC_ERR_NULL, f"{name} must be a tensor")
    _contig(t, name)
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise McError(_lib.MC_ERR_SHAPE, f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if dtype is not None and t.dtype != dtype:
        raise McError(_lib.MC_ERR_DTYPE, f"{name} has dtype {t.dtype}, expected {dtype}")
    if device is not None and t.device != device:
        raise McError(_lib.MC_ERR_LAYOUT, f"{name} is on {t.device}, expected {device}")
    return t


def _lora_factors(A, B):
    """FusedLoRAOp::new (src/backend/custom_ops.rs:118-148): A [K, r] and B [r, N]."""
    for t, n in ((A, "A"), (B, "B")):
        if not isinstance(t, torch.Tensor):
            raise McError(_lib.MC_ERR_NULL, f"{n} must be a tensor")
    if A.dim() != 2 or B.dim() != 2:
        raise McError(_lib.MC_ERR_SHAPE,
                      f"LoRA matrices must be 2D, got shapes {list(A.shape)} and {list(B.shape)}")
    if A.shape[1] != B.shape[0]:
        raise McError(_lib.MC_ERR_SHAPE, "Incompatible LoRA matrix dimensions: "
                      f"{A.shape[0]}\u00d7{A.shape[1]} and {B.shape[0]}\u00d7{B.shape[1]}")
    return A.shape[0], A.shape[1], B.shape[1]


def _rows_of(x, name):
    if not isinstance(x, torch.Tensor):
        raise McError(_lib.MC_ERR_NULL, f"{name} must be a tensor")
    if x.dim() < 1:
        raise McError(_lib.MC_ERR_SHAPE, "Input must have at least 1 dimension")
    _contig(x, name)
    _dtype_code(x)
    D = x.shape[-1]
    return (x.numel() // D if D else 0), D


def _workspace(nbytes, device):
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def lora_desc(tokens, in_features, out_features, rank, scale, dropout_p=0.0, dtype=torch.bfloat16):
    return LoraDesc(tokens, in_features, out_features, rank, scale, dropout_p, _DTYPES[dtype])


def lora_forward(x, A, B, scale, W=None, bias=None, mask=None, dropout_p=0.0, save_hidden=True):
    """y = x.W^T + bias + scale*((x.A) (.) mask/(1-p)).B ; returns (y, h_save).

    x [..., K] (float32 or bfloat16), A [K, r] and B [r, N] float32, W [N, K]
    and bias [N] in x's dtype, mask uint8 [T, r] (T = the leading dims of x
    folded); all contiguous on x's device. Shape errors keep the reference's
    messages (custom_ops.rs:123-139, 153-174)."""
    K, r, N = _lora_factors(A, B)
    if not isinstance(x, torch.Tensor) or x.dim() < 1:
        raise McError(_lib.MC_ERR_SHAPE, "Input must have at least 1 dimension")
    _contig(x, "x")
    code = _dtype_code(x)
    if x.shape[-1] != K:
        raise McError(_lib.MC_ERR_SHAPE, f"Input feature dimension mismatch: expected {K}, got {x.shape[-1]}")
    T = x.numel() // K if K else 0
    dev = x.device
    _expect(A, "A", dtype=torch.float32, device=dev)
    _expect(B, "B", dtype=torch.float32, device=dev)
    _expect(W, "W", shape=(N, K), dtype=x.dtype, device=dev)
    _expect(bias, "bias", shape=(N,), dtype=x.dtype, device=dev)
    _expect(mask, "mask", shape=(T, r), dtype=torch.uint8, device=dev)
    d = LoraDesc(T, K, N, r, float(scale), float(dropout_p), code)
    y = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=dev)
    h = torch.empty(r, T, dtype=torch.float32, device=dev) if save_hidden else None
    ws_n = lib().mc_lora_fwd_workspace_size(ctypes.byref(d))  # 0 for an invalid descriptor
    ws = _workspace(ws_n, dev)
    check(lib().mc_lora_fwd(ctypes.byref(d), _ptr(x), _ptr(W), _ptr(bias), _ptr(A), _ptr(B), _ptr(mask),
                            _ptr(y), _ptr(h), _ptr(ws), ws_n, _stream(x)))
    return y, h


def lora_backward(x, A, B, dY, scale, W=None, mask=None, dropout_p=0.0, h_save=None,
                  need_dx=True, need_dA=True, need_dB=True):
    """(dX, dA, dB) with W frozen; entries not requested are None.

    dY [..., N] with x [..., K] over the same leading dims (x may be None
    when dA is not requested), h_save [r, T] float32 from lora_forward
    (required for dB), other tensors as in lora_forward."""
    K, r, N = _lora_factors(A, B)
    if not isinstance(dY, torch.Tensor) or dY.dim() < 1:
        raise McError(_lib.MC_ERR_SHAPE, "dY must have at least 1 dimension")
    _contig(dY, "dY")
    code = _dtype_code(dY)
    if dY.shape[-1] != N:
        raise McError(_lib.MC_ERR_SHAPE, f"dY feature dimension mismatch: expected {N}, got {dY.shape[-1]}")
    T = dY.numel() // N if N else 0
    dev = dY.device
    _expect(A, "A", dtype=torch.float32, device=dev)
    _expect(B, "B", dtype=torch.float32, device=dev)
    _expect(x, "x", shape=tuple(dY.shape[:-1]) + (K,), dtype=dY.dtype, device=dev)
    _expect(W, "W", shape=(N, K), dtype=dY.dtype, device=dev)
    _expect(mask, "mask", shape=(T, r), dtype=torch.uint8, device=dev)
    _expect(h_save, "h_save", shape=(r, T), dtype=torch.float32, device=dev)
    d = LoraDesc(T, K, N, r, float(scale), float(dropout_p), code)
    dX = torch.empty(*dY.shape[:-1], K, dtype=dY.dtype, device=dev) if need_dx else None
    dA = torch.empty(K, r, dtype=torch.float32, device=dev) if need_dA else None
    dB = torch.empty(r, N, dtype=torch.float32, device=dev) if need_dB else None
    ws_n = lib().mc_lora_bwd_workspace_size(ctypes.byref(d))  # 0 for an invalid descriptor
    ws = _workspace(ws_n, dev)
    check(lib().mc_lora_bwd(ctypes.byref(d), _ptr(x), _ptr(W), _ptr(A), _ptr(B), _ptr(mask), _ptr(h_save),
                            _ptr(dY), _ptr(dX), _ptr(dA), _ptr(dB), _ptr(ws), ws_n, _stream(dY)))
    return dX, dA, dB


def _ptr_array(ts):
    return (ctypes.c_void_p * len(ts))(*[None if t is None else t.data_ptr() for t in ts])


def _group_table(x, projs, dropout_p, lead=None, like=None):
    """Validate a grouped call's projections (dicts with W, bias, A, B, mask)
    against the shared x [..., K] and build the C table; returns (table, K,
    r, T, [N_g]). With x None, the leading dims come from `lead`, K from the
    first projection's A and the dtype / device from the tensor `like`."""
    if not isinstance(projs, (list, tuple)) or not 1 <= len(projs) <= _lib.MC_LORA_MAX_GROUP:
        raise McError(_lib.MC_ERR_SHAPE, f"a group holds 1 to {_lib.MC_LORA_MAX_GROUP} projections")
    if x is None:
        if not isinstance(projs[0], dict) or not isinstance(projs[0].get("A"), torch.Tensor) or projs[0]["A"].dim() != 2:
            raise McError(_lib.MC_ERR_SHAPE, "lora_a must be 2D")
        K = projs[0]["A"].shape[0]
        T = 1
        for n in lead:
            T *= n
        dtype, device = like.dtype, like.device
    else:
        if not isinstance(x, torch.Tensor) or x.dim() < 1:
            raise McError(_lib.MC_ERR_SHAPE, "Input must have at least 1 dimension")
        _contig(x, "x")
        K = x.shape[-1]
        T = x.numel() // K if K else 0
        dtype, device = x.dtype, x.device
    if dtype != torch.bfloat16:
        raise McError(_lib.MC_ERR_DTYPE, "grouped projections run in bfloat16 only")
    table = (LoraProj * len(projs))()
    r0, Ns = None, []
    for g, p in enumerate(projs):
        Kg, r, N = _lora_factors(p["A"], p["B"])
        if Kg != K:
            raise McError(_lib.MC_ERR_SHAPE, f"Input feature dimension mismatch: expected {Kg}, got {K}")
        if r0 is not None and r != r0:
            raise McError(_lib.MC_ERR_SHAPE, f"projection {g}: rank {r} differs from the group's {r0}")
        r0 = r
        _expect(p["A"], "A", dtype=torch.float32, device=device)
        _expect(p["B"], "B", dtype=torch.float32, device=device)
        _expect(p.get("W"), "W", shape=(N, K), dtype=dtype, device=device)
        _expect(p.get("bias"), "bias", shape=(N,), dtype=dtype, device=device)
        _expect(p.get("mask"), "mask", shape=(T, r), dtype=torch.uint8, device=device)
        _expect(p.get("Wt"), "Wt", shape=(K, N), dtype=dtype, device=device)
        table[g] = LoraProj(N, *[None if p.get(k) is None else p[k].data_ptr()
                                 for k in ("W", "bias", "A", "B", "mask", "Wt")])
        Ns.append(N)
    return table, K, r0, T, Ns


def lora_group_forward(x, projs, scale, dropout_p=0.0, save_hidden=True):
    """The LoRA projections of one input x [..., K] in one call
    (mc_lora_group_fwd): projs is a list of 1-4 dicts with W [N_g, K], bias
    [N_g] (or None), A [K, r], B [r, N_g], mask [T, r] (or None) and,
    optionally, Wt = transpose_weight(W) for the backward. Returns ([y_g],
    [h_save_g]); each y_g equals lora_forward's for that projection."""
    table, K, r, T, Ns = _group_table(x, projs, dropout_p)
    d = LoraDesc(T, K, Ns[0], r, float(scale), float(dropout_p), _lib.MC_BF16)
    ys = [torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=x.device) for N in Ns]
    hs = [torch.empty(r, T, dtype=torch.float32, device=x.device) if save_hidden else None for _ in Ns]
    n = len(Ns)
    ws_n = lib().mc_lora_group_fwd_workspace_size(ctypes.byref(d), table, n)
    ws = _workspace(ws_n, x.device)
    check(lib().mc_lora_group_fwd(ctypes.byref(d), _ptr(x), table, n, _ptr_array(ys), _ptr_array(hs), _ptr(ws), ws_n,
                                  _stream(x)))
    return ys, hs


def lora_group_backward(x, projs, dYs, scale, dropout_p=0.0, h_saves=None, need_dx=True, need_dA=True, need_dB=True):
    """Backward of lora_group_forward (mc_lora_group_bwd): returns (dX, [dA_g],
    [dB_g]) where dX [..., K] is the sum of every projection's input gradient.
    x may be None when dA is not requested (as in lora_backward); the leading
    dims then come from dYs[0] and K from the projections' A."""
    if not isinstance(dYs, (list, tuple)) or len(dYs) < 1:
        raise McError(_lib.MC_ERR_SHAPE, "one dY per projection")
    if x is None:
        if need_dA:
            raise McError(_lib.MC_ERR_NULL, "LoRA backward: dA requires x")
        if not isinstance(dYs[0], torch.Tensor) or dYs[0].dim() < 1:
            raise McError(_lib.MC_ERR_SHAPE, "dY must have at least 1 dimension")
        lead = tuple(dYs[0].shape[:-1])
        table, K, r, T, Ns = _group_table(None, projs, dropout_p, lead=lead, like=dYs[0])
    else:
        table, K, r, T, Ns = _group_table(x, projs, dropout_p)
        lead = tuple(x.shape[:-1])
    if len(dYs) != len(Ns):
        raise McError(_lib.MC_ERR_SHAPE, "one dY per projection")
    dev = dYs[0].device if x is None else x.device
    for g, (dy, N) in enumerate(zip(dYs, Ns)):
        _expect(dy, f"dY[{g}]", shape=lead + (N,), dtype=torch.bfloat16, device=dev)
    if h_saves is not None:
        for g, h in enumerate(h_saves):
            _expect(h, f"h_save[{g}]", shape=(r, T), dtype=torch.float32, device=dev)
    d = LoraDesc(T, K, Ns[0], r, float(scale), float(dropout_p), _lib.MC_BF16)
    dX = torch.empty(*lead, K, dtype=torch.bfloat16, device=dev) if need_dx else None
    dAs = [torch.empty(K, r, dtype=torch.float32, device=dev) if need_dA else None for _ in Ns]
    dBs = [torch.empty(r, N, dtype=torch.float32, device=dev) if need_dB else None for N in Ns]
    n = len(Ns)
    ws_n = lib().mc_lora_group_bwd_workspace_size(ctypes.byref(d), table, n)
    ws = _workspace(ws_n, dev)
    hp = _ptr_array(h_saves) if h_saves is not None else None
    check(lib().mc_lora_group_bwd(ctypes.byref(d), _ptr(x), table, n, hp, _ptr_array(dYs), _ptr(dX), _ptr_array(dAs),
                                  _ptr_array(dBs), _ptr(ws), ws_n, _stream(dYs[0])))
    return dX, dAs, dBs


def transpose_weight(W):
    """W^T [K, N] of a frozen bf16 base weight W [N, K] (mc_transpose_bf16):
    built once and passed as a projection's Wt, the grouped backward reads it
    instead of transposing W on every call."""
    _contig(W, "W")
    if W.dim() != 2:
        raise McError(_lib.MC_ERR_SHAPE, "W must be 2-D")
    if W.dtype != torch.bfloat16:
        raise McError(_lib.MC_ERR_DTYPE, "transpose_weight takes a bfloat16 W")
    Wt = torch.empty(W.shape[1], W.shape[0], dtype=W.dtype, device=W.device)
    check(lib().mc_transpose_bf16(W.shape[0], W.shape[1], _ptr(W), _ptr(Wt), _stream(W)))
    return Wt


def rms_norm_forward(x, eps, w=None, save_rstd=True):
    """RMSNorm over the last dim: (y, rstd). w [dim] in x's dtype or None."""
    rows, D = _rows_of(x, "x")
    _expect(w, "w", shape=(D,), dtype=x.dtype, device=x.device)
    y = torch.empty_like(x)
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device) if save_rstd else None
    check(lib().mc_rmsnorm_fwd(rows, D, float(eps), _dtype_code(x), _ptr(x), _ptr(w), _ptr(y), _ptr(rstd),
                               _stream(x)))
    return y, rstd


def rms_norm_backward(x, dy, eps, w=None, rstd=None, need_dw=True):
    """(dx, dw) of RMSNorm; rstd [rows] float32 from the forward or None."""
    rows, D = _rows_of(x, "x")
    _expect(dy, "dy", shape=x.shape, dtype=x.dtype, device=x.device)
    _expect(w, "w", shape=(D,), dtype=x.dtype, device=x.device)
    _expect(rstd, "rstd", shape=(rows,), dtype=torch.float32, device=x.device)
    dx = torch.empty_like(x)
    dw = torch.empty(D, dtype=torch.float32, device=x.device) if need_dw else None
    ws_n = lib().mc_rmsnorm_bwd_workspace_size(rows, D) if need_dw else 0
    ws = _workspace(ws_n, x.device)
    check(lib().mc_rmsnorm_bwd(rows, D, float(eps), _dtype_code(x), _ptr(x), _ptr(w), _ptr(rstd), _ptr(dy),
                               _ptr(dx), _ptr(dw), _ptr(ws), ws_n, _stream(x)))
    return dx, dw


def softmax_forward(s, causal_rows=0):
    rows, D = _rows_of(s, "s")
    p = torch.empty_like(s)
    check(lib().mc_softmax_fwd(rows, D, int(causal_rows), _dtype_code(s), _ptr(s), _ptr(p), _stream(s)))
    return p


def softmax_backward(p, dp, causal_rows=0):
    rows, D = _rows_of(p, "p")
    _expect(dp, "dp", shape=p.shape, dtype=p.dtype, device=p.device)
    ds = torch.empty_like(p)
    check(lib().mc_softmax_bwd(rows, D, int(causal_rows), _dtype_code(p), _ptr(p), _ptr(dp), _ptr(ds),
                               _stream(p)))
    return ds


def attention_desc(q, k, causal, scale):
    B, H, S, D = q.shape
    return AttnDesc(B, S, H, k.shape[1], D, int(bool(causal)), float(scale), _dtype_code(q))


def _attn_inputs(q, k, v, mask):
    """q [B, H, S, D]; k, v [B, Hkv, S, D] in q's dtype; mask fp32 [S, S] or None."""
    if not isinstance(q, torch.Tensor) or q.dim() != 4:
        raise McError(_lib.MC_ERR_SHAPE, "q must be [batch, heads, seq, head_dim]")
    _contig(q, "q")
    _dtype_code(q)
    B, H, S, D = q.shape
    if not isinstance(k, torch.Tensor) or k.dim() != 4:
        raise McError(_lib.MC_ERR_SHAPE, "k must be [batch, kv_heads, seq, head_dim]")
    Hkv = k.shape[1]
    _expect(k, "k", shape=(B, Hkv, S, D), dtype=q.dtype, device=q.device)
    _expect(v, "v", shape=(B, Hkv, S, D), dtype=q.dtype, device=q.device)
    _expect(mask, "mask", shape=(S, S), dtype=torch.float32, device=q.device)
    return B, H, S, D


def attention_forward(q, k, v, causal=False, scale=None, mask=None, save_lse=True):
    """Attention core of Attention::forward (src/models/transformer.rs:258-283):
    q [B, H, S, D], k, v [B, Hkv, S, D] -> (o [B, S, H*D], lse [B, H, S])."""
    B, H, S, D = _attn_inputs(q, k, v, mask)
    if scale is None:
        scale = D ** -0.5
    d = attention_desc(q, k, causal, scale)
    o = torch.empty(B, S, H * D, dtype=q.dtype, device=q.device)
    lse = torch.empty(B, H, S, dtype=torch.float32, device=q.device) if save_lse else None
    ws_n = lib().mc_attention_fwd_workspace_size(ctypes.byref(d))
    ws = _workspace(ws_n, q.device)
    check(lib().mc_attention_fwd(ctypes.byref(d), _ptr(q), _ptr(k), _ptr(v), _ptr(mask), _ptr(o), _ptr(lse),
                                 _ptr(ws), ws_n, _stream(q)))
    return o, lse


def attention_backward(q, k, v, o, lse, dout, causal=False, scale=None, mask=None):
    """(dq, dk, dv) of attention_forward; o and lse come from the forward."""
    B, H, S, D = _attn_inputs(q, k, v, mask)
    _expect(o, "o", shape=(B, S, H * D), dtype=q.dtype, device=q.device)
    _expect(dout, "dout", shape=(B, S, H * D), dtype=q.dtype, device=q.device)
    _expect(lse, "lse", shape=(B, H, S), dtype=torch.float32, device=q.device)
    if o is None or lse is None or dout is None:
        raise McError(_lib.MC_ERR_NULL, "attention backward: o, lse and dout are required")
    if scale is None:
        scale = D ** -0.5
    d = attention_desc(q, k, causal, scale)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws_n = lib().mc_attention_bwd_workspace_size(ctypes.byref(d))
    ws = _workspace(ws_n, q.device)
    check(lib().mc_attention_bwd(ctypes.byref(d), _ptr(q), _ptr(k), _ptr(v), _ptr(mask), _ptr(o), _ptr(lse),
                                 _ptr(dout), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(ws), ws_n, _stream(q)))
    return dq, dk, dv


def layer_norm_forward(x, eps, w=None, b=None, save_stats=True):
    """LayerNorm over the last dim: (y, mean, rstd). w, b [dim] in x's dtype or None."""
    rows, D = _rows_of(x, "x")
    _expect(w, "w", shape=(D,), dtype=x.dtype, device=x.device)
    _expect(b, "b", shape=(D,), dtype=x.dtype, device=x.device)
    y = torch.empty_like(x)
    mean = torch.empty(rows, dtype=torch.float32, device=x.device) if save_stats else None
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device) if save_stats else None
    check(lib().mc_layernorm_fwd(rows, D, float(eps), _dtype_code(x), _ptr(x), _ptr(w), _ptr(b), _ptr(y), _ptr(mean),
                                 _ptr(rstd), _stream(x)))
    return y, mean, rstd


def layer_norm_backward(x, dy, eps, w=None, mean=None, rstd=None, need_dw=True, need_db=True):
    """(dx, dw, db) of LayerNorm; dw / db are fp32 [D] (None when not requested)."""
    rows, D = _rows_of(x, "x")
    _expect(dy, "dy", shape=x.shape, dtype=x.dtype, device=x.device)
    _expect(w, "w", shape=(D,), dtype=x.dtype, device=x.device)
    _expect(mean, "mean", shape=(rows,), dtype=torch.float32, device=x.device)
    _expect(rstd, "rstd", shape=(rows,), dtype=torch.float32, device=x.device)
    dx = torch.empty_like(x)
    dw = torch.empty(D, dtype=torch.float32, device=x.device) if need_dw else None
    db = torch.empty(D, dtype=torch.float32, device=x.device) if need_db else None
    ws_n = lib().mc_layernorm_bwd_workspace_size(rows, D) if (need_dw or need_db) else 0
    ws = _workspace(ws_n, x.device)
    check(lib().mc_layernorm_bwd(rows, D, float(eps), _dtype_code(x), _ptr(x), _ptr(w), _ptr(mean), _ptr(rstd),
                                 _ptr(dy), _ptr(dx), _ptr(dw), _ptr(db), _ptr(ws), ws_n, _stream(x)))
    return dx, dw, db


def log_softmax_forward(x):
    rows, D = _rows_of(x, "x")
    y = torch.empty_like(x)
    check(lib().mc_log_softmax_fwd(rows, D, _dtype_code(x), _ptr(x), _ptr(y), _stream(x)))
    return y


def log_softmax_backward(y, dy):
    rows, D = _rows_of(y, "y")
    _expect(dy, "dy", shape=y.shape, dtype=y.dtype, device=y.device)
    dx = torch.empty_like(y)
    check(lib().mc_log_softmax_bwd(rows, D, _dtype_code(y), _ptr(y), _ptr(dy), _ptr(dx), _stream(y)))
    return dx


def _xent_desc(logits, ignore_index, smoothing):
    rows, V = _rows_of(logits, "logits")
    return XentDesc(rows, V, -1 if ignore_index is None else int(ignore_index), float(smoothing),
                    _dtype_code(logits))


def _targets(targets, logits):
    """uint32 targets [rows] as the kernels read them: torch.uint32, or
    torch.int32 (the same bytes for ids below 2^31); int64 ids are converted
    explicitly (a copy), so their low 32 bits are what the kernels see."""
    rows = logits.numel() // logits.shape[-1]
    if not isinstance(targets, torch.Tensor):
        raise McError(_lib.MC_ERR_NULL, "targets must be a tensor")
    if targets.dtype == torch.int64:
        targets = targets.to(torch.int32)
    if targets.dtype not in (torch.int32, torch.uint32):
        raise McError(_lib.MC_ERR_DTYPE, f"targets have dtype {targets.dtype}, expected uint32 (or int32 / int64 ids)")
    _expect(targets, "targets", device=logits.device)
    if targets.numel() != rows:
        raise McError(_lib.MC_ERR_SHAPE, f"targets have {targets.numel()} entries, expected {rows} (one per row)")
    return targets


def cross_entropy_forward(logits, targets, ignore_index=None, smoothing=0.0):
    """cross_entropy_loss (src/training/loss.rs:58-245) over logits [..., V] and
    uint32 targets [...]: (loss fp32 [1], stats fp32 [rows + 1])."""
    d = _xent_desc(logits, ignore_index, smoothing)
    targets = _targets(targets, logits)
    loss = torch.empty(1, dtype=torch.float32, device=logits.device)
    stats = torch.empty(d.rows + 1, dtype=torch.float32, device=logits.device)
    ws_n = lib().mc_cross_entropy_workspace_size(ctypes.byref(d))
    ws = _workspace(ws_n, logits.device)
    check(lib().mc_cross_entropy_fwd(ctypes.byref(d), _ptr(logits), _ptr(targets), _ptr(loss), _ptr(stats), _ptr(ws),
                                     ws_n, _stream(logits)))
    return loss, stats


def cross_entropy_backward(logits, targets, stats, dloss=None, ignore_index=None, smoothing=0.0):
    """d loss / d logits (times dloss, a fp32 [1] device tensor; default 1)."""
    d = _xent_desc(logits, ignore_index, smoothing)
    targets = _targets(targets, logits)
    _expect(stats, "stats", shape=(d.rows + 1,), dtype=torch.float32, device=logits.device)
    if stats is None:
        raise McError(_lib.MC_ERR_NULL, "stats from cross_entropy_forward are required")
    if dloss is None:
        dloss = torch.ones(1, dtype=torch.float32, device=logits.device)
    _expect(dloss, "dloss", shape=(1,), dtype=torch.float32, device=logits.device)
    dlogits = torch.empty_like(logits)
    check(lib().mc_cross_entropy_bwd(ctypes.byref(d), _ptr(logits), _ptr(targets), _ptr(stats), _ptr(dloss),
                                     _ptr(dlogits), _stream(logits)))
    return dlogits


def adamw_step(params, grads, ms, vs, steps, lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01,
               outs=None):
    """AdamW::step (src/training/optimizer.rs:227-281) for a list of fp32
    tensors in one call: m and v are updated in place; the new parameters go
    to outs (default: the params themselves, in place). steps: one step count
    per tensor (or one int for all)."""
    n = len(params)
    if isinstance(steps, int):
        steps = [steps] * n
    outs = params if outs is None else outs
    for group, name in ((params, "param"), (grads, "grad"), (ms, "m"), (vs, "v"), (outs, "param_out")):
        if len(group) != n:
            raise McError(_lib.MC_ERR_SHAPE, f"{name} list has {len(group)} entries, expected {n}")
        for t in group:
            _contig(t, name)
            if t.dtype != torch.float32:
                raise McError(_lib.MC_ERR_DTYPE, f"{name} must be float32")
    table = (AdamWTensor * max(n, 1))()
    for i in range(n):
        numel = params[i].numel()
        for t in (grads[i], ms[i], vs[i], outs[i]):
            if t.numel() != numel:
                raise McError(_lib.MC_ERR_SHAPE, f"tensor {i}: element counts differ")
        table[i] = AdamWTensor(params[i].data_ptr(), grads[i].data_ptr(), ms[i].data_ptr(), vs[i].data_ptr(),
                               outs[i].data_ptr(), numel, int(steps[i]))
    cfg = AdamWConfig(lr, beta1, beta2, eps, weight_decay)
    stream = _stream(params[0]) if n else None
    check(lib().mc_adamw_step(ctypes.byref(cfg), table, n, stream))
    return outs


def dropout_mask(seed, p, rows, rank):
    """Host-generated keep-mask (uint8 [rows, rank]) as a CPU torch tensor."""
    m = torch.empty(rows, rank, dtype=torch.uint8)
    check(lib().mc_dropout_mask(int(seed), float(p), int(rows), int(rank), ctypes.c_void_p(m.data_ptr())))
    return m
