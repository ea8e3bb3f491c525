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
from ._lib import AdamWConfig, AdamWTensor, AttnDesc, LoraDesc, McError, XentDesc, check, lib

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


def _workspace(nbytes, device):
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def lora_desc(tokens, in_features, out_features, rank, scale, dropout_p=0.0, dtype=torch.bfloat16):
    return LoraDesc(tokens, in_features, out_features, rank, scale, dropout_p, _DTYPES[dtype])


def lora_forward(x, A, B, scale, W=None, bias=None, mask=None, dropout_p=0.0, save_hidden=True):
    """y = x.W^T + bias + scale*((x.A) (.) mask/(1-p)).B ; returns (y, h_save)."""
    _contig(x, "x"), _contig(W, "W"), _contig(A, "A"), _contig(B, "B")
    K = x.shape[-1]
    T = x.numel() // K
    r, N = B.shape
    d = LoraDesc(T, K, N, r, float(scale), float(dropout_p), _dtype_code(x))
    y = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=x.device)
    h = torch.empty(r, T, dtype=torch.float32, device=x.device) if save_hidden else None
    ws_n = lib().mc_lora_fwd_workspace_size(ctypes.byref(d))  # 0 for an invalid descriptor
    ws = _workspace(ws_n, x.device)
    check(lib().mc_lora_fwd(ctypes.byref(d), _ptr(x), _ptr(W), _ptr(bias), _ptr(A), _ptr(B), _ptr(mask),
                            _ptr(y), _ptr(h), _ptr(ws), ws_n, _stream(x)))
    return y, h


def lora_backward(x, A, B, dY, scale, W=None, mask=None, dropout_p=0.0, h_save=None,
                  need_dx=True, need_dA=True, need_dB=True):
    """(dX, dA, dB) with W frozen; entries not requested are None."""
    K = A.shape[0]
    r, N = B.shape
    T = dY.numel() // N
    d = LoraDesc(T, K, N, r, float(scale), float(dropout_p), _dtype_code(dY))
    dX = torch.empty(*dY.shape[:-1], K, dtype=dY.dtype, device=dY.device) if need_dx else None
    dA = torch.empty(K, r, dtype=torch.float32, device=dY.device) if need_dA else None
    dB = torch.empty(r, N, dtype=torch.float32, device=dY.device) if need_dB else None
    ws_n = lib().mc_lora_bwd_workspace_size(ctypes.byref(d))  # 0 for an invalid descriptor
    ws = _workspace(ws_n, dY.device)
    check(lib().mc_lora_bwd(ctypes.byref(d), _ptr(x), _ptr(W), _ptr(A), _ptr(B), _ptr(mask), _ptr(h_save),
                            _ptr(dY), _ptr(dX), _ptr(dA), _ptr(dB), _ptr(ws), ws_n, _stream(dY)))
    return dX, dA, dB


def rms_norm_forward(x, eps, w=None, save_rstd=True):
    D = x.shape[-1]
    rows = x.numel() // D if D else 0
    y = torch.empty_like(x)
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device) if save_rstd else None
    check(lib().mc_rmsnorm_fwd(rows, D, float(eps), _dtype_code(x), _ptr(x), _ptr(w), _ptr(y), _ptr(rstd),
                               _stream(x)))
    return y, rstd


def rms_norm_backward(x, dy, eps, w=None, rstd=None, need_dw=True):
    D = x.shape[-1]
    rows = x.numel() // D if D else 0
    dx = torch.empty_like(x)
    dw = torch.empty(D, dtype=torch.float32, device=x.device) if need_dw else None
    ws_n = lib().mc_rmsnorm_bwd_workspace_size(rows, D) if need_dw else 0
    ws = _workspace(ws_n, x.device)
    check(lib().mc_rmsnorm_bwd(rows, D, float(eps), _dtype_code(x), _ptr(x), _ptr(w), _ptr(rstd), _ptr(dy),
                               _ptr(dx), _ptr(dw), _ptr(ws), ws_n, _stream(x)))
    return dx, dw


def softmax_forward(s, causal_rows=0):
    D = s.shape[-1]
    rows = s.numel() // D if D else 0
    p = torch.empty_like(s)
    check(lib().mc_softmax_fwd(rows, D, int(causal_rows), _dtype_code(s), _ptr(s), _ptr(p), _stream(s)))
    return p


def softmax_backward(p, dp, causal_rows=0):
    D = p.shape[-1]
    rows = p.numel() // D if D else 0
    ds = torch.empty_like(p)
    check(lib().mc_softmax_bwd(rows, D, int(causal_rows), _dtype_code(p), _ptr(p), _ptr(dp), _ptr(ds),
                               _stream(p)))
    return ds


def attention_desc(q, k, causal, scale):
    B, H, S, D = q.shape
    return AttnDesc(B, S, H, k.shape[1], D, int(bool(causal)), float(scale), _dtype_code(q))


def attention_forward(q, k, v, causal=False, scale=None, mask=None, save_lse=True):
    """Attention core of Attention::forward (src/models/transformer.rs:258-283):
    q [B, H, S, D], k, v [B, Hkv, S, D] -> (o [B, S, H*D], lse [B, H, S])."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (mask, "mask")):
        _contig(t, n)
    B, H, S, D = q.shape
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
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (o, "o"), (lse, "lse"), (dout, "dout"), (mask, "mask")):
        _contig(t, n)
    D = q.shape[-1]
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
    """LayerNorm over the last dim: (y, mean, rstd)."""
    D = x.shape[-1]
    rows = x.numel() // D
    y = torch.empty_like(x)
    mean = torch.empty(rows, dtype=torch.float32, device=x.device) if save_stats else None
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device) if save_stats else None
    check(lib().mc_layernorm_fwd(rows, D, float(eps), _dtype_code(x), _ptr(x), _ptr(w), _ptr(b), _ptr(y), _ptr(mean),
                                 _ptr(rstd), _stream(x)))
    return y, mean, rstd


def layer_norm_backward(x, dy, eps, w=None, mean=None, rstd=None, need_dw=True, need_db=True):
    """(dx, dw, db) of LayerNorm; dw / db are fp32 [D] (None when not requested)."""
    D = x.shape[-1]
    rows = x.numel() // D
    dx = torch.empty_like(x)
    dw = torch.empty(D, dtype=torch.float32, device=x.device) if need_dw else None
    db = torch.empty(D, dtype=torch.float32, device=x.device) if need_db else None
    ws_n = lib().mc_layernorm_bwd_workspace_size(rows, D) if (need_dw or need_db) else 0
    ws = _workspace(ws_n, x.device)
    check(lib().mc_layernorm_bwd(rows, D, float(eps), _dtype_code(x), _ptr(x), _ptr(w), _ptr(mean), _ptr(rstd),
                                 _ptr(dy), _ptr(dx), _ptr(dw), _ptr(db), _ptr(ws), ws_n, _stream(x)))
    return dx, dw, db


def log_softmax_forward(x):
    D = x.shape[-1]
    y = torch.empty_like(x)
    check(lib().mc_log_softmax_fwd(x.numel() // D, D, _dtype_code(x), _ptr(x), _ptr(y), _stream(x)))
    return y


def log_softmax_backward(y, dy):
    D = y.shape[-1]
    dx = torch.empty_like(y)
    check(lib().mc_log_softmax_bwd(y.numel() // D, D, _dtype_code(y), _ptr(y), _ptr(dy), _ptr(dx), _stream(y)))
    return dx


def _xent_desc(logits, ignore_index, smoothing):
    V = logits.shape[-1]
    return XentDesc(logits.numel() // V, V, -1 if ignore_index is None else int(ignore_index), float(smoothing),
                    _dtype_code(logits))


def cross_entropy_forward(logits, targets, ignore_index=None, smoothing=0.0):
    """cross_entropy_loss (src/training/loss.rs:58-245) over logits [..., V] and
    uint32 targets [...]: (loss fp32 [1], stats fp32 [rows + 1])."""
    _contig(logits, "logits"), _contig(targets, "targets")
    d = _xent_desc(logits, ignore_index, smoothing)
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
    if dloss is None:
        dloss = torch.ones(1, dtype=torch.float32, device=logits.device)
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
