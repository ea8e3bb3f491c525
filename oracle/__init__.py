"""numpy front end of the CPU oracle (liboracle.so, built from oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker. The product path never imports
this package. See oracle.h for the reference file:line each function restates
and the checks that pin it.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# MC_ORACLE_LIB names another build of oracle.c (the sanitizer build that
# tests/test_sanitizers_cpu.py loads); the default is the optimised library.
_LIB_PATH = os.environ.get("MC_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i64 = ctypes.c_int64


def build():
    """Compile liboracle.so with the committed Makefile."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built; run `make -C oracle`")
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_philox4x32_10.argtypes = [_u32p, _u32p, _u32p]
        L.oracle_dropout_mask.argtypes = [ctypes.c_uint64, ctypes.c_float, _i64, ctypes.c_int32, _u8p]
        L.oracle_lora_fwd.argtypes = [_i64, _i64, _i64, ctypes.c_int32, ctypes.c_float, ctypes.c_float,
                                      _f32p, _f32p, _f32p, _f32p, _f32p, _u8p, _f32p, _f32p, ctypes.c_int]
        L.oracle_lora_bwd.argtypes = [_i64, _i64, _i64, ctypes.c_int32, ctypes.c_float, ctypes.c_float,
                                      _f32p, _f32p, _f32p, _f32p, _u8p, _f32p, _f32p, _f32p, _f32p,
                                      ctypes.c_int]
        L.oracle_rmsnorm_fwd.argtypes = [_i64, _i64, ctypes.c_float, _f32p, _f32p, _f32p, _f32p, ctypes.c_int]
        L.oracle_rmsnorm_bwd.argtypes = [_i64, _i64, ctypes.c_float, _f32p, _f32p, _f32p, _f32p, _f32p,
                                         ctypes.c_int]
        L.oracle_softmax_fwd.argtypes = [_i64, _i64, _i64, _f32p, _f32p, ctypes.c_int]
        L.oracle_softmax_bwd.argtypes = [_i64, _i64, _i64, _f32p, _f32p, _f32p, ctypes.c_int]
        L.oracle_round_bf16.argtypes = [_f32p, _f32p, _i64]
        _i32 = ctypes.c_int32
        L.oracle_attention_fwd.argtypes = [_i64, _i32, _i32, _i64, _i32, ctypes.c_float, ctypes.c_int,
                                           _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, ctypes.c_int]
        L.oracle_layernorm_fwd.argtypes = [_i64, _i64, ctypes.c_float, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                           ctypes.c_int]
        L.oracle_layernorm_bwd.argtypes = [_i64, _i64, ctypes.c_float, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                           ctypes.c_int]
        L.oracle_log_softmax_fwd.argtypes = [_i64, _i64, _f32p, _f32p, ctypes.c_int]
        L.oracle_log_softmax_bwd.argtypes = [_i64, _i64, _f32p, _f32p, _f32p, ctypes.c_int]
        L.oracle_cross_entropy_fwd.argtypes = [_i64, _i64, _f32p, _u32p, _i64, ctypes.c_float, _f32p,
                                               ctypes.POINTER(ctypes.c_double)]
        L.oracle_cross_entropy_fwd.restype = ctypes.c_double
        L.oracle_cross_entropy_bwd.argtypes = [_i64, _i64, _f32p, _u32p, _i64, ctypes.c_float, ctypes.c_float,
                                               _f32p]
        L.oracle_adamw_step.argtypes = [_i64, ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                        ctypes.c_float, _i64, _f32p, _f32p, _f32p, _f32p, _f32p]
        L.oracle_attention_bwd.argtypes = [_i64, _i32, _i32, _i64, _i32, ctypes.c_float, ctypes.c_int,
                                           _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                           ctypes.c_int]
        _i64p = ctypes.POINTER(ctypes.c_int64)
        L.oracle_softmax_fwd_rows.argtypes = [_i64, _i64, _i64, _i64p, _f32p, _f32p, ctypes.c_int]
        L.oracle_softmax_bwd_rows.argtypes = [_i64, _i64, _i64, _i64p, _f32p, _f32p, _f32p, ctypes.c_int]
        _lib = L
    return _lib


def _f(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f32p)


def _c32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def philox4x32_10(ctr, key):
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().oracle_philox4x32_10(c.ctypes.data_as(_u32p), k.ctypes.data_as(_u32p), out.ctypes.data_as(_u32p))
    return out


def dropout_mask(seed, p, rows, rank):
    m = np.zeros((rows, rank), dtype=np.uint8)
    lib().oracle_dropout_mask(seed, p, rows, rank, m.ctypes.data_as(_u8p))
    return m


def round_bf16(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty_like(a)
    lib().oracle_round_bf16(_f(a), _f(out), a.size)
    return out


def lora_fwd(x, A, B, scale, W=None, bias=None, mask=None, p=0.0, threads=0, return_hidden=False):
    """y[..., N] for x[..., K]; W [N, K], A [K, r], B [r, N]."""
    x = _c32(x)
    K = x.shape[-1]
    T = x.size // K if K else 0
    A, B, W, bias = _c32(A), _c32(B), _c32(W), _c32(bias)
    r, N = B.shape
    y = np.empty(x.shape[:-1] + (N,), dtype=np.float32)
    hd = np.empty((T, r), dtype=np.float32) if return_hidden else None
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
    lib().oracle_lora_fwd(T, K, N, r, scale, p, _f(x), _f(W), _f(bias), _f(A), _f(B),
                          None if m is None else m.ctypes.data_as(_u8p), _f(y), _f(hd), threads)
    return (y, hd) if return_hidden else y


def lora_bwd(x, A, B, dy, scale, W=None, mask=None, p=0.0, threads=0, need_dx=True, need_dA=True,
             need_dB=True):
    """(dx, dA, dB) of lora_fwd with W frozen (entries not requested are None)."""
    x, A, B, W, dy = _c32(x), _c32(A), _c32(B), _c32(W), _c32(dy)
    K = x.shape[-1]
    T = x.size // K if K else 0
    r, N = B.shape
    dx = np.empty_like(x) if need_dx else None
    dA = np.empty_like(A) if need_dA else None
    dB = np.empty_like(B) if need_dB else None
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
    lib().oracle_lora_bwd(T, K, N, r, scale, p, _f(x), _f(W), _f(A), _f(B),
                          None if m is None else m.ctypes.data_as(_u8p), _f(dy), _f(dx), _f(dA), _f(dB),
                          threads)
    return dx, dA, dB


def rmsnorm_fwd(x, eps, w=None, threads=0):
    x, w = _c32(x), _c32(w)
    D = x.shape[-1]
    rows = x.size // D if D else 0
    y = np.empty_like(x)
    rstd = np.empty(rows, dtype=np.float32)
    lib().oracle_rmsnorm_fwd(rows, D, eps, _f(x), _f(w), _f(y), _f(rstd), threads)
    return y, rstd


def rmsnorm_bwd(x, dy, eps, w=None, threads=0):
    x, w, dy = _c32(x), _c32(w), _c32(dy)
    D = x.shape[-1]
    rows = x.size // D if D else 0
    dx = np.empty_like(x)
    dw = np.empty(D, dtype=np.float32)
    lib().oracle_rmsnorm_bwd(rows, D, eps, _f(x), _f(w), _f(dy), _f(dx), _f(dw), threads)
    return dx, dw


def _ids(row_ids):
    ids = np.ascontiguousarray(row_ids, dtype=np.int64)
    return ids, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))


def softmax_fwd(s, causal_rows=0, threads=0, row_ids=None):
    """Softmax over the last dim; row_ids gives each row's index in the full
    tensor when s is a sample of its rows (for the causal mask)."""
    s = _c32(s)
    D = s.shape[-1]
    rows = s.size // D if D else 0
    p = np.empty_like(s)
    if row_ids is None:
        lib().oracle_softmax_fwd(rows, D, causal_rows, _f(s), _f(p), threads)
    else:
        ids, ip = _ids(row_ids)
        assert ids.size == rows
        lib().oracle_softmax_fwd_rows(rows, D, causal_rows, ip, _f(s), _f(p), threads)
    return p


def softmax_bwd(p, dp, causal_rows=0, threads=0, row_ids=None):
    p, dp = _c32(p), _c32(dp)
    D = p.shape[-1]
    rows = p.size // D if D else 0
    ds = np.empty_like(p)
    if row_ids is None:
        lib().oracle_softmax_bwd(rows, D, causal_rows, _f(p), _f(dp), _f(ds), threads)
    else:
        ids, ip = _ids(row_ids)
        assert ids.size == rows
        lib().oracle_softmax_bwd_rows(rows, D, causal_rows, ip, _f(p), _f(dp), _f(ds), threads)
    return ds


def attention_fwd(q, k, v, scale, causal=False, mask=None, threads=0):
    """(o [B, S, H*D], lse [B, H, S]) for q [B, H, S, D], k, v [B, Hkv, S, D]."""
    q, k, v, mask = _c32(q), _c32(k), _c32(v), _c32(mask)
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    o = np.empty((B, S, H * D), dtype=np.float32)
    lse = np.empty((B, H, S), dtype=np.float32)
    lib().oracle_attention_fwd(B, H, Hkv, S, D, scale, int(causal), _f(q), _f(k), _f(v), _f(mask), _f(o),
                               _f(lse), threads)
    return o, lse


def attention_bwd(q, k, v, dout, scale, causal=False, mask=None, threads=0):
    """(dq, dk, dv) of attention_fwd for dout [B, S, H*D]."""
    q, k, v, mask, dout = _c32(q), _c32(k), _c32(v), _c32(mask), _c32(dout)
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    lib().oracle_attention_bwd(B, H, Hkv, S, D, scale, int(causal), _f(q), _f(k), _f(v), _f(mask), _f(dout),
                               _f(dq), _f(dk), _f(dv), threads)
    return dq, dk, dv


def adamw_step(param, grad, m, v, step, lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01):
    """One AdamW::step: returns (param_new, m_new, v_new); the inputs are not modified."""
    p, g = _c32(param).copy(), _c32(grad)
    m, v = _c32(m).copy(), _c32(v).copy()
    out = np.empty_like(p)
    lib().oracle_adamw_step(p.size, lr, beta1, beta2, eps, weight_decay, step, _f(p), _f(g), _f(m), _f(v), _f(out))
    return out, m, v


def layernorm_fwd(x, eps, w=None, b=None, threads=0):
    """(y, mean, rstd) of LayerNorm over the last dim."""
    x, w, b = _c32(x), _c32(w), _c32(b)
    D = x.shape[-1]
    rows = x.size // D
    y = np.empty_like(x)
    mean = np.empty(rows, np.float32)
    rstd = np.empty(rows, np.float32)
    lib().oracle_layernorm_fwd(rows, D, eps, _f(x), _f(w), _f(b), _f(y), _f(mean), _f(rstd), threads)
    return y, mean, rstd


def layernorm_bwd(x, dy, eps, w=None, threads=0):
    """(dx, dw, db) of LayerNorm."""
    x, w, dy = _c32(x), _c32(w), _c32(dy)
    D = x.shape[-1]
    rows = x.size // D
    dx = np.empty_like(x)
    dw = np.empty(D, np.float32)
    db = np.empty(D, np.float32)
    lib().oracle_layernorm_bwd(rows, D, eps, _f(x), _f(w), _f(dy), _f(dx), _f(dw), _f(db), threads)
    return dx, dw, db


def log_softmax_fwd(x, threads=0):
    x = _c32(x)
    D = x.shape[-1]
    y = np.empty_like(x)
    lib().oracle_log_softmax_fwd(x.size // D, D, _f(x), _f(y), threads)
    return y


def log_softmax_bwd(y, dy, threads=0):
    y, dy = _c32(y), _c32(dy)
    D = y.shape[-1]
    dx = np.empty_like(y)
    lib().oracle_log_softmax_bwd(y.size // D, D, _f(y), _f(dy), _f(dx), threads)
    return dx


def cross_entropy_fwd(logits, targets, ignore_index=-1, smoothing=0.0):
    """(loss, lse [rows], count) for logits [rows, V] and uint32 targets [rows]."""
    x = _c32(logits)
    V = x.shape[-1]
    rows = x.size // V
    t = np.ascontiguousarray(targets, dtype=np.uint32).reshape(-1)
    assert t.size == rows
    lse = np.empty(rows, np.float32)
    cnt = ctypes.c_double()
    loss = lib().oracle_cross_entropy_fwd(rows, V, _f(x), t.ctypes.data_as(_u32p), ignore_index, smoothing, _f(lse),
                                          ctypes.byref(cnt))
    return loss, lse, cnt.value


def cross_entropy_bwd(logits, targets, ignore_index=-1, smoothing=0.0, dloss=1.0):
    x = _c32(logits)
    V = x.shape[-1]
    rows = x.size // V
    t = np.ascontiguousarray(targets, dtype=np.uint32).reshape(-1)
    d = np.empty_like(x)
    lib().oracle_cross_entropy_bwd(rows, V, _f(x), t.ctypes.data_as(_u32p), ignore_index, smoothing, dloss, _f(d))
    return d
