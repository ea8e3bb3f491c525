"""ctypes binding of libmc_hip.so, the C ABI declared in include/mc_hip.h.

The library is loaded from this package directory. There is no fallback: if
it is missing or fails to load, every entry point raises.
"""
import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmc_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "mc_hip.h")

MC_OK = 0
MC_ERR_NULL = 1
MC_ERR_SHAPE = 2
MC_ERR_DTYPE = 3
MC_ERR_LAYOUT = 4
MC_ERR_VALUE = 5
MC_ERR_WORKSPACE = 6
MC_ERR_HIP = 7

MC_F32 = 0
MC_BF16 = 1

STATUS_NAMES = {
    0: "MC_OK", 1: "MC_ERR_NULL", 2: "MC_ERR_SHAPE", 3: "MC_ERR_DTYPE", 4: "MC_ERR_LAYOUT",
    5: "MC_ERR_VALUE", 6: "MC_ERR_WORKSPACE", 7: "MC_ERR_HIP",
}


class McError(RuntimeError):
    """A non-zero mc_status, with the library's per-thread message."""

    def __init__(self, code, message):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


class LoraDesc(ctypes.Structure):
    _fields_ = [
        ("tokens", ctypes.c_int64),
        ("in_features", ctypes.c_int64),
        ("out_features", ctypes.c_int64),
        ("rank", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("dropout_p", ctypes.c_float),
        ("act_dtype", ctypes.c_int32),
    ]


class LoraProj(ctypes.Structure):
    _fields_ = [
        ("out_features", ctypes.c_int64),
        ("W", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("A", ctypes.c_void_p),
        ("B", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("Wt", ctypes.c_void_p),
    ]


MC_LORA_MAX_GROUP = 4


class AttnDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64),
        ("seq", ctypes.c_int64),
        ("heads", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


class XentDesc(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int64),
        ("vocab", ctypes.c_int64),
        ("ignore_index", ctypes.c_int64),
        ("smoothing", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


class AdamWConfig(ctypes.Structure):
    _fields_ = [
        ("learning_rate", ctypes.c_float),
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("epsilon", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
    ]


class AdamWTensor(ctypes.Structure):
    _fields_ = [
        ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("m", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("param_out", ctypes.c_void_p),
        ("numel", ctypes.c_int64),
        ("step", ctypes.c_int64),
    ]


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_dp = ctypes.POINTER(LoraDesc)
_ap = ctypes.POINTER(AttnDesc)

_SIGNATURES = {
    "mc_version": (ctypes.c_char_p, []),
    "mc_last_error": (ctypes.c_char_p, []),
    "mc_lora_fwd_workspace_size": (_sz, [_dp]),
    "mc_lora_bwd_workspace_size": (_sz, [_dp]),
    "mc_lora_fwd": (ctypes.c_int, [_dp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mc_lora_bwd": (ctypes.c_int, [_dp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mc_lora_group_fwd_workspace_size": (_sz, [_dp, ctypes.POINTER(LoraProj), _i32]),
    "mc_lora_group_bwd_workspace_size": (_sz, [_dp, ctypes.POINTER(LoraProj), _i32]),
    "mc_lora_group_fwd": (ctypes.c_int, [_dp, _vp, ctypes.POINTER(LoraProj), _i32, ctypes.POINTER(_vp),
                                         ctypes.POINTER(_vp), _vp, _sz, _vp]),
    "mc_lora_group_bwd": (ctypes.c_int, [_dp, _vp, ctypes.POINTER(LoraProj), _i32, ctypes.POINTER(_vp),
                                         ctypes.POINTER(_vp), _vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _vp,
                                         _sz, _vp]),
    "mc_transpose_bf16": (ctypes.c_int, [_i64, _i64, _vp, _vp, _vp]),
    "mc_rmsnorm_fwd": (ctypes.c_int, [_i64, _i64, _f32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "mc_rmsnorm_bwd_workspace_size": (_sz, [_i64, _i64]),
    "mc_rmsnorm_bwd": (ctypes.c_int, [_i64, _i64, _f32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mc_rmsnorm_bwd_noalloc": (ctypes.c_int, [_i64, _i64, _f32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mc_softmax_fwd": (ctypes.c_int, [_i64, _i64, _i64, _i32, _vp, _vp, _vp]),
    "mc_softmax_bwd": (ctypes.c_int, [_i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp]),
    "mc_attention_fwd_workspace_size": (_sz, [_ap]),
    "mc_attention_fwd": (ctypes.c_int, [_ap, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mc_attention_bwd_workspace_size": (_sz, [_ap]),
    "mc_attention_bwd": (ctypes.c_int, [_ap, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mc_layernorm_fwd": (ctypes.c_int, [_i64, _i64, _f32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mc_layernorm_bwd_workspace_size": (_sz, [_i64, _i64]),
    "mc_layernorm_bwd": (ctypes.c_int, [_i64, _i64, _f32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                        _vp]),
    "mc_log_softmax_fwd": (ctypes.c_int, [_i64, _i64, _i32, _vp, _vp, _vp]),
    "mc_log_softmax_bwd": (ctypes.c_int, [_i64, _i64, _i32, _vp, _vp, _vp, _vp]),
    "mc_cross_entropy_workspace_size": (_sz, [ctypes.POINTER(XentDesc)]),
    "mc_cross_entropy_fwd": (ctypes.c_int, [ctypes.POINTER(XentDesc), _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mc_cross_entropy_bwd": (ctypes.c_int, [ctypes.POINTER(XentDesc), _vp, _vp, _vp, _vp, _vp, _vp]),
    "mc_adamw_step": (ctypes.c_int, [ctypes.POINTER(AdamWConfig), ctypes.POINTER(AdamWTensor), _i32, _vp]),
    "mc_dropout_mask": (ctypes.c_int, [ctypes.c_uint64, _f32, _i64, _i32, _vp]),
    "mc_profile_enable": (ctypes.c_int, [_i32]),
    "mc_profile_collect": (ctypes.c_int, []),
    "mc_profile_read": (ctypes.c_int, [_i32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64),
                                       ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "mc_profile_reset": (ctypes.c_int, []),
}

PROFILE_KINDS = {"gemm": 0, "lowrank": 1, "rmsnorm": 2, "softmax": 3, "attention": 4, "adamw": 5, "rowops": 6}

_lib = None


def lib():
    """Load libmc_hip.so (once) and declare the C signatures."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: run __graft_entry__.build() (or make -C metal-candle_amd)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def header_symbols():
    """Names of the functions include/mc_hip.h declares."""
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mc_[a-z0-9_]+)\s*\(", text)))


def check(status):
    if status != MC_OK:
        msg = lib().mc_last_error()
        raise McError(status, msg.decode() if msg else "")


def profile_read(kind):
    """(elapsed_ms, launches, flops, bytes) accumulated for a kernel class."""
    ms, fl, by = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    n = ctypes.c_int64()
    check(lib().mc_profile_read(PROFILE_KINDS[kind], ctypes.byref(ms), ctypes.byref(n), ctypes.byref(fl),
                                ctypes.byref(by)))
    return ms.value, n.value, fl.value, by.value


def last_error():
    msg = lib().mc_last_error()
    return msg.decode() if msg else ""
