"""Loader for libquipsharp_hip.so (the C ABI declared in include/quipsharp_hip.h).

The library is mandatory: every compute entry point of quipsharp_amd goes
through it, and there is no CPU or pure-PyTorch substitute.  A missing or
unloadable library raises immediately.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libquipsharp_hip.so")

QS_OK = 0
QS_STAGE_E8P = 0
QS_STAGE_E8_1BIT = 1
QS_DTYPE_F32, QS_DTYPE_F16, QS_DTYPE_BF16 = 0, 1, 2
QS_LAYOUT_ROWMAJOR, QS_LAYOUT_TILED = 0, 1
QS_SIGNS_BITS = 0x100  # layout flag: su / sv are packed sign bits
QS_MAX_STAGES = 4
QS_MAX_KRON = 64
QS_MAX_GROUP = 4
QS_NOALLOC_SCRATCH_BYTES = 32 << 20
QS_PREOP_RMSNORM, QS_PREOP_SILU_MUL = 1, 2

_vp = ctypes.c_void_p


class LinearJob(ctypes.Structure):
    """qs_linear_job (include/quipsharp_hip.h)."""
    _fields_ = [("codes0", ctypes.c_void_p), ("codes1", ctypes.c_void_p), ("m", ctypes.c_int64),
                ("su", ctypes.c_void_p), ("sv", ctypes.c_void_p), ("kron_pm", ctypes.c_int),
                ("kron_m", ctypes.c_void_p), ("s0", ctypes.c_float), ("s1", ctypes.c_float),
                ("layer_scale", ctypes.c_float), ("bias", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("ldy", ctypes.c_int64), ("sign_bits", ctypes.c_int)]



class PreOp(ctypes.Structure):
    """qs_preop (include/quipsharp_hip.h)."""
    _fields_ = [("kind", ctypes.c_int), ("x2", ctypes.c_void_p), ("ldx2", ctypes.c_int64),
                ("weight", ctypes.c_void_p), ("h_out", ctypes.c_void_p), ("ldo", ctypes.c_int64),
                ("eps", ctypes.c_float)]

_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_int_p = ctypes.POINTER(ctypes.c_int)
_f32_p = ctypes.POINTER(ctypes.c_float)

_SIGNATURES = {
    "qs_last_error": ([], ctypes.c_char_p),
    "qs_abi_version": ([], _int),
    "qs_e8p_abs_table": ([_vp], _int),
    "qs_e81_table": ([_vp], _int),
    "qs_rvq_encode": ([_vp, _i64, _i64, _int, _int_p, _f32_p, _f32, _f32, _vp, _i64, _vp, _int, _i64, _i64,
                       _vp], _int),
    "qs_div_f32": ([_vp, _vp, _i64, _f32, _vp], _int),
    "qs_rvq_decode": ([_vp, _int, _i64, _i64, _int, _int_p, _f32_p, _f32, _vp, _vp], _int),
    "qs_ldlq_step": ([_vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _int, _int_p, _f32_p,
                      _vp, _int, _i64, _i64, _vp], _int),
    "qs_ldlq_chunk": ([_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _int, _int, _i64, _int, _int_p,
                       _f32_p, _vp, _int, _i64, _i64, _vp], _int),
    "qs_rht_f32": ([_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _int, _vp, _vp], _int),
    "qs_pack_codes": ([_vp, _int, _i64, _i64, _int, _int, _vp, _vp], _int),
    "qs_linear_workspace_bytes": ([_i64, _i64, _i64, _int], ctypes.c_size_t),
    "qs_linear_forward": ([_vp, _int, _i64, _i64, _i64, _i64, _vp, _vp, _int, _int, _vp, _vp, _int, _vp,
                           _int, _vp, _f32, _f32, _f32, _vp, _vp, _int, _i64, _vp, ctypes.c_size_t, _vp, _vp,
                           _vp], _int),
    "qs_linear_forward_noalloc": ([_vp, _int, _i64, _i64, _i64, _i64, _vp, _vp, _int, _int, _vp, _vp, _int, _vp,
                                   _int, _vp, _f32, _f32, _f32, _vp, _vp, _int, _i64, _vp], _int),
    "qs_decode_matvec": ([_vp, _int, _i64, _i64, _i64, _i64, _vp, _vp, _int, _int, _f32, _f32, _f32, _vp, _int,
                          _i64, _vp, ctypes.c_size_t, _vp], _int),
    "qs_linear_group_workspace_bytes": ([_i64, _i64, _int, ctypes.POINTER(ctypes.c_int64)], ctypes.c_size_t),
    "qs_linear_forward_group": ([_vp, _int, _i64, _i64, _i64, _int, _vp, _int, ctypes.POINTER(LinearJob), _int,
                                 _vp, ctypes.c_size_t, _vp, _vp, _vp], _int),
    "qs_linear_forward_group_pre": ([_vp, _i64, _i64, _i64, _int, _vp, _int, ctypes.POINTER(LinearJob),
                                     ctypes.POINTER(PreOp), _int, _vp, ctypes.c_size_t, _vp], _int),
    "qs_busy_wait": ([_i64, _vp], _int),
    "qs_dec_rmsnorm": ([_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _vp], _int),
    "qs_dec_qk_norm_rope": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _int, _int, _int, _i64,
                             _f32, _vp], _int),
    "qs_dec_attention_workspace_bytes": ([_i64, _int, _i64], _i64),
    "qs_dec_attention": ([_vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _int, _int, _int, _i64, _f32, _vp], _int),
    "qs_dec_attention_rope": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _int,
                               _int, _int, _i64, _f32, _f32, _vp], _int),
    "qs_dec_silu_mul": ([_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp], _int),
}

EXPORTED = tuple(_SIGNATURES)

_lib = None


class QuipHipError(RuntimeError):
    """An entry point of libquipsharp_hip.so returned an error."""


def lib():
    """The loaded library (loaded on first use, after torch)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m quipsharp_amd.build` "
                "(quipsharp_amd has no fallback implementation)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def check(rc):
    if rc != QS_OK:
        raise QuipHipError(lib().qs_last_error().decode(errors="replace") or f"error {rc}")


def ptr(t):
    return None if t is None else _vp(t.data_ptr())


def stream_of(t):
    return _vp(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*tensors, what="quipsharp_amd"):
    """Every compute path runs on the GPU; CPU tensors are rejected, not emulated."""
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(f"{what} runs on the GPU (MI355X / gfx950); got a tensor on {t.device}")


def int_array(vals):
    arr = (ctypes.c_int * len(vals))(*vals)
    return arr


def float_array(vals):
    return (ctypes.c_float * len(vals))(*vals)


def dtype_code(dt):
    if dt == torch.float32:
        return QS_DTYPE_F32
    if dt == torch.float16:
        return QS_DTYPE_F16
    if dt == torch.bfloat16:
        return QS_DTYPE_BF16
    raise TypeError(f"unsupported dtype {dt} (float32, float16 or bfloat16)")
