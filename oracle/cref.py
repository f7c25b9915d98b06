"""ctypes wrapper around the C oracle ``oracle/liboracle.so`` (test infrastructure).

Each wrapper names the reference routine it restates; the C source carries the
file:line citations.  Arrays are numpy, contiguous, C order.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64


def build():
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.qso_e8p_abs_table.argtypes = [_f32p]
        L.qso_e8p_abs_table.restype = ctypes.c_int
        L.qso_e81_table.argtypes = [_f32p]
        L.qso_e81_table.restype = ctypes.c_int
        L.qso_e8p_decode.argtypes = [_i64p, _i64, _f32p, _f32p]
        L.qso_e8p_encode.argtypes = [_f32p, _i64, _f32p, _i64p, _f32p]
        L.qso_e8p_bruteforce_d2.argtypes = [_f32p, _i64, _f32p, _f64p]
        L.qso_e81_encode.argtypes = [_f32p, _i64, _f32p, _i64p, _f32p]
        L.qso_rvq_encode.argtypes = [_f32p, _i64, ctypes.c_int, _i32p, _f32p, _f32p, _f32p, _i64p, _f32p]
        L.qso_rvq_decode.argtypes = [_i64p, _i64, ctypes.c_int, _i32p, _f32p, ctypes.c_float, _f32p, _f32p, _f32p]
        L.qso_fwht.argtypes = [_f32p, _i64, _i64, _i64]
        _lib = L
    return _lib


def _vec8(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.shape[-1] == 8
    return x.reshape(-1, 8), x.shape[:-1]


def e8p_abs_table():
    """quipsharp/codebooks/e8p.py:84-89 build_abs_table -> (256, 8) fp32."""
    t = np.zeros((256, 8), np.float32)
    n = lib().qso_e8p_abs_table(t)
    assert n == 227
    return t


def e81_table():
    """quipsharp/codebooks/e8_1bit.py:66-70 build_table -> (256, 8) fp32."""
    t = np.zeros((256, 8), np.float32)
    n = lib().qso_e81_table(t)
    assert n == 256
    return t


_E8P = None
_E81 = None


def _tables():
    global _E8P, _E81
    if _E8P is None:
        _E8P, _E81 = e8p_abs_table(), e81_table()
    return _E8P, _E81


def e8p_decode(codes):
    """quipsharp/codebooks/e8p.py:197-199 E8PCodebook.dequantize."""
    c = np.ascontiguousarray(codes, dtype=np.int64)
    out = np.zeros(c.shape + (8,), np.float32)
    lib().qso_e8p_decode(c.reshape(-1), c.size, _tables()[0], out.reshape(-1, 8))
    return out


def e8p_encode(x):
    """quipsharp/codebooks/e8p.py:190-195 E8PCodebook.quantize -> (vals, code int64)."""
    xv, shp = _vec8(x)
    codes = np.zeros(xv.shape[0], np.int64)
    vals = np.zeros_like(xv)
    lib().qso_e8p_encode(xv, xv.shape[0], _tables()[0], codes, vals)
    return vals.reshape(shp + (8,)), codes.reshape(shp)


def e8p_bruteforce_d2(x):
    """Minimum squared distance (fp64) to all 65,536 E8P codewords."""
    xv, shp = _vec8(x)
    out = np.zeros(xv.shape[0], np.float64)
    lib().qso_e8p_bruteforce_d2(xv, xv.shape[0], _tables()[0], out)
    return out.reshape(shp)


def e81_encode(x):
    """quipsharp/codebooks/e8_1bit.py:80-83 E8OneBitCodebook.quantize -> (vals, idx)."""
    xv, shp = _vec8(x)
    idx = np.zeros(xv.shape[0], np.int64)
    vals = np.zeros_like(xv)
    lib().qso_e81_encode(xv, xv.shape[0], _tables()[1], idx, vals)
    return vals.reshape(shp + (8,)), idx.reshape(shp)


E8P, E81 = 0, 1


def rvq_encode(x, kinds, scales):
    """quipsharp/rvq.py:69-80 rvq_quantize -> (total vals, codes [S, ...])."""
    xv, shp = _vec8(x)
    k = np.asarray(kinds, np.int32)
    s = np.asarray(scales, np.float32)
    codes = np.zeros((len(k), xv.shape[0]), np.int64)
    tot = np.zeros_like(xv)
    e8p, e81 = _tables()
    lib().qso_rvq_encode(xv, xv.shape[0], len(k), k, s, e8p, e81, codes, tot)
    return tot.reshape(shp + (8,)), codes.reshape((len(k),) + shp)


def rvq_decode(codes, kinds, scales, layer_scale=1.0):
    """quipsharp/rvq.py:83-88 followed by the ``* layer.scale`` of quantize.py:113."""
    k = np.asarray(kinds, np.int32)
    s = np.asarray(scales, np.float32)
    c = np.ascontiguousarray(codes, dtype=np.int64)
    assert c.shape[0] == len(k)
    n = c[0].size
    out = np.zeros((n, 8), np.float32)
    e8p, e81 = _tables()
    lib().qso_rvq_decode(c.reshape(len(k), -1), n, len(k), k, s, np.float32(layer_scale), e8p, e81, out)
    return out.reshape(c.shape[1:] + (8,))


def fwht(x, axis=-1):
    """quipsharp/hadamard.py:17-40 fwht(x, dim), bit-level restatement."""
    y = np.array(x, dtype=np.float32, copy=True)
    axis = axis % y.ndim
    n = y.shape[axis]
    outer = int(np.prod(y.shape[:axis], dtype=np.int64))
    inner = int(np.prod(y.shape[axis + 1:], dtype=np.int64))
    y = np.ascontiguousarray(y)
    lib().qso_fwht(y.reshape(-1), outer, n, inner)
    return y
