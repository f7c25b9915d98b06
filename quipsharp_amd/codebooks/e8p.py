"""The E8P 2-bit lattice codebook on gfx950 (quipsharp/codebooks/e8p.py).

code = [abs_idx : 8][sign bits of coordinates 0..6 : 7][shift : 1]; the sign
of coordinate 7 is the parity of the seven stored bits; shift 1 adds +1/4,
shift 0 adds -1/4.  The 256 x 8 table lives in the library's constant memory
(generated at compile time); ``build_abs_table`` returns a host copy of it.

``E8PCodebook.quantize`` runs the library's nearest-codeword search, which
reproduces the reference's greedy parity-repair search bit for bit, ties
included; ``dequantize`` runs the library's decoder.
"""
import ctypes

import torch
from torch import Tensor

from .. import _lib

CODE_DIM = 8
ABS_TABLE_SIZE = 256


def build_abs_table() -> Tensor:
    """(256, 8) fp32 table of canonical D8-hat representatives
    (quipsharp/codebooks/e8p.py:84-89), as built into the library."""
    t = torch.empty(ABS_TABLE_SIZE, CODE_DIM, dtype=torch.float32)
    _lib.check(_lib.lib().qs_e8p_abs_table(ctypes.c_void_p(t.data_ptr())))
    return t


def _same_as_builtin(abs_table: Tensor) -> bool:
    return abs_table.shape == (ABS_TABLE_SIZE, CODE_DIM) and torch.equal(
        abs_table.detach().float().cpu(), build_abs_table())


def decode_from_table(abs_idx: Tensor, sign_bits7: Tensor, shift_bit: Tensor, abs_table: Tensor) -> Tensor:
    """Decode unpacked fields against an arbitrary table
    (quipsharp/codebooks/e8p.py:92-101); elementwise tensor algebra on the
    inputs' device.  The packed-code hot path is ``E8PCodebook.dequantize``."""
    base = abs_table[abs_idx]
    parity = sign_bits7.sum(-1) % 2
    flips = torch.cat([sign_bits7, parity.unsqueeze(-1)], dim=-1)
    signed = base * (1 - 2 * flips.to(base.dtype))
    shift = (2 * shift_bit.to(base.dtype) - 1) * 0.25
    return signed + shift.unsqueeze(-1)


def pack_code(abs_idx: Tensor, sign_bits7: Tensor, shift_bit: Tensor) -> Tensor:
    """[abs_idx:8][sign_bits7:7][shift_bit:1] (quipsharp/codebooks/e8p.py:165-171)."""
    weights = torch.tensor([64, 32, 16, 8, 4, 2, 1], dtype=torch.int64, device=sign_bits7.device)
    sign_int = (sign_bits7.to(torch.int64) * weights).sum(-1)
    return (abs_idx.to(torch.int64) << 8) | (sign_int << 1) | shift_bit.to(torch.int64)


def unpack_code(code: Tensor):
    """Inverse of pack_code (quipsharp/codebooks/e8p.py:174-180)."""
    code = code.to(torch.int64)
    abs_idx = (code >> 8) & 0xFF
    shift_bit = code & 1
    shifts = torch.arange(6, -1, -1, dtype=torch.int64, device=code.device)
    sign_bits7 = ((code >> 1).unsqueeze(-1) >> shifts) & 1
    return abs_idx, sign_bits7, shift_bit


def _encode(x: Tensor, kinds, scales, in_div=1.0, out_mul=1.0):
    """Residual-VQ encode of x (..., 8) fp32 on the GPU -> (vals, codes int64 [S, ...]).
    The input is divided by ``in_div`` and the result multiplied by ``out_mul``
    inside the kernel (IEEE fp32)."""
    _lib.require_gpu(x, what="E8P encode")
    if x.shape[-1] != CODE_DIM:
        raise ValueError(f"expected last dim {CODE_DIM}, got {x.shape[-1]}")
    xf = x.float().reshape(-1, CODE_DIM).contiguous()
    nvec = xf.shape[0]
    S = len(kinds)
    vals = torch.empty_like(xf)
    codes = torch.empty(S, nvec, dtype=torch.int64, device=x.device)
    _lib.check(_lib.lib().qs_rvq_encode(
        _lib.ptr(xf), CODE_DIM, nvec, S, _lib.int_array(kinds), _lib.float_array(scales), float(in_div),
        float(out_mul), _lib.ptr(vals), CODE_DIM, _lib.ptr(codes), 8, nvec, 1, _lib.stream_of(xf)))
    return vals.reshape(x.shape[:-1] + (CODE_DIM,)), codes.reshape((S,) + tuple(x.shape[:-1]))


def _decode(codes: Tensor, kinds, scales, out_scale=1.0):
    """codes int [S, ...] -> (..., 8) fp32: sum_s Q_s(code_s) * scale_s, times out_scale."""
    _lib.require_gpu(codes, what="decode")
    S = len(kinds)
    c = codes.to(torch.int64).reshape(S, -1).contiguous()
    nvec = c.shape[1]
    out = torch.empty(nvec, CODE_DIM, dtype=torch.float32, device=codes.device)
    _lib.check(_lib.lib().qs_rvq_decode(
        _lib.ptr(c), 8, nvec, nvec, S, _lib.int_array(kinds), _lib.float_array(scales), float(out_scale),
        _lib.ptr(out), _lib.stream_of(c)))
    return out.reshape(tuple(codes.shape[1:]) + (CODE_DIM,))


def encode_to_table(x: Tensor, abs_table: Tensor):
    """Nearest E8P codeword of x (..., 8) (quipsharp/codebooks/e8p.py:131-162)
    -> (abs_idx, sign_bits7, shift_bit, vals).  The search runs in the library
    against its built-in table, which ``abs_table`` must equal."""
    if not _same_as_builtin(abs_table):
        raise NotImplementedError("encode_to_table searches the built-in E8P table only")
    vals, codes = _encode(x, [_lib.QS_STAGE_E8P], [1.0])
    abs_idx, sign_bits7, shift_bit = unpack_code(codes[0])
    return abs_idx, sign_bits7, shift_bit, vals


class E8PCodebook:
    """2-bit, 8-dimensional E8P codebook (quipsharp/codebooks/e8p.py:183-199)."""

    stage_kind = _lib.QS_STAGE_E8P

    def native_stages(self):
        """(kinds, scales) of this codebook as a residual-VQ chain."""
        return [self.stage_kind], [1.0]

    def __init__(self, device=None):
        self.abs_table = build_abs_table().to(device=device)

    def quantize(self, x: Tensor):
        """x (..., 8) -> (vals, code int64 (...))."""
        vals, codes = _encode(x, [_lib.QS_STAGE_E8P], [1.0])
        return vals, codes[0]

    def dequantize(self, code: Tensor) -> Tensor:
        return _decode(code.unsqueeze(0), [_lib.QS_STAGE_E8P], [1.0])
