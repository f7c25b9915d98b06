"""QuIP# without fine-tuning (Algorithm 1) and the quantized-linear forward
(Algorithm 2) on gfx950 -- quipsharp/quantize.py.

``linear_forward`` never materializes the dense weight: the codes are packed
once into the kernel layout and decoded on the fly inside the matrix-core
matvec, between the two randomized-Hadamard transforms.
"""
import ctypes
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _lib
from .codebooks.e8p import _decode
from .hadamard import hartley_matrix, kron_factor
from .incoherence import incoherence_process_auto
from .ldlq import block_ldl, block_ldlq, block_ldlq_native
from .rvq import RVQStage, rvq_dequantize, rvq_quantize


@dataclass
class QuantizedLayer:
    """quipsharp/quantize.py:22-28."""
    codes: Tensor  # (m, T) or (S, m, T), per-block codes
    signs: object  # IncoherenceSigns / KronSigns
    g: int
    shape: tuple
    scale: float


class RVQCodebookAdapter:
    """Residual-VQ stages behind the single-codebook protocol (quipsharp/quantize.py:31-45)."""

    def __init__(self, stages):
        self.stages = stages

    def native_stages(self):
        """(kinds, scales) when every stage is one of the library's codebooks."""
        kinds, scales = [], []
        for st in self.stages:
            nat = getattr(st.codebook, "native_stages", None)
            if nat is None:
                return None
            k, s = nat()
            if len(k) != 1 or s[0] != 1.0:
                return None
            kinds.append(k[0])
            scales.append(float(st.scale))
        return kinds, scales

    def quantize(self, x: Tensor):
        vals, codes = rvq_quantize(x, self.stages)
        return vals, torch.stack(codes, dim=0)

    def dequantize(self, code: Tensor) -> Tensor:
        return rvq_dequantize([code[i] for i in range(code.shape[0])], self.stages)


def _stages_of(codebook):
    nat = getattr(codebook, "native_stages", None)
    return nat() if nat is not None else None


def _div(x: Tensor, d: float) -> Tensor:
    """x / d with an IEEE fp32 divide (torch's GPU division by a Python float
    multiplies by a rounded reciprocal instead)."""
    xf = x.float().contiguous()
    out = torch.empty_like(xf)
    _lib.check(_lib.lib().qs_div_f32(_lib.ptr(xf), _lib.ptr(out), xf.numel(), float(d), _lib.stream_of(xf)))
    return out


def quantize_linear(W: Tensor, H: Tensor, codebook, g: int = 8, damping: float = 1e-2, generator=None,
                    codebook_scale: float = 1.0, tune_iters: int = 10, transform: str = "auto"):
    """Algorithm 1 for one linear layer (quipsharp/quantize.py:48-104) on the
    GPU.  Returns (QuantizedLayer, W_hat_q) like the reference.  ``transform``:
    "auto" (Walsh-Hadamard RHT for power-of-two dims, else the Kronecker RHT)
    or "rfft" (the reference's choice for non-power-of-two dims, for
    checkpoints that must match its format)."""
    _lib.require_gpu(W, H, what="quantize_linear")
    W = W.float()
    H = H.float()
    H = H + damping * H.diagonal().mean() * torch.eye(H.shape[0], device=H.device, dtype=H.dtype)
    what, hhat, signs = incoherence_process_auto(W, H, generator=generator, transform=transform)
    L, _ = block_ldl(hhat, g, damping=0.0)
    rms = what.double().pow(2).mean().float().sqrt().item()
    layer_scale = rms * codebook_scale
    what_scaled = _div(what, layer_scale)
    stages = _stages_of(codebook)
    if stages is not None and g == 8:
        what_q_scaled, codes = block_ldlq_native(what_scaled, L, stages[0], stages[1], H=hhat,
                                                 tune_iters=tune_iters)
        codes_stacked = codes[0] if len(stages[0]) == 1 else codes
    else:
        T = what.shape[1] // g
        blocks = [None] * T

        def quantize_fn(target, k):
            vals, code = codebook.quantize(target)
            blocks[k] = code  # keyed by block index; blocks are revisited
            return vals

        what_q_scaled = block_ldlq(what_scaled, L, g, quantize_fn, H=hhat, tune_iters=tune_iters)
        codes_stacked = torch.stack(blocks, dim=-1)
    what_q = what_q_scaled * layer_scale
    layer = QuantizedLayer(codes=codes_stacked, signs=signs, g=g, shape=tuple(W.shape), scale=layer_scale)
    return layer, what_q


def dequantize_linear(layer: QuantizedLayer, codebook) -> Tensor:
    """Dense W_hat from the codes (quipsharp/quantize.py:107-113), bit-exact."""
    m, n = layer.shape
    stages = _stages_of(codebook)
    if stages is not None:
        codes = layer.codes if layer.codes.dim() == 3 else layer.codes.unsqueeze(0)
        out = _decode(codes, stages[0], stages[1], out_scale=layer.scale)
        return out.reshape(m, n)
    T = n // layer.g
    blocks = [codebook.dequantize(layer.codes[..., k]) for k in range(T)]
    return torch.cat(blocks, dim=-1) * layer.scale


# ---------------------------------------------------------------------------
# forward
# ---------------------------------------------------------------------------
class PackedCodes:
    """Codes of one layer in the layout the forward kernels stream."""

    def __init__(self, codes: Tensor, m: int, n: int, kinds):
        _lib.require_gpu(codes, what="pack_codes")
        S = codes.shape[0] if codes.dim() == 3 else 1
        codes = codes if codes.dim() == 3 else codes.unsqueeze(0)
        if S > 2:
            raise NotImplementedError("the forward kernels take one or two residual stages")
        if kinds[0] != _lib.QS_STAGE_E8P:
            raise NotImplementedError("the first stage must be E8P")
        tiled = m % 16 == 0 and n % 256 == 0 and (S == 1 or kinds[1] == _lib.QS_STAGE_E8_1BIT)
        self.layout = _lib.QS_LAYOUT_TILED if tiled else _lib.QS_LAYOUT_ROWMAJOR
        self.m, self.n = m, n
        self.kind1 = kinds[1] if S == 2 else _lib.QS_STAGE_E8_1BIT
        T = n // 8
        lib = _lib.lib()
        stream = _lib.stream_of(codes)
        self.codes0 = torch.empty(m * T, dtype=torch.int16, device=codes.device)
        self.codes1 = None
        c0 = codes[0].contiguous()
        _lib.check(lib.qs_pack_codes(_lib.ptr(c0), c0.element_size(), m, n, _lib.QS_STAGE_E8P, self.layout,
                                     _lib.ptr(self.codes0), stream))
        if S == 2:
            c1 = codes[1].contiguous()
            if self.kind1 == _lib.QS_STAGE_E8P:
                self.codes1 = torch.empty(m * T, dtype=torch.int16, device=codes.device)
            else:
                self.codes1 = torch.empty(m * T, dtype=torch.uint8, device=codes.device)
            _lib.check(lib.qs_pack_codes(_lib.ptr(c1), c1.element_size(), m, n, self.kind1, self.layout,
                                         _lib.ptr(self.codes1), stream))

    def nbytes(self):
        return self.codes0.numel() * 2 + (0 if self.codes1 is None else self.codes1.numel() *
                                          self.codes1.element_size())


def pack_signs(s: Tensor) -> Tensor:
    """+-1 sign vector -> int32 words for the forward's packed-sign format
    (QS_SIGNS_BITS): bit i % 32 of word i // 32 set where s[i] < 0.  A 32nd of
    the fp32 bytes, which every work-group of the transforms reads."""
    flat = s.reshape(-1)
    n = flat.numel()
    nw = (n + 31) // 32
    neg = torch.zeros(nw * 32, dtype=torch.int64, device=s.device)
    neg[:n] = (flat < 0).to(torch.int64)
    w = (neg.view(nw, 32) << torch.arange(32, device=s.device)).sum(1)
    return (w - ((w >= 2 ** 31).to(torch.int64) << 32)).to(torch.int32)  # two's-complement words


def _sign_format(su: Tensor, sv: Tensor) -> bool:
    """True for packed sign bits (int32 words), False for fp32 sign vectors."""
    bits = su.dtype == torch.int32
    if bits != (sv.dtype == torch.int32):
        raise ValueError("su and sv must both be fp32 signs or both packed sign bits")
    return bits


def check_linear_args(x: Tensor, m: int, n: int, su: Tensor, sv: Tensor, bias: Tensor = None,
                      out: Tensor = None, workspace: Tensor = None) -> bool:
    """Host-side checks of one linear's tensors before their pointers go to
    the library, which reads su / sv as m / n fp32 values (or as packed sign
    words), bias as m fp32 values and writes out / workspace on x's device.
    Returns True for packed sign bits.  Raises ValueError on a tensor that
    would make the kernels read or write out of bounds or on another device."""
    dev = x.device
    bits = _sign_format(su, sv)
    for name, t, length in (("su", su, m), ("sv", sv, n)):
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, x on {dev}")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        if bits:
            if t.numel() < (length + 31) // 32:
                raise ValueError(f"{name}: {t.numel()} sign words for {length} signs")
        elif t.dtype != torch.float32 or t.numel() != length:
            raise ValueError(f"{name} must be {length} float32 signs, got {t.numel()} x {t.dtype}")
    if bias is not None:
        if bias.device != dev or bias.dtype != torch.float32 or bias.numel() != m or not bias.is_contiguous():
            raise ValueError(f"bias must be {m} contiguous float32 values on {dev}, got {bias.numel()} x "
                             f"{bias.dtype} on {bias.device}")
    if out is not None and out.device != dev:
        raise ValueError(f"out is on {out.device}, x on {dev}")
    if workspace is not None and (workspace.device != dev or not workspace.is_contiguous()
                                  or workspace.dtype != torch.uint8):
        raise ValueError(f"workspace must be a contiguous uint8 tensor on {dev}")
    return bits


def sign_bits_ok(x: Tensor, m: int, n: int) -> bool:
    """Whether the library takes packed sign bits for a forward of x at
    (m, n): both sizes on the chunk scheme of every path (multiples of 256 up
    to 12288), or a call of 1-2 rows that the one-launch kernel covers with
    its output transform in the launch (multiples of 256 up to 32768, n up to
    16384 for fp16 / fp32 activations, rows 8-byte aligned, 16-byte for
    fp32)."""
    fits = lambda d: d % 256 == 0 and d <= 12288
    if fits(m) and fits(n):
        return True
    rows = x.numel() // n if n and x.dim() else 0
    nmax = 32768 if x.dtype == torch.bfloat16 else 16384
    if not (1 <= rows <= 2 and m % 256 == 0 and m <= 32768 and n % 256 == 0 and n <= nmax):
        return False
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1:
        return True  # the forward copies it into a fresh (aligned) buffer
    return x2.data_ptr() % (16 if x2.dtype == torch.float32 else 8) == 0 and x2.stride(0) % 4 == 0


def _out_rows(out: Tensor, B: int, m: int) -> Tensor:
    """``out`` as B rows of m outputs written in place: a (B, m) view with unit
    column stride (its row stride is passed to the library), never a copy."""
    if out.shape[-1] != m or out.numel() != B * m:
        raise ValueError(f"out has shape {tuple(out.shape)}, expected (..., {m}) with {B} rows")
    y = out.reshape(B, m)
    if y.untyped_storage().data_ptr() != out.untyped_storage().data_ptr() or (B > 0 and y.stride(1) != 1):
        raise ValueError("out must be viewable as (rows, m) with unit column stride without a copy")
    return y


def _ld(y: Tensor, m: int) -> int:
    """Row stride of the (B, m) output view (any stride >= m serves one row)."""
    return y.stride(0) if y.shape[0] > 1 else max(y.stride(0), m)


def forward_packed(x: Tensor, packed: PackedCodes, su: Tensor, sv: Tensor, s0: float, s1: float,
                   layer_scale: float, bias: Tensor = None, out_dtype=None, workspace: Tensor = None,
                   out: Tensor = None, mv_events=None) -> Tensor:
    """y = su (.) T_m(layer_scale * W_hat @ T_n(sv (.) x)) + bias for x (..., n),
    computed in the library (fp32 accumulation; output in ``out_dtype``,
    default x.dtype)."""
    _lib.require_gpu(x, su, sv, bias, what="linear forward")
    m, n = packed.m, packed.n
    if x.shape[-1] != n:
        raise ValueError(f"expected last dim {n}, got {x.shape[-1]}")
    bits = check_linear_args(x, m, n, su, sv, bias, out, workspace)
    if packed.codes0.device != x.device:
        raise ValueError(f"codes are on {packed.codes0.device}, x on {x.device}")
    out_dtype = out_dtype or x.dtype
    lead = x.shape[:-1]
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    B = x2.shape[0]
    y = _out_rows(out, B, m) if out is not None else torch.empty(B, m, dtype=out_dtype, device=x.device)
    if B == 0:
        return out if out is not None else y.reshape(*lead, m)
    fm, fn = kron_factor(m), kron_factor(n)
    if fm is None or fn is None:
        raise ValueError(f"dims ({m}, {n}) need the form p * 2^k with odd p <= {_lib.QS_MAX_KRON}")
    Km = hartley_matrix(fm[0], x.device) if fm[0] > 1 else None
    Kn = hartley_matrix(fn[0], x.device) if fn[0] > 1 else None
    lib = _lib.lib()
    need = lib.qs_linear_workspace_bytes(m, n, B, packed.layout)
    if workspace is None or workspace.numel() < need:
        # zero-initialised: the first 256 bytes are the fused kernel's counter
        workspace = torch.zeros(max(need, 256), dtype=torch.uint8, device=x.device)
    _lib.check(lib.qs_linear_forward(
        _lib.ptr(x2), _lib.dtype_code(x2.dtype), x2.stride(0), B, n, m, _lib.ptr(packed.codes0),
        _lib.ptr(packed.codes1), packed.kind1, packed.layout | (_lib.QS_SIGNS_BITS if bits else 0),
        _lib.ptr(sv), _lib.ptr(su), fn[0], _lib.ptr(Kn),
        fm[0], _lib.ptr(Km), float(s0), float(s1), float(layer_scale), _lib.ptr(bias), _lib.ptr(y),
        _lib.dtype_code(y.dtype), _ld(y, m), _lib.ptr(workspace), workspace.numel(),
        None if mv_events is None else _lib._vp(mv_events[0]), None if mv_events is None else _lib._vp(mv_events[1]),
        _lib.stream_of(x2)))
    return out if out is not None else y.reshape(*lead, m)


def decode_matvec(x: Tensor, packed: PackedCodes, s0: float, s1: float, layer_scale: float,
                  out_dtype=None, workspace: Tensor = None) -> Tensor:
    """y = layer_scale * W_hat @ x with no transforms (qs_decode_matvec): the
    forward of a layer whose transforms run elsewhere (the reference's RFFT
    layers).  x (..., n) already in the transformed basis."""
    _lib.require_gpu(x, what="decode-matvec")
    m, n = packed.m, packed.n
    if x.shape[-1] != n:
        raise ValueError(f"expected last dim {n}, got {x.shape[-1]}")
    out_dtype = out_dtype or x.dtype
    lead = x.shape[:-1]
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    B = x2.shape[0]
    y = torch.empty(B, m, dtype=out_dtype, device=x.device)
    if B == 0:
        return y.reshape(*lead, m)
    lib = _lib.lib()
    need = lib.qs_linear_workspace_bytes(m, n, B, packed.layout)
    if workspace is None or workspace.numel() < need:
        workspace = torch.zeros(max(need, 256), dtype=torch.uint8, device=x.device)
    _lib.check(lib.qs_decode_matvec(
        _lib.ptr(x2), _lib.dtype_code(x2.dtype), x2.stride(0), B, n, m, _lib.ptr(packed.codes0),
        _lib.ptr(packed.codes1), packed.kind1, packed.layout, float(s0), float(s1), float(layer_scale), _lib.ptr(y),
        _lib.dtype_code(y.dtype), m, _lib.ptr(workspace), workspace.numel(), _lib.stream_of(x2)))
    return y.reshape(*lead, m)


def forward_packed_group(x: Tensor, linears, out_dtype=None, workspace: Tensor = None, outs=None,
                         mv_events=None, pre: dict = None):
    """Several linears that read the same x in one launch (qs_linear_forward_group):
    ``linears`` is a sequence of (packed, su, sv, s0, s1, layer_scale, bias);
    returns the list of outputs, each equal to ``forward_packed`` of that
    linear.  Needs the tiled layout and n a multiple of 256 (one launch at 1-2
    rows; from 3 rows with n up to 12288 one launch per stage -- input
    transforms, decode-matvecs, output transforms -- for the whole group, the
    wide GEMM one launch per linear; one forward per linear otherwise).  No
    counterpart in the reference (one linear per call there).

    ``pre`` (qs_linear_forward_group_pre): the linears read the rows a
    pre-operation makes of the bf16 ``x`` inside the same launch --
    ``{"kind": "rmsnorm", "delta": Tensor or None, "weight": Tensor, "h_out":
    Tensor or None, "eps": float}`` (input = RMSNorm(x + delta), x + delta
    written to h_out); 1-2 rows, or 3-16 on the chunk scheme (``pre_ok``),
    bit-identical to ``qs_dec_rmsnorm`` followed by the grouped forward."""
    count = len(linears)
    if not 1 <= count <= _lib.QS_MAX_GROUP:
        raise ValueError(f"1..{_lib.QS_MAX_GROUP} linears per group, got {count}")
    n = linears[0][0].n
    if x.shape[-1] != n or any(lin[0].n != n for lin in linears):
        raise ValueError("all linears of a group read the same input width")
    _lib.require_gpu(x, *[t for lin in linears for t in (lin[1], lin[2], lin[6])], what="linear forward")
    out_dtype = out_dtype or x.dtype
    lead = x.shape[:-1]
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    B = x2.shape[0]
    fn = kron_factor(n)
    if fn is None:
        raise ValueError(f"n = {n} needs the form p * 2^k with odd p <= {_lib.QS_MAX_KRON}")
    Kn = hartley_matrix(fn[0], x.device) if fn[0] > 1 else None
    jobs = (_lib.LinearJob * count)()
    ys = []
    formats = set()
    for g, (packed, su, sv, s0, s1, layer_scale, bias) in enumerate(linears):
        m = packed.m
        formats.add(check_linear_args(x, m, n, su, sv, bias, None if outs is None else outs[g], workspace))
        if packed.codes0.device != x.device:
            raise ValueError(f"linear {g}: codes are on {packed.codes0.device}, x on {x.device}")
        if len(formats) > 1:
            raise ValueError("all linears of a group pass their signs in one format (fp32 or packed bits)")
        fm = kron_factor(m)
        if fm is None:
            raise ValueError(f"m = {m} needs the form p * 2^k with odd p <= {_lib.QS_MAX_KRON}")
        Km = hartley_matrix(fm[0], x.device) if fm[0] > 1 else None
        y = _out_rows(outs[g], B, m) if outs is not None else torch.empty(B, m, dtype=out_dtype, device=x.device)
        ys.append(y)
        jobs[g] = _lib.LinearJob(packed.codes0.data_ptr(), None if packed.codes1 is None else packed.codes1.data_ptr(),
                                 m, su.data_ptr(), sv.data_ptr(), fm[0], None if Km is None else Km.data_ptr(),
                                 float(s0), float(s1), float(layer_scale),
                                 None if bias is None else bias.data_ptr(), y.data_ptr(), _ld(y, m) if B else m,
                                 1 if True in formats else 0)
        if packed.layout != _lib.QS_LAYOUT_TILED:
            raise ValueError("grouped forward needs the tiled code layout")
    if B == 0:
        return list(outs) if outs is not None else [y.reshape(*lead, y.shape[-1]) for y in ys]
    if len({y.dtype for y in ys}) != 1:
        raise ValueError("all outputs of a group share one dtype")
    lib = _lib.lib()
    ms = (ctypes.c_int64 * count)(*[lin[0].m for lin in linears])
    need = lib.qs_linear_group_workspace_bytes(n, B, count, ms)
    if workspace is None or workspace.numel() < need:
        workspace = torch.zeros(max(need, 256), dtype=torch.uint8, device=x.device)
    if pre is not None:
        op = _pre_struct(x2, pre, n)
        _lib.check(lib.qs_linear_forward_group_pre(
            _lib.ptr(x2), x2.stride(0), B, n, fn[0], _lib.ptr(Kn), count, jobs, ctypes.byref(op),
            _lib.dtype_code(ys[0].dtype), _lib.ptr(workspace), workspace.numel(), _lib.stream_of(x2)))
        return list(outs) if outs is not None else [y.reshape(*lead, y.shape[-1]) for y in ys]
    _lib.check(lib.qs_linear_forward_group(
        _lib.ptr(x2), _lib.dtype_code(x2.dtype), x2.stride(0), B, n, fn[0], _lib.ptr(Kn), count, jobs,
        _lib.dtype_code(ys[0].dtype), _lib.ptr(workspace), workspace.numel(),
        None if mv_events is None else _lib._vp(mv_events[0]), None if mv_events is None else _lib._vp(mv_events[1]),
        _lib.stream_of(x2)))
    return list(outs) if outs is not None else [y.reshape(*lead, y.shape[-1]) for y in ys]


def _rows_of(t: Tensor, n: int, B: int, what: str) -> Tensor:
    """``t`` as B bf16 rows of n with unit column stride on x's device (no copy)."""
    if t.dtype != torch.bfloat16 or t.shape[-1] != n or t.numel() != B * n:
        raise ValueError(f"{what} must be {B} bf16 rows of {n}, got {tuple(t.shape)} {t.dtype}")
    r = t.reshape(B, n)
    if r.stride(-1) != 1 or r.untyped_storage().data_ptr() != t.untyped_storage().data_ptr():
        raise ValueError(f"{what} must be viewable as ({B}, {n}) rows with unit column stride")
    return r


def pre_ok(x: Tensor, n: int, pre: dict) -> bool:
    """Whether a grouped forward of x can run ``pre`` in its launches: the
    norm, bf16 rows, 8-byte aligned; 1-2 rows with n a multiple of 256 up to
    16384 (in the one-launch kernel), or 3-16 rows with n on the multi-row
    kernels' chunk scheme -- a multiple of 256 up to 12288 whose power-of-two
    part is at least 256 -- (in the input-transform launch)
    (qs_linear_forward_group_pre)."""
    rows = x.numel() // n if n else 0
    others = [pre.get("delta"), pre.get("h_out")]
    fn = kron_factor(n) if n else None
    if 1 <= rows <= 2:
        shape_ok = n % 256 == 0 and n <= 16384
    else:
        shape_ok = 3 <= rows <= 16 and fn is not None and n % 256 == 0 and n <= 12288 and n // fn[0] >= 256
    return (pre.get("kind") == "rmsnorm" and x.dtype == torch.bfloat16 and shape_ok
            and all(t is None or (t.dtype == torch.bfloat16 and t.data_ptr() % 8 == 0) for t in others)
            and x.data_ptr() % 8 == 0 and (rows == 1 or x.reshape(-1, n).stride(0) % 4 == 0))


def _pre_struct(x2: Tensor, pre: dict, n: int):
    """The qs_preop of ``pre`` for the rows x2 (B x n bf16)."""
    B = x2.shape[0]
    dev = x2.device
    kind = pre["kind"]
    if kind == "rmsnorm":
        delta, weight, h_out = pre.get("delta"), pre["weight"], pre.get("h_out")
        if weight.dtype != torch.bfloat16 or weight.numel() != n or not weight.is_contiguous():
            raise ValueError(f"norm weight must be {n} contiguous bf16 values")
        _lib.require_gpu(weight, delta, h_out, what="rmsnorm pre-operation")
        d = _rows_of(delta, n, B, "delta") if delta is not None else None
        o = _rows_of(h_out, n, B, "h_out") if h_out is not None else None
        for t in (weight, d, o):
            if t is not None and t.device != dev:
                raise ValueError(f"pre-operation tensors must be on {dev}")
        return _lib.PreOp(_lib.QS_PREOP_RMSNORM, _lib.ptr(d), d.stride(0) if d is not None and B > 1 else n,
                          _lib.ptr(weight), _lib.ptr(o), o.stride(0) if o is not None and B > 1 else n,
                          float(pre.get("eps", 1e-6)))
    raise ValueError(f"unknown pre-operation {kind!r}")


def _forward_params(codebook, num_stages):
    stages = _stages_of(codebook)
    if stages is None:
        raise NotImplementedError("linear_forward decodes the library's codebooks (E8P, E8 1-bit residual VQ)")
    kinds, scales = stages
    if len(kinds) != num_stages:
        raise ValueError(f"codebook has {len(kinds)} stages, codes have {num_stages}")
    s0 = scales[0]
    s1 = scales[1] if len(scales) > 1 else 0.0
    return kinds, s0, s1


def linear_forward(x: Tensor, layer: QuantizedLayer, codebook) -> Tensor:
    """Algorithm 2 (quipsharp/quantize.py:116-124) with the fused kernels; x
    (..., n) -> (..., m) in x.dtype.  The packed codes are cached on ``layer``."""
    m, n = layer.shape
    S = layer.codes.shape[0] if layer.codes.dim() == 3 else 1
    kinds, s0, s1 = _forward_params(codebook, S)
    packed = getattr(layer, "_packed", None)
    if packed is None or packed[0] is not layer.codes:
        packed = (layer.codes, PackedCodes(layer.codes, m, n, kinds))
        layer._packed = packed
    signs = layer.signs
    if getattr(signs, "kind", None) == "rfft":
        # the reference's RFFT layers: FFT transforms (hipFFT) around the decode-matvec
        x2 = signs.transform_input(x.float())
        return signs.transform_output(decode_matvec(x2, packed[1], s0, s1, layer.scale, out_dtype=torch.float32))
    if not hasattr(signs, "su"):
        raise NotImplementedError("linear_forward supports Hadamard, Kronecker and RFFT transforms")
    return forward_packed(x, packed[1], signs.su.float().contiguous(), signs.sv.float().contiguous(), s0, s1,
                          layer.scale)
