"""Residual vector quantization (quipsharp/rvq.py) on gfx950.

When every stage uses one of the library's codebooks (E8P, E8 1-bit), the
whole stage chain runs in one kernel: per stage Q(residual / s) with an IEEE
fp32 divide, total += q*s, residual -= q*s -- the reference's op order, so
codes and values are bit-exact.  Stages with other codebook objects fall back
to calling those objects in the same order.
"""
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _lib
from .codebooks.e8p import _decode, _encode


@dataclass
class RVQStage:
    """quipsharp/rvq.py:22-25."""
    codebook: object
    scale: float


def _native_kinds(stages):
    kinds = []
    for st in stages:
        k = getattr(st.codebook, "stage_kind", None)
        if k is None:
            return None
        kinds.append(k)
    if not 1 <= len(kinds) <= _lib.QS_MAX_STAGES:
        return None
    return kinds


def rvq_quantize(x: Tensor, stages):
    """quipsharp/rvq.py:69-80 -> (total vals, list of per-stage codes)."""
    kinds = _native_kinds(stages)
    if kinds is not None:
        vals, codes = _encode(x, kinds, [float(st.scale) for st in stages])
        return vals, [codes[i] for i in range(len(stages))]
    residual = x
    total = torch.zeros_like(x)
    codes = []
    for stage in stages:
        vals, code = stage.codebook.quantize(residual / stage.scale)
        total = total + vals * stage.scale
        residual = residual - vals * stage.scale
        codes.append(code)
    return total, codes


def rvq_dequantize(codes, stages) -> Tensor:
    """quipsharp/rvq.py:83-88."""
    kinds = _native_kinds(stages)
    if kinds is not None:
        return _decode(torch.stack([c.to(torch.int64) for c in codes]), kinds,
                       [float(st.scale) for st in stages])
    total = None
    for stage, code in zip(stages, codes):
        vals = stage.codebook.dequantize(code) * stage.scale
        total = vals if total is None else total + vals
    return total


def _sweep_scale(x: Tensor, codebook, candidates) -> float:
    """The candidate s minimizing mean ||x - s Q(x/s)||^2 (quipsharp/rvq.py:28-37);
    the first best wins ties.  For the library's codebooks x/s and Q(.)*s are
    IEEE fp32 operations inside the encode kernel (as on the reference's CPU
    path); the error is accumulated in fp64 on the GPU."""
    native = getattr(codebook, "native_stages", None)
    stages = native() if native is not None else None
    best_scale, best_mse = None, float("inf")
    for s in candidates:
        s = s.item()
        if stages is not None:
            approx, _ = _encode(x, stages[0], stages[1], in_div=s, out_mul=s)
        else:
            vals, _ = codebook.quantize(x / s)
            approx = vals * s
        mse = (x - approx).pow(2).double().mean().item()
        if mse < best_mse:
            best_mse, best_scale = mse, s
    return best_scale


def _samples(n_samples, dim, seed, device):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n_samples, dim, generator=g)
    return x.to(device) if device is not None else x


def fit_stage_scale(codebook, dim: int = 8, n_samples: int = 200_000, candidates=None, seed: int = 0,
                    device=None) -> float:
    """quipsharp/rvq.py:40-50: x ~ N(0, I) drawn on the CPU generator, sweep
    over linspace(0.5, 4, 71)."""
    if candidates is None:
        candidates = torch.linspace(0.5, 4.0, 71)
    return _sweep_scale(_samples(n_samples, dim, seed, device), codebook, candidates)


def fit_residual_stage_scale(prev_stages, codebook, dim: int = 8, n_samples: int = 200_000,
                             candidates=None, seed: int = 0, device=None) -> float:
    """quipsharp/rvq.py:53-66: sweep over linspace(0.05, 2, 79) on the
    residual left by ``prev_stages``."""
    if candidates is None:
        candidates = torch.linspace(0.05, 2.0, 79)
    x = _samples(n_samples, dim, seed, device)
    vals, _ = rvq_quantize(x, prev_stages)
    return _sweep_scale(x - vals, codebook, candidates)
