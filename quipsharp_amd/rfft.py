"""Randomized-FFT incoherence (quipsharp/rfft.py), kept so that checkpoints
quantized by the reference with its RFFT transform (every layer with a
non-power-of-two dimension) load and run here.

The transform is the reference's: reshape n reals into n/2 complex numbers,
multiply by a unit-modulus phase, unitary DFT, reshape back (enter); inverse
DFT, conjugate phase (exit).  The DFTs run in hipFFT on the GPU through
``torch.fft``; the quantized forward between them is the library's
decode-matvec (``qs_decode_matvec``).  New quantizations here use the
Kronecker RHT instead (``incoherence.kron_incoherence_process``).
"""
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _lib


def random_phase(n_half: int, device=None, generator=None) -> Tensor:
    """quipsharp/rfft.py:31-34: uniform unit-modulus complex vector of length
    n_half.  The angles are drawn on the generator's device (the CPU default
    generator when none is given), as ``hadamard.rademacher`` does, so seeded
    draws match the reference's CPU run; the result moves to ``device``."""
    gdev = generator.device if generator is not None else torch.device("cpu")
    theta = torch.rand(n_half, device=gdev, generator=generator) * (2 * torch.pi)
    ph = torch.polar(torch.ones_like(theta), theta)
    return ph.to(device) if device is not None else ph


def _enter(x: Tensor, phase: Tensor) -> Tensor:
    n = x.shape[-1]
    assert n == 2 * phase.shape[-1], f"{phase.shape[-1]} phases pair {2 * phase.shape[-1]} values per row; the rows have {n}"
    shape = x.shape
    xc = torch.view_as_complex(x.reshape(*shape[:-1], n // 2, 2).contiguous())
    return torch.view_as_real(torch.fft.fft(xc * phase, norm="ortho")).reshape(shape)


def _exit(y: Tensor, phase: Tensor) -> Tensor:
    n = y.shape[-1]
    assert n == 2 * phase.shape[-1], f"{phase.shape[-1]} phases pair {2 * phase.shape[-1]} values per row; the rows have {n}"
    shape = y.shape
    yc = torch.view_as_complex(y.reshape(*shape[:-1], n // 2, 2).contiguous())
    return torch.view_as_real(torch.fft.ifft(yc, norm="ortho") * torch.conj(phase)).reshape(shape)


def to_transformed_space(x: Tensor, phase: Tensor, dim: int = -1) -> Tensor:
    """quipsharp/rfft.py:37-48: phase, then unitary FFT, along ``dim``."""
    _lib.require_gpu(x, phase, what="rfft transform")
    return _enter(x.movedim(dim, -1), phase).movedim(-1, dim)


def from_transformed_space(y: Tensor, phase: Tensor, dim: int = -1) -> Tensor:
    """quipsharp/rfft.py:51-60: unitary inverse FFT, then conjugate phase."""
    _lib.require_gpu(y, phase, what="rfft transform")
    return _exit(y.movedim(dim, -1), phase).movedim(-1, dim)


@dataclass
class RFFTPhases:
    """quipsharp/rfft.py:63-77."""
    phase_u: Tensor  # (m // 2,) complex64
    phase_v: Tensor  # (n // 2,) complex64
    kind = "rfft"

    def transform_input(self, x: Tensor) -> Tensor:
        return to_transformed_space(x, self.phase_v, dim=-1)

    def transform_output(self, y: Tensor) -> Tensor:
        return from_transformed_space(y, self.phase_u, dim=-1)

    def reconstruct_weight(self, what: Tensor) -> Tensor:
        return reconstruct_weight(what, self)


def rfft_incoherence_process(W: Tensor, H: Tensor, generator=None):
    """quipsharp/rfft.py:80-95 (Algorithm 4): W_hat, H_hat and the phases.
    Phase draw order u then v, as the reference."""
    m, n = W.shape
    assert m % 2 == 0 and n % 2 == 0, f"the FFT pairs neighbouring entries: {m} x {n} has an odd side"
    assert H.shape == (n, n), f"H is {tuple(H.shape)}, W has {n} columns"
    phase_u = random_phase(m // 2, device=W.device, generator=generator)
    phase_v = random_phase(n // 2, device=W.device, generator=generator)
    what = to_transformed_space(to_transformed_space(W, phase_u, dim=0), phase_v, dim=1)
    hhat = to_transformed_space(to_transformed_space(H, phase_v, dim=0), phase_v, dim=1)
    return what, hhat, RFFTPhases(phase_u=phase_u, phase_v=phase_v)


def reconstruct_weight(what: Tensor, phases: RFFTPhases) -> Tensor:
    """quipsharp/rfft.py:98-101."""
    return from_transformed_space(from_transformed_space(what, phases.phase_v, dim=1), phases.phase_u, dim=0)


def reconstruct_hessian(hhat: Tensor, phases: RFFTPhases) -> Tensor:
    """quipsharp/rfft.py:104-107."""
    return from_transformed_space(from_transformed_space(hhat, phases.phase_v, dim=1), phases.phase_v, dim=0)
