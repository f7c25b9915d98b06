"""Incoherence processing with the randomized Hadamard transform, on gfx950.

Mirrors quipsharp/incoherence.py.  Forward (quantization time):
    W_hat = T_m (S_u W S_v) T_n,    H_hat = T_n (S_v H S_v) T_n
and the inference-time activation transforms (:86-93)
    x2 = T_n(S_v x),                y = S_u T_m(y1).
For power-of-two dimensions T is the Walsh-Hadamard transform and every
result is bit-exact with the reference.  For other dimensions the reference
switches to its randomized FFT (quipsharp/rfft.py); here both dimensions use
the Kronecker transform K_p (x) H_{2^k} instead (``KronSigns``), which keeps
the real, sign-flip-plus-orthogonal structure and the same transform protocol.
"""
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _lib
from .hadamard import hartley_matrix, is_pow2, kron_factor, rademacher


def _two_sided(X: Tensor, left: Tensor, right: Tensor) -> Tensor:
    """T_rows(left (.) X (.) right) along dim 0, then T_cols along dim 1 --
    the ``fwht(fwht(Z, dim=0), dim=1)`` order of quipsharp/incoherence.py:65-69,
    with the sign scalings fused into the first pass."""
    _lib.require_gpu(X, what="incoherence processing")
    X = X.float().contiguous()
    m, n = X.shape
    fm, fn = kron_factor(m), kron_factor(n)
    if fm is None or fn is None:
        raise ValueError(f"dims ({m}, {n}) need the form p * 2^k with odd p <= {_lib.QS_MAX_KRON}")
    Km = hartley_matrix(fm[0], X.device) if fm[0] > 1 else None
    Kn = hartley_matrix(fn[0], X.device) if fn[0] > 1 else None
    L = _lib.lib()
    s = _lib.stream_of(X)
    out = torch.empty_like(X)
    # dim 0: [outer=1][m][inner=n]
    _lib.check(L.qs_rht_f32(_lib.ptr(X), _lib.ptr(out), 1, m, n, _lib.ptr(left), _lib.ptr(right), None,
                            fm[0], _lib.ptr(Km), s))
    # dim 1: [outer=m][n][inner=1]
    _lib.check(L.qs_rht_f32(_lib.ptr(out), _lib.ptr(out), m, n, 1, None, None, None, fn[0], _lib.ptr(Kn), s))
    return out


def _two_sided_inverse(X: Tensor, left: Tensor, right: Tensor) -> Tensor:
    """(T_m X T_n) (.) left[:, None] (.) right[None, :] (quipsharp/incoherence.py:74-83)."""
    _lib.require_gpu(X, what="incoherence processing")
    X = X.float().contiguous()
    m, n = X.shape
    fm, fn = kron_factor(m), kron_factor(n)
    Km = hartley_matrix(fm[0], X.device) if fm[0] > 1 else None
    Kn = hartley_matrix(fn[0], X.device) if fn[0] > 1 else None
    L = _lib.lib()
    s = _lib.stream_of(X)
    out = torch.empty_like(X)
    _lib.check(L.qs_rht_f32(_lib.ptr(X), _lib.ptr(out), 1, m, n, None, None, None, fm[0], _lib.ptr(Km), s))
    _lib.check(L.qs_rht_f32(_lib.ptr(out), _lib.ptr(out), m, n, 1, None, None, None, fn[0], _lib.ptr(Kn), s))
    return out * left.unsqueeze(1) * right.unsqueeze(0)


def _rows(x: Tensor, pre: Tensor = None, post: Tensor = None) -> Tensor:
    """post (.) T_n(pre (.) x) along the last dim of x (..., n)."""
    _lib.require_gpu(x, pre, post, what="transform")
    n = x.shape[-1]
    f = kron_factor(n)
    if f is None:
        raise ValueError(f"length {n} is not p * 2^k with odd p <= {_lib.QS_MAX_KRON}")
    xf = x.float().reshape(-1, n).contiguous()
    out = torch.empty_like(xf)
    K = hartley_matrix(f[0], x.device) if f[0] > 1 else None
    _lib.check(_lib.lib().qs_rht_f32(_lib.ptr(xf), _lib.ptr(out), xf.shape[0], n, 1, _lib.ptr(pre), None,
                                     _lib.ptr(post), f[0], _lib.ptr(K), _lib.stream_of(xf)))
    return out.reshape(x.shape)


@dataclass
class IncoherenceSigns:
    """quipsharp/incoherence.py:29-45."""
    su: Tensor  # (m,) row signs
    sv: Tensor  # (n,) column signs

    kind = "rht"

    def transform_input(self, x: Tensor) -> Tensor:
        return transform_input(x, self.sv)

    def transform_output(self, y: Tensor) -> Tensor:
        return transform_output(y, self.su)

    def reconstruct_weight(self, what: Tensor) -> Tensor:
        return reconstruct_weight(what, self)


@dataclass
class KronSigns(IncoherenceSigns):
    """Signs of a layer processed with the Kronecker transform (non-power-of-two
    dims).  Same protocol as IncoherenceSigns; the transform is selected by
    the lengths of su and sv."""

    kind = "krht"


def _process(W: Tensor, H: Tensor, generator, cls):
    m, n = W.shape
    assert H.shape == (n, n)
    su = rademacher(m, device=W.device, dtype=torch.float32, generator=generator)
    sv = rademacher(n, device=W.device, dtype=torch.float32, generator=generator)
    what = _two_sided(W, su, sv)
    hhat = _two_sided(H, sv, sv)
    return what, hhat, cls(su=su, sv=sv)


def incoherence_process(W: Tensor, H: Tensor, generator=None):
    """Algorithm 3, IP-RHT (quipsharp/incoherence.py:48-71).  Power-of-two
    dims only (ValueError otherwise); bit-exact with the reference given the
    same signs, which are drawn in the same order (su, then sv)."""
    m, n = W.shape
    if not (is_pow2(m) and is_pow2(n)):
        raise ValueError(
            f"incoherence_process requires power-of-two dims, got ({m}, {n}); "
            "use incoherence_process_auto for other sizes")
    return _process(W, H, generator, IncoherenceSigns)


def kron_incoherence_process(W: Tensor, H: Tensor, generator=None):
    """IP-RHT with the Kronecker transform for dims n = p * 2^k (p odd, p <= 64)."""
    m, n = W.shape
    if kron_factor(m) is None or kron_factor(n) is None:
        raise ValueError(f"dims ({m}, {n}) need the form p * 2^k with odd p <= {_lib.QS_MAX_KRON}")
    return _process(W, H, generator, KronSigns)


def reconstruct_weight(what: Tensor, signs: IncoherenceSigns) -> Tensor:
    """quipsharp/incoherence.py:74-77."""
    return _two_sided_inverse(what, signs.su, signs.sv)


def reconstruct_hessian(hhat: Tensor, signs: IncoherenceSigns) -> Tensor:
    """quipsharp/incoherence.py:80-83."""
    return _two_sided_inverse(hhat, signs.sv, signs.sv)


def transform_input(x: Tensor, sv: Tensor) -> Tensor:
    """x -> T_n(S_v x) (quipsharp/incoherence.py:86-88)."""
    return _rows(x, pre=sv.float().contiguous())


def transform_output(y: Tensor, su: Tensor) -> Tensor:
    """y -> S_u T_m(y) (quipsharp/incoherence.py:91-93)."""
    return _rows(y, post=su.float().contiguous())


def linear_via_transformed(x: Tensor, what: Tensor, signs: IncoherenceSigns) -> Tensor:
    """Dense check of Algorithm 2 with the unquantized W_hat (quipsharp/incoherence.py:96-105)."""
    x2 = transform_input(x, signs.sv)
    y1 = x2 @ what.T
    return transform_output(y1, signs.su)


def incoherence_mu(W: Tensor) -> float:
    """mu = max|W| sqrt(mn) / ||W||_F (quipsharp/incoherence.py:108-112)."""
    m, n = W.shape
    return (W.abs().max() * (m * n) ** 0.5 / W.norm()).item()


def incoherence_process_auto(W: Tensor, H: Tensor, generator=None, transform: str = "auto"):
    """quipsharp/incoherence.py:115-131: the Walsh-Hadamard RHT when both dims
    are powers of two; otherwise the Kronecker RHT (where the reference uses
    its RFFT on both sides).  transform="rfft" takes the reference's branch
    for non-power-of-two dims (quipsharp_amd.rfft)."""
    m, n = W.shape
    if transform not in ("auto", "rfft"):
        raise ValueError(f"transform must be 'auto' or 'rfft', got {transform!r}")
    if is_pow2(m) and is_pow2(n):
        return incoherence_process(W, H, generator=generator)
    if transform == "rfft":
        from .rfft import rfft_incoherence_process
        return rfft_incoherence_process(W, H, generator=generator)
    return kron_incoherence_process(W, H, generator=generator)
