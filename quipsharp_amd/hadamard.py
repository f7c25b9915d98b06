"""Walsh-Hadamard transform and randomized-Hadamard building blocks on gfx950.

Mirrors quipsharp/hadamard.py (``is_pow2``, ``next_pow2``, ``fwht``,
``rademacher``) and adds the Kronecker transform used for dimensions that are
not powers of two: n = p * 2^k with p odd is transformed by K_p (x) H_{2^k},
K_p the normalized discrete Hartley matrix (orthogonal, symmetric, K_p^2 = I),
so the transform stays its own inverse like H_n.
"""
import math

import torch
from torch import Tensor

from . import _lib


def is_pow2(n: int) -> bool:
    """quipsharp/hadamard.py:9-10."""
    return n > 0 and (n & (n - 1)) == 0


def next_pow2(n: int) -> int:
    """quipsharp/hadamard.py:13-14."""
    return 1 << (n - 1).bit_length()


def kron_factor(n: int):
    """(p, L) with n = p * L, L a power of two and p odd, or None if p exceeds
    the largest odd factor the kernels accept."""
    if n <= 0:
        return None
    L = n & -n
    p = n // L
    if p > _lib.QS_MAX_KRON:
        return None
    return p, L


_KRON_CACHE = {}


def hartley_matrix(p: int, device=None) -> Tensor:
    """Normalized discrete Hartley matrix cas(2 pi a b / p) / sqrt(p), fp32.
    Symmetric and orthogonal, hence an involution."""
    key = (p, str(device))
    K = _KRON_CACHE.get(key)
    if K is None:
        a = torch.arange(p, dtype=torch.int64)
        ab = (a[:, None] * a[None, :]) % p
        ang = ab.to(torch.float64) * (2.0 * math.pi / p)
        K = ((torch.cos(ang) + torch.sin(ang)) / math.sqrt(p)).to(torch.float32).contiguous()
        K = K.to(device)
        _KRON_CACHE[key] = K
    return K


def rht(x: Tensor, dim: int = -1, pre: Tensor = None, post: Tensor = None) -> Tensor:
    """post (.) T_n(pre (.) x) along ``dim`` (fp32, GPU).  T_n is the
    orthonormal Walsh-Hadamard transform for power-of-two n and K_p (x) H_L
    otherwise.  ``pre``/``post`` are length-n vectors (e.g. the +-1 signs)."""
    _lib.require_gpu(x, pre, post, what="rht")
    dim = dim % x.dim()
    n = x.shape[dim]
    f = kron_factor(n)
    if f is None:
        raise ValueError(f"rht needs n = p * 2^k with odd p <= {_lib.QS_MAX_KRON}, got {n}")
    p, _ = f
    orig_dtype = x.dtype
    xf = x.float().contiguous()
    outer = math.prod(xf.shape[:dim])
    inner = math.prod(xf.shape[dim + 1:])
    out = torch.empty_like(xf)
    K = hartley_matrix(p, x.device) if p > 1 else None
    pre = None if pre is None else pre.float().contiguous()
    post = None if post is None else post.float().contiguous()
    _lib.check(_lib.lib().qs_rht_f32(_lib.ptr(xf), _lib.ptr(out), outer, n, inner, _lib.ptr(pre), None,
                                     _lib.ptr(post), p, _lib.ptr(K), _lib.stream_of(xf)))
    return out if orig_dtype == torch.float32 else out.to(orig_dtype)


def fwht(x: Tensor, dim: int = -1) -> Tensor:
    """Orthonormal fast Walsh-Hadamard transform along ``dim``
    (quipsharp/hadamard.py:17-40), bit-exact with the reference's fp32 stage
    order.  Requires a power-of-two length (ValueError otherwise)."""
    n = x.shape[dim]
    if not is_pow2(n):
        raise ValueError(f"fwht requires a power-of-two size along dim, got {n}")
    return rht(x, dim)


def rademacher(n: int, device=None, dtype=torch.float32, generator=None) -> Tensor:
    """Uniform +-1 vector (quipsharp/hadamard.py:43-46).  The bits are drawn
    on the generator's device -- the CPU generator (global CPU RNG when
    ``generator`` is None) unless a device generator is given -- then moved
    to ``device``, so a seeded run draws the same signs as the reference's
    CPU run."""
    gdev = generator.device if generator is not None else torch.device("cpu")
    bits = torch.randint(0, 2, (n,), device=gdev, generator=generator)
    return (bits.to(dtype) * 2 - 1).to(device)
