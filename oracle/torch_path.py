"""torch-CPU restatement of the reference's quantize / forward pipeline.

TEST INFRASTRUCTURE ONLY: the timed CPU baseline of bench.py and an
end-to-end check of the restatement itself (tests/test_oracle_torch_path.py).
It uses the same torch CPU tensor operations, shapes and fp32 op order as
numbersletter/quipsharp, so its cost and its results are the reference's:

  fwht                   quipsharp/hadamard.py:17-40
  rfft transforms        quipsharp/rfft.py:37-60   (non-power-of-two dims)
  E8P / E8 1-bit encode  quipsharp/codebooks/e8p.py:104-162, e8_1bit.py:80-83
  decode                 quipsharp/codebooks/e8p.py:92-101, 174-180
  block_ldl, block_ldlq  quipsharp/ldlq.py:39-141
  quantize_linear        quipsharp/quantize.py:48-104
  linear_forward         quipsharp/quantize.py:107-124 (dense dequantize loop)
"""
import numpy as np
import torch

from . import cref

_TAB = None


def tables():
    global _TAB
    if _TAB is None:
        _TAB = (torch.from_numpy(cref.e8p_abs_table()), torch.from_numpy(cref.e81_table()))
    return _TAB


def fwht(x, dim=-1):
    x = x.movedim(dim, -1)
    n = x.shape[-1]
    shape = x.shape
    y = x.reshape(-1, n).contiguous()
    h = 1
    while h < n:
        v = y.view(-1, n // (2 * h), 2, h)
        y = torch.stack((v[:, :, 0] + v[:, :, 1], v[:, :, 0] - v[:, :, 1]), dim=2).reshape(-1, n)
        h *= 2
    return (y * (n ** -0.5)).view(shape).movedim(-1, dim)


def to_rfft(x, phase):
    n = x.shape[-1]
    xc = torch.view_as_complex(x.reshape(*x.shape[:-1], n // 2, 2).contiguous())
    return torch.view_as_real(torch.fft.fft(xc * phase, norm="ortho")).reshape(x.shape)


def from_rfft(y, phase):
    n = y.shape[-1]
    yc = torch.view_as_complex(y.reshape(*y.shape[:-1], n // 2, 2).contiguous())
    return torch.view_as_real(torch.fft.ifft(yc, norm="ortho") * torch.conj(phase)).reshape(y.shape)


def e8p_encode(x):
    """Brute force over the 256 rows for both 1/4-cosets at once; returns
    (vals, codes).  Same per-element fp32 ops as the reference."""
    T = tables()[0]
    xs = torch.stack((x + 0.25, x - 0.25))             # (2, N, 8): shift bit 0 then 1
    prod = xs.unsqueeze(-2) * T                        # (2, N, 256, 8)
    flip = (prod < 0).to(torch.int64)
    odd = flip.sum(-1) % 2 == 1
    j = prod.abs().argmin(-1, keepdim=True)
    flip = flip.scatter(-1, j, flip.gather(-1, j) ^ odd.to(torch.int64).unsqueeze(-1))
    vals = T * (1 - 2 * flip)
    d2 = (xs.unsqueeze(-2) - vals).pow(2).sum(-1)      # (2, N, 256)
    r = d2.argmin(-1)                                  # (2, N)
    best = d2.gather(-1, r.unsqueeze(-1)).squeeze(-1)
    sb = (best[0] > best[1]).to(torch.int64)           # shift bit 0 wins ties
    rr = torch.where(sb == 0, r[0], r[1])
    sel = lambda t: torch.where((sb == 0)[:, None], t[0].gather(1, r[0][:, None, None].expand(-1, 1, 8)).squeeze(1),
                                t[1].gather(1, r[1][:, None, None].expand(-1, 1, 8)).squeeze(1))
    f = sel(flip)
    v = sel(vals) + torch.where(sb == 0, -0.25, 0.25).unsqueeze(-1)
    sign = (f[:, :7] * torch.tensor([64, 32, 16, 8, 4, 2, 1])).sum(-1)
    return v, (rr << 8) | (sign << 1) | sb


def e8p_decode(code):
    T = tables()[0]
    a, sh = (code >> 8) & 0xFF, code & 1
    bits = torch.stack([(code >> (7 - i)) & 1 for i in range(7)], -1)
    f = torch.cat([bits, bits.sum(-1, keepdim=True) % 2], -1)
    return T[a] * (1 - 2 * f.float()) + ((2 * sh.float() - 1) * 0.25).unsqueeze(-1)


def block_ldl(H, g):
    n = H.shape[0]
    T = n // g
    L0 = torch.linalg.cholesky(H)
    DL = torch.diagonal(L0.reshape(T, g, T, g), dim1=0, dim2=2).permute(2, 0, 1).clone()
    DL_inv = torch.linalg.inv(DL)
    L = L0.reshape(n, T, g)
    for i in range(T):
        L[:, i, :] = L[:, i, :] @ DL_inv[i]
    return L.reshape(n, n)


def quantize_steps(W, L, H, k_list, tune=False, Wq=None, targets=None):
    """Runs the reference's per-block work for the listed blocks (timing
    sample): feedback (or full-residual tune) product, then the E8P encode.
    Wq: the quantized weights so far (updated in place; zeros if None);
    targets: a list that receives each block's target."""
    m, n = W.shape
    g = 8
    Wq = torch.zeros_like(W) if Wq is None else Wq
    out = []
    dinv = None
    if tune:
        T = n // g
        dinv = torch.linalg.inv(torch.stack([H[k * g:(k + 1) * g, k * g:(k + 1) * g] for k in range(T)]))
    for k in k_list:
        ck = slice(k * g, (k + 1) * g)
        if tune:
            resid = W - Wq
            target = Wq[:, ck] + resid @ H[:, ck] @ dinv[k]
        else:
            tail = slice((k + 1) * g, n)
            target = W[:, ck] + (W[:, tail] - Wq[:, tail]) @ L[tail, ck]
        if targets is not None:
            targets.append(target.clone())
        vals, code = e8p_encode(target)
        Wq[:, ck] = vals
        out.append(code)
    return out


def dequantize_linear(codes, scale):
    """quipsharp/quantize.py:107-113: one decode per block column, then cat."""
    T = codes.shape[-1]
    blocks = [e8p_decode(codes[..., k]) for k in range(T)]
    return torch.cat(blocks, dim=-1) * scale


def linear_forward(x, codes, scale, su=None, sv=None, phase_u=None, phase_v=None):
    """quipsharp/quantize.py:116-124 with RHT signs (power-of-two dims) or RFFT phases."""
    what_q = dequantize_linear(codes, scale)
    x2 = fwht(x * sv) if sv is not None else to_rfft(x, phase_v)
    y1 = x2 @ what_q.T
    return fwht(y1) * su if su is not None else from_rfft(y1, phase_u)


def random_codes(m, n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 65536, (m, n // 8), generator=g)


def as_numpy(t):
    return t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)
