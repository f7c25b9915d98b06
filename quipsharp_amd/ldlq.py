"""BlockLDLQ (quipsharp/ldlq.py) on the GPU.

``block_ldl`` factors H = L blockdiag(D) L^T with torch-ROCm linear algebra
(rocSOLVER Cholesky, batched block inverses).  ``block_ldlq`` runs the
reference's rounding schedule -- base pass over blocks T-1..0 with feedback
from the already-rounded tail, then ``tune_iters`` refinement sweeps with the
full Hessian -- keeping the residual W - Wq up to date block by block instead
of recomputing it.  With one of the library's codebooks,
``block_ldlq_native`` fuses each step's target formation, residual-VQ
encode, and the Wq / residual / code updates into a single kernel launch;
the feedback products stay on rocBLAS.
"""
import torch
from torch import Tensor

from . import _lib


def _cholesky_escalating(M: Tensor, scale: float, base: float):
    """Lower Cholesky factor of M.  Failure semantics of the reference
    (quipsharp/ldlq.py:58-75): when the fp32 factorization breaks down the
    matrix is promoted to fp64 and factored again, and on further failures
    diagonal loading grows tenfold per attempt (base, 10 base, 100 base times
    the mean diagonal `scale`), four fp64 attempts in all.  Returns the factor
    and the extra loading added (0.0 when fp32 sufficed)."""
    try:
        return torch.linalg.cholesky(M), 0.0
    except torch.linalg.LinAlgError:
        pass
    M64 = M.double()
    eye = torch.eye(M.shape[0], device=M.device, dtype=torch.float64)
    added = 0.0
    for attempt in range(4):
        try:
            return torch.linalg.cholesky(M64), added
        except torch.linalg.LinAlgError:
            if attempt == 3:
                raise
            loading = scale * base * 10.0 ** attempt
            M64 = M64 + loading * eye
            added += loading


def block_ldl(H: Tensor, g: int, damping: float = 1e-2):
    """g-block LDL, H = L @ blockdiag(D) @ L^T (quipsharp/ldlq.py:39-84).
    Returns L (n, n) unit block-lower-triangular and D (T, g, g)."""
    n = H.shape[0]
    assert n % g == 0, f"block_ldl: n = {n} is not a multiple of the block size {g}"
    T = n // g
    mean_diag = float(H.diagonal().mean())
    M = H + damping * mean_diag * torch.eye(n, device=H.device, dtype=H.dtype) if damping else H.clone()
    L0, added = _cholesky_escalating(M, mean_diag, damping if damping else 1e-2)
    if L0.dtype != H.dtype:
        print(f"[quipsharp_amd] {n}x{n} Hessian: Cholesky needed fp64 and {added / mean_diag:.0e} x mean(diag) "
              "of extra diagonal loading", flush=True)
    # the g x g diagonal blocks of the Cholesky factor, then each block column
    # of L0 times the inverse of its diagonal block (one batched product)
    DL = torch.diagonal(L0.reshape(T, g, T, g), dim1=0, dim2=2).permute(2, 0, 1).contiguous()
    D = DL @ DL.transpose(-1, -2)
    L = torch.matmul(L0.reshape(n, T, g).transpose(0, 1), torch.linalg.inv(DL)).transpose(0, 1).reshape(n, n)
    return L.to(H.dtype), D.to(H.dtype)


def block_diag_from_stack(D: Tensor) -> Tensor:
    """(T, g, g) -> (n, n) block-diagonal (quipsharp/ldlq.py:87-94)."""
    return torch.block_diag(*D.unbind(0))


def _diag_inv(H: Tensor, g: int) -> Tensor:
    n = H.shape[0]
    T = n // g
    blocks = torch.diagonal(H.reshape(T, g, T, g), dim1=0, dim2=2).permute(2, 0, 1).contiguous()
    return torch.linalg.inv(blocks)


def block_ldlq(W: Tensor, L: Tensor, g: int, quantize_fn, H: Tensor = None, tune_iters: int = 10) -> Tensor:
    """BlockLDLQ with a caller-supplied rounding callback
    (quipsharp/ldlq.py:97-141).  quantize_fn(target (m, g), k) -> (m, g)."""
    _lib.require_gpu(W, L, H, what="block_ldlq")
    m, n = W.shape
    assert n % g == 0
    T = n // g
    Wq = torch.zeros_like(W)
    E = W.clone()  # W - Wq, updated block by block
    for k in reversed(range(T)):
        ck = slice(k * g, (k + 1) * g)
        tail = slice((k + 1) * g, n)
        target = W[:, ck] + E[:, tail] @ L[tail, ck]
        Wq[:, ck] = quantize_fn(target, k)
        E[:, ck] = W[:, ck] - Wq[:, ck]
    if H is not None and tune_iters > 0:
        dinv = _diag_inv(H, g)
        for _ in range(tune_iters):
            for k in reversed(range(T)):
                ck = slice(k * g, (k + 1) * g)
                target = Wq[:, ck] + (E @ H[:, ck]) @ dinv[k]
                Wq[:, ck] = quantize_fn(target, k)
                E[:, ck] = W[:, ck] - Wq[:, ck]
    return Wq


_TUNE_CHUNK = 16  # blocks per chunk of the refinement pass (qs_ldlq_chunk: at most 16)
_TUNE_CHUNKED = True  # False: the refinement forms E @ H[:, block] for each block (ldlq.py:136-138's form)


def block_ldlq_native(W: Tensor, L: Tensor, kinds, scales, H: Tensor = None, tune_iters: int = 10):
    """BlockLDLQ with the library's residual-VQ codebook (g = 8), one fused
    kernel per rounding step.  Returns (Wq (m, n), codes int64 (S, m, T))."""
    _lib.require_gpu(W, L, H, what="block_ldlq")
    g = 8
    W = W.float().contiguous()
    L = L.float().contiguous()
    m, n = W.shape
    assert n % g == 0
    T = n // g
    S = len(kinds)
    Wq = torch.zeros_like(W)
    E = W.clone()
    codes = torch.zeros(S, m, T, dtype=torch.int64, device=W.device)
    fb = torch.empty(m, g, dtype=torch.float32, device=W.device)
    kinds_c = _lib.int_array(kinds)
    scales_c = _lib.float_array([float(s) for s in scales])
    lib = _lib.lib()
    stream = _lib.stream_of(W)
    esz = W.element_size()
    wp, wqp, ep, cp = W.data_ptr(), Wq.data_ptr(), E.data_ptr(), codes.data_ptr()

    def step(k, base_ptr, dinv_ptr):
        _lib.check(lib.qs_ldlq_step(
            base_ptr, n, fb.data_ptr(), dinv_ptr, wp + k * g * esz, n, wqp + k * g * esz, n,
            ep + k * g * esz, n, m, S, kinds_c, scales_c, cp + k * 8, 8, m * T, T, stream))

    for k in reversed(range(T)):
        ck = slice(k * g, (k + 1) * g)
        tail = slice((k + 1) * g, n)
        if k == T - 1:
            fb.zero_()
        else:
            torch.mm(E[:, tail], L[tail, ck], out=fb)
        step(k, wp + k * g * esz, None)
    if H is not None and tune_iters > 0:
        H = H.float().contiguous()
        dinv = _diag_inv(H, g).contiguous()
        dp = dinv.data_ptr()
        if not _TUNE_CHUNKED:
            for _ in range(tune_iters):
                for k in reversed(range(T)):
                    ck = slice(k * g, (k + 1) * g)
                    torch.mm(E, H[:, ck], out=fb)
                    step(k, wqp + k * g * esz, dp + k * g * g * 4)
            return Wq, codes
        # E @ H[:, ck] for each block, with E as the pass leaves it: within a
        # chunk of blocks only the chunk's columns of E change, so the product
        # with the other columns is formed once per chunk (P = E @ H[:, cc] -
        # E[:, cc] @ H[cc, cc]) and one launch runs the chunk's blocks, adding
        # the chunk's current columns itself (qs_ldlq_chunk): E is read once
        # per chunk, and there is one launch per chunk instead of two per block
        C = min(_TUNE_CHUNK, T)
        P = torch.empty(m, C * g, dtype=torch.float32, device=W.device)
        hp = H.data_ptr()
        for _ in range(tune_iters):
            for c0 in reversed(range(0, T, C)):
                c1 = min(c0 + C, T)
                cc = slice(c0 * g, c1 * g)
                Pc = P if c1 - c0 == C else torch.empty(m, (c1 - c0) * g, dtype=torch.float32, device=W.device)
                torch.mm(E, H[:, cc], out=Pc)
                Pc.addmm_(E[:, cc], H[cc, cc], alpha=-1.0)
                _lib.check(lib.qs_ldlq_chunk(wp, n, wqp, n, ep, n, Pc.data_ptr(), Pc.stride(0), hp + c0 * g * n * 4, n,
                                             dp, c0, c1 - c0, m, S, kinds_c, scales_c, cp, 8, m * T, T, stream))
    return Wq, codes
