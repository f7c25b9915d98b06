"""GPU parity: randomized Hadamard transforms.  The Walsh-Hadamard transform is
bit-exact with the reference's fwht (golden outputs); the Kronecker transform
for non-power-of-two lengths is checked against a dense fp64 matrix."""
import math

import numpy as np
import pytest
import torch

from conftest import golden
from oracle import cref

pytestmark = pytest.mark.gpu


def sylvester(n):
    H = np.array([[1.0]])
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H / np.sqrt(n)


def hartley(p):
    a = np.arange(p)
    ang = 2 * np.pi * ((a[:, None] * a[None, :]) % p) / p
    return (np.cos(ang) + np.sin(ang)) / np.sqrt(p)


def dense_T(n):
    L = n & -n
    p = n // L
    return np.kron(hartley(p), sylvester(L)) if p > 1 else sylvester(n)


@pytest.mark.parametrize("k", range(15))
def test_fwht_golden_bit_exact(dev, k):
    from quipsharp_amd.hadamard import fwht
    f = golden("fwht.npz")
    n = 1 << k
    print("case: fwht n =", n, flush=True)
    y = fwht(torch.from_numpy(f[f"x{n}"]).to(dev)).cpu().numpy()
    assert np.array_equal(y, f[f"y{n}"])


def test_fwht_dim0_golden(dev):
    from quipsharp_amd.hadamard import fwht
    f = golden("fwht.npz")
    y = fwht(torch.from_numpy(f["xdim0"]).to(dev), dim=0).cpu().numpy()
    assert np.array_equal(y, f["ydim0"])


@pytest.mark.parametrize("shape,dim", [((3, 4096, 5), 1), ((2, 16384, 70), 1), ((128, 4096), 0),
                                       ((7, 32768), 1), ((1, 2048, 3), 1)])
def test_fwht_strided_bit_exact_vs_oracle(dev, shape, dim):
    from quipsharp_amd.hadamard import fwht
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(shape).astype(np.float32)
    y = fwht(torch.from_numpy(x).to(dev), dim=dim).cpu().numpy()
    assert np.array_equal(y, cref.fwht(x, dim))


def test_fwht_errors(dev):
    from quipsharp_amd.hadamard import fwht
    with pytest.raises(ValueError):
        fwht(torch.randn(3, device=dev))


@pytest.mark.parametrize("n", [3 * 64, 43 * 256, 7 * 2048, 37 * 512, 5 * 1024, 25 * 1024, 7 * 512, 43])
def test_kron_transform_vs_dense(dev, n):
    from quipsharp_amd.hadamard import rht
    rng = np.random.default_rng(n)
    x = rng.standard_normal((3, n)).astype(np.float32)
    y = rht(torch.from_numpy(x).to(dev)).cpu().numpy()
    want = x.astype(np.float64) @ dense_T(n).T
    assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max() * math.sqrt(n / 64) + 1e-6
    # involution
    back = rht(torch.from_numpy(y).to(dev)).cpu().numpy()
    assert np.allclose(back, x, atol=1e-4)


@pytest.mark.parametrize("m,n", [(11008, 64), (96, 43 * 64)])
def test_kron_transform_columns_vs_dense(dev, m, n):
    from quipsharp_amd.hadamard import rht
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, n)).astype(np.float32)
    y = rht(torch.from_numpy(x).to(dev), dim=0).cpu().numpy()
    want = dense_T(m) @ x.astype(np.float64)
    assert np.abs(y - want).max() <= 1e-4


def test_incoherence_process_bit_exact(dev):
    """W_hat = H_m (S_u W S_v) H_n, H_hat likewise (quipsharp/incoherence.py:48-71):
    same signs (CPU generator, su then sv) and bit-exact transforms."""
    from quipsharp_amd.incoherence import incoherence_process, reconstruct_weight, reconstruct_hessian
    rng = np.random.default_rng(5)
    m, n = 256, 128
    W = rng.standard_normal((m, n)).astype(np.float32)
    A = rng.standard_normal((n, n)).astype(np.float32)
    H = (A @ A.T + np.eye(n)).astype(np.float32)
    g = torch.Generator().manual_seed(42)
    what, hhat, signs = incoherence_process(torch.from_numpy(W).to(dev), torch.from_numpy(H).to(dev), generator=g)
    g2 = torch.Generator().manual_seed(42)
    su = (torch.randint(0, 2, (m,), generator=g2).float() * 2 - 1).numpy()
    sv = (torch.randint(0, 2, (n,), generator=g2).float() * 2 - 1).numpy()
    assert np.array_equal(signs.su.cpu().numpy(), su) and np.array_equal(signs.sv.cpu().numpy(), sv)
    Z = W * su[:, None] * sv[None, :]
    assert np.array_equal(what.cpu().numpy(), cref.fwht(cref.fwht(Z, 0), 1))
    Y = H * sv[:, None] * sv[None, :]
    assert np.array_equal(hhat.cpu().numpy(), cref.fwht(cref.fwht(Y, 0), 1))
    assert np.allclose(reconstruct_weight(what, signs).cpu().numpy(), W, atol=1e-4)
    assert np.allclose(reconstruct_hessian(hhat, signs).cpu().numpy(), H, atol=1e-3)


def test_transform_order_identity(dev):
    """quipsharp tests/test_incoherence.py:37-51 (x @ W^T through the transforms),
    for the Walsh-Hadamard and the Kronecker kinds."""
    from quipsharp_amd.incoherence import incoherence_process_auto, linear_via_transformed
    for m, n in ((16, 32), (48, 144), (11008 // 8, 4096 // 8 * 3)):
        torch.manual_seed(2)
        W = torch.randn(m, n, device=dev)
        what, _, signs = incoherence_process_auto(W, torch.eye(n, device=dev))
        x = torch.randn(5, n, device=dev)
        y = linear_via_transformed(x, what, signs)
        assert torch.allclose(y, x @ W.T, atol=1e-3), (m, n)


def test_incoherence_reduces_mu(dev):
    """quipsharp tests/test_incoherence.py:54-67 and tests/test_rfft.py:87-97."""
    from quipsharp_amd.incoherence import incoherence_mu, incoherence_process_auto
    for m, n in ((64, 64), (40, 60)):
        torch.manual_seed(3)
        W = torch.randn(m, n, device=dev) * 0.1
        W[3, 5] = 50.0
        what, _, _ = incoherence_process_auto(W, torch.eye(n, device=dev))
        assert incoherence_mu(what) < incoherence_mu(W) / 5
