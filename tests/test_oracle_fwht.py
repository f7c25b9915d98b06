"""Walsh-Hadamard oracle: bit-exact with the reference's fwht, and the dense
Sylvester matrix / involution properties of quipsharp tests/test_hadamard.py."""
import numpy as np
import pytest

from conftest import golden
from oracle import cref


def sylvester(n):
    H = np.array([[1.0]])
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H / np.sqrt(n)


@pytest.mark.parametrize("k", range(15))
def test_fwht_bit_exact_with_reference(k):
    f = golden("fwht.npz")
    n = 1 << k
    assert np.array_equal(cref.fwht(f[f"x{n}"], -1), f[f"y{n}"])


def test_fwht_dim0_bit_exact():
    f = golden("fwht.npz")
    assert np.array_equal(cref.fwht(f["xdim0"], 0), f["ydim0"])


@pytest.mark.parametrize("n", [1, 2, 4, 8, 16, 32, 128, 1024])
def test_fwht_matches_dense_matrix(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((5, n)).astype(np.float32)
    assert np.allclose(cref.fwht(x), x.astype(np.float64) @ sylvester(n).T, atol=1e-5)


def test_fwht_involution_and_norm():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 64)).astype(np.float32)
    y = cref.fwht(x)
    assert np.allclose(cref.fwht(y), x, atol=1e-5)
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), atol=1e-5)


def test_fwht_stage_order_matters():
    """A reversed stage order is mathematically equal but not bit-identical,
    so the golden comparison above pins the order."""
    f = golden("fwht.npz")
    x = f["x4096"].astype(np.float32)
    y = x.copy()
    n = 4096
    h = n // 2
    while h >= 1:
        for b in range(0, n, 2 * h):
            a, d = y[:, b:b + h].copy(), y[:, b + h:b + 2 * h].copy()
            y[:, b:b + h], y[:, b + h:b + 2 * h] = a + d, a - d
        h //= 2
    y = y * np.float32(n ** -0.5)
    assert not np.array_equal(y, f["y4096"])
