"""The C ABI library: loads without a GPU, exports every entry point declared
in include/quipsharp_hip.h, and rejects bad arguments on the host (nothing is
launched by these calls)."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT
from oracle import cref


@pytest.fixture(scope="module")
def L():
    from quipsharp_amd import _lib
    return _lib.lib()


def declared():
    text = open(os.path.join(ROOT, "include", "quipsharp_hip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(qs_[a-z0-9_]+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = declared()
    assert "qs_linear_forward" in names and "qs_rvq_encode" in names and len(names) >= 12


def test_library_exports_every_declared_symbol(L):
    lib = ctypes.CDLL(os.path.join(ROOT, "quipsharp_amd", "libquipsharp_hip.so"))
    for name in declared():
        assert hasattr(lib, name), name


def test_python_binding_covers_the_header():
    from quipsharp_amd import _lib
    assert sorted(_lib.EXPORTED) == declared()


def test_abi_version(L):
    assert L.qs_abi_version() == 1


def test_tables_equal_oracle(L):
    a = np.zeros((256, 8), np.float32)
    b = np.zeros((256, 8), np.float32)
    assert L.qs_e8p_abs_table(a.ctypes.data) == 0
    assert L.qs_e81_table(b.ctypes.data) == 0
    assert np.array_equal(a, cref.e8p_abs_table())
    assert np.array_equal(b, cref.e81_table())


def test_argument_errors_are_reported(L):
    from quipsharp_amd import _lib
    rc = L.qs_rvq_encode(ctypes.c_void_p(16), 8, 4, 0, _lib.int_array([0]), _lib.float_array([1.0]), 1.0, 1.0, None, 8,
                         None, 8, 4, 1, None)
    assert rc == 1 and b"nstages" in L.qs_last_error()
    rc = L.qs_rht_f32(ctypes.c_void_p(16), ctypes.c_void_p(16), 1, 12, 1, None, None, None, 1, None, None)
    assert rc == 1 and b"power of two" in L.qs_last_error()
    rc = L.qs_rht_f32(ctypes.c_void_p(16), ctypes.c_void_p(16), 1, 11008, 1, None, None, None, 43, None, None)
    assert rc == 1 and b"kron_mat" in L.qs_last_error()
    rc = L.qs_pack_codes(ctypes.c_void_p(16), 8, 20, 512, 0, 1, ctypes.c_void_p(16), None)
    assert rc == 1 and b"tiled" in L.qs_last_error()
    rc = L.qs_div_f32(ctypes.c_void_p(16), ctypes.c_void_p(16), 4, 0.0, None)
    assert rc == 1 and b"divisor" in L.qs_last_error()


def test_zero_sized_calls_are_noops(L):
    from quipsharp_amd import _lib
    assert L.qs_rvq_encode(None, 8, 0, 1, _lib.int_array([0]), _lib.float_array([1.0]), 1.0, 1.0, None, 8,
                           None, 8, 0, 1, None) == 0
    assert L.qs_div_f32(None, None, 0, 2.0, None) == 0


def test_workspace_size(L):
    from quipsharp_amd import _lib
    a = L.qs_linear_workspace_bytes(4096, 4096, 1, _lib.QS_LAYOUT_TILED)
    b = L.qs_linear_workspace_bytes(4096, 11008, 16, _lib.QS_LAYOUT_TILED)
    assert a >= 4096 * 2 + 4096 * 4 and b > a and a % 256 == 0


def test_noalloc_bound(L):
    """The allocation-free forward's array is the size the header states, and
    the shapes the header says fit do: every m, n <= 32768 (multiples of 256)
    at 1..128 rows; a wide prefill batch (11008 x 4096 at 4096 rows) does not
    (qs_linear_forward_noalloc refuses what exceeds the array)."""
    from quipsharp_amd import _lib
    text = open(os.path.join(ROOT, "include", "quipsharp_hip.h")).read()
    mib = int(re.search(r"#define QS_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << 20\)", text).group(1))
    cap = _lib.QS_NOALLOC_SCRATCH_BYTES
    assert cap == mib << 20
    dims = range(256, 32769, 256)
    ws = L.qs_linear_workspace_bytes
    tiled = _lib.QS_LAYOUT_TILED
    worst = max(ws(m, n, b, tiled) for m in dims for n in dims for b in (1, 2, 4, 8, 9, 16, 17, 32, 64, 128))
    assert worst <= cap, (worst, cap)
    assert ws(11008, 4096, 4096, tiled) > cap


def test_group_argument_errors(L):
    import ctypes as ct
    from quipsharp_amd import _lib
    ms = (ct.c_int64 * 2)(4096, 11008)
    assert L.qs_linear_group_workspace_bytes(4096, 1, 2, ms) > L.qs_linear_workspace_bytes(4096, 4096, 1, 1)
    assert L.qs_linear_group_workspace_bytes(4096, 1, 0, ms) == 0
    jobs = (_lib.LinearJob * 5)()
    rc = L.qs_linear_forward_group(ct.c_void_p(256), 0, 4096, 1, 4096, 1, None, 5, jobs, 0, ct.c_void_p(256), 1 << 20,
                                   None, None, None)
    assert rc == 1 and b"count" in L.qs_last_error()
    rc = L.qs_linear_forward_group(ct.c_void_p(256), 0, 384, 3, 384, 3, ct.c_void_p(256), 1, jobs, 0,
                                   ct.c_void_p(256), 1 << 20, None, None, None)  # n = 3 x 128: not a multiple of 256
    assert rc == 1 and b"grouped forward needs n" in L.qs_last_error()


def test_out_rows_views_without_copy():
    """Output views for the forward: (rows, m) in place with their row stride,
    never a copy; views that would need one are refused (host logic only)."""
    import torch
    from quipsharp_amd.quantize import _ld, _out_rows
    big = torch.zeros(4, 40)
    y = _out_rows(big[:, 8:24], 4, 16)
    assert y.data_ptr() == big[:, 8:24].data_ptr() and y.stride() == (40, 1) and _ld(y, 16) == 40
    y3 = _out_rows(torch.zeros(2, 3, 16), 6, 16)
    assert y3.shape == (6, 16) and _ld(y3, 16) == 16
    one = torch.zeros(16, 1).T  # a single row: contiguous along m, any row stride
    assert _ld(_out_rows(one, 1, 16), 16) == 16
    with pytest.raises(ValueError):
        _out_rows(torch.zeros(16, 4).T, 4, 16)  # rows not contiguous along m
    with pytest.raises(ValueError):
        _out_rows(torch.zeros(4, 15), 4, 16)
    y4 = _out_rows(torch.zeros(2, 3, 40)[:, :, :16], 6, 16)  # the two leading dims collapse: row stride 40
    assert y4.stride() == (40, 1) and _ld(y4, 16) == 40
    with pytest.raises(ValueError):
        _out_rows(torch.zeros(2, 3, 40)[:, :2, :16], 4, 16)  # (4, 16) only as a copy


def test_pack_signs_words():
    """Bit i % 32 of word i // 32 is set where s[i] < 0 (int32 two's complement),
    the tail of the last word zero."""
    import torch
    from quipsharp_amd.quantize import pack_signs
    rng = np.random.default_rng(3)
    for n in (1, 31, 32, 33, 256, 4160):
        s = rng.choice([-1.0, 1.0], n).astype(np.float32)
        w = pack_signs(torch.from_numpy(s)).numpy().view(np.uint32)
        assert w.shape == ((n + 31) // 32,)
        bits = np.unpackbits(w.view(np.uint8), bitorder="little")
        assert np.array_equal(bits[:n], (s < 0).astype(np.uint8))
        assert not bits[n:].any()
    assert pack_signs(torch.tensor([-1.0] * 32)).item() == -1
