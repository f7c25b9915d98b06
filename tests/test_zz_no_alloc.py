"""GPU: qs_linear_forward_noalloc (workspace in the library's device array)
against qs_linear_forward (caller's workspace), through the C ABI: outputs
bit-identical on consecutive calls, each smaller than the one before, on the
one-launch, batched and wide paths; a replayed HIP graph of the
allocation-free call; and the size limit reported before any launch."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _linear(dev, m, n, seed, bits, bias):
    from quipsharp_amd.hadamard import hartley_matrix, kron_factor
    from quipsharp_amd.quantize import PackedCodes, pack_signs
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 65536, (m, n // 8), generator=g).to(dev)
    su = (torch.randint(0, 2, (m,), generator=g).float() * 2 - 1).to(dev)
    sv = (torch.randint(0, 2, (n,), generator=g).float() * 2 - 1).to(dev)
    b = torch.randn(m, generator=g).to(dev) if bias else None
    if bits:
        su, sv = pack_signs(su), pack_signs(sv)
    pm, pn = kron_factor(m)[0], kron_factor(n)[0]
    return dict(packed=PackedCodes(codes, m, n, [0]), su=su, sv=sv, bias=b, m=m, n=n, bits=bits, pm=pm, pn=pn,
                Km=hartley_matrix(pm, dev) if pm > 1 else None, Kn=hartley_matrix(pn, dev) if pn > 1 else None)


def _args(L, x, y):
    from quipsharp_amd import _lib
    p = L["packed"]
    layout = p.layout | (_lib.QS_SIGNS_BITS if L["bits"] else 0)
    return [_lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), x.shape[0], L["n"], L["m"], _lib.ptr(p.codes0),
            None, 0, layout, _lib.ptr(L["sv"]), _lib.ptr(L["su"]), L["pn"], _lib.ptr(L["Kn"]), L["pm"],
            _lib.ptr(L["Km"]), 1.0, 0.0, 0.0135, _lib.ptr(L["bias"]), _lib.ptr(y), _lib.dtype_code(y.dtype),
            y.stride(0)]


def _with_workspace(L, x):
    from quipsharp_amd import _lib
    lib = _lib.lib()
    y = torch.empty(x.shape[0], L["m"], dtype=x.dtype, device=x.device)
    need = lib.qs_linear_workspace_bytes(L["m"], L["n"], x.shape[0], L["packed"].layout)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=x.device)
    _lib.check(lib.qs_linear_forward(*_args(L, x, y), _lib.ptr(ws), ws.numel(), None, None, _lib.stream_of(x)))
    return y


def _noalloc(L, x, y=None):
    from quipsharp_amd import _lib
    y = torch.empty(x.shape[0], L["m"], dtype=x.dtype, device=x.device) if y is None else y
    _lib.check(_lib.lib().qs_linear_forward_noalloc(*_args(L, x, y), _lib.stream_of(x)))
    return y


@pytest.mark.parametrize("calls", [
    # (m, n, rows, packed sign bits, bias): each call smaller than the previous one
    [(4096, 4096, 16, False, True), (1024, 4096, 1, True, False)],
    [(11008, 4096, 2, True, True), (4096, 11008, 1, True, False)],       # odd-factor output / input
    [(4096, 4096, 24, True, False), (4096, 4096, 5, False, True), (512, 1024, 2, True, True)],
    [(14336, 4096, 8, False, False), (4096, 4096, 2, True, False)],      # m off the chunk scheme
    [(25600, 5120, 16, False, True), (25600, 5120, 8, False, False), (5120, 25600, 1, False, False)],  # Qwen3-32B MLP
])
def test_noalloc_equals_workspace_forward(dev, calls):
    for i, (m, n, rows, bits, bias) in enumerate(calls):
        print(f"case: noalloc call {i}: m={m} n={n} rows={rows} bits={bits} bias={bias}", flush=True)
        L = _linear(dev, m, n, 100 + i, bits, bias)
        x = torch.randn(rows, n, generator=torch.Generator().manual_seed(i)).to(dev).bfloat16()
        want = _with_workspace(L, x)
        got = _noalloc(L, x)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (m, n, rows)


def test_noalloc_graph_replays(dev):
    """Captured in a HIP graph (the callers it is for) and replayed, with
    eager calls of another shape between the replays."""
    L = _linear(dev, 4096, 4096, 7, True, True)
    L2 = _linear(dev, 1024, 4096, 8, True, False)
    x = torch.randn(1, 4096, device=dev).bfloat16()
    x2 = torch.randn(16, 4096, device=dev).bfloat16()
    want = _with_workspace(L, x)
    y = torch.empty(1, 4096, dtype=torch.bfloat16, device=dev)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        _noalloc(L, x, y)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _noalloc(L, x, y)
    for _ in range(4):
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want)
        _noalloc(L2, x2)
        torch.cuda.synchronize()


@pytest.mark.parametrize("m,n,rows", [(12288, 12288, 512), (25600, 25600, 256)])
def test_noalloc_rejects_oversized(dev, m, n, rows):
    """A shape whose workspace exceeds the array (wide prefill batches; every
    m, n <= 32768 fits at 1-128 rows): QS_ERR_UNSUPPORTED on the host,
    nothing launched, the output untouched."""
    from quipsharp_amd import _lib
    lib = _lib.lib()
    need = lib.qs_linear_workspace_bytes(m, n, rows, _lib.QS_LAYOUT_TILED)
    assert need > _lib.QS_NOALLOC_SCRATCH_BYTES
    L = _linear(dev, m, n, 9, False, False)
    x = torch.zeros(rows, n, dtype=torch.bfloat16, device=dev)
    y = torch.full((rows, m), 7.0, dtype=torch.bfloat16, device=dev)
    rc = lib.qs_linear_forward_noalloc(*_args(L, x, y), _lib.stream_of(x))
    assert rc == 3 and b"allocation-free forward has" in lib.qs_last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
    assert np.isfinite(need)
