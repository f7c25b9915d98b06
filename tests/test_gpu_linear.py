"""GPU parity: the fused quantized-linear forward (decode + transforms +
matvec) against the reference's golden outputs and a dense fp64 oracle at the
Llama-2-7B layer shapes.  Tolerance: relative 1e-3 (norm-wise) with fp32
accumulation; dequantization is bit-exact."""
import numpy as np
import pytest
import torch

from conftest import golden
from oracle import cref

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def fwht64(x, axis=-1):
    """fp64 orthonormal Walsh-Hadamard along axis (numpy)."""
    x = np.moveaxis(np.array(x, dtype=np.float64), axis, -1)
    n = x.shape[-1]
    shp = x.shape
    y = x.reshape(-1, n)
    h = 1
    while h < n:
        y = y.reshape(-1, n // (2 * h), 2, h)
        y = np.stack((y[:, :, 0] + y[:, :, 1], y[:, :, 0] - y[:, :, 1]), axis=2)
        h *= 2
    return np.moveaxis(y.reshape(shp) / np.sqrt(n), -1, axis)


def hartley(p):
    a = np.arange(p)
    ang = 2 * np.pi * ((a[:, None] * a[None, :]) % p) / p
    return (np.cos(ang) + np.sin(ang)) / np.sqrt(p)


def T64(x):
    """fp64 transform along the last dim: K_p (x) H_L (H_n when p == 1)."""
    n = x.shape[-1]
    L = n & -n
    p = n // L
    y = fwht64(x.reshape(x.shape[:-1] + (p, L)), -1)
    if p > 1:
        y = np.einsum("ab,...bl->...al", hartley(p), y)
    return y.reshape(x.shape)


def dense_forward(x, codes0, codes1, s0, s1, su, sv, scale, bias=None):
    m, T = codes0.shape
    W = cref.e8p_decode(codes0).reshape(m, T * 8).astype(np.float64) * s0
    if codes1 is not None:
        W += cref.e81_table()[codes1].reshape(m, T * 8).astype(np.float64) * s1
    x2 = T64(x.astype(np.float64) * sv)
    y = T64(x2 @ W.T * scale) * su
    return y if bias is None else y + bias


def rel_err(got, want):
    return np.linalg.norm(got - want) / np.linalg.norm(want)


def run(dev, x, codes0, codes1, s0, s1, su, sv, scale, bias=None, out_dtype=torch.float32):
    from quipsharp_amd.quantize import PackedCodes, forward_packed
    m, T = codes0.shape
    kinds = [0] if codes1 is None else [0, 1]
    c = torch.from_numpy(codes0.astype(np.int64)).to(dev)
    if codes1 is not None:
        c = torch.stack([c, torch.from_numpy(codes1.astype(np.int64)).to(dev)])
    packed = PackedCodes(c, m, T * 8, kinds)
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
    xt = x if isinstance(x, torch.Tensor) else t(x)
    y = forward_packed(xt, packed, t(su), t(sv), s0, s1, scale, bias=t(bias), out_dtype=out_dtype)
    return y, packed


def test_linear_forward_golden(dev):
    """linear_forward on the reference's random-code layers (golden y)."""
    from quipsharp_amd.codebooks.e8p import E8PCodebook
    from quipsharp_amd.codebooks.e8_1bit import E8OneBitCodebook
    from quipsharp_amd.incoherence import IncoherenceSigns
    from quipsharp_amd.quantize import QuantizedLayer, RVQCodebookAdapter, dequantize_linear, linear_forward
    from quipsharp_amd.rvq import RVQStage
    lf = golden("linear.npz")
    cb = E8PCodebook(dev)
    books = {"e8p": cb, "rvq3": RVQCodebookAdapter([RVQStage(cb, 1.03), RVQStage(E8OneBitCodebook(dev), 0.47)])}
    for name, book in books.items():
        codes = torch.from_numpy(lf[name + "_codes"].astype(np.int64)).to(dev)
        m, n = lf[name + "_deq"].shape
        signs = IncoherenceSigns(su=torch.from_numpy(lf[name + "_su"]).to(dev),
                                 sv=torch.from_numpy(lf[name + "_sv"]).to(dev))
        layer = QuantizedLayer(codes=codes, signs=signs, g=8, shape=(m, n), scale=float(lf[name + "_scale"]))
        deq = dequantize_linear(layer, book).cpu().numpy()
        assert np.array_equal(deq, lf[name + "_deq"]), name
        y = linear_forward(torch.from_numpy(lf[name + "_x"]).to(dev), layer, book).cpu().numpy()
        err = rel_err(y, lf[name + "_y"])
        print(f"{name}: rel err vs reference {err:.2e}", flush=True)
        assert err < REL_TOL, (name, err)


@pytest.mark.parametrize("m,n", [(4096, 4096), (11008, 4096), (4096, 11008), (1024, 4096), (3584, 3584)])
@pytest.mark.parametrize("B", [1, 4, 16])
def test_forward_vs_dense_fp64(dev, m, n, B):
    print(f"case: forward m={m} n={n} B={B}", flush=True)
    rng = np.random.default_rng(m * 7 + n + B)
    codes = rng.integers(0, 65536, (m, n // 8))
    su = rng.choice([-1.0, 1.0], m)
    sv = rng.choice([-1.0, 1.0], n)
    x = rng.standard_normal((B, n)).astype(np.float32)
    scale = float(np.float32(0.0135))
    y, packed = run(dev, x, codes, None, 1.0, 0.0, su, sv, scale)
    assert packed.layout == 1
    want = dense_forward(x, codes, None, 1.0, 0.0, su, sv, scale)
    err = rel_err(y.cpu().numpy(), want)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < REL_TOL


@pytest.mark.parametrize("B", [1, 17])
def test_forward_rvq3_vs_dense(dev, B):
    m, n = 4096, 4096
    rng = np.random.default_rng(B)
    c0 = rng.integers(0, 65536, (m, n // 8))
    c1 = rng.integers(0, 256, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    x = rng.standard_normal((B, n)).astype(np.float32)
    y, packed = run(dev, x, c0, c1, 0.95, 0.5, su, sv, 0.01)
    assert packed.layout == 1
    want = dense_forward(x, c0, c1, 0.95, 0.5, su, sv, 0.01)
    assert rel_err(y.cpu().numpy(), want) < REL_TOL


@pytest.mark.parametrize("m,n", [(40, 96), (48, 144), (200, 64)])
def test_forward_rowmajor_fallback(dev, m, n):
    rng = np.random.default_rng(m + n)
    codes = rng.integers(0, 65536, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    x = rng.standard_normal((3, n)).astype(np.float32)
    bias = rng.standard_normal(m)
    y, packed = run(dev, x, codes, None, 1.0, 0.0, su, sv, 0.02, bias=bias)
    assert packed.layout == 0
    want = dense_forward(x, codes, None, 1.0, 0.0, su, sv, 0.02, bias)
    assert rel_err(y.cpu().numpy(), want) < 1e-5


def test_forward_bf16_io_and_bias(dev):
    m, n = 4096, 4096
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 65536, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    bias = rng.standard_normal(m).astype(np.float32) * 0.1
    xb = torch.from_numpy(rng.standard_normal((2, n)).astype(np.float32)).to(dev).bfloat16()
    y, _ = run(dev, xb, codes, None, 1.0, 0.0, su, sv, 0.0135, bias=bias, out_dtype=torch.bfloat16)
    assert y.dtype == torch.bfloat16
    want = dense_forward(xb.float().cpu().numpy(), codes, None, 1.0, 0.0, su, sv, 0.0135, bias)
    got = y.float().cpu().numpy()
    # bf16 output: within rounding of the fp32 result plus the 1e-3 path tolerance
    assert np.all(np.abs(got - want) <= 2 ** -8 * np.abs(want) + 2e-3 * np.abs(want).max())


def test_forward_large_activation_range(dev):
    """Activations far outside fp16 range are handled by the per-row
    power-of-two scaling of the input transform."""
    m, n = 1024, 4096
    rng = np.random.default_rng(9)
    codes = rng.integers(0, 65536, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    x = (rng.standard_normal((2, n)) * np.array([[3e5], [1e-6]])).astype(np.float32)
    y, _ = run(dev, x, codes, None, 1.0, 0.0, su, sv, 0.01)
    want = dense_forward(x, codes, None, 1.0, 0.0, su, sv, 0.01)
    g = y.cpu().numpy()
    for b in range(2):
        assert rel_err(g[b], want[b]) < REL_TOL


@pytest.mark.parametrize("m,n,B", [(4096, 4096, 1), (11008, 4096, 1), (4096, 11008, 2)])
def test_forward_graph_replays(dev, m, n, B):
    """The single-launch path keeps its completion counter in the workspace and
    resets it in-kernel: captured in a HIP graph, every replay (with eager work
    and synchronizations in between) must equal the eager result."""
    from quipsharp_amd.quantize import PackedCodes, forward_packed
    rng = np.random.default_rng(m + n + B)
    codes = torch.from_numpy(rng.integers(0, 65536, (m, n // 8))).to(dev)
    packed = PackedCodes(codes, m, n, [0])
    su = torch.from_numpy(rng.choice([-1.0, 1.0], m).astype(np.float32)).to(dev)
    sv = torch.from_numpy(rng.choice([-1.0, 1.0], n).astype(np.float32)).to(dev)
    x = torch.randn(B, n, device=dev).bfloat16()
    ws = torch.zeros(1 << 22, dtype=torch.uint8, device=dev)
    out = torch.empty(B, m, device=dev, dtype=torch.bfloat16)
    eager = forward_packed(x, packed, su, sv, 1.0, 0.0, 0.0135, workspace=ws).clone()
    forward_packed(x, packed, su, sv, 1.0, 0.0, 0.0135, workspace=ws, out=out)
    assert torch.equal(out, eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        forward_packed(x, packed, su, sv, 1.0, 0.0, 0.0135, workspace=ws, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        forward_packed(x, packed, su, sv, 1.0, 0.0, 0.0135, workspace=ws, out=out)
    for rep in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
        # unrelated eager work between replays
        _ = forward_packed(x, packed, su, sv, 1.0, 0.0, 0.0135, workspace=ws)
        torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B", [1, 2, 5])
def test_forward_strided_unaligned_input(dev, dtype, B):
    """Rows with a stride that is not a multiple of 4 and a start that is not
    8-byte aligned take the element-wise activation loads."""
    m, n = 4096, 4096
    rng = np.random.default_rng(40 + B)
    codes = rng.integers(0, 65536, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    full = torch.from_numpy(rng.standard_normal((B, n + 3)).astype(np.float32)).to(dev).to(dtype)
    x = full[:, 1:n + 1]
    assert x.stride(0) == n + 3 and x.data_ptr() % 8 != 0
    y, _ = run(dev, x, codes, None, 1.0, 0.0, su, sv, 0.0135)
    want = dense_forward(x.float().cpu().numpy(), codes, None, 1.0, 0.0, su, sv, 0.0135)
    assert rel_err(y.float().cpu().numpy(), want) < REL_TOL


@pytest.mark.parametrize("m,n,B", [(11008, 4096, 2), (3584, 3584, 1), (11008, 4096, 7)])
def test_forward_odd_factor_output_bias(dev, m, n, B):
    """Odd-factor outputs go through the chunked output kernel (one work-group
    per output chunk), with bias."""
    rng = np.random.default_rng(m + 3 * B)
    codes = rng.integers(0, 65536, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    bias = rng.standard_normal(m).astype(np.float32)
    x = rng.standard_normal((B, n)).astype(np.float32)
    y, _ = run(dev, x, codes, None, 1.0, 0.0, su, sv, 0.0135, bias=bias)
    want = dense_forward(x, codes, None, 1.0, 0.0, su, sv, 0.0135, bias)
    assert rel_err(y.cpu().numpy(), want) < REL_TOL


@pytest.mark.parametrize("m,n", [(256, 256), (768, 512), (512, 768), (1280, 256)])
@pytest.mark.parametrize("B", [1, 3])
def test_forward_small_chunk_counts(dev, m, n, B):
    """One to five 256-chunks per side (768 = 3 x 256 and 1280 = 5 x 256 take
    the odd-factor stage), single-launch and batched paths."""
    rng = np.random.default_rng(m * 5 + n + B)
    codes = rng.integers(0, 65536, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    bias = rng.standard_normal(m).astype(np.float32)
    x = rng.standard_normal((B, n)).astype(np.float32)
    y, packed = run(dev, x, codes, None, 1.0, 0.0, su, sv, 0.02, bias=bias)
    assert packed.layout == 1
    want = dense_forward(x, codes, None, 1.0, 0.0, su, sv, 0.02, bias)
    assert rel_err(y.cpu().numpy(), want) < REL_TOL


def _rand_linear(dev, rng, m, n, stages=1, bias=False):
    from quipsharp_amd.quantize import PackedCodes
    c = torch.from_numpy(rng.integers(0, 65536, (m, n // 8))).to(dev)
    kinds = [0]
    if stages == 2:
        c = torch.stack([c, torch.from_numpy(rng.integers(0, 256, (m, n // 8))).to(dev)])
        kinds = [0, 1]
    packed = PackedCodes(c, m, n, kinds)
    su = torch.from_numpy(rng.choice([-1.0, 1.0], m).astype(np.float32)).to(dev)
    sv = torch.from_numpy(rng.choice([-1.0, 1.0], n).astype(np.float32)).to(dev)
    b = torch.from_numpy(rng.standard_normal(m).astype(np.float32)).to(dev) if bias else None
    return (packed, su, sv, 0.97, 0.45 if stages == 2 else 0.0, 0.0135, b)


@pytest.mark.parametrize("shapes,n,B,stages,bias", [
    ([4096, 4096, 4096], 4096, 1, 1, False),   # q, k, v
    ([4096, 4096, 4096], 4096, 2, 1, True),
    ([11008, 11008], 4096, 1, 1, True),        # gate, up (odd-factor outputs)
    ([4096, 1024, 11008, 512], 4096, 2, 1, False),
    ([4096, 1024], 4096, 1, 2, False),         # 3-bit residual VQ
    ([4096, 4096], 11008, 1, 1, False),        # odd-factor input
    ([4096, 4096, 4096], 4096, 3, 1, False),   # 16-row pass: input transforms, decode-matvecs,
    ([4096, 1024, 1024], 4096, 16, 1, True),   # output transforms one launch each for the group
    ([11008, 11008], 4096, 8, 2, False),
    ([4096, 14336], 4096, 8, 1, False),        # m = 56 x 256 outside the chunk scheme: own output kernel
    ([4096, 4096], 11008, 5, 1, True),
    ([4096, 1024, 1024], 4096, 24, 1, False),  # wide: one GEMM per linear between the grouped transforms
    ([11008, 11008], 4096, 40, 2, True),
    ([4096, 14336], 4096, 33, 1, False),
    ([4096, 1024, 11008, 512], 4096, 16, 1, True),  # four linears, one of each output size
    ([4096, 1024, 11008, 512], 4096, 24, 1, False),
])
def test_forward_group_equals_single(dev, shapes, n, B, stages, bias):
    """Each output of a grouped launch is bit-identical to the single-linear
    call (same slices per work-group, same reduction order; at 3 or more rows
    the same kernels with the linears' work-groups in one grid)."""
    print(f"case: group {shapes} n={n} B={B} stages={stages}", flush=True)
    from quipsharp_amd.quantize import forward_packed, forward_packed_group
    rng = np.random.default_rng(sum(shapes) + n + B)
    lins = [_rand_linear(dev, rng, m, n, stages, bias) for m in shapes]
    x = torch.randn(B, n, device=dev).bfloat16()
    ys = forward_packed_group(x, lins)
    for lin, y in zip(lins, ys):
        want = forward_packed(x, *lin)
        assert y.shape == want.shape and torch.equal(y, want)
    # and against the dense oracle for one of them
    packed, su, sv, s0, s1, sc, b = lins[0]
    codes = lins[0][0]
    m0 = shapes[0]
    if stages == 1:
        rng2 = np.random.default_rng(sum(shapes) + n + B)
        c0 = rng2.integers(0, 65536, (m0, n // 8))
        su_np = rng2.choice([-1.0, 1.0], m0)
        sv_np = rng2.choice([-1.0, 1.0], n)
        b_np = rng2.standard_normal(m0).astype(np.float32) if bias else None
        want = dense_forward(x.float().cpu().numpy(), c0, None, s0, 0.0, su_np, sv_np, sc, b_np)
        got = ys[0].float().cpu().numpy()
        assert np.all(np.abs(got - want) <= 2 ** -8 * np.abs(want) + 2e-3 * np.abs(want).max())


@pytest.mark.parametrize("B", [1, 16, 24])
def test_forward_group_graph_replays(dev, B):
    from quipsharp_amd import _lib
    from quipsharp_amd.quantize import forward_packed_group
    print(f"case: group graph B={B}", flush=True)
    rng = np.random.default_rng(77)
    lins = [_rand_linear(dev, rng, m, 4096) for m in (4096, 4096, 11008)]
    x = torch.randn(B, 4096, device=dev).bfloat16()
    lib = _lib.lib()
    import ctypes
    ms = (ctypes.c_int64 * 3)(4096, 4096, 11008)
    ws = torch.zeros(lib.qs_linear_group_workspace_bytes(4096, B, 3, ms), dtype=torch.uint8, device=dev)
    outs = [torch.empty(B, m, device=dev, dtype=torch.bfloat16) for m in (4096, 4096, 11008)]
    eager = [y.clone() for y in forward_packed_group(x, lins, workspace=ws)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        forward_packed_group(x, lins, workspace=ws, outs=outs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        forward_packed_group(x, lins, workspace=ws, outs=outs)
    for rep in range(3):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), rep
        forward_packed_group(x, lins, workspace=ws)
        torch.cuda.synchronize()


@pytest.mark.parametrize("seed", range(12))
def test_forward_group_random_sweep(dev, seed):
    """Seeded random groups: 1-4 linears with output sizes inside and outside
    the chunk scheme, inputs of 512..4096 columns (some with an odd factor),
    1..40 rows, one or two stages.  Every output is bit-identical to its
    single-linear call; the first is checked against the dense fp64 oracle."""
    from quipsharp_amd.quantize import forward_packed, forward_packed_group
    rng = np.random.default_rng(1000 + seed)
    count = int(rng.integers(1, 5))
    n = int(rng.choice([512, 768, 1024, 2048, 3072, 4096]))
    ms = [int(rng.choice([256, 512, 768, 1024, 2304, 4096, 11008, 14336])) for _ in range(count)]
    B = int(rng.choice([1, 2, 3, 5, 8, 16, 17, 24, 40]))
    stages = int(rng.choice([1, 2]))
    bias = bool(rng.integers(0, 2))
    print(f"case: sweep seed={seed} n={n} ms={ms} B={B} stages={stages} bias={bias}", flush=True)
    from quipsharp_amd.quantize import PackedCodes
    lins, host = [], []
    for m in ms:
        c0 = rng.integers(0, 65536, (m, n // 8))
        c1 = rng.integers(0, 256, (m, n // 8)) if stages == 2 else None
        su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
        bv = rng.standard_normal(m).astype(np.float32) if bias else None
        c = torch.from_numpy(c0).to(dev) if c1 is None else torch.stack(
            [torch.from_numpy(c0), torch.from_numpy(c1)]).to(dev)
        packed = PackedCodes(c, m, n, [0] if c1 is None else [0, 1])
        t = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float32)).to(dev)
        lins.append((packed, t(su), t(sv), 0.97, 0.45 if stages == 2 else 0.0, 0.0135,
                     None if bv is None else t(bv)))
        host.append((c0, c1, su, sv, bv))
    x = torch.from_numpy(rng.standard_normal((B, n)).astype(np.float32)).to(dev).bfloat16()
    ys = forward_packed_group(x, lins)
    for lin, y in zip(lins, ys):
        assert torch.equal(y, forward_packed(x, *lin))
    c0, c1, su, sv, bv = host[0]
    _, _, _, s0, s1, sc, _ = lins[0]
    want = dense_forward(x.float().cpu().numpy(), c0, c1, s0, s1, su, sv, sc, bv)
    err = rel_err(ys[0].float().cpu().numpy(), want)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < 1e-2  # bf16 output rounding


@pytest.mark.parametrize("B", [1, 16, 24])
def test_forward_into_strided_outputs(dev, B):
    """out / outs may be column slices of wider buffers: the results land in
    place (row stride passed to the library), the other columns stay as they
    were, and the values equal those of contiguous outputs."""
    from quipsharp_amd.quantize import forward_packed, forward_packed_group
    rng = np.random.default_rng(60 + B)
    lins = [_rand_linear(dev, rng, m, 1024, 1, True) for m in (512, 768)]
    x = torch.randn(B, 1024, device=dev).bfloat16()
    want = [forward_packed(x, *lin) for lin in lins]
    big = torch.full((B, 512 + 768 + 64), 7.0, device=dev, dtype=torch.bfloat16)
    outs = [big[:, 0:512], big[:, 512:1280]]
    got = forward_packed_group(x, lins, outs=outs)
    assert got[0] is outs[0] and got[1] is outs[1]
    for w, o in zip(want, outs):
        assert torch.equal(o, w)
    assert torch.all(big[:, 1280:] == 7.0)
    big2 = torch.full((B, 600), 7.0, device=dev, dtype=torch.bfloat16)
    y = forward_packed(x, *lins[0], out=big2[:, 40:552])
    assert torch.equal(y, want[0]) and torch.all(big2[:, :40] == 7.0) and torch.all(big2[:, 552:] == 7.0)
    if B > 1:  # rows that are not contiguous along m: refused, never written to a copy
        with pytest.raises(ValueError):
            forward_packed(x, *lins[0], out=torch.empty(512, B, device=dev, dtype=torch.bfloat16).T)


def test_forward_group_workspace_reused_across_row_counts(dev):
    """One group workspace serves calls of any row count in any order: the
    one-launch kernel's completion counters sit at fixed places, so a wider
    call before a 1- or 2-row call cannot leave them non-zero."""
    from quipsharp_amd import _lib
    from quipsharp_amd.quantize import forward_packed, forward_packed_group
    import ctypes
    rng = np.random.default_rng(31)
    shapes = (1024, 2048, 1024)
    lins = [_rand_linear(dev, rng, m, 1024) for m in shapes]
    ms = (ctypes.c_int64 * 3)(*shapes)
    lib = _lib.lib()
    ws = torch.zeros(max(lib.qs_linear_group_workspace_bytes(1024, B, 3, ms) for B in (1, 2, 16, 40)),
                     dtype=torch.uint8, device=dev)
    for B in (40, 2, 1, 16, 2, 33, 1):
        print(f"case: reuse B={B}", flush=True)
        x = torch.randn(B, 1024, device=dev).bfloat16()
        ys = forward_packed_group(x, lins, workspace=ws)
        for lin, y in zip(lins, ys):
            assert torch.equal(y, forward_packed(x, *lin)), B


def test_forward_group_rejects(dev):
    from quipsharp_amd._lib import QuipHipError
    from quipsharp_amd.quantize import forward_packed_group
    rng = np.random.default_rng(5)
    a = _rand_linear(dev, rng, 1024, 4096)
    b = _rand_linear(dev, rng, 1024, 4096, stages=2)
    x = torch.randn(1, 4096, device=dev)
    with pytest.raises(ValueError):
        forward_packed_group(x, [a] * 5)
    with pytest.raises(QuipHipError, match="stages"):
        forward_packed_group(x, [a, b])


def _dense_weights(codes0, codes1, s0, s1):
    W = cref.e8p_decode(codes0).reshape(codes0.shape[0], -1).astype(np.float64) * s0
    if codes1 is not None:
        W += cref.e81_table()[codes1].reshape(codes1.shape[0], -1).astype(np.float64) * s1
    return W


def _check_shape(dev, m, n, batches, stages, seed):
    """Forward at (m, n) for each batch size against one fp64 dense oracle."""
    rng = np.random.default_rng(seed)
    c0 = rng.integers(0, 65536, (m, n // 8))
    c1 = rng.integers(0, 256, (m, n // 8)) if stages == 2 else None
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    s0, s1, scale = (0.93, 0.41, 0.011) if stages == 2 else (1.0, 0.0, 0.0135)
    W = _dense_weights(c0, c1, s0, s1)
    for B in batches:
        print(f"case: m={m} n={n} B={B} stages={stages}", flush=True)
        x = rng.standard_normal((B, n)).astype(np.float32)
        y, packed = run(dev, x, c0, c1, s0, s1, su, sv, scale)
        assert packed.layout == 1
        want = T64(T64(x.astype(np.float64) * sv) @ W.T * scale) * su
        err = rel_err(y.cpu().numpy(), want)
        print(f"  rel err {err:.2e}", flush=True)
        assert err < REL_TOL, (m, n, B, err)


@pytest.mark.parametrize("m,n", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_llama3_8b_rvq3_shapes(dev, m, n):
    """3-bit residual VQ (E8P + E8 1-bit) at the Llama-3-8B layer shapes, batch 1 / 4 / 16
    (14336 = 7 x 2048 takes the odd-factor transform)."""
    _check_shape(dev, m, n, [1, 4, 16], 2, m + n)


@pytest.mark.parametrize("m,n", [(3584, 3584), (512, 3584), (18944, 3584), (3584, 18944)])
def test_qwen25_7b_shapes(dev, m, n):
    """Qwen2.5-7B layer shapes (3584 = 7 x 512, 18944 = 37 x 512), batch 1."""
    _check_shape(dev, m, n, [1], 1, m * 3 + n)


@pytest.mark.parametrize("m,n", [(8192, 5120), (1024, 5120), (5120, 8192), (25600, 5120), (5120, 25600)])
def test_qwen3_32b_shapes(dev, m, n):
    """Qwen3-32B layer shapes (5120 = 5 x 1024, 25600 = 25 x 1024), batch 1 and 8."""
    _check_shape(dev, m, n, [1, 8], 1, m + 7 * n)


@pytest.mark.gpu
@pytest.mark.parametrize("m,n", [(4096, 4096), (11008, 4096), (4096, 11008), (1536, 768)])
@pytest.mark.parametrize("B", [1, 2, 16, 24])
def test_packed_sign_bits_bit_identical(dev, m, n, B):
    """su / sv as packed sign bits (QS_SIGNS_BITS) give outputs bit-identical
    to the fp32 sign vectors, single and grouped, on every path (one launch at
    1-2 rows, the batched passes, the wide GEMM)."""
    from quipsharp_amd.quantize import forward_packed, forward_packed_group, pack_signs
    print(f"case: sign bits m={m} n={n} B={B}", flush=True)
    rng = np.random.default_rng(77 + B)
    lins = [_rand_linear(dev, rng, m, n, stages=s, bias=bool(s - 1)) for s in (1, 2)]
    x = torch.from_numpy(rng.standard_normal((B, n)).astype(np.float32)).to(dev).bfloat16()
    for lin in lins:
        packed, su, sv, s0, s1, ls, bias = lin
        bits = (packed, pack_signs(su), pack_signs(sv), s0, s1, ls, bias)
        want = forward_packed(x, packed, su, sv, s0, s1, ls, bias)
        got = forward_packed(x, packed, bits[1], bits[2], s0, s1, ls, bias)
        assert torch.equal(got, want)
        g_want = forward_packed_group(x, [lin, lin])
        g_got = forward_packed_group(x, [bits, bits])
        for a, b in zip(g_got, g_want):
            assert torch.equal(a, b)
        assert torch.equal(g_want[0], want)


@pytest.mark.gpu
def test_packed_sign_bits_rejected_outside_chunk_scheme(dev):
    from quipsharp_amd._lib import QuipHipError
    from quipsharp_amd.quantize import forward_packed, pack_signs
    rng = np.random.default_rng(9)
    packed, su, sv, s0, s1, ls, bias = _rand_linear(dev, rng, 13312, 1024)  # m = 52 chunks of 256, beyond 48
    x3 = torch.randn(3, 1024, device=dev)  # three rows: the multi-row kernels' chunk scheme ends at 48
    forward_packed(x3, packed, su, sv, s0, s1, ls)
    with pytest.raises(QuipHipError):
        forward_packed(x3, packed, pack_signs(su), pack_signs(sv), s0, s1, ls)
    x = torch.randn(1, 1024, device=dev)  # one row: the one-launch kernel takes them
    assert torch.equal(forward_packed(x, packed, pack_signs(su), pack_signs(sv), s0, s1, ls),
                       forward_packed(x, packed, su, sv, s0, s1, ls))
    with pytest.raises(ValueError):
        forward_packed(x, packed, pack_signs(su), sv, s0, s1, ls)
    from quipsharp_amd.quantize import forward_packed_group
    rng2 = np.random.default_rng(10)
    a = _rand_linear(dev, rng2, 1024, 1024)
    bits = (a[0], pack_signs(a[1]), pack_signs(a[2])) + a[3:]
    with pytest.raises(ValueError, match="one format"):       # refused on the host
        forward_packed_group(x, [bits, a])
    # and by the library itself, for callers of the C ABI
    from quipsharp_amd import _lib
    y = torch.empty(2, 1, 1024, device=dev)
    jobs = (_lib.LinearJob * 2)()
    for g, (lin, fmt) in enumerate(((bits, 1), (a, 0))):
        jobs[g] = _lib.LinearJob(lin[0].codes0.data_ptr(), None, 1024, lin[1].data_ptr(), lin[2].data_ptr(), 1, None,
                                 lin[3], lin[4], lin[5], None, y[g].data_ptr(), 1024, fmt)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    rc = _lib.lib().qs_linear_forward_group(_lib.ptr(x), _lib.QS_DTYPE_F32, 1024, 1, 1024, 1, None, 2, jobs,
                                            _lib.QS_DTYPE_F32, _lib.ptr(ws), ws.numel(), None, None,
                                            _lib.stream_of(x))
    assert rc == 1 and b"same sign format" in _lib.lib().qs_last_error()
