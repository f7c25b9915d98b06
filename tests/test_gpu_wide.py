"""GPU parity of the wide-batch forward (17 or more activation rows: the codes
are decoded into fp16 weight chunks once per call and multiplied on the
matrix cores) against the dense fp64 oracle.  Tolerance: relative 1e-3
(norm-wise), as for the narrow paths; the dequantized weights are exact in
fp16, so the error is the fp16 operand rounding and fp32 accumulation."""
import numpy as np
import pytest
import torch

from test_gpu_linear import REL_TOL, T64, _dense_weights, dense_forward, rel_err, run

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n,B", [
    (4096, 4096, 17),     # smallest wide batch: one tile per wave, three waves idle
    (4096, 4096, 32),     # one tile per wave for two waves
    (4096, 4096, 100),    # batch not a multiple of 16
    (11008, 4096, 48),    # odd-factor outputs (43 x 256), 86 weight row tiles
    (4096, 11008, 40),    # odd-factor inputs: 43 slices in 3 slice groups of 15, 15, 13
    (768, 512, 33),       # small: one chunk shorter than the chunk size
    (256, 256, 40),       # one slice, one weight row tile (two 16-row blocks past the end)
    (1024, 2048, 300),    # four activation tiles per wave, ragged last work-group column
    (2048, 1024, 129),    # two tiles per wave, one row past a tile
    (1024, 2048, 500),    # two work-group columns of 256 rows, the second ragged
    (784, 1024, 420),     # 49 row blocks: the last work-group row holds one; m = 49 x 16
    (4096, 2048, 300),    # 64 work-group tiles: K split in 4 slice groups (the 4-group output kernel)
    (1024, 2048, 1031),   # more rows than two transform work-groups per CU: two or three rows each
    (512, 11008, 515),    # three chunks per wave in the transforms, two or three rows per work-group
])
def test_wide_vs_dense_fp64(dev, m, n, B):
    print(f"case: wide m={m} n={n} B={B}", flush=True)
    rng = np.random.default_rng(m * 3 + n + B)
    codes = rng.integers(0, 65536, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    x = rng.standard_normal((B, n)).astype(np.float32)
    y, packed = run(dev, x, codes, None, 1.0, 0.0, su, sv, 0.0135)
    assert packed.layout == 1
    want = dense_forward(x, codes, None, 1.0, 0.0, su, sv, 0.0135)
    err = rel_err(y.cpu().numpy(), want)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < REL_TOL


@pytest.mark.parametrize("m,n,B", [(4096, 4096, 64), (14336, 4096, 33), (2048, 1024, 200)])
def test_wide_rvq3_vs_dense(dev, m, n, B):
    """3-bit residual VQ: the E8 1-bit stage is a second set of MFMAs and
    accumulators, combined with its own scale at the end (14336 = 7 x 2048
    output rows; 200 rows: two tiles per wave)."""
    print(f"case: wide rvq3 m={m} n={n} B={B}", flush=True)
    rng = np.random.default_rng(m + B)
    c0 = rng.integers(0, 65536, (m, n // 8))
    c1 = rng.integers(0, 256, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    x = rng.standard_normal((B, n)).astype(np.float32)
    y, _ = run(dev, x, c0, c1, 0.93, 0.41, su, sv, 0.011)
    want = dense_forward(x, c0, c1, 0.93, 0.41, su, sv, 0.011)
    err = rel_err(y.cpu().numpy(), want)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < REL_TOL


@pytest.mark.parametrize("m,n,B", [(25600, 5120, 32), (5120, 25600, 32)])
def test_wide_large_factor_shapes(dev, m, n, B):
    """Qwen3-32B MLP shapes: 25600 = 25 x 1024 is transformed by the
    LDS-radix row kernels, not the chunk-scheme ones."""
    print(f"case: wide m={m} n={n} B={B}", flush=True)
    rng = np.random.default_rng(m + 5 * n)
    c0 = rng.integers(0, 65536, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    W = _dense_weights(c0, None, 1.0, 0.0)
    x = rng.standard_normal((B, n)).astype(np.float32)
    y, _ = run(dev, x, c0, None, 1.0, 0.0, su, sv, 0.0135)
    want = T64(T64(x.astype(np.float64) * sv) @ W.T * 0.0135) * su
    err = rel_err(y.cpu().numpy(), want)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < REL_TOL


def test_wide_bf16_strided_bias(dev):
    """bf16 activations read through a row stride, bf16 output, bias, and a
    sign vector that is not 16-byte aligned (the LDS-radix input kernel)."""
    m, n, B = 11008, 4096, 40
    print(f"case: wide bf16 strided m={m} n={n} B={B}", flush=True)
    rng = np.random.default_rng(77)
    codes = rng.integers(0, 65536, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    bias = rng.standard_normal(m).astype(np.float32)
    x = rng.standard_normal((B, n)).astype(np.float32)
    xb = torch.zeros(B, n + 64, dtype=torch.bfloat16, device=dev)
    xb[:, :n] = torch.from_numpy(x).to(dev)
    xs = xb[:, :n]
    x_used = xs.float().cpu().numpy()
    y, packed = run(dev, xs, codes, None, 1.0, 0.0, su, sv, 0.0135, bias=bias, out_dtype=torch.bfloat16)
    assert y.dtype == torch.bfloat16
    want = dense_forward(x_used, codes, None, 1.0, 0.0, su, sv, 0.0135, bias)
    err = rel_err(y.float().cpu().numpy(), want)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < 1e-2  # bf16 output rounding

    from quipsharp_amd.quantize import forward_packed
    svt = torch.from_numpy(np.concatenate([[0.0], sv]).astype(np.float32)).to(dev)[1:]
    sut = torch.from_numpy(su.astype(np.float32)).to(dev)
    y2 = forward_packed(torch.from_numpy(x).to(dev), packed, sut, svt, 1.0, 0.0, 0.0135,
                        bias=torch.from_numpy(bias).to(dev), out_dtype=torch.float32)
    err2 = rel_err(y2.cpu().numpy(), dense_forward(x, codes, None, 1.0, 0.0, su, sv, 0.0135, bias))
    print(f"  unaligned sv: rel err {err2:.2e}", flush=True)
    assert err2 < REL_TOL


def test_wide_matches_narrow_path(dev):
    """The first 16 rows of a wide call agree with a 16-row (batched path)
    call on the same rows."""
    m, n = 4096, 4096
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 65536, (m, n // 8))
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    x = rng.standard_normal((64, n)).astype(np.float32)
    yw, _ = run(dev, x, codes, None, 1.0, 0.0, su, sv, 0.0135)
    yn, _ = run(dev, x[:16], codes, None, 1.0, 0.0, su, sv, 0.0135)
    assert rel_err(yw[:16].cpu().numpy(), yn.cpu().numpy().astype(np.float64)) < 2e-4


@pytest.mark.parametrize("shapes,n,B", [
    ([4096, 4096, 4096], 4096, 300),  # 3 x 64 tiles: one shared launch, one slice group (4 alone)
    ([2048, 2048], 2048, 140),        # 2 x 16 tiles: one shared launch, 8 slice groups as alone
    ([11008, 11008], 4096, 300),      # 2 x 172 tiles, more than one round: one launch each
    ([4096, 1024], 4096, 300),        # two shapes: one launch each
])
def test_wide_group_shared_gemm(dev, shapes, n, B):
    """Linears of one shape above 128 rows whose GEMM tiles fit one round over
    the CUs share one wp_kernel launch, with the slice groups chosen for the
    group: each output equals the single call up to the fp32 summation order
    (bit-identical when they take one launch each) and matches the dense fp64
    oracle."""
    print(f"case: wide group {shapes} n={n} B={B}", flush=True)
    from test_gpu_linear import _rand_linear
    from quipsharp_amd.quantize import forward_packed, forward_packed_group
    seed = sum(shapes) + n + B + 5
    rng = np.random.default_rng(seed)
    lins = [_rand_linear(dev, rng, m, n, 1, True) for m in shapes]
    x = torch.randn(B, n, generator=torch.Generator().manual_seed(seed)).to(dev).bfloat16()
    ys = forward_packed_group(x, lins)
    # the library's choice (wide_group_splits): one shape, 4 column tiles per
    # work-group (B > 128), and the group's GEMM tiles of 128 rows x 256
    # columns fit one round over the device's CUs
    ncu = torch.cuda.get_device_properties(dev).multi_processor_count
    tiles = -(-shapes[0] // 128) * -(-B // 256) * len(shapes)
    shared = len(set(shapes)) == 1 and B > 128 and tiles <= ncu
    for lin, y in zip(lins, ys):
        want = forward_packed(x, *lin)
        assert y.shape == want.shape
        if shared:
            a, b = y.float().cpu().numpy(), want.float().cpu().numpy()
            assert np.all(np.abs(a - b) <= 2 ** -7 * np.abs(b) + 1e-4 * np.abs(b).max())
        else:
            assert torch.equal(y, want)
    # the first linear against the dense oracle (its draws repeated)
    rng2 = np.random.default_rng(seed)
    m0 = shapes[0]
    c0 = rng2.integers(0, 65536, (m0, n // 8))
    su_np = rng2.choice([-1.0, 1.0], m0)
    sv_np = rng2.choice([-1.0, 1.0], n)
    b_np = rng2.standard_normal(m0).astype(np.float32)
    packed, su, sv, s0, s1, sc, b = lins[0]
    want = dense_forward(x.float().cpu().numpy(), c0, None, s0, 0.0, su_np, sv_np, sc, b_np)
    got = ys[0].float().cpu().numpy()  # bf16 outputs: half an ulp of bf16 on top of the forward's error
    print(f"  rel err {rel_err(got, want):.2e}", flush=True)
    assert np.all(np.abs(got - want) <= 2 ** -8 * np.abs(want) + 2e-3 * np.abs(want).max())
