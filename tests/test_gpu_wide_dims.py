"""GPU parity of the one-launch forward beyond 12288: n and m up to 32768 =
128 chunks of 256 at 1-2 rows (the Llama-3-8B 14336, Qwen2.5-7B 18944,
Qwen3-32B 25600 and Llama-2-70B 28672 intermediates), with the input
transform chunk combination first and the output transform in two levels.
Against the dense fp64 oracle (tolerance: relative 1e-3, norm-wise, as for
every forward), and bit-identity between sign formats, single and grouped
calls."""
import numpy as np
import pytest
import torch

from test_gpu_linear import REL_TOL, T64, _dense_weights, _rand_linear, rel_err

pytestmark = pytest.mark.gpu


def _oracle_case(dev, m, n, B, stages, seed, dtype=torch.bfloat16, bias=False):
    from quipsharp_amd.quantize import PackedCodes, forward_packed
    rng = np.random.default_rng(seed)
    c0 = rng.integers(0, 65536, (m, n // 8))
    c1 = rng.integers(0, 256, (m, n // 8)) if stages == 2 else None
    su, sv = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    s0, s1, scale = (0.93, 0.41, 0.011) if stages == 2 else (1.0, 0.0, 0.0135)
    bv = rng.standard_normal(m) if bias else None
    c = torch.from_numpy(c0).to(dev)
    if c1 is not None:
        c = torch.stack([c, torch.from_numpy(c1).to(dev)])
    packed = PackedCodes(c, m, n, [0] if c1 is None else [0, 1])
    t = lambda a: None if a is None else torch.from_numpy(np.asarray(a, dtype=np.float32)).to(dev)
    x = torch.from_numpy(rng.standard_normal((B, n)).astype(np.float32)).to(dev).to(dtype)
    y = forward_packed(x, packed, t(su), t(sv), s0, s1, scale, bias=t(bv), out_dtype=torch.float32)
    W = _dense_weights(c0, c1, s0, s1)
    want = T64(T64(x.double().cpu().numpy() * sv) @ W.T * scale) * su
    if bv is not None:
        want = want + bv
    return rel_err(y.cpu().numpy(), want)


@pytest.mark.parametrize("m,n", [
    (1024, 25600),   # 100 input chunks (two rounds of activation loads), K_25 (x) H_4 across chunks
    (25600, 1024),   # 100 output chunks: two-level output transform with K_25
    (256, 32768),    # 128 input chunks, Hadamard only
    (32768, 256),    # 128 output chunks
    (768, 18944),    # 74 input chunks, K_37 (x) H_2
    (14336, 512),    # 56 output chunks, K_7 (x) H_8
    (28672, 512),    # 112 output chunks, K_7 (x) H_16
])
@pytest.mark.parametrize("B", [1, 2])
def test_wide_dims_vs_dense(dev, m, n, B):
    print(f"case: wide dims m={m} n={n} B={B} bf16", flush=True)
    err = _oracle_case(dev, m, n, B, 1, m + 3 * n + B, bias=(B == 2))
    print(f"  rel err {err:.2e}", flush=True)
    assert err < REL_TOL, (m, n, B, err)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("m,n", [(512, 16384), (20480, 768)])
def test_wide_dims_fp16_fp32_activations(dev, dtype, m, n):
    """fp16 / fp32 activations keep a second (low-part) chunk table plane, so
    the one-launch kernel takes n up to 16384 for them."""
    print(f"case: wide dims m={m} n={n} {dtype}", flush=True)
    for B in (1, 2):
        err = _oracle_case(dev, m, n, B, 1, m + n + B, dtype=dtype)
        print(f"  B={B} rel err {err:.2e}", flush=True)
        assert err < REL_TOL, (m, n, B, dtype, err)


def test_wide_dims_rvq3(dev):
    """Two-stage codes (E8P + E8 1-bit) at 14336 x 4096-like widths."""
    for m, n in ((1024, 14336), (14336, 1024)):
        print(f"case: wide dims rvq3 m={m} n={n}", flush=True)
        err = _oracle_case(dev, m, n, 1, 2, m + n)
        print(f"  rel err {err:.2e}", flush=True)
        assert err < REL_TOL, (m, n, err)


@pytest.mark.parametrize("m,n", [(25600, 1024), (1024, 25600), (14336, 14336)])
@pytest.mark.parametrize("B", [1, 2])
def test_wide_dims_sign_bits_and_groups(dev, m, n, B):
    """Packed sign bits are taken by the one-launch kernel at these sizes and
    give outputs bit-identical to fp32 signs; grouped outputs equal single
    calls."""
    from quipsharp_amd.quantize import forward_packed, forward_packed_group, pack_signs, sign_bits_ok
    print(f"case: wide dims bits/group m={m} n={n} B={B}", flush=True)
    rng = np.random.default_rng(m + n + 11 * B)
    lins = [_rand_linear(dev, rng, m, n, bias=True), _rand_linear(dev, rng, m, n)]
    x = torch.from_numpy(rng.standard_normal((B, n)).astype(np.float32)).to(dev).bfloat16()
    assert sign_bits_ok(x, m, n)
    want = [forward_packed(x, *lin) for lin in lins]
    bits = [(lin[0], pack_signs(lin[1]), pack_signs(lin[2])) + lin[3:] for lin in lins]
    for lin, w in zip(bits, want):
        assert torch.equal(forward_packed(x, *lin), w)
    for group in (lins, bits):
        for y, w in zip(forward_packed_group(x, group), want):
            assert torch.equal(y, w)


def test_wide_dims_rows_beyond_one_launch(dev):
    """Three rows at n = 25600: outside every multi-row kernel's chunk scheme,
    the grouped call runs one forward per linear (equal to single calls), and
    packed sign bits are refused there."""
    from quipsharp_amd._lib import QuipHipError
    from quipsharp_amd.quantize import forward_packed, forward_packed_group, pack_signs, sign_bits_ok
    rng = np.random.default_rng(3)
    lins = [_rand_linear(dev, rng, 1024, 25600), _rand_linear(dev, rng, 512, 25600, bias=True)]
    x = torch.randn(3, 25600, device=dev).bfloat16()
    ys = forward_packed_group(x, lins)
    for lin, y in zip(lins, ys):
        assert torch.equal(y, forward_packed(x, *lin))
    assert not sign_bits_ok(x, 1024, 25600)
    packed, su, sv, s0, s1, ls, b = lins[0]
    with pytest.raises(QuipHipError):
        forward_packed(x, packed, pack_signs(su), pack_signs(sv), s0, s1, ls)


def test_wide_dims_graph_replays(dev):
    """The two-level output transform under HIP graph replay: every replay
    equals the eager call (the tags advance per launch, the chunk-transform
    slots of the previous launch never pass for this one's)."""
    from quipsharp_amd.quantize import forward_packed_group
    rng = np.random.default_rng(21)
    lins = [_rand_linear(dev, rng, 25600, 1024), _rand_linear(dev, rng, 25600, 1024, bias=True)]
    x = torch.randn(1, 1024, device=dev).bfloat16()
    ws = torch.zeros(1 << 24, dtype=torch.uint8, device=dev)
    outs = [torch.empty(1, 25600, device=dev, dtype=torch.bfloat16) for _ in lins]
    eager = [y.clone() for y in forward_packed_group(x, lins, workspace=ws)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        forward_packed_group(x, lins, workspace=ws, outs=outs)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            forward_packed_group(x, lins, workspace=ws, outs=outs)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(4):
        for o in outs:
            o.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), rep


@pytest.mark.parametrize("m,n", [(5120, 25600), (5120, 8192), (8192, 5120)])
def test_qwen3_32b_shapes_bf16_one_launch(dev, m, n):
    """Qwen3-32B's down (n = 25600: 7 slice groups into the two-level output
    transform), o and q shapes with bf16 activations on the one-launch path."""
    for B in (1, 2):
        print(f"case: qwen3 shape m={m} n={n} B={B} bf16", flush=True)
        err = _oracle_case(dev, m, n, B, 1, 5 * m + n + B, bias=(B == 2))
        print(f"  rel err {err:.2e}", flush=True)
        assert err < REL_TOL, (m, n, B, err)


def test_shared_workspace_across_job_lists(dev):
    """One workspace for grouped calls with different job lists and single
    calls (a decoder layer's q+k+v, o, gate+up, down at Qwen3-32B shapes, as
    a caller that keeps one workspace may issue them), eager and replayed
    from a HIP graph: every output equals its own call on a fresh workspace."""
    from quipsharp_amd.quantize import forward_packed, forward_packed_group
    rng = np.random.default_rng(32)
    shapes = {"q": (8192, 5120), "k": (1024, 5120), "v": (1024, 5120), "o": (5120, 8192),
              "gate": (25600, 5120), "up": (25600, 5120), "down": (5120, 25600)}
    lin = {k: _rand_linear(dev, rng, m, n, bias=(k == "o")) for k, (m, n) in shapes.items()}
    plan = [("q", "k", "v"), ("o",), ("gate", "up"), ("down",)]
    src = {"q": "x", "o": "q", "gate": "o", "down": "gate"}
    x = torch.randn(1, 5120, device=dev).bfloat16()
    buf = {k: torch.empty(1, m, device=dev, dtype=torch.bfloat16) for k, (m, _) in shapes.items()}
    buf["x"] = x
    import ctypes
    from quipsharp_amd import _lib
    L = _lib.lib()
    need = max(L.qs_linear_group_workspace_bytes(shapes[g[0]][1], 1, len(g),
                                                (ctypes.c_int64 * len(g))(*[shapes[k][0] for k in g]))
               for g in plan)
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)

    def step(layers=3):
        for _ in range(layers):
            for g in plan:
                forward_packed_group(buf[src[g[0]]], [lin[k] for k in g], workspace=ws, outs=[buf[k] for k in g])
            forward_packed(buf["o"], *lin["gate"], workspace=ws, out=buf["gate"])  # a single call in between

    # the same chain with a fresh workspace per call
    want = {}
    cur = {"x": x}
    for _ in range(3):
        for g in plan:
            ys = forward_packed_group(cur[src[g[0]]], [lin[k] for k in g])
            cur.update(dict(zip(g, ys)))
        cur["gate"] = forward_packed(cur["o"], *lin["gate"])
    want = {k: v.clone() for k, v in cur.items()}
    step()
    torch.cuda.synchronize()
    for k in shapes:
        assert torch.equal(buf[k], want[k]), ("eager", k)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(4):
        for k in shapes:
            buf[k].fill_(0)
        g.replay()
        torch.cuda.synchronize()
        for k in shapes:
            assert torch.equal(buf[k], want[k]), (rep, k)


@pytest.mark.parametrize("m,n", [
    (25600, 1024),   # output: 100 chunks, K_25 (x) H_4, 7 work-groups per row
    (1024, 25600),   # input: 100 chunks over 7 slice groups of 16
    (14336, 512),    # K_7 (x) H_8
    (768, 18944),    # K_37 (x) H_2
    (32768, 256),    # 128 output chunks, Hadamard only
    (256, 32768),    # 128 input chunks
    (28672, 512),    # K_7 (x) H_16
])
@pytest.mark.parametrize("B", [3, 8, 16, 40])
def test_wide_dims_multi_row(dev, m, n, B):
    """Three rows and more beyond 12288: the per-row transforms run as
    work-groups of 16 chunks (qs_linear_big.hip) around the 16-row
    decode-matvec (3-16 rows) or the wide GEMM (40 rows)."""
    print(f"case: wide dims multi-row m={m} n={n} B={B} bf16", flush=True)
    err = _oracle_case(dev, m, n, B, 1, m + 5 * n + B, bias=(B == 8))
    print(f"  rel err {err:.2e}", flush=True)
    assert err < REL_TOL, (m, n, B, err)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_wide_dims_multi_row_fp16_fp32(dev, dtype):
    """fp16 / fp32 rows: the 16-chunk input kernel keeps a low-part plane (n up
    to 16384); beyond that the row kernel of any length takes them."""
    for m, n, B in ((512, 16384, 5), (512, 18944, 4), (14336, 1024, 6)):
        print(f"case: wide dims multi-row m={m} n={n} B={B} {dtype}", flush=True)
        err = _oracle_case(dev, m, n, B, 1, m + n + B, dtype=dtype)
        print(f"  rel err {err:.2e}", flush=True)
        assert err < REL_TOL, (m, n, B, dtype, err)


def test_wide_dims_multi_row_rvq3(dev):
    for m, n, B in ((1024, 14336, 4), (14336, 1024, 16)):
        print(f"case: wide dims multi-row rvq3 m={m} n={n} B={B}", flush=True)
        err = _oracle_case(dev, m, n, B, 2, m + n + B)
        print(f"  rel err {err:.2e}", flush=True)
        assert err < REL_TOL, (m, n, B, err)


@pytest.mark.parametrize("B", [8, 40])
def test_wide_dims_multi_row_group_equals_single(dev, B):
    """Linears of one input with outputs beyond 12288 (gate / up of the
    Qwen3-32B MLP) share one output-transform launch; each output equals its
    single call bit for bit."""
    from quipsharp_amd.quantize import forward_packed, forward_packed_group
    rng = np.random.default_rng(41 + B)
    lins = [_rand_linear(dev, rng, 25600, 1024, bias=True), _rand_linear(dev, rng, 25600, 1024),
            _rand_linear(dev, rng, 4096, 1024)]
    x = torch.from_numpy(rng.standard_normal((B, 1024)).astype(np.float32)).to(dev).bfloat16()
    ys = forward_packed_group(x, lins)
    for lin, y in zip(lins, ys):
        assert torch.equal(y, forward_packed(x, *lin))
