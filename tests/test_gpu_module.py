"""GPU: QuantizedLinear drop-in behaviour and row independence of the forward.

* A non-finite activation row must not reach the other rows' outputs (the
  reference computes rows independently: quipsharp/quantize.py:116-124).
* After ``.half()`` / ``.to(torch.bfloat16)`` the module keeps the reference's
  semantics (quipsharp/checkpoint.py:131-146): buffers take the new dtype, the
  forward promotes signs and bias to fp32 and reads the rounded scale.
* Linears grouped by the library whose signs cannot all be packed bits (an
  output size off the chunk scheme) still run, eagerly and under capture.
* A buffer changed in place and next used under HIP graph capture.
* ``replace_with_quantized_linear_`` (quipsharp/checkpoint.py:149-156)."""
import copy

import pytest
import torch

pytestmark = pytest.mark.gpu


def _layer(dev, m, n, seed):
    from quipsharp_amd.hadamard import is_pow2
    from quipsharp_amd.incoherence import IncoherenceSigns, KronSigns
    from quipsharp_amd.quantize import QuantizedLayer
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 65536, (m, n // 8), generator=g)
    su = torch.randint(0, 2, (m,), generator=g).float() * 2 - 1
    sv = torch.randint(0, 2, (n,), generator=g).float() * 2 - 1
    cls = IncoherenceSigns if is_pow2(m) and is_pow2(n) else KronSigns
    return QuantizedLayer(codes=codes.to(dev), signs=cls(su=su.to(dev), sv=sv.to(dev)), g=8, shape=(m, n),
                          scale=0.0135)


def _qlin(dev, m, n, seed, bias=False):
    from quipsharp_amd.checkpoint import QuantizedLinear
    from quipsharp_amd.codebooks.e8p import E8PCodebook
    b = torch.randn(m, generator=torch.Generator().manual_seed(seed + 1)).to(dev) if bias else None
    q = QuantizedLinear.from_quantized_layer(_layer(dev, m, n, seed), bias=b).to(dev)
    q.codebook = E8PCodebook(device=dev)
    return q


@pytest.mark.parametrize("m,n", [(4096, 4096), (11008, 4096)])
@pytest.mark.parametrize("B", [2, 16, 24])
@pytest.mark.parametrize("bias", [False, True])
def test_nonfinite_row_stays_in_its_row(dev, m, n, B, bias):
    """Row 0 = +inf: rows 1.. are bit-identical to the same call with a finite
    row 0 (one-launch path at 2 rows, batched at 16, wide at 24)."""
    print(f"case: nonfinite row m={m} n={n} B={B} bias={bias}", flush=True)
    q = _qlin(dev, m, n, 7, bias)
    x = torch.randn(B, n, generator=torch.Generator().manual_seed(B)).to(dev).bfloat16()
    want = q(x)
    xi = x.clone()
    xi[0] = float("inf")
    got = q(xi)
    assert torch.equal(got[1:], want[1:])
    assert not torch.isfinite(got[0].float()).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_module_cast_keeps_reference_semantics(dev, dtype):
    """module.to(dtype): su / sv / bias / scale take dtype like the reference's
    buffers; the forward equals the fp32 module whose scale and bias hold the
    same rounded values, bit for bit."""
    from quipsharp_amd.checkpoint import grouped_forward
    for m, n in ((4096, 4096), (14336, 4096)):   # packed-sign and fp32-sign paths
        q = _qlin(dev, m, n, 3, bias=True)
        qc = copy.deepcopy(q).to(dtype)
        qc.codebook = q.codebook
        assert qc.su.dtype == dtype and qc.bias.dtype == dtype and qc.scale.dtype == dtype
        ref = copy.deepcopy(q)
        ref.codebook = q.codebook
        with torch.no_grad():
            ref.scale.copy_(q.scale.to(dtype).float())
            ref.bias.copy_(q.bias.to(dtype).float())
        for B in (1, 16, 24):
            x = torch.randn(B, n, device=dev).to(dtype)
            y = qc(x)
            assert y.dtype == dtype
            assert torch.equal(y, ref(x)), (m, n, B)
        assert torch.equal(grouped_forward(x, [qc])[0], ref(x))


@pytest.mark.parametrize("B", [1, 2, 16])
def test_grouped_mixed_output_sizes(dev, B):
    """A 4096-row member (packed sign bits) grouped with a 14336-row member
    (fp32 signs: 56 chunks of 256, off the chunk scheme): one sign format for
    the launch, each output bit-identical to its own call."""
    from quipsharp_amd.checkpoint import grouped_forward
    a = _qlin(dev, 4096, 4096, 11)
    b = _qlin(dev, 14336, 4096, 12, bias=True)
    assert a.signs()[0].dtype == torch.int32 and b.signs()[0].dtype == torch.float32
    x = torch.randn(B, 4096, device=dev).bfloat16()
    ya, yb = grouped_forward(x, [a, b])
    assert torch.equal(ya, a(x)) and torch.equal(yb, b(x))


@pytest.mark.parametrize("B", [1, 16])
def test_linked_mixed_group_under_capture(dev, B):
    """Linked siblings of mixed output sizes called one by one inside a HIP
    graph: the first call runs the grouped forward for both; every replay
    equals the eager outputs."""
    a = _qlin(dev, 4096, 4096, 21)
    b = _qlin(dev, 14336, 4096, 22)
    for mod in (a, b):
        mod._siblings = [a, b]
    x = torch.randn(B, 4096, device=dev).bfloat16()
    want_a, want_b = a(x).clone(), b(x).clone()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        a(x), b(x)          # warm-up outside capture: workspaces and packed signs exist
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ya = a(x)
        yb = b(x)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ya, want_a) and torch.equal(yb, want_b)
        a(x)                # eager work between replays
        torch.cuda.synchronize()


def test_changed_buffer_first_used_under_capture(dev):
    """A bf16 module whose bias changed in place after its last forward, next
    called under HIP graph capture: the fp32 copy of the bias is made uncached
    there (cached, it would live in the graph's pool, unwritten until a
    replay), so an eager call before the first replay, and every replay,
    equal a copy of the module run eagerly.  A forward that would have to pack
    the codes (the first after a cast) refuses capture with a clear error."""
    q = _qlin(dev, 4096, 4096, 31, bias=True).bfloat16()
    x = torch.randn(2, 4096, generator=torch.Generator().manual_seed(3)).to(dev).bfloat16()
    q(x)                    # workspace, packed codes and signs, fp32 copies
    torch.cuda.synchronize()
    with torch.no_grad():
        q.bias.add_(0.5)    # a new version of the bias
    want = copy.deepcopy(q)(x).clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = q(x)
    got = q(x)              # eager, before any replay
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    for _ in range(2):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want)
    q2 = _qlin(dev, 4096, 4096, 32).half()
    with pytest.raises(RuntimeError, match="run one forward outside capture first"):
        with torch.cuda.graph(torch.cuda.CUDAGraph()):
            q2(x.half())


def test_replace_with_quantized_linear(dev):
    """quipsharp/checkpoint.py:149-156: the parent's attribute becomes a
    QuantizedLinear built from the layer, the codebook is assigned, the bias
    is carried verbatim, and the forward is linear_forward(x) + bias."""
    from quipsharp_amd.checkpoint import QuantizedLinear, replace_with_quantized_linear_
    from quipsharp_amd.codebooks.e8p import E8PCodebook
    from quipsharp_amd.quantize import linear_forward
    parent = torch.nn.Module()
    parent.proj = torch.nn.Linear(512, 256)
    layer = _layer(dev, 256, 512, 5)
    cb = E8PCodebook(device=dev)
    bias = torch.randn(256, device=dev)
    q = replace_with_quantized_linear_(parent, "proj", layer, cb, bias=bias)
    assert parent.proj is q and isinstance(q, QuantizedLinear) and q.codebook is cb
    assert q.transform_kind == "rht" and (q.in_features, q.out_features) == (512, 256)
    assert torch.equal(q.bias.to(dev), bias)
    assert torch.equal(q.codes.to(torch.int64) & 0xFFFF, layer.codes.cpu())
    q = q.to(dev)
    x = torch.randn(3, 512, device=dev)
    assert torch.allclose(q(x), linear_forward(x, layer, cb) + bias, atol=1e-5, rtol=1e-5)
    nb = replace_with_quantized_linear_(parent, "proj", layer, cb)
    assert nb.bias is None and parent.proj is nb
