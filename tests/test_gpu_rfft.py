"""GPU parity for the reference's RFFT layers (quipsharp/rfft.py): transforms
against the reference's golden outputs, the decode-matvec without
transforms, the RFFT forward against a dense fp64 oracle, and checkpoint
save / load of RFFT and Hadamard layers."""
import numpy as np
import pytest
import torch

from conftest import golden
from oracle import cref

pytestmark = pytest.mark.gpu


def test_rfft_transforms_golden(dev):
    from quipsharp_amd.rfft import from_transformed_space, to_transformed_space
    g = golden("rfft.npz")
    phase = torch.view_as_complex(torch.from_numpy(g["phase"])).to(dev)
    x = torch.from_numpy(g["x"]).to(dev)
    fwd = to_transformed_space(x, phase).cpu().numpy()
    inv = from_transformed_space(x, phase).cpu().numpy()
    scale = np.abs(g["fwd"]).max()
    assert np.abs(fwd - g["fwd"]).max() <= 1e-5 * scale
    assert np.abs(inv - g["inv"]).max() <= 1e-5 * np.abs(g["inv"]).max()
    # exact inverse up to rounding, along another dim too
    y = torch.randn(6, 2 * phase.shape[0], 3, device=dev)
    back = from_transformed_space(to_transformed_space(y, phase, dim=1), phase, dim=1)
    assert torch.allclose(back, y, atol=1e-5)


@pytest.mark.parametrize("m,n,B", [(4096, 4096, 1), (11008, 4096, 2), (4096, 11008, 3), (512, 96, 5)])
def test_decode_matvec_identity(dev, m, n, B):
    """qs_decode_matvec = layer_scale * W_hat @ x (fp64 oracle), tiled and row-major layouts."""
    from quipsharp_amd.quantize import PackedCodes, decode_matvec
    rng = np.random.default_rng(m + n + B)
    codes = rng.integers(0, 65536, (m, n // 8))
    packed = PackedCodes(torch.from_numpy(codes).to(dev), m, n, [0])
    x = rng.standard_normal((B, n)).astype(np.float32)
    y = decode_matvec(torch.from_numpy(x).to(dev), packed, 1.0, 0.0, 0.0135, out_dtype=torch.float32)
    W = cref.e8p_decode(codes).reshape(m, n).astype(np.float64)
    want = x.astype(np.float64) @ W.T * 0.0135
    err = np.linalg.norm(y.cpu().numpy() - want) / np.linalg.norm(want)
    assert err < 1e-3, err


def test_rfft_quantized_linear_forward(dev):
    """An RFFT-transformed QuantizedLinear (the reference's format for
    non-power-of-two dims) against su/sv-free dense fp64 math."""
    from quipsharp_amd.checkpoint import QuantizedLinear, build_codebook
    from quipsharp_amd.rfft import random_phase
    m, n = 11008, 4096
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 65536, (m, n // 8))
    g = torch.Generator().manual_seed(3)
    pu, pv = random_phase(m // 2, generator=g), random_phase(n // 2, generator=g)
    mod = QuantizedLinear(n, m, 8, "rfft", has_bias=True)
    with torch.no_grad():
        mod.codes.copy_(torch.from_numpy(codes.astype(np.int64)).to(torch.int16))
        mod.scale.fill_(0.0135)
        mod.phase_u.copy_(pu)
        mod.phase_v.copy_(pv)
        mod.bias.copy_(torch.from_numpy(rng.standard_normal(m).astype(np.float32)))
    mod = mod.to(dev)
    mod.codebook, _ = build_codebook("2bit", dev, 0)
    x = torch.from_numpy(rng.standard_normal((2, n)).astype(np.float32))
    y = mod(x.to(dev).bfloat16()).float().cpu().numpy()
    # fp64 oracle: the reference's transforms in complex128
    def enter(v, ph):
        c = v[..., 0::2] + 1j * v[..., 1::2]
        f = np.fft.fft(c * ph, norm="ortho")
        return np.stack([f.real, f.imag], -1).reshape(v.shape)
    def leave(v, ph):
        c = v[..., 0::2] + 1j * v[..., 1::2]
        f = np.fft.ifft(c, norm="ortho") * np.conj(ph)
        return np.stack([f.real, f.imag], -1).reshape(v.shape)
    xb = x.bfloat16().double().numpy()
    W = cref.e8p_decode(codes).reshape(m, n).astype(np.float64) * mod.codebook.native_stages()[1][0]
    y1 = enter(xb, pv.numpy().astype(np.complex128)) @ W.T * float(np.float32(0.0135))
    want = leave(y1, pu.numpy().astype(np.complex128)) + mod.bias.cpu().double().numpy()
    assert np.all(np.abs(y - want) <= 2 ** -8 * np.abs(want) + 2e-3 * np.abs(want).max())


def test_checkpoint_round_trip(dev, tmp_path):
    """save_quantized_checkpoint / load_quantized_checkpoint with an RHT and an
    RFFT layer: same buffers, same outputs."""
    from torch import nn
    from quipsharp_amd.checkpoint import (QuantizedLinear, build_codebook, is_quantized_checkpoint,
                                          load_quantized_checkpoint, save_quantized_checkpoint)
    from quipsharp_amd.rfft import random_phase

    class Net(nn.Module):
        def __init__(self):
            super().__init__()
            self.a = nn.Linear(512, 256, bias=False)
            self.b = nn.Linear(256, 768, bias=True)

    rng = np.random.default_rng(2)
    net = Net()
    cb, _ = build_codebook("2bit", dev, 0)
    qa = QuantizedLinear(512, 256, 8, "rht")
    qb = QuantizedLinear(256, 768, 8, "rfft", has_bias=True)
    with torch.no_grad():
        for q, (m, n) in ((qa, (256, 512)), (qb, (768, 256))):
            q.codes.copy_(torch.from_numpy(rng.integers(0, 65536, (m, n // 8)).astype(np.int64)).to(torch.int16))
            q.scale.fill_(0.02)
        qa.su.copy_(torch.from_numpy(rng.choice([-1.0, 1.0], 256).astype(np.float32)))
        qa.sv.copy_(torch.from_numpy(rng.choice([-1.0, 1.0], 512).astype(np.float32)))
        g = torch.Generator().manual_seed(0)
        qb.phase_u.copy_(random_phase(384, generator=g))
        qb.phase_v.copy_(random_phase(128, generator=g))
        qb.bias.copy_(torch.from_numpy(rng.standard_normal(768).astype(np.float32)))
    net.a, net.b = qa, qb
    net = net.to(dev)
    for q in (net.a, net.b):
        q.codebook = cb
    x = torch.randn(3, 512, device=dev)
    want = net.b(net.a(x))
    mods = [{"name": "a", "in_features": 512, "out_features": 256, "transform_kind": "rht", "has_bias": False},
            {"name": "b", "in_features": 256, "out_features": 768, "transform_kind": "rfft", "has_bias": True}]
    save_quantized_checkpoint(net, "local/test", tmp_path, "2bit", 8, 0, mods)
    assert is_quantized_checkpoint(tmp_path)
    with torch.device("meta"):
        skel = Net()
    loaded = load_quantized_checkpoint(tmp_path, device=dev, model=skel)
    got = loaded.b(loaded.a(x))
    assert torch.equal(got, want)
    for k, v in net.state_dict().items():
        assert torch.equal(loaded.state_dict()[k], v), k


def test_quantize_with_rfft_transform(dev):
    """quantize_linear(transform="rfft") takes the reference's branch for
    non-power-of-two dims; the forward of the result equals x @ W_q^T with
    W_q reconstructed through the inverse transforms."""
    from quipsharp_amd.checkpoint import QuantizedLinear, build_codebook
    from quipsharp_amd.quantize import linear_forward, quantize_linear
    from quipsharp_amd.rfft import RFFTPhases
    g = torch.Generator().manual_seed(0)
    m, n = 384, 768
    W = (torch.randn(m, n, generator=g) * 0.02).to(dev)
    X = torch.randn(1024, n, generator=g).to(dev)
    H = X.T @ X / 1024
    cb, s = build_codebook("2bit", dev, 0)
    layer, what_q = quantize_linear(W, H, cb, codebook_scale=s, tune_iters=2, transform="rfft",
                                    generator=torch.Generator().manual_seed(1))
    assert isinstance(layer.signs, RFFTPhases)
    Wq = layer.signs.reconstruct_weight(what_q)
    rel = ((Wq - W).norm() / W.norm()).item()
    assert rel < 0.5, rel
    x = torch.randn(4, n, device=dev)
    y = linear_forward(x, layer, cb)
    want = x @ Wq.T
    assert ((y - want).norm() / want.norm()).item() < 1e-3
    mod = QuantizedLinear.from_quantized_layer(layer).to(dev)
    mod.codebook = cb
    assert ((mod(x) - want).norm() / want.norm()).item() < 1e-3
