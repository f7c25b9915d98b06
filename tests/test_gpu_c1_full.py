"""GPU quantize of the full 4096 x 4096 layer against the reference's own run
(tests/golden/c1_full.npz, written by make_golden.py from
quipsharp/quantize.py:48-104 on the CPU): W = 0.02 N(0,1), H = X^T X / 2048
with X in R^{2048 x 4096}, x in R^4096, drawn from Generator().manual_seed(0)
in that order; torch.manual_seed(0) before quantize_linear; E8P 2-bit,
damping 1e-2, 10 refinement sweeps.

Codes cannot be bit-exact end to end (the feedback products and the Cholesky
factor come from rocBLAS / rocSOLVER instead of MKL, and one near-tie flip
changes the rest of its row's feedback), so the contract is: signs
bit-exact, the layer scale the same fp32 value, code agreement at least 99 %
(measured 0.9916), relative proxy loss tr(E H E^T) / tr(W H W^T) in the
transformed basis no worse than 1.01x the reference's (measured 1.000x; both
under the same H_hat, the reference's codes decoded bit-exactly), the
forward on the reference's own codes within 1e-3 of its y, and our y as
close to the unquantized W x as the reference's (within 1 %).  Our y differs from the
reference's by a few percent: the ~1 % of rows that take another code after
a near-tie flip carry their difference into every output through T_m."""
import hashlib

import numpy as np
import pytest
import torch

from conftest import golden

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def c1(dev):
    from quipsharp_amd.checkpoint import build_codebook
    from quipsharp_amd.quantize import quantize_linear
    ref = golden("c1_full.npz")
    g = torch.Generator().manual_seed(0)
    W = torch.randn(4096, 4096, generator=g) * 0.02
    X = torch.randn(2048, 4096, generator=g)
    x = torch.randn(4096, generator=g)
    H = X.T @ X / 2048   # on the host CPU, like the reference
    cb, s = build_codebook("2bit", dev, 0)
    Wd, Hd = W.to(dev), H.to(dev)
    torch.manual_seed(0)
    layer, what_q = quantize_linear(Wd, Hd, cb, g=8, damping=1e-2, codebook_scale=s, tune_iters=10)
    torch.cuda.synchronize()
    return dict(ref=ref, W=Wd, H=Hd, x=x.to(dev), cb=cb, layer=layer, what_q=what_q)


def test_c1_fixture_integrity():
    ref = golden("c1_full.npz")
    assert ref["codes"].shape == (4096, 512) and ref["codes"].dtype == np.uint16
    assert hashlib.sha256(ref["codes"].tobytes()).digest() == ref["codes_sha256"].tobytes()


def test_c1_signs_and_scale(c1):
    ref, layer = c1["ref"], c1["layer"]
    assert np.array_equal(layer.signs.su.cpu().numpy(), ref["su"].astype(np.float32))
    assert np.array_equal(layer.signs.sv.cpu().numpy(), ref["sv"].astype(np.float32))
    rs = float(ref["layer_scale"])
    ia, ib = (np.array([v], np.float32).view(np.int32)[0] for v in (layer.scale, rs))
    gap = abs(int(ia) - int(ib))
    print(f"C1 layer scale: ours {layer.scale!r}, reference {rs!r}, {gap} fp32 ulp apart", flush=True)
    assert gap == 0  # the same fp32 value


def test_c1_codes_proxy_and_forward(c1):
    from quipsharp_amd.incoherence import incoherence_process
    from quipsharp_amd.quantize import QuantizedLayer, dequantize_linear, linear_forward
    ref, layer, cb, dev = c1["ref"], c1["layer"], c1["cb"], c1["W"].device
    codes = layer.codes.cpu().numpy().astype(np.uint16)
    agree = float((codes == ref["codes"]).mean())
    rows_exact = float((codes == ref["codes"]).all(axis=1).mean())
    # the reference's quantized weight, decoded bit-exactly from its codes
    ref_layer = QuantizedLayer(codes=torch.from_numpy(ref["codes"].astype(np.int64)).to(dev), signs=layer.signs,
                               g=8, shape=(4096, 4096), scale=float(ref["layer_scale"]))
    what_q_ref = dequantize_linear(ref_layer, cb)
    H = c1["H"]
    Hd = H + 1e-2 * H.diagonal().mean() * torch.eye(4096, device=dev)
    what, hhat, _ = incoherence_process(c1["W"], Hd, generator=torch.Generator().manual_seed(0))
    Hh, Wh = hhat.double(), what.double()
    den = torch.trace(Wh @ Hh @ Wh.T).item()

    def proxy(q):
        E = (q.double() - Wh)
        return torch.trace(E @ Hh @ E.T).item() / den

    ours, theirs = proxy(c1["what_q"]), proxy(what_q_ref)
    x = c1["x"]
    y = linear_forward(x, layer, cb).double().cpu().numpy()
    y_refcodes = linear_forward(x, ref_layer, cb).double().cpu().numpy()   # our forward, the reference's codes
    y_ref = ref["y"].astype(np.float64)
    y_true = (c1["W"].double() @ x.double()).cpu().numpy()                # the unquantized layer
    rel = lambda a, b: float(np.linalg.norm(a - b) / np.linalg.norm(b))
    print(f"C1 4096x4096: code agreement {agree:.4f} (rows identical {rows_exact:.4f}); relative proxy loss "
          f"ours {ours:.5e}, reference {theirs:.5e} (reference's own figure {float(ref['proxy_rel']):.5e}); "
          f"forward on the reference's codes vs its y {rel(y_refcodes, y_ref):.2e}; y vs W x: ours "
          f"{rel(y, y_true):.4f}, reference {rel(y_ref, y_true):.4f}; ours vs reference {rel(y, y_ref):.3e}",
          flush=True)
    # the reference's proxy recomputed here agrees with its own figure
    assert abs(theirs - float(ref["proxy_rel"])) <= 1e-3 * float(ref["proxy_rel"])
    assert ours <= 1.01 * theirs
    assert agree >= 0.99
    # the forward at full size: the reference's own codes give the reference's y
    assert rel(y_refcodes, y_ref) < 1e-3
    # our quantization serves the layer as well as the reference's
    assert rel(y, y_true) <= 1.01 * rel(y_ref, y_true)
    # the rows that took another code after a near-tie move y by a few percent
    assert rel(y, y_ref) < 0.07
