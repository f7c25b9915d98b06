"""The torch-CPU restatement used as bench.py's CPU baseline reproduces the
reference's CPU results (golden fixtures) on this machine."""
import numpy as np
import torch

from conftest import golden
from oracle import cref, torch_path


def test_encode_matches_golden_and_c_oracle():
    e = golden("encode.npz")
    v, c = torch_path.e8p_encode(torch.from_numpy(e["x"]))
    assert np.array_equal(c.numpy().astype(np.uint16), e["e8p_code"])
    assert np.array_equal(v.numpy(), cref.e8p_decode(c.numpy()))


def test_decode_and_forward_match_golden():
    lf = golden("linear.npz")
    codes = torch.from_numpy(lf["e8p_codes"].astype(np.int64))
    deq = torch_path.dequantize_linear(codes, float(lf["e8p_scale"]))
    assert np.array_equal(deq.numpy(), lf["e8p_deq"])
    y = torch_path.linear_forward(torch.from_numpy(lf["e8p_x"]), codes, float(lf["e8p_scale"]),
                                  su=torch.from_numpy(lf["e8p_su"]), sv=torch.from_numpy(lf["e8p_sv"]))
    assert np.allclose(y.numpy(), lf["e8p_y"], rtol=1e-5, atol=1e-5)


def test_fwht_and_rfft_match_golden():
    f = golden("fwht.npz")
    assert np.array_equal(torch_path.fwht(torch.from_numpy(f["x4096"])).numpy(), f["y4096"])
    r = golden("rfft.npz")
    ph = torch.view_as_complex(torch.from_numpy(r["phase"]))
    assert np.allclose(torch_path.to_rfft(torch.from_numpy(r["x"]), ph).numpy(), r["fwd"], atol=1e-6)
    assert np.allclose(torch_path.from_rfft(torch.from_numpy(r["x"]), ph).numpy(), r["inv"], atol=1e-6)


def test_quantize_steps_teacher_forced():
    """The first base-pass steps of the golden 2-bit run give the golden codes."""
    q = golden("quantize2.npz")
    t = torch.from_numpy(q["targets"][:4])
    for i in range(4):
        _, c = torch_path.e8p_encode(t[i])
        assert np.array_equal(c.numpy(), q["target_codes"][i])


def test_random_phase_draws_the_reference_phases():
    """quipsharp_amd.rfft.random_phase with the fixture's generator seed draws
    the reference's phases bit for bit (CPU draw, quipsharp/rfft.py:31-34)."""
    import torch
    from quipsharp_amd.rfft import random_phase
    g = golden("rfft.npz")
    ph = random_phase(72, generator=torch.Generator().manual_seed(3))
    assert np.array_equal(torch.view_as_real(ph).numpy(), g["phase"])


def test_block_ldl_matches_golden():
    """torch_path.block_ldl (the CPU baseline's factorization) against the
    reference's block_ldl output (quipsharp/ldlq.py:39-94, golden ldl.npz:
    H = A A^T + I, g = 8, no damping), and the identity H = L D L^T with the
    golden block diagonal D."""
    g = golden("ldl.npz")
    H = torch.from_numpy(g["H"])
    L = torch_path.block_ldl(H.clone(), 8)
    assert np.allclose(L.numpy(), g["L"], rtol=1e-4, atol=1e-5)
    D = torch.block_diag(*torch.from_numpy(g["D"]))
    back = (L.double() @ D.double() @ L.double().T).numpy()
    assert np.abs(back - g["H"]).max() <= 1e-4 * np.abs(g["H"]).max()
    # unit block diagonal: each 8x8 diagonal block of L is the identity
    for k in range(8):
        assert np.allclose(L[8 * k:8 * k + 8, 8 * k:8 * k + 8].numpy(), np.eye(8), atol=1e-5)


def _golden_run_inputs(q):
    """The reference's transformed, scaled weight and Hessian for a golden
    quantize run (quipsharp/quantize.py:48-104): damping 1e-2, RHT with the
    run's signs, divide by the layer scale."""
    W = torch.from_numpy(q["W"])
    H = torch.from_numpy(q["H"])
    su, sv = torch.from_numpy(q["su"]), torch.from_numpy(q["sv"])
    Hd = H + 1e-2 * H.diagonal().mean() * torch.eye(H.shape[0])
    hhat = torch_path.fwht(torch_path.fwht(Hd * sv[:, None] * sv[None, :], 0), 1)
    what = torch_path.fwht(torch_path.fwht(W * su[:, None] * sv[None, :], 0), 1)
    return what / torch.tensor(float(q["layer_scale"]), dtype=torch.float32), hhat


def test_quantize_steps_feedback_targets_match_golden():
    """The CPU baseline's BlockLDLQ products (quantize_steps) reproduce the
    targets the reference handed its codebook in the golden 2-bit run: the
    base pass (blocks last to first, feedback through L) and the first tune
    sweep (full residual through H and the inverse diagonal blocks)."""
    q = golden("quantize2.npz")
    Ws, hhat = _golden_run_inputs(q)
    T = Ws.shape[1] // 8
    L = torch_path.block_ldl(hhat.clone(), 8)
    got = []
    Wq = torch.zeros_like(Ws)
    torch_path.quantize_steps(Ws, L, hhat, list(range(T - 1, -1, -1)), Wq=Wq, targets=got)
    ref = q["targets"]
    # the first block has no feedback: its target is the scaled weight itself
    assert np.allclose(got[0].numpy(), ref[0], rtol=1e-5, atol=1e-6)
    for i in range(T):
        assert np.allclose(got[i].numpy(), ref[i], rtol=1e-3, atol=1e-4), i
    # a planted mistake (feedback from the unquantized instead of the residual) fails
    bad = []
    torch_path.quantize_steps(Ws, L, hhat, [T - 1, T - 2], Wq=torch.zeros_like(Ws), targets=bad)
    wrong = Ws[:, 8 * (T - 2):8 * (T - 1)] + Ws[:, 8 * (T - 1):] @ L[8 * (T - 1):, 8 * (T - 2):8 * (T - 1)]
    assert not np.allclose(wrong.numpy(), ref[1], rtol=1e-3, atol=1e-4)
    # first tune sweep, with the base pass's codes as the current Wq
    tgot = []
    order = list(range(T - 1, -1, -1))
    torch_path.quantize_steps(Ws, L, hhat, order, tune=True, Wq=Wq, targets=tgot)
    assert np.allclose(tgot[0].numpy(), ref[T], rtol=1e-3, atol=1e-4)
