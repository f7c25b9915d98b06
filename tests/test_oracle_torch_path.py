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
