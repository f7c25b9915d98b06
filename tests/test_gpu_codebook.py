"""GPU parity: codebook encode/decode kernels through the C ABI vs the oracle
and the reference's golden fixtures.  Integer codes and decoded values must
match bit for bit."""
import hashlib
import json

import numpy as np
import pytest
import torch

from conftest import golden
from oracle import cref

pytestmark = pytest.mark.gpu


def enc(x, kinds, scales, dev, in_div=1.0, out_mul=1.0):
    from quipsharp_amd.codebooks.e8p import _encode
    v, c = _encode(torch.from_numpy(np.ascontiguousarray(x)).to(dev), kinds, scales, in_div, out_mul)
    return v.cpu().numpy(), c.cpu().numpy()


def test_e8p_encode_golden(dev):
    e = golden("encode.npz")
    print("case: e8p encode golden", e["x"].shape, flush=True)
    vals, codes = enc(e["x"], [0], [1.0], dev)
    assert np.array_equal(codes[0].astype(np.uint16), e["e8p_code"])
    assert np.array_equal(vals, cref.e8p_decode(codes[0]))


def test_e81_encode_golden(dev):
    e = golden("encode.npz")
    vals, idx = enc(e["x"], [1], [1.0], dev)
    assert np.array_equal(idx[0].astype(np.uint8), e["e81_idx"])
    assert np.array_equal(vals, cref.e81_table()[idx[0]])


@pytest.mark.parametrize("name,kinds,scales", [("rvq3", [0, 1], [1.03, 0.47]), ("rvq4", [0, 0], [1.03, 0.29])])
def test_rvq_encode_golden(dev, name, kinds, scales):
    e, r = golden("encode.npz"), golden("rvq.npz")
    tot, codes = enc(e["x"], kinds, scales, dev)
    assert np.array_equal(codes, r[name + "_codes"])
    assert hashlib.sha256(tot.tobytes()).digest() == r[name + "_sha256"].tobytes()


def test_teacher_forced_ldlq_targets(dev):
    q2 = golden("quantize2.npz")
    _, c = enc(q2["targets"], [0], [1.0], dev)
    assert np.array_equal(c[0], q2["target_codes"])
    q3, sc = golden("quantize3.npz"), golden("scales.json")["3bit"]["stage_scales"]
    t = q3["targets"]
    _, c3 = enc(t, [0, 1], sc, dev)
    assert np.array_equal(c3.transpose(1, 0, 2), q3["target_codes"])


@pytest.mark.parametrize("n", [1, 63, 64, 65, 4096, 20011])
def test_random_encode_vs_oracle(dev, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((n, 8)) * rng.choice([0.3, 1.0, 3.0], (n, 1))).astype(np.float32)
    for kinds, scales in (([0], [1.0]), ([1], [1.0]), ([0, 1], [0.95, 0.5]), ([0, 0, 1], [1.1, 0.3, 0.2])):
        tot, codes = enc(x, kinds, scales, dev)
        ot, oc = cref.rvq_encode(x, kinds, scales)
        assert np.array_equal(codes, oc), (n, kinds)
        assert np.array_equal(tot, ot), (n, kinds)


def test_in_div_out_mul(dev):
    """codebook.quantize(x / s) then vals * s as one kernel (IEEE divide, as the
    reference's CPU sweep does) equals the oracle on pre-divided inputs."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((3000, 8)).astype(np.float32)
    for s in (0.55, 1.05, 2.35):
        v, c = enc(x, [0], [1.0], dev, in_div=s, out_mul=s)
        ov, oc = cref.e8p_encode(x / np.float32(s))
        assert np.array_equal(c[0], oc)
        assert np.array_equal(v, ov * np.float32(s))


def test_decode_all_codes(dev):
    from quipsharp_amd.codebooks.e8p import E8PCodebook
    cb = E8PCodebook(dev)
    d = cb.dequantize(torch.arange(65536, device=dev)).cpu().numpy()
    assert hashlib.sha256(d.tobytes()).digest() == golden("tables.npz")["e8p_decode_all_sha256"].tobytes()


def test_e81_decode(dev):
    from quipsharp_amd.codebooks.e8_1bit import E8OneBitCodebook
    d = E8OneBitCodebook(dev).dequantize(torch.arange(256, device=dev)).cpu().numpy()
    assert np.array_equal(d, cref.e81_table())


def test_codebook_api_roundtrip(dev):
    """quipsharp tests/test_e8p.py:86-92 and tests/test_rvq.py:22-27, 52-63."""
    from quipsharp_amd.codebooks.e8p import E8PCodebook
    from quipsharp_amd.codebooks.e8_1bit import E8OneBitCodebook
    from quipsharp_amd.rvq import RVQStage, rvq_quantize, rvq_dequantize
    torch.manual_seed(1)
    x = torch.randn(100, 8, device=dev) * 0.5
    cb = E8PCodebook(dev)
    vals, code = cb.quantize(x)
    assert code.dtype == torch.int64 and torch.equal(cb.dequantize(code), vals)
    ob = E8OneBitCodebook(dev)
    v1, i1 = ob.quantize(x)
    assert torch.equal(ob.dequantize(i1), v1)
    st = [RVQStage(cb, 0.95), RVQStage(ob, 0.5)]
    tv, tc = rvq_quantize(x, st)
    assert torch.equal(rvq_dequantize(tc, st), tv)


def test_encode_to_table_fields(dev):
    from quipsharp_amd.codebooks import e8p
    e = golden("encode.npz")
    x = torch.from_numpy(e["x"][:500]).to(dev)
    abs_idx, s7, sh, vals = e8p.encode_to_table(x, e8p.build_abs_table())
    packed = e8p.pack_code(abs_idx, s7, sh).cpu().numpy()
    assert np.array_equal(packed.astype(np.uint16), e["e8p_code"][:500])


def test_fitted_scales_match_reference(dev):
    """build_codebook's scale sweeps (quipsharp/checkpoint.py:60-77) choose the
    reference's scales (golden), with the same seeds and sample counts."""
    from quipsharp_amd.checkpoint import build_codebook
    sc = golden("scales.json")
    cb2, s2 = build_codebook("2bit", dev, 0)
    assert s2 == sc["2bit"]["scale"]
    cb3, s3 = build_codebook("3bit", dev, 0)
    assert s3 == sc["3bit"]["scale"]
    assert [st.scale for st in cb3.stages] == sc["3bit"]["stage_scales"]


def test_ldlq_step_kernel(dev):
    """Fused BlockLDLQ step: target = base + delta @ dinv, encode, wq / resid /
    code updates through strided views."""
    from quipsharp_amd import _lib
    rng = np.random.default_rng(11)
    m, n, k = 300, 64, 3
    W = rng.standard_normal((m, n)).astype(np.float32)
    Wq = rng.standard_normal((m, n)).astype(np.float32)
    delta = rng.standard_normal((m, 8)).astype(np.float32)
    dinv = rng.standard_normal((8, 8)).astype(np.float32)
    tW, tWq, tE = (torch.from_numpy(a).to(dev) for a in (W, Wq, np.zeros_like(W)))
    tD, tI = torch.from_numpy(delta).to(dev), torch.from_numpy(dinv).to(dev)
    codes = torch.zeros(m, n // 8, dtype=torch.int16, device=dev)
    L = _lib.lib()
    base_ptr = tWq.data_ptr() + k * 32
    _lib.check(L.qs_ldlq_step(base_ptr, n, tD.data_ptr(), tI.data_ptr(), tW.data_ptr() + k * 32, n,
                              tWq.data_ptr() + k * 32, n, tE.data_ptr() + k * 32, n, m, 1, _lib.int_array([0]),
                              _lib.float_array([1.0]), codes.data_ptr() + k * 2, 2, 0, n // 8,
                              _lib.stream_of(tW)))
    torch.cuda.synchronize()
    adj = (delta.astype(np.float64) @ dinv.astype(np.float64)).astype(np.float32)
    target = Wq[:, k * 8:(k + 1) * 8] + adj
    ov, oc = cref.e8p_encode(target)
    got_c = codes[:, k].cpu().numpy().astype(np.int64) & 0xFFFF
    # the 8-term product may round differently from fp64: allow rare near-tie flips
    assert (got_c == oc).mean() > 0.99
    wq = tWq.cpu().numpy()
    assert np.array_equal(wq[:, k * 8:(k + 1) * 8], cref.e8p_decode(got_c))
    assert np.array_equal(tE.cpu().numpy()[:, k * 8:(k + 1) * 8], W[:, k * 8:(k + 1) * 8] - wq[:, k * 8:(k + 1) * 8])
    assert np.array_equal(np.delete(wq, range(k * 8, k * 8 + 8), 1), np.delete(Wq, range(k * 8, k * 8 + 8), 1))
