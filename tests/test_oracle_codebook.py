"""The CPU oracle (oracle/qs_oracle.c) pinned against the reference's own
known answers and golden fixtures, plus brute-force optimality checks."""
import hashlib
import itertools

import numpy as np
import pytest

from conftest import golden
from oracle import cref


def test_abs_table_known_answers():
    """quipsharp tests/test_e8p.py:14-37: 227 enumerated rows, 256 total,
    even row sums, unique rows, the Appendix C.2 row present."""
    t = cref.e8p_abs_table()
    assert t.shape == (256, 8)
    assert np.all(t.sum(-1) % 2 == 0)
    assert np.unique(t, axis=0).shape[0] == 256
    assert (t == np.array([0.5, 0.5, 0.5, 1.5, 0.5, 0.5, 0.5, -0.5], np.float32)).all(-1).any()
    # first 227 rows: squared norm <= 10 and sorted lexicographically by |x|
    a = np.abs(t[:227])
    assert np.all((a ** 2).sum(-1) <= 10) and np.all((np.abs(t[227:]) ** 2).sum(-1) == 12)
    assert all(tuple(a[i]) < tuple(a[i + 1]) for i in range(226))


def test_tables_match_reference():
    g = golden("tables.npz")
    assert np.array_equal(cref.e8p_abs_table(), g["e8p_abs"])
    assert np.array_equal(cref.e81_table(), g["e81"])


def test_decode_all_codes_match_reference():
    dec = cref.e8p_decode(np.arange(65536))
    assert hashlib.sha256(dec.astype(np.float32).tobytes()).digest() == golden("tables.npz")[
        "e8p_decode_all_sha256"].tobytes()


def test_paper_worked_example():
    """quipsharp tests/test_e8p.py:40-69: row (.5,.5,.5,1.5,.5,.5,.5,-.5), free
    flips at coordinates 0,1,4,6, shift +1/4."""
    t = cref.e8p_abs_table()
    row = np.array([0.5, 0.5, 0.5, 1.5, 0.5, 0.5, 0.5, -0.5], np.float32)
    a = int(np.nonzero((t == row).all(-1))[0][0])
    bits = [1, 1, 0, 0, 1, 0, 1]
    code = (a << 8) | (sum(b << (6 - i) for i, b in enumerate(bits)) << 1) | 1
    want = np.array([-0.25, -0.25, 0.75, 1.75, -0.25, 0.75, -0.25, -0.25], np.float32)
    assert np.array_equal(cref.e8p_decode(np.array([code]))[0], want)


def test_decoded_points_in_e8_plus_quarter():
    """Every codeword minus its shift is in E8 (all-integer or all-half-integer
    coordinates, even sum) -- quipsharp tests/test_e8p.py:95-108, exhaustively."""
    c = np.arange(65536)
    v = cref.e8p_decode(c).astype(np.float64)
    v -= np.where(c & 1, 0.25, -0.25)[:, None]
    twice = v * 2
    assert np.all(twice == np.round(twice))
    is_int = np.all(v == np.round(v), -1)
    is_half = np.all(twice % 2 != 0, -1)
    assert np.all(is_int | is_half)
    assert np.all(np.round(v.sum(-1)) % 2 == 0)


def test_e81_table_known_answers():
    """quipsharp tests/test_rvq.py:10-19: the 240-vector kissing shell, 256 unique rows."""
    t = cref.e81_table()
    assert np.all(t[0] == 0)
    assert np.all((t[1:241].astype(np.float64) ** 2).sum(-1) == 2)
    assert np.all((t[241:].astype(np.float64) ** 2).sum(-1) == 4)
    assert np.unique(t, axis=0).shape[0] == 256


def test_encode_matches_reference_golden():
    e = golden("encode.npz")
    _, codes = cref.e8p_encode(e["x"])
    assert np.array_equal(codes.astype(np.uint16), e["e8p_code"])
    _, idx = cref.e81_encode(e["x"])
    assert np.array_equal(idx.astype(np.uint8), e["e81_idx"])


@pytest.mark.parametrize("name,kinds,scales", [("rvq3", [0, 1], [1.03, 0.47]), ("rvq4", [0, 0], [1.03, 0.29])])
def test_rvq_matches_reference_golden(name, kinds, scales):
    e, r = golden("encode.npz"), golden("rvq.npz")
    tot, codes = cref.rvq_encode(e["x"], kinds, scales)
    assert np.array_equal(codes, r[name + "_codes"])
    assert hashlib.sha256(tot.tobytes()).digest() == r[name + "_sha256"].tobytes()


def test_teacher_forced_targets_match_reference():
    """Every target the reference's BlockLDLQ handed its codebook (quantize2 / quantize3)."""
    q2 = golden("quantize2.npz")
    _, c = cref.e8p_encode(q2["targets"])
    assert np.array_equal(c, q2["target_codes"])
    q3, sc = golden("quantize3.npz"), golden("scales.json")["3bit"]["stage_scales"]
    t = q3["targets"]
    _, c3 = cref.rvq_encode(t.reshape(-1, 8), [0, 1], sc)
    assert np.array_equal(c3.reshape(2, t.shape[0], t.shape[1]).transpose(1, 0, 2), q3["target_codes"])


def test_encode_is_optimal_over_all_codewords():
    """Brute force over all 65,536 decoded codewords (fp64 distances): the
    greedy search of e8p.py:104-162 finds a nearest codeword."""
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((192, 8)) * rng.choice([0.5, 1.0, 2.0], (192, 1))).astype(np.float32)
    vals, _ = cref.e8p_encode(x)
    got = ((x.astype(np.float64) - vals) ** 2).sum(-1)
    best = cref.e8p_bruteforce_d2(x)
    assert np.all(got <= best * (1 + 1e-6) + 1e-9)


def test_greedy_parity_repair_vs_128_patterns():
    """quipsharp tests/test_e8p.py:111-140: the chosen codeword is never beaten
    by any of the 128 even-parity signings of its own table row."""
    rng = np.random.default_rng(3)
    t = cref.e8p_abs_table().astype(np.float64)
    # the oracle's chosen codeword is never beaten by any even signing of its row
    x = rng.standard_normal((64, 8)).astype(np.float32)
    vals, codes = cref.e8p_encode(x)
    for k in range(64):
        r, sb = codes[k] >> 8, codes[k] & 1
        sh = 0.25 if sb else -0.25
        d = ((x[k].astype(np.float64) - vals[k]) ** 2).sum()
        for b in itertools.product([0, 1], repeat=7):
            s = np.array([1 - 2 * f for f in (list(b) + [sum(b) % 2])])
            assert d <= ((x[k] - (t[r] * s + sh)) ** 2).sum() + 1e-9


def test_special_inputs():
    """A codeword encodes to itself; x = 0 ties across both shifts and the -1/4
    coset (shift bit 0) wins, as use_plus = d+ <= d- does in e8p.py:156."""
    c = np.array([0, 1, 12345, 65535, 40000])
    v = cref.e8p_decode(c)
    v2, c2 = cref.e8p_encode(v)
    assert np.array_equal(v2, v) and np.array_equal(c2, c)
    _, cz = cref.e8p_encode(np.zeros((1, 8), np.float32))
    assert cz[0] & 1 == 0


def test_decode_of_rvq_matches_reference_dequant():
    lf = golden("linear.npz")
    d = cref.rvq_decode(lf["e8p_codes"][None], [0], [1.0], lf["e8p_scale"])
    assert np.array_equal(d.reshape(lf["e8p_deq"].shape), lf["e8p_deq"])
    d3 = cref.rvq_decode(lf["rvq3_codes"], [0, 1], [1.03, 0.47], lf["rvq3_scale"])
    assert np.array_equal(d3.reshape(lf["rvq3_deq"].shape), lf["rvq3_deq"])


def test_planted_mistakes_fail():
    """The checks above catch plausible slips in the oracle: a swapped tie rule
    or a wrong flip bit order changes golden codes."""
    e = golden("encode.npz")
    _, codes = cref.e8p_encode(e["x"])
    # reversed sign-bit order
    rev = (codes & ~0xFE) | sum((((codes >> (7 - i)) & 1) << (1 + i)) for i in range(7))
    assert not np.array_equal(rev.astype(np.uint16), e["e8p_code"])
    # ties resolved toward shift bit 1 instead of 0: exact-tie inputs flip
    zero = np.zeros((1, 8), np.float32)
    _, cz = cref.e8p_encode(zero)
    assert (cz[0] ^ 1) & 1 != e["e8p_code"][3 * 1536 + 512] & 1
