"""Host-side logic that runs without a GPU: the power-of-two helpers against
the reference's known answers, and the argument checks that guard every
pointer handed to the library (a tensor of the wrong dtype, length, layout
or device must be refused before the kernels could read past it)."""
import pytest
import torch

from quipsharp_amd.hadamard import is_pow2, next_pow2
from quipsharp_amd.quantize import check_linear_args, pack_signs


def test_is_pow2_and_next_pow2_known_answers():
    """quipsharp tests/test_hadamard.py:54-60."""
    assert [is_pow2(n) for n in [1, 2, 3, 4, 5, 8, 15, 16]] == \
        [True, True, False, True, False, True, False, True]
    assert next_pow2(1) == 1
    assert next_pow2(5) == 8
    assert next_pow2(129) == 256
    assert next_pow2(256) == 256


def test_pow2_helpers_brute_force():
    """Against the definitions: n is a power of two iff some 2^k equals it;
    next_pow2(n) is the smallest 2^k >= n (n >= 1).  Zero and negatives are
    not powers of two."""
    pows = {1 << k for k in range(20)}
    for n in range(-4, 1 << 12):
        assert is_pow2(n) == (n in pows), n
    for n in range(1, 1 << 12):
        want = min(p for p in pows if p >= n)
        assert next_pow2(n) == want, n


def test_pack_signs_layout():
    """bit i % 32 of word i // 32 set where s[i] < 0 (two's-complement int32)."""
    g = torch.Generator().manual_seed(0)
    s = torch.randint(0, 2, (100,), generator=g).float() * 2 - 1
    w = pack_signs(s)
    assert w.dtype == torch.int32 and w.numel() == 4
    for i in range(100):
        bit = (int(w[i // 32]) >> (i % 32)) & 1
        assert bit == (1 if s[i] < 0 else 0)
    assert torch.equal(pack_signs(-torch.ones(32)), torch.tensor([-1], dtype=torch.int32))


def _args(m=512, n=256, **over):
    kw = dict(x=torch.zeros(2, n), m=m, n=n, su=torch.ones(m), sv=torch.ones(n), bias=None, out=None,
              workspace=None)
    kw.update(over)
    return kw


def test_linear_args_accepts_fp32_and_bits():
    assert check_linear_args(**_args()) is False
    assert check_linear_args(**_args(su=pack_signs(torch.ones(512)), sv=pack_signs(torch.ones(256)))) is True
    assert check_linear_args(**_args(bias=torch.zeros(512), workspace=torch.zeros(64, dtype=torch.uint8))) is False


@pytest.mark.parametrize("bad,msg", [
    (dict(su=torch.ones(512, dtype=torch.float16)), "float32 signs"),        # after module.half()
    (dict(sv=torch.ones(256, dtype=torch.bfloat16)), "float32 signs"),
    (dict(su=torch.ones(511)), "float32 signs"),                              # short: reads past the end
    (dict(sv=torch.ones(512)[::2]), "contiguous"),
    (dict(su=torch.zeros(15, dtype=torch.int32), sv=torch.zeros(8, dtype=torch.int32)), "sign words"),
    (dict(su=torch.zeros(16, dtype=torch.int32)), "both be fp32 signs or both packed"),
    (dict(bias=torch.zeros(512, dtype=torch.float16)), "bias"),
    (dict(bias=torch.zeros(500)), "bias"),
    (dict(bias=torch.zeros(1024)[::2]), "bias"),
    (dict(out=torch.zeros(2, 512, device="meta")), "out is on"),
    (dict(workspace=torch.zeros(64, dtype=torch.uint8, device="meta")), "workspace"),
    (dict(workspace=torch.zeros(64, dtype=torch.float32)), "workspace"),
    (dict(su=torch.ones(512, device="meta")), "su is on"),
])
def test_linear_args_rejects(bad, msg):
    with pytest.raises(ValueError, match=msg):
        check_linear_args(**_args(**bad))


def test_checkpoint_placement():
    """Where a checkpoint loads (quipsharp/checkpoint.py:228-263 places it on
    gpu_devices[0] when it fits the budget): one GPU listed and over the budget
    -> still that GPU, with a warning (naming the CPU share the reference
    would have offloaded when cpu_budget_bytes is set); several GPUs over the
    budget -> NotImplementedError that names the ways out."""
    from quipsharp_amd.checkpoint import checkpoint_placement
    assert checkpoint_placement(10, "cuda:3") == ("cuda:3", None)
    assert checkpoint_placement(10, "cpu", ["cuda:1"], None) == ("cuda:1", None)
    assert checkpoint_placement(10, "cpu", ["cuda:1", "cuda:2"], 10) == ("cuda:1", None)
    dev, note = checkpoint_placement(26 << 30, "cpu", ["cuda:0"], 20 << 30, 0)
    assert dev == "cuda:0" and "all of it goes on cuda:0" in note and "CPU" not in note
    dev, note = checkpoint_placement(26 << 30, "cpu", ["cuda:0"], 20 << 30, 60 << 30)
    assert dev == "cuda:0" and "on the CPU" in note
    with pytest.raises(NotImplementedError, match="pass one device"):
        checkpoint_placement(26 << 30, "cpu", ["cuda:0", "cuda:1"], 20 << 30, 60 << 30)
