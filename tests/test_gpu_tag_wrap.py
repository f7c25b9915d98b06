"""GPU: the launch with the last tag counter value (the counter wrap) on the
real kernels -- the one-launch forward with one and with two output levels,
the 16-row decode-matvec that applies the output transform itself, and
grouped launches where only one job wraps.

The epoch word of the job is set so that the next call is the wrap launch,
and words carrying tags are planted past the call's own workspace regions.
The wrap launch must give the same output as any other launch, remove every
word carrying a tag of its own job index from the workspace (the counter
then starts again at 1), leave other jobs' tags and other data alone, and
set the wrap word back to zero; the launch after it continues at counter 1
with the same output."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TAG_BASE = 0x7FC00000
LAST = 0xFFFFF
WRAP_WORD = 16   # unsigned index of job 0's wrap word
F1E30 = int(np.array([1e30], np.float32).view(np.uint32)[0])


def tag(c, g):
    return TAG_BASE | (c << 2) | g


def slot(t, bits=F1E30):
    return (t << 32) | bits


def counter(word):
    return (int(word) >> 2) & LAST


def _rand_linear(dev, rng, m, n, bias):
    from quipsharp_amd.quantize import PackedCodes
    c = torch.from_numpy(rng.integers(0, 65536, (m, n // 8))).to(dev)
    su = torch.from_numpy(rng.choice([-1.0, 1.0], m).astype(np.float32)).to(dev)
    sv = torch.from_numpy(rng.choice([-1.0, 1.0], n).astype(np.float32)).to(dev)
    b = torch.from_numpy(rng.standard_normal(m).astype(np.float32)).to(dev) if bias else None
    return (PackedCodes(c, m, n, [0]), su, sv, 0.97, 0.0, 0.0135, b)


def _plant(ws, need, wrap_job, other_job):
    """Words past the call's regions (bytes need ..): 64-bit word index ->
    planted value, and which of them the wrap must clear."""
    w64 = ws.view(torch.int64)
    first = (need + 255) // 8 // 32 * 32 + 32
    plan = {
        first: (slot(tag(1, wrap_job)), True),            # the next era's first tag of the wrapping job
        first + 5: (slot(tag(LAST, wrap_job)), True),
        first + 9: (slot(tag(3, other_job)), False),       # another job's tag
        first + 17: (slot(0x3F800000, 0x3F800000), False),  # ordinary data (1.0f, 1.0f)
        w64.numel() - 1: (slot(tag(77, wrap_job)), True),  # the workspace's last word
    }
    for i, (v, _) in plan.items():
        w64[i] = v
    return plan


def _check_after_wrap(ws, plan, wrap_job):
    w32 = ws.view(torch.int32).cpu().numpy().view(np.uint32)
    w64 = ws.view(torch.int64).cpu().numpy()
    assert counter(w32[wrap_job]) == LAST and (w32[wrap_job] & 3) == wrap_job, hex(w32[wrap_job])
    assert w32[WRAP_WORD + wrap_job] == 0
    for i, (v, cleared) in plan.items():
        assert w64[i] == (0 if cleared else v), (i, hex(int(w64[i])), hex(v))


@pytest.mark.parametrize("m,n,B", [
    (4096, 4096, 1),    # one-launch forward, output transform in the first work-group
    (8192, 4096, 2),    # one-launch forward, two output levels
    (11008, 4096, 1),   # two output levels with an odd factor (43)
    (4096, 4096, 8),    # 16-row decode-matvec with the output transform in its tail
    (4096, 4096, 16),
])
def test_wrap_launch_single(dev, m, n, B):
    from quipsharp_amd import _lib
    from quipsharp_amd.quantize import forward_packed
    print(f"case: tag wrap single m={m} n={n} B={B}", flush=True)
    rng = np.random.default_rng(m + n + B)
    lin = _rand_linear(dev, rng, m, n, bias=True)
    x = torch.randn(B, n, generator=torch.Generator().manual_seed(B)).to(dev).bfloat16()
    need = _lib.lib().qs_linear_workspace_bytes(m, n, B, lin[0].layout)
    ws = torch.zeros(need + 4096, dtype=torch.uint8, device=dev)
    want = forward_packed(x, *lin, workspace=ws).clone()
    torch.cuda.synchronize()
    assert counter(ws.view(torch.int32)[0].item() & 0xFFFFFFFF) == 1  # a tagged kernel ran
    ws.view(torch.int32)[0] = tag(LAST - 1, 0)
    plan = _plant(ws, need, 0, 1)
    torch.cuda.synchronize()
    y = forward_packed(x, *lin, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y, want)
    _check_after_wrap(ws, plan, 0)
    y = forward_packed(x, *lin, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y, want)
    assert counter(ws.view(torch.int32)[0].item() & 0xFFFFFFFF) == 1


@pytest.mark.parametrize("shapes,B,wrap_job", [
    ([4096, 1024], 1, 0),
    ([4096, 1024], 1, 1),
    ([8192, 4096, 1024], 2, 2),
    ([4096, 1024], 8, 1),    # decode-matvecs of the group with their output transforms
])
def test_wrap_launch_group(dev, shapes, B, wrap_job):
    from quipsharp_amd import _lib
    from quipsharp_amd.quantize import forward_packed, forward_packed_group
    print(f"case: tag wrap group {shapes} B={B} wrapping job {wrap_job}", flush=True)
    n = 4096
    rng = np.random.default_rng(sum(shapes) + B)
    lins = [_rand_linear(dev, rng, m, n, bias=g == 0) for g, m in enumerate(shapes)]
    x = torch.randn(B, n, generator=torch.Generator().manual_seed(B)).to(dev).bfloat16()
    ms = (ctypes.c_int64 * len(shapes))(*shapes)
    need = _lib.lib().qs_linear_group_workspace_bytes(n, B, len(shapes), ms)
    ws = torch.zeros(need + 4096, dtype=torch.uint8, device=dev)
    want = [forward_packed(x, *lin) for lin in lins]
    ys = forward_packed_group(x, lins, workspace=ws)
    torch.cuda.synchronize()
    for y, w in zip(ys, want):
        assert torch.equal(y, w)
    w32 = ws.view(torch.int32).cpu().numpy().view(np.uint32)
    assert all(counter(w32[g]) == 1 for g in range(len(shapes))), [hex(v) for v in w32[:4]]
    ws.view(torch.int32)[wrap_job] = tag(LAST - 1, wrap_job)
    other = (wrap_job + 1) % len(shapes)
    plan = _plant(ws, need, wrap_job, other)
    torch.cuda.synchronize()
    for rep in range(2):
        ys = forward_packed_group(x, lins, workspace=ws)
        torch.cuda.synchronize()
        for y, w in zip(ys, want):
            assert torch.equal(y, w), rep
        if rep == 0:
            _check_after_wrap(ws, plan, wrap_job)
            w32 = ws.view(torch.int32).cpu().numpy().view(np.uint32)
            assert counter(w32[other]) == 2    # the other jobs go on counting
    w32 = ws.view(torch.int32).cpu().numpy().view(np.uint32)
    assert counter(w32[wrap_job]) == 1
