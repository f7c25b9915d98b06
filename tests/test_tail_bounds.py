"""CPU bounds check of the index math of the forward kernels' tails.

The output transforms that run inside the decode-matvec kernels read and
write tagged 64-bit slots in the workspace and take dummy loads for absent
operands.  For every shape the kernels accept, each index they form under
their own guards is enumerated here and checked against the size of the
region it addresses; a plausible slip (a dropped guard, B where the region
holds 2 rows, a stride of m + 256) fails one of these cases.

Index forms (qs_forward_dev.h, qs_linear_fused.hip, qs_linear_batched.hip):
  poll_load / poll_issue / poll_finish: y1t + ((g B + b) m + 256 c + lane + 64 j)
      for c = w + 16 u < S_m, g < SG, b < B, lane < 64, j < 4; re-polls only
      reload entries whose first load was a real one
  bm_kernel reduction store: ((sg B + bc) m + 16 rb + row), rb < m / 16, row < 16
  store_h2 / poll_columns: h2t + (b m + 256 c + 16 g + tt), c < S_m, g < 16, tt < 16
  output index and dummy loads: 256 r + t, r < S_m, t < 256 (su words: that / 32)
Region sizes (ws_layout, fused_block in qs_linear.hip): one-launch slots
SG_f 2 m, its chunk transforms 2 m, the 16-row decode-matvec's slots SG B m.
"""
import numpy as np
import pytest


def slot_indices(m, B, SG):
    """Every slot a tail work-group polls: poll_load's address under its guards."""
    Sm = m // 256
    g, b, w, u, lane, j = np.meshgrid(np.arange(SG), np.arange(B), np.arange(16), np.arange(3),
                                      np.arange(64), np.arange(4), indexing="ij", sparse=True)
    c = w + 16 * u
    idx = (g * B + b) * m + 256 * c + lane + 64 * j
    return idx[np.broadcast_to(c < Sm, idx.shape)]


def reduction_indices(m, B, SG):
    sg, bc, rb, row = np.meshgrid(np.arange(SG), np.arange(B), np.arange(m // 16), np.arange(16),
                                  indexing="ij", sparse=True)
    return ((sg * B + bc) * m + 16 * rb + row).ravel()


def column_indices(m, B):
    """poll_columns: v = tid + 1024 k -> (c, tt) = (v / 16, v % 16), column group g."""
    Sm = m // 256
    b, g, v = np.meshgrid(np.arange(B), np.arange(16), np.arange(2048), indexing="ij", sparse=True)
    c, tt = v >> 4, v & 15
    idx = b * m + 256 * c + 16 * g + tt
    return idx[np.broadcast_to(c < Sm, idx.shape)]


def output_indices(m):
    r, t = np.meshgrid(np.arange(m // 256), np.arange(256), indexing="ij")
    return (256 * r + t).ravel()


def check(idx, cap, what):
    assert idx.size > 0, what
    assert idx.min() >= 0 and idx.max() < cap, f"{what}: index {idx.max()} outside {cap}"


@pytest.mark.parametrize("S", [1, 2, 3, 7, 16, 20, 43, 48])
@pytest.mark.parametrize("B", [3, 8, 15, 16])
@pytest.mark.parametrize("SG", [1, 2, 3])
def test_batched_tail_slots_in_bounds(S, B, SG):
    m = 256 * S
    cap = SG * B * m  # the 16-row decode-matvec's tagged slots
    check(slot_indices(m, B, SG), cap, "poll")
    red = reduction_indices(m, B, SG)
    check(red, cap, "reduction store")
    assert np.unique(red).size == cap  # every slot written once: each poll finds its value


@pytest.mark.parametrize("S", [1, 4, 16, 20, 43, 64, 100, 128])
@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("SG", [1, 2, 5, 8])
def test_one_launch_tail_in_bounds(S, B, SG):
    m = 256 * S
    if S <= 16:  # one work-group polls the slots (m <= 4096)
        check(slot_indices(m, B, SG), SG * 2 * m, "one-launch poll")
    else:  # two levels: chunk transforms as slots, then 16 column groups
        check(column_indices(m, B), 2 * m, "column poll")
        c, lane, j = np.meshgrid(np.arange(S), np.arange(64), np.arange(4), indexing="ij", sparse=True)
        for b in range(B):
            check((b * m + 256 * c + lane + 64 * j).ravel(), 2 * m, "store_h2")


@pytest.mark.parametrize("S", [1, 16, 43, 48, 128])
def test_output_and_dummy_indices_in_bounds(S):
    m = 256 * S
    o = output_indices(m)
    check(o, m, "output / bias / su")
    check(o >> 5, -(-m // 32), "su sign-bit words")
    # a dummy source stands in for an absent bias: the slots hold >= 2 m floats
    check(o, 2 * m, "dummy load from the slots")


def test_a_planted_slip_is_caught():
    """A poll that skipped its c < S_m guard would read past the region."""
    m, B, SG = 256 * 20, 16, 2
    g, b, w, u, lane, j = np.meshgrid(np.arange(SG), np.arange(B), np.arange(16), np.arange(3),
                                      np.arange(64), np.arange(4), indexing="ij", sparse=True)
    unguarded = ((g * B + b) * m + 256 * (w + 16 * u) + lane + 64 * j).ravel()
    with pytest.raises(AssertionError):
        check(unguarded, SG * B * m, "unguarded poll")
