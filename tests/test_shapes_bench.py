"""Host logic of the per-configuration measurement harness (no GPU)."""
import torch

from quipsharp_amd import shapes_bench as sb


def test_make_weights_seeded_and_heavy_tailed():
    W1, X1 = sb.make_weights(64, 256, True, 5)
    W2, X2 = sb.make_weights(64, 256, True, 5)
    assert torch.equal(W1, W2) and torch.equal(X1, X2)
    assert X1.shape == (4096, 256)
    W0, _ = sb.make_weights(64, 256, False, 5)
    changed = (W1 != W0).float().mean().item()
    assert 0.005 < changed < 0.02  # about 1 % of the entries replaced
    assert W1.abs().max() > W0.abs().max()  # Student-t(3) tails


def test_linear_bytes_counts_stages():
    # 2-byte E8P codes per 8 weights (+1 byte per 8 for the E8 1-bit stage),
    # bf16 activations, bit-packed signs, one fp16 scale
    assert sb.linear_bytes(4096, 4096, 1, 1) == 4096 * 512 * 2 + 2 * 8192 + 1024 + 2
    assert sb.linear_bytes(4096, 4096, 1, 2) - sb.linear_bytes(4096, 4096, 1, 1) == 4096 * 512
