"""GPU Hessian accumulation (quipsharp/hessian.py:14-29) against fp64 X^T X / N."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_accumulator_matches_fp64(dev):
    from quipsharp_amd.hessian import HessianAccumulator
    g = torch.Generator().manual_seed(0)
    xs = [torch.randn(b, 7, 384, generator=g) for b in (3, 5, 2)]
    acc = HessianAccumulator(384, device=dev)
    for x in xs:
        acc.update(x.to(dev).bfloat16())
    X = torch.cat([x.reshape(-1, 384) for x in xs]).bfloat16().double()
    want = (X.T @ X / X.shape[0]).numpy()
    got = acc.hessian.cpu().double().numpy()
    assert acc.count == 70
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
