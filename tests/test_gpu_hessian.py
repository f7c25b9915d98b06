"""GPU Hessian accumulation (quipsharp/hessian.py:14-266) against fp64 X^T X / N,
group aliasing, and the save / load cache."""
import numpy as np
import pytest
import torch
from torch import nn

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


def test_collect_groups_and_cache(dev, tmp_path):
    from quipsharp_amd.hessian import collect_hessians, load_hessians, save_hessians

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.q = nn.Linear(64, 64)
            self.k = nn.Linear(64, 32)
            self.o = nn.Linear(64, 64)

        def forward(self, x):
            return self.o(self.q(x)) + self.k(x).sum()

    torch.manual_seed(0)
    net = Block().to(dev)
    batches = [torch.randn(4, 64, device=dev) for _ in range(3)]
    H = collect_hessians(net, batches, groups=[["q", "k"]], device=dev)
    assert set(H) == {"q", "k", "o"} and H["q"] is H["k"]
    X = torch.cat(batches).double()
    assert torch.allclose(H["q"].double(), X.T @ X / 12, atol=1e-5)
    save_hessians(H, "toy", root=tmp_path)
    back = load_hessians("toy", ["q", "k", "o"], root=tmp_path, device=dev)
    assert back["q"] is back["k"] and torch.equal(back["o"], H["o"])
    assert load_hessians("toy", ["q", "missing"], root=tmp_path) is None
