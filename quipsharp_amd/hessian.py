"""Calibration Hessian accumulation on the GPU (quipsharp/hessian.py:14-29):
H = E[x x^T] over a layer's input activations, accumulated in fp32 with one
GEMM per batch (rocBLAS / hipBLASLt through torch on the device), so a
Hessian feeds ``quantize_linear`` without a host round trip.  Collecting
Hessians over a calibration dataset and caching them on disk are outside
this library."""
import torch
from torch import Tensor

from . import _lib


class HessianAccumulator:
    """quipsharp/hessian.py:14-29: H = sum_i x_i x_i^T, then H / count."""

    def __init__(self, n: int, device="cuda", dtype=torch.float32):
        self.n = n
        self.H = torch.zeros(n, n, device=device, dtype=dtype)
        _lib.require_gpu(self.H, what="Hessian accumulation")
        self.count = 0

    def update(self, x: Tensor) -> None:
        x = x.reshape(-1, self.n).to(device=self.H.device, dtype=self.H.dtype)
        self.H.addmm_(x.T, x)
        self.count += x.shape[0]

    @property
    def hessian(self) -> Tensor:
        return self.H / max(self.count, 1)
