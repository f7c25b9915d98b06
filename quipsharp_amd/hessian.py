"""Calibration Hessians on the GPU (quipsharp/hessian.py:14-115): H = E[x x^T]
over a layer's input activations, accumulated in fp32 with one GEMM per batch
(rocBLAS / hipBLASLt through torch on the device, so calibration feeds
``quantize_linear`` without a host round trip)."""
import json
from pathlib import Path

import torch
from torch import nn, Tensor

from . import _lib

ALIAS_MANIFEST_NAME = "_aliases.json"


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


def collect_hessians(model: nn.Module, calibration_batches, layer_names=None, groups=None,
                     device="cuda") -> dict:
    """quipsharp/hessian.py:32-91: forward hooks on the nn.Linear submodules
    accumulate E[x x^T] over ``model(batch)`` for each calibration batch.
    ``groups``: lists of layer names that read the same activations (q/k/v,
    gate/up); only the first of each is hooked and the others share its
    Hessian by object identity."""
    representative_of = {}
    for group in groups or []:
        for name in group:
            representative_of[name] = group[0]
    accumulators = {}
    hooks = []

    def make_hook(name, n):
        acc = HessianAccumulator(n, device=device)
        accumulators[name] = acc

        def hook(module, inputs, output):
            acc.update(inputs[0].detach())

        return hook

    for name, module in model.named_modules():
        if not (isinstance(module, nn.Linear) and (layer_names is None or name in layer_names)):
            continue
        if name in representative_of and representative_of[name] != name:
            continue
        hooks.append(module.register_forward_hook(make_hook(name, module.in_features)))
    if not hooks:
        raise ValueError("no matching nn.Linear layers found to hook")
    model.eval()
    with torch.no_grad():
        for batch in calibration_batches:
            model(batch)
    for h in hooks:
        h.remove()
    hessians = {name: acc.hessian for name, acc in accumulators.items()}
    for name, rep in representative_of.items():
        if name != rep and rep in hessians:
            hessians[name] = hessians[rep]
    return hessians


def save_hessians(hessians: dict, model_name: str, root: str = "hess") -> None:
    """quipsharp/hessian.py:94-129: <root>/<model_name>/<layer>.pt, shared
    tensors written once and the other names recorded in an alias manifest
    (merged with an existing one)."""
    out_dir = Path(root) / model_name
    out_dir.mkdir(parents=True, exist_ok=True)
    manifest_path = out_dir / ALIAS_MANIFEST_NAME
    aliases = json.loads(manifest_path.read_text()) if manifest_path.exists() else {}
    written = {}
    for name, H in hessians.items():
        if id(H) in written:
            aliases[name] = written[id(H)]
            continue
        written[id(H)] = name
        torch.save(H.cpu(), out_dir / f"{name}.pt")
    if aliases:
        manifest_path.write_text(json.dumps(aliases, indent=2))


def load_hessians(model_name: str, layer_names, root: str = "hess", device="cuda"):
    """quipsharp/hessian.py:234-266: the saved Hessians of ``layer_names``, or
    None when the cache is missing or incomplete (so the caller recomputes
    instead of mixing stale and fresh data).  Aliases share one tensor;
    files are read with ``torch.load(weights_only=True)`` (tensors only)."""
    out_dir = Path(root) / model_name
    if not out_dir.exists():
        return None
    manifest_path = out_dir / ALIAS_MANIFEST_NAME
    aliases = json.loads(manifest_path.read_text()) if manifest_path.exists() else {}
    loaded = {}
    out = {}
    for name in layer_names:
        src = aliases.get(name, name)
        if src not in loaded:
            path = out_dir / f"{src}.pt"
            if not path.exists():
                return None
            loaded[src] = torch.load(path, map_location="cpu", weights_only=True).to(device)
        out[name] = loaded[src]
    return out
