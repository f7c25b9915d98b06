"""Import root with the reference's package name (numbersletter/quipsharp), so
its scripts bind unchanged: ``from quipsharp.checkpoint import ...``,
``from quipsharp.model_loading import load_eval_model`` (scripts/eval_ppl.py:18).

Each hot-path module of the reference is this library's module of the same
name (``sys.modules`` aliases, so ``quipsharp.checkpoint is
quipsharp_amd.checkpoint``): hadamard, incoherence, rfft, codebooks (e8p,
e8_1bit), rvq, ldlq, quantize, checkpoint, architectures, hessian,
model_loading.  The reference's lazy hub loaders (lazy_weights) and its
calibration scripts are not part of this library."""
import importlib
import sys

import quipsharp_amd

_MODULES = ("hadamard", "incoherence", "rfft", "codebooks", "codebooks.e8p", "codebooks.e8_1bit", "rvq", "ldlq",
            "quantize", "checkpoint", "architectures", "hessian", "model_loading")

for _name in _MODULES:
    _mod = importlib.import_module("quipsharp_amd." + _name)
    sys.modules[__name__ + "." + _name] = _mod
    if "." not in _name:
        globals()[_name] = _mod

__version__ = quipsharp_amd.__version__
