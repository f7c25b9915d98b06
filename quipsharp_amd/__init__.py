"""quipsharp_amd -- the QuIP# quantize/dequantize hot path on AMD MI355X (gfx950).

Same public API as numbersletter/quipsharp's ``hadamard``, ``incoherence``,
``codebooks``, ``rvq``, ``ldlq``, ``quantize`` and ``checkpoint`` modules;
the computation runs in libquipsharp_hip.so (hand-written HIP kernels for
gfx950, C ABI in include/quipsharp_hip.h) on torch-ROCm device memory and
streams.  There is no CPU fallback: CPU tensors are rejected.
"""
from . import _lib

__version__ = "0.1.0"


def library_path():
    return _lib.LIB_PATH
