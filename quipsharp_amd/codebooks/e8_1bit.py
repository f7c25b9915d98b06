"""The 1-bit E8 codebook used as the second residual stage of 3-bit QuIP#
(quipsharp/codebooks/e8_1bit.py): the zero vector, the 240 norm^2 = 2 vectors
of E8 and 15 norm^2 = 4 vectors, 256 entries, nearest-neighbour search by
brute force in the library (first index wins ties, as torch.argmin does)."""
import ctypes

import torch
from torch import Tensor

from .. import _lib
from .e8p import _decode, _encode

CODE_DIM = 8
TABLE_SIZE = 256


def build_table() -> Tensor:
    """(256, 8) fp32 table (quipsharp/codebooks/e8_1bit.py:66-70), as built into the library."""
    t = torch.empty(TABLE_SIZE, CODE_DIM, dtype=torch.float32)
    _lib.check(_lib.lib().qs_e81_table(ctypes.c_void_p(t.data_ptr())))
    return t


def norm2_shell() -> Tensor:
    """The 240 minimal vectors of E8 (table rows 1..240)."""
    return build_table()[1:241]


class E8OneBitCodebook:
    """quipsharp/codebooks/e8_1bit.py:73-87."""

    stage_kind = _lib.QS_STAGE_E8_1BIT

    def native_stages(self):
        """(kinds, scales) of this codebook as a residual-VQ chain."""
        return [self.stage_kind], [1.0]

    def __init__(self, device=None):
        self.table = build_table().to(device=device)

    def quantize(self, x: Tensor):
        vals, codes = _encode(x, [_lib.QS_STAGE_E8_1BIT], [1.0])
        return vals, codes[0]

    def dequantize(self, idx: Tensor) -> Tensor:
        return _decode(idx.unsqueeze(0), [_lib.QS_STAGE_E8_1BIT], [1.0])
