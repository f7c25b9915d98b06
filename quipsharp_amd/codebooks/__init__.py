"""Lattice codebooks (quipsharp/codebooks/__init__.py)."""
from .e8p import (E8PCodebook, build_abs_table, decode_from_table, encode_to_table, pack_code,
                  unpack_code)
from .e8_1bit import E8OneBitCodebook, build_table

__all__ = [
    "E8PCodebook", "build_abs_table", "encode_to_table", "decode_from_table",
    "pack_code", "unpack_code", "E8OneBitCodebook", "build_table",
]
