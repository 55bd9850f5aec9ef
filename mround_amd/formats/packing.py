"""MLX uint32 packing on MI355X (``mround/formats/packing.py:84-206``).

Same names, layouts, validation and messages as the reference; the packing
itself is ``mr_pack_codes`` / ``mr_unpack_codes``. Codes are expected in one
byte each (uint8, or int8 with ``offset``) -- the form the tuning path keeps
them in (``mround/formats/mlx_export.py:109-125``); wider integer tensors are
narrowed after their range has been checked.

Portions follow MRound (Copyright 2026 The MRound Authors, Apache License 2.0);
see NOTICE.
"""

from __future__ import annotations

import torch

from mround_amd import kernels as K
from mround_amd.schemes import SUPPORTED_BITS

__all__ = ["pack_codes", "packed_width", "unpack_codes"]

WORD_BITS = 32
MATRIX_NDIM = 2


def _validate_bits(bits: int) -> None:
    if bits not in SUPPORTED_BITS:
        supported = ", ".join(str(b) for b in sorted(SUPPORTED_BITS))
        msg = f"bits must be one of {{{supported}}}, got {bits}"
        raise ValueError(msg)


def packed_width(in_features: int, bits: int) -> int:
    """Words per row (``mround/formats/packing.py:84-116``)."""
    _validate_bits(bits)
    if WORD_BITS % bits == 0:
        per_word = WORD_BITS // bits
        if in_features % per_word:
            msg = f"in_features={in_features} is not a multiple of {per_word} codes per word at {bits} bits"
            raise ValueError(msg)
        return in_features // per_word
    if in_features % WORD_BITS:
        msg = (
            f"in_features={in_features} is not a multiple of 32, which the "
            f"cross-word bitstream layout requires at {bits} bits"
        )
        raise ValueError(msg)
    return in_features // WORD_BITS * bits


def pack_codes(codes: torch.Tensor, bits: int, *, offset: int = 0) -> torch.Tensor:
    """Pack unsigned codes into uint32 words (``mround/formats/packing.py:119-163``).

    ``offset`` is added first (``2**(bits-1)`` turns symmetric signed codes
    into stored unsigned ones, ``mround/formats/mlx_export.py:219-221``).

    Raises:
        ValueError: If a code leaves ``[0, 2**bits - 1]`` or the row does not tile.
    """
    _validate_bits(bits)
    if codes.ndim != MATRIX_NDIM:
        msg = f"expected a 2-D code matrix, got shape {tuple(codes.shape)}"
        raise ValueError(msg)
    rows, cols = codes.shape
    words = packed_width(cols, bits)
    hi = 2**bits - 1
    if codes.dtype in (torch.uint8, torch.int8):
        narrow = codes.contiguous()
    else:
        lo_seen, hi_seen = int(codes.min()) + offset, int(codes.max()) + offset
        if lo_seen < 0 or hi_seen > hi:
            msg = f"codes must lie in [0, {hi}] at {bits} bits, got [{lo_seen}, {hi_seen}]"
            raise ValueError(msg)
        narrow = (codes.to(torch.int32) + offset).to(torch.uint8).contiguous()
        offset = 0
    packed = torch.empty((rows, words), dtype=torch.uint32, device=codes.device)
    rng = torch.empty(2, dtype=torch.int32, device=codes.device)
    K.pack_codes(narrow, bits, signed=narrow.dtype == torch.int8, offset=offset, packed_out=packed,
                 range_out=rng)
    if rows and cols:
        lo_seen, hi_seen = (int(x) for x in rng.tolist())
        if lo_seen < 0 or hi_seen > hi:
            msg = f"codes must lie in [0, {hi}] at {bits} bits, got [{lo_seen}, {hi_seen}]"
            raise ValueError(msg)
    return packed


def unpack_codes(packed: torch.Tensor, in_features: int, bits: int) -> torch.Tensor:
    """Inverse of :func:`pack_codes` (``mround/formats/packing.py:166-206``), uint8 codes."""
    _validate_bits(bits)
    expected = packed_width(in_features, bits)
    if packed.shape[1] != expected:
        msg = (
            f"expected {expected} words per row for in_features={in_features} "
            f"at {bits} bits, got {packed.shape[1]}"
        )
        raise ValueError(msg)
    rows = packed.shape[0]
    codes = torch.empty((rows, in_features), dtype=torch.uint8, device=packed.device)
    K.unpack_codes(packed.contiguous(), rows, in_features, bits, codes)
    return codes
