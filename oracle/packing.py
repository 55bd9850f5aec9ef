"""MLX uint32 packing and the affine export convention (oracle).

Restates ``mround/reference/packing.py:38-168`` (pack/unpack, both layouts) and
``mround/formats/mlx_export.py:109-125, 159-195`` (narrow_codes, to_affine).
``mlx_style_pack`` is the second, independent construction the reference's
tests use (explode to bits, regroup by 32, reassemble;
``tests/unit/test_reference_packing.py:180-225``).
"""

from __future__ import annotations

import numpy as np

WORD_BITS = 32
SUPPORTED_BITS = (2, 3, 4, 5, 6, 7, 8)


def packed_width(in_features: int, bits: int) -> int:
    """``mround/reference/packing.py:38-70``."""
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"bits must be one of {{2, 3, 4, 5, 6, 7, 8}}, got {bits}")
    if WORD_BITS % bits == 0:
        per_word = WORD_BITS // bits
        if in_features % per_word:
            raise ValueError(
                f"in_features={in_features} is not a multiple of {per_word} codes per word at {bits} bits"
            )
        return in_features // per_word
    if in_features % WORD_BITS:
        raise ValueError(
            f"in_features={in_features} is not a multiple of 32, which the cross-word "
            f"bitstream layout requires at {bits} bits"
        )
    return in_features // WORD_BITS * bits


def pack_codes(codes, bits: int) -> np.ndarray:
    """``mround/reference/packing.py:73-122``: element 0 in the least significant bits."""
    codes = np.asarray(codes)
    if codes.ndim != 2:
        raise ValueError(f"expected a 2-D code matrix, got shape {codes.shape}")
    hi = 2**bits - 1
    if codes.min(initial=0) < 0 or codes.max(initial=0) > hi:
        raise ValueError(f"codes must lie in [0, {hi}] at {bits} bits, got [{codes.min()}, {codes.max()}]")
    rows, cols = codes.shape
    words = packed_width(cols, bits)
    wide = codes.astype(np.uint64)
    if WORD_BITS % bits == 0:
        per_word = WORD_BITS // bits
        blocks = wide.reshape(rows, words, per_word)
        shifts = (np.arange(per_word, dtype=np.uint64) * np.uint64(bits)).reshape(1, 1, -1)
        return np.bitwise_or.reduce(blocks << shifts, axis=-1).astype(np.uint32)
    out = np.zeros((rows, words), dtype=np.uint64)
    for i in range(cols):
        word, offset = divmod(i * bits, WORD_BITS)
        out[:, word] |= wide[:, i] << np.uint64(offset)
        spill = offset + bits - WORD_BITS
        if spill > 0:
            out[:, word + 1] |= wide[:, i] >> np.uint64(bits - spill)
    return (out & np.uint64(0xFFFFFFFF)).astype(np.uint32)


def unpack_codes(packed, in_features: int, bits: int) -> np.ndarray:
    """``mround/reference/packing.py:125-168``."""
    packed = np.asarray(packed)
    expected = packed_width(in_features, bits)
    if packed.shape[1] != expected:
        raise ValueError(
            f"expected {expected} words per row for in_features={in_features} at {bits} bits, "
            f"got {packed.shape[1]}"
        )
    rows = packed.shape[0]
    mask = np.uint64(2**bits - 1)
    wide = packed.astype(np.uint64)
    if WORD_BITS % bits == 0:
        per_word = WORD_BITS // bits
        shifts = (np.arange(per_word, dtype=np.uint64) * np.uint64(bits)).reshape(1, 1, -1)
        return ((wide[:, :, None] >> shifts) & mask).reshape(rows, -1)[:, :in_features].astype(np.int64)
    out = np.zeros((rows, in_features), dtype=np.uint64)
    for i in range(in_features):
        word, offset = divmod(i * bits, WORD_BITS)
        value = wide[:, word] >> np.uint64(offset)
        spill = offset + bits - WORD_BITS
        if spill > 0:
            value |= wide[:, word + 1] << np.uint64(bits - spill)
        out[:, i] = value & mask
    return out.astype(np.int64)


def mlx_style_pack(codes, bits: int) -> np.ndarray:
    """Independent construction: explode to bits, regroup by 32, reassemble."""
    codes = np.asarray(codes)
    rows = codes.shape[0]
    exploded = ((codes[:, :, None].astype(np.uint32) >> np.arange(bits, dtype=np.uint32)) & 1)
    words = exploded.reshape(rows, -1).reshape(rows, -1, 32).astype(np.uint64)
    place = np.uint64(1) << np.arange(32, dtype=np.uint64)
    return (words * place).sum(axis=-1).astype(np.uint32)


def narrow_codes(codes, bits: int, symmetric: bool) -> np.ndarray:
    """``mround/formats/mlx_export.py:109-125``: one byte per code."""
    return np.asarray(codes).astype(np.int8 if symmetric else np.uint8)


def _round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 -> ``dtype`` -> float32 (round half to even)."""
    from oracle.quantize import round_to_bf16

    x = np.asarray(x, dtype=np.float32)
    if dtype == "bfloat16":
        return round_to_bf16(x)
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    return x


def to_affine(scale, zero_point, bits: int, dtype: str = "bfloat16"):
    """``mround/formats/mlx_export.py:159-195``, values returned as float32.

    ``scales = dtype(scale)``; ``biases = dtype(-scales * dtype(zero_point))``,
    with the fixed ``2**(bits-1)`` for a symmetric scheme. A bf16/fp16 product
    is formed exactly in float32 and rounded once, as MLX's half-precision
    arithmetic does.
    """
    scales = _round_to(scale, dtype)
    if zero_point is None:
        biases = _round_to(-scales * np.float32(2 ** (bits - 1)), dtype)
    else:
        biases = _round_to(-scales * _round_to(zero_point, dtype), dtype)
    return scales, biases
