"""bfloat16 narrowing on the device against its bit-pattern rule.

Every kernel narrows float32 to bfloat16 with gfx950's conversion instruction
(``mround_amd/csrc/mr_common.h``: ``pack_bf16x2``, ``f32_to_bf16``). The rule
it must follow is torch's and MLX's: round to nearest, ties to even, on the bit
pattern (``(u + 0x7fff + ((u >> 16) & 1)) >> 16``), and a NaN keeps its sign
and high payload bits and is made quiet (``(u >> 16) | 0x40``). The oracle's
``round_to_bf16`` states the same rule on finite values. ``mr_cast_f32_bf16``
runs both forms (paired conversion on 16-byte rows, the single one otherwise);
here it converts all 2^32 float32 bit patterns and a ragged tail of special
values.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from mround_amd import kernels as K
from oracle import quantize as OQ

pytestmark = pytest.mark.gpu

CHUNK = 1 << 28


def _rule(u: torch.Tensor) -> torch.Tensor:
    """The expected bfloat16 bits (int64, 0..65535) of float32 bits u (int64, 0..2^32-1)."""
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return torch.where(nan, (u >> 16) | 0x40, rounded) & 0xFFFF


def _bits(u: torch.Tensor) -> torch.Tensor:
    """int64 values 0..2^32-1 as the int32 tensor with those bits."""
    return torch.where(u >= (1 << 31), u - (1 << 32), u).to(torch.int32)


def test_narrowing_matches_the_rule_on_every_float32():
    print("case bf16 narrowing, all 2^32 inputs", flush=True, file=sys.stderr)
    y = torch.empty(CHUNK, dtype=torch.bfloat16, device="cuda")
    for c in range((1 << 32) // CHUNK):
        u = torch.arange(c * CHUNK, (c + 1) * CHUNK, dtype=torch.int64, device="cuda")
        x = _bits(u).view(torch.float32)
        K.cast_bf16(x, y)
        got = y.view(torch.int16).to(torch.int64) & 0xFFFF
        want = _rule(u)
        bad = (got != want).nonzero()
        assert bad.numel() == 0, (c, [(hex(int(u[i])), hex(int(got[i])), hex(int(want[i])))
                                      for i in bad[:8, 0].tolist()])
        del u, x, got, want


def test_single_conversions_on_a_ragged_tail():
    specials = np.array([0x00000000, 0x80000000, 0x00000001, 0x807FFFFF, 0x3F808000, 0x3F818000,
                         0x3F80FFFF, 0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x7F800001, 0xFFC12345,
                         0x7FBFFFFF, 0x477FE000, 0x33800000], dtype=np.uint32)
    rng = np.random.default_rng(0)
    u = np.concatenate([specials, rng.integers(0, 1 << 32, size=4094, dtype=np.uint64).astype(np.uint32)])
    assert u.size % 4 != 0
    x = torch.from_numpy(u.view(np.int32)).cuda().view(torch.float32)
    y = torch.empty(u.size, dtype=torch.bfloat16, device="cuda")
    K.cast_bf16(x, y)
    got = (y.view(torch.int16).cpu().numpy().view(np.uint16)).astype(np.int64)
    want = _rule(torch.from_numpy(u.astype(np.int64))).numpy()
    assert np.array_equal(got, want)
    finite = np.isfinite(u.view(np.float32))
    ref = OQ.round_to_bf16(u.view(np.float32)[finite])
    assert np.array_equal(y.float().cpu().numpy()[finite].view(np.uint32), ref.view(np.uint32))
