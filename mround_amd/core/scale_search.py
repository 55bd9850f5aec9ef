"""The v2 candidate-scale grid search (mround/core/scale_search.py).

Before the rounding is learned, a symmetric scheme below 4 bits picks each
group's initial scale by trying a line of clipping thresholds and keeping
the one with the least importance-weighted reconstruction error
(``mr_search_scales``, one GPU thread per group). The searched scale then
enters fake quantization as ``init_scale`` with ``beta`` learning a factor
around it (``ScaleInit.SEARCHED``).
"""

from __future__ import annotations

import dataclasses

import torch

from mround_amd import kernels as K
from mround_amd.schemes import QuantScheme, Symmetry

_TWO_BIT_HALF_COUNT = 90
_TWO_BIT_STEP = 0.01
_GRID = 200


@dataclasses.dataclass(frozen=True, slots=True)
class SearchGrid:
    """The candidate family (mround/reference/scale_search.py:66-100): step and
    half-count; 2 bits use a fixed finer window (0.01, 90), other widths
    ``span = nmax * ratio``, ``step = span / 200 * 2``, ``half = int(span / step)``."""

    ratio: float = 0.75

    def steps(self, bits: int) -> tuple[float, int]:
        if bits == 2:
            return _TWO_BIT_STEP, _TWO_BIT_HALF_COUNT
        nmax = float(2 ** (bits - 1))
        span = nmax * self.ratio
        step = span / _GRID * 2
        return step, int(span / step)


def search_scales(weight: torch.Tensor, scheme: QuantScheme, *,
                  importance: torch.Tensor | None = None,
                  grid: SearchGrid | None = None) -> torch.Tensor:
    """One signed scale per group, ``(n_groups, 1)`` fp32 on the weight's device
    (mround/core/scale_search.py:71-127). Zero for an all-zero group.

    Raises ``ValueError`` for a non-symmetric scheme, a weight that does not
    group evenly, or an importance whose length is not the input width.
    """
    if scheme.symmetry is not Symmetry.SYMMETRIC:
        raise ValueError("the searched initialization is defined for symmetric schemes only")
    if weight.dim() != 2 or weight.shape[-1] % scheme.group_size:
        raise ValueError(f"search expects a 2-D weight whose last dimension is a multiple of "
                         f"group_size={scheme.group_size}, got shape {tuple(weight.shape)}")
    imp = None
    if importance is not None:
        imp = importance.to(device=weight.device, dtype=torch.float32).reshape(-1).contiguous()
        if imp.numel() != weight.shape[-1]:
            raise ValueError(f"importance has {imp.numel()} channels but the weight has "
                             f"{weight.shape[-1]} input features")
    rows, cols = weight.shape
    step, half = (grid or SearchGrid()).steps(scheme.bits)
    w = weight if weight.dtype in (torch.float32, torch.bfloat16) else weight.float()
    out = torch.empty(rows * (cols // scheme.group_size), 1, dtype=torch.float32, device=weight.device)
    K.search_scales(w.contiguous(), bits=scheme.bits, group_size=scheme.group_size, step=step,
                    half_count=half, scale_out=out, importance=imp)
    return out
