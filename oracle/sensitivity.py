"""DeltaLoss and storage cost (oracle).

Restates ``mround/planner/sensitivity.py:190-349`` and the per-batch term of
``mround/pipeline/scoring.py:238-266``.
"""

from __future__ import annotations

import numpy as np

from oracle.quantize import fake_quantize


def delta_loss(weight, quantized_weight, gradient) -> float:
    """``sum |g * (Wq - W)|`` in float64 (``mround/planner/sensitivity.py:190-229``)."""
    w = np.asarray(weight, dtype=np.float64)
    q = np.asarray(quantized_weight, dtype=np.float64)
    g = np.asarray(gradient, dtype=np.float64)
    if not (w.shape == q.shape == g.shape):
        raise ValueError("weight, quantized weight, and gradient must share one shape")
    return float(np.sum(np.abs(g * (q - w))))


def delta_terms_f32(weight, gradient, *, bits, group_size, mode, eps=1e-8) -> np.ndarray:
    """The float32 terms ``|g * (rtn(W) - W)|`` the scoring pass sums.

    ``mround/pipeline/scoring.py:213-221, 262``: the perturbation is the
    round-to-nearest reconstruction in float32 less the float32 weight.
    """
    w = np.asarray(weight, dtype=np.float32)
    q, _, _, _ = fake_quantize(w, None, None, None, bits=bits, group_size=group_size, mode=mode,
                               eps=eps, dtype=np.float32)
    return np.abs(np.asarray(gradient, dtype=np.float32) * (q - w))


def groups_per_row(in_features: int, group_size: int) -> int:
    """``mround/planner/sensitivity.py:271-294``."""
    if group_size == -1:
        return 1
    if group_size <= 0 or in_features % group_size:
        raise ValueError(f"in_features {in_features} is not a multiple of group size {group_size}")
    return in_features // group_size


def storage_bits(shape, bits: int, group_size: int, *, dtype_bits: int = 16) -> int:
    """``mround/planner/sensitivity.py:232-268``: codes plus a scale and bias per group."""
    out_features, in_features = shape
    groups = out_features * groups_per_row(in_features, group_size)
    return out_features * in_features * bits + 2 * groups * dtype_bits


def mixed_budget_bits(shapes, average_bits: float, group_size: int, *, dtype_bits: int = 16) -> int:
    """``mround/planner/sensitivity.py:297-349``."""
    elements = 0
    metadata = 0
    for out_features, in_features in shapes.values():
        elements += out_features * in_features
        metadata += 2 * out_features * groups_per_row(in_features, group_size) * dtype_bits
    return int(elements * average_bits) + metadata
