"""Per-layer sensitivity and storage cost (mround/planner/sensitivity.py:190-432).

DeltaLoss scores a layer at a candidate width as ``sum |g * (Q_b(W) - W)|``,
with ``g`` the loss gradient at the quantized weights from a calibration
backward pass. The per-batch term runs on the GPU (``mr_delta_loss``: every
candidate width in one read of W and g, each term accumulated in fp64); the
storage cost and the allocator's input are host arithmetic.

Portions follow MRound (Copyright 2026 The MRound Authors, Apache License 2.0);
see NOTICE.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence

import numpy as np
import torch

from mround_amd import kernels as K
from mround_amd.core.quantizer import mode_of
from mround_amd.exceptions import SchemeError
from mround_amd.planner.allocator import LayerOption
from mround_amd.schemes import DEFAULT_EPS_FP32, QuantScheme

SENSITIVITY_SAMPLES = 128  # mround/planner/sensitivity.py:91-92
SENSITIVITY_SEQ_LEN = 1024
SENSITIVITY_BATCH_TOKENS = 2048
OWN_WIDTH_FROM_WEIGHTS = 2_500_000_000
GRADIENT_SOURCES = ("auto", "own_width", "widest")


def gradient_source_for(requested: str, scored_weights: int) -> str:
    """``"own_width"`` from 2.5 B scored weights up, else ``"widest"``, unless
    asked for explicitly (mround/planner/sensitivity.py:128-156)."""
    if requested not in GRADIENT_SOURCES:
        raise SchemeError("sensitivity_gradients must be one of "
                          f"{', '.join(repr(s) for s in GRADIENT_SOURCES)}, got {requested!r}")
    if requested != "auto":
        return requested
    return "own_width" if int(scored_weights) >= OWN_WIDTH_FROM_WEIGHTS else "widest"


def scoring_batch_size(n_samples: int, seq_len: int, *,
                       budget_tokens: int = SENSITIVITY_BATCH_TOKENS) -> int:
    """Sequences per scoring batch at a fixed token budget (sensitivity.py:159-187)."""
    per_batch = max(1, int(budget_tokens) // max(1, int(seq_len)))
    return max(1, min(int(n_samples), per_batch))


def delta_loss(weight, quantized_weight, gradient) -> float:
    """``sum |g (Wq - W)|`` in float64 for one layer at one width
    (mround/planner/sensitivity.py:190-229)."""
    w = torch.as_tensor(weight).double()
    q = torch.as_tensor(quantized_weight).double()
    g = torch.as_tensor(gradient).double()
    if not (w.shape == q.shape == g.shape):
        raise ValueError(f"weight {tuple(w.shape)}, quantized weight {tuple(q.shape)}, and gradient "
                         f"{tuple(g.shape)} must share one shape")
    return float((g * (q - w)).abs().sum())


class DeltaLossAccumulator:
    """Running DeltaLoss per layer and width over calibration batches, on the
    device (the per-batch ``_accumulate`` of mround/pipeline/scoring.py:238-266,
    with round-to-nearest perturbations at every candidate width)."""

    def __init__(self, widths: Sequence[int], scheme: QuantScheme, *,
                 eps: float = DEFAULT_EPS_FP32) -> None:
        if not widths:
            raise ValueError("no candidate widths")
        self.widths = tuple(int(b) for b in widths)
        self.scheme = scheme
        self.eps = eps
        self._scores: dict[str, torch.Tensor] = {}

    def add(self, name: str, weight: torch.Tensor, gradient: torch.Tensor) -> None:
        """Add one batch's terms for layer ``name``: weight (rows, cols) in its
        model dtype, gradient fp32 (rows, cols), both on the device."""
        acc = self._scores.get(name)
        if acc is None:
            acc = torch.zeros(len(self.widths), dtype=torch.float64, device=weight.device)
            self._scores[name] = acc
        K.delta_loss(weight.contiguous(), gradient.contiguous().float(),
                     group_size=self.scheme.group_size, bits_list=list(self.widths),
                     mode=mode_of(self.scheme), eps=self.eps, scores_out=acc)

    def scores(self) -> dict[str, dict[int, float]]:
        return {n: dict(zip(self.widths, acc.cpu().tolist())) for n, acc in self._scores.items()}


def groups_per_row(in_features: int, group_size: int) -> int:
    """Scales per output channel, ``-1`` meaning one (sensitivity.py:271-294)."""
    if group_size == -1:
        return 1
    if group_size <= 0 or in_features % group_size:
        raise ValueError(f"in_features {in_features} is not a multiple of group size {group_size}; "
                         "this layer stays dense and has no quantized cost")
    return in_features // group_size


def storage_bits(shape: tuple[int, int], bits: int, group_size: int, *, dtype_bits: int = 16) -> int:
    """Packed codes plus a scale and a bias per group (sensitivity.py:232-268)."""
    out_features, in_features = shape
    if out_features <= 0 or in_features <= 0:
        raise ValueError(f"shape must be positive, got {shape}")
    groups = out_features * groups_per_row(in_features, group_size)
    return out_features * in_features * bits + 2 * groups * dtype_bits


def mixed_budget_bits(shapes: Mapping[str, tuple[int, int]], average_bits: float, group_size: int,
                      *, dtype_bits: int = 16) -> int:
    """``int(elements * average) + metadata`` (sensitivity.py:297-349)."""
    if not shapes:
        raise ValueError("no layers to budget over")
    if average_bits <= 0:
        raise ValueError(f"average_bits must be positive, got {average_bits}")
    elements = 0
    metadata = 0
    for name, (out_features, in_features) in shapes.items():
        if out_features <= 0 or in_features <= 0:
            raise ValueError(f"layer {name!r} with shape {(out_features, in_features)} cannot be grouped")
        try:
            groups = groups_per_row(in_features, group_size)
        except ValueError as exc:
            raise ValueError(f"layer {name!r} with shape {(out_features, in_features)} cannot be "
                             "grouped") from exc
        elements += out_features * in_features
        metadata += 2 * out_features * groups * dtype_bits
    return int(elements * average_bits) + metadata


def score_layer_options(scores: Mapping[str, Mapping[int, float]],
                        shapes: Mapping[str, tuple[int, int]], base_scheme: QuantScheme, *,
                        dtype_bits: int = 16) -> dict[str, list[LayerOption]]:
    """Per-layer per-width scores into the allocator's input (sensitivity.py:352-432)."""
    if set(scores) != set(shapes):
        only_scores = sorted(set(scores) - set(shapes))
        only_shapes = sorted(set(shapes) - set(scores))
        raise ValueError(f"scores and shapes must cover the same layers; only scored: {only_scores}, "
                         f"only shaped: {only_shapes}")
    if not scores:
        raise ValueError("no layers to score")
    widths: set[int] | None = None
    for name, per_width in scores.items():
        if widths is None:
            widths = set(per_width)
            if not widths:
                raise ValueError(f"layer {name!r} has no scored widths")
        elif set(per_width) != widths:
            raise ValueError(f"layer {name!r} is scored at widths {sorted(per_width)} but others at "
                             f"{sorted(widths)}; every layer must come from the same scoring passes")
    options: dict[str, list[LayerOption]] = {}
    for name, per_width in scores.items():
        out_features, in_features = shapes[name]
        candidates = []
        for width in sorted(per_width):
            score = per_width[width]
            if not np.isfinite(score) or score < 0.0:
                raise ValueError(f"layer {name!r} at {width} bits has invalid score {score!r}")
            candidates.append(LayerOption(
                bits=width,
                cost_bits=storage_bits(shapes[name], width, base_scheme.group_size,
                                       dtype_bits=dtype_bits),
                delta_loss=float(score), elements=out_features * in_features))
        options[name] = candidates
    return options
