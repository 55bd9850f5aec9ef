"""Whole-model sensitivity scoring for mixed precision (mround/pipeline/scoring.py).

For every block layer and candidate width, DeltaLoss ``sum |g (Q_b(W) - W)|``
summed over calibration batches, with ``g`` the gradient of the model's causal
cross-entropy at the quantized model (``CausalLM``) and ``Q_b`` round to
nearest at width b (the searched grid where the scheme searches, without
importance, scoring.py:196-211). Two schedules, as the reference's:

* ``"own_width"`` (scoring.py:269-315): per width, the model quantized at that
  width, one backward per batch, that width's perturbation;
* ``"widest"`` (scoring.py:318-365): the model at the widest width, one
  backward per batch, every width's perturbation against it.

Each block's gradients are reduced as its backward ends, by
``mr_delta_loss_mapped`` reading the fused gradient operand in place (every
width in one pass, terms in fp32, sums in fp64), so no model-sized gradient or
perturbation is ever held.
"""

from __future__ import annotations

import dataclasses
import time
from collections.abc import Callable, Sequence

import torch

from mround_amd import kernels as K
from mround_amd.core.quantizer import mode_of
from mround_amd.core.scale_search import search_scales
from mround_amd.pipeline.block import LAYERS, placements
from mround_amd.pipeline.causal_lm import CausalLM
from mround_amd.schemes import DEFAULT_EPS_FP32, QuantScheme, ScaleInit

__all__ = ["ScoringProgress", "SensitivityScores", "eligible_block_layers", "score_widths"]

GRADIENT_SCHEDULES = ("own_width", "widest")


@dataclasses.dataclass
class SensitivityScores:
    """What one scoring run measured (mround/pipeline/scoring.py:84-105):
    ``scores[path][width]`` DeltaLoss, ``shapes[path]`` (out, in), the layers
    no width can quantize with the reason, and the wall clock."""

    scores: dict[str, dict[int, float]]
    shapes: dict[str, tuple[int, int]]
    skipped: tuple[tuple[str, str], ...]
    seconds: float


@dataclasses.dataclass(frozen=True)
class ScoringProgress:
    """One reportable moment of a scoring pass (mround/pipeline/scoring.py:108-180):
    ``stage`` is ``"perturbations"`` (the widest schedule's grids),
    ``"width"`` (a quantized copy built) or ``"backward"`` (a batch done)."""

    stage: str
    index: int
    total: int
    seconds: float
    peak_memory_bytes: int
    stage_seconds: float = 0.0
    preparations_left: int = 0
    preparation_seconds: float = 0.0

    @property
    def projected_seconds(self) -> float:
        if self.index < 1:
            return 0.0
        return self.stage_seconds / self.index * self.total

    @property
    def remaining_seconds(self) -> float:
        left = max(0.0, self.projected_seconds - self.stage_seconds)
        return left + self.preparations_left * self.preparation_seconds

    def describe(self) -> str:
        peak = "" if not self.peak_memory_bytes else f", peak memory {self.peak_memory_bytes / 1e9:.2f} GB"
        if self.stage == "perturbations":
            return f"  scoring: perturbations for {self.total} widths ready in {self.seconds:.1f}s{peak}"
        if self.stage == "width":
            return (f"  scoring: quantized copy {self.index} of {self.total} ready "
                    f"at {self.seconds:.0f}s{peak}")
        return (f"  scoring: backward {self.index}/{self.total} at {self.seconds:.0f}s, "
                f"about {self.remaining_seconds:.0f}s remaining{peak}")


def eligible_block_layers(model, group_size: int):
    """The block layers a mixed run plans over (mround/pipeline/scoring.py:368-422):
    every block linear whose input width divides into whole groups.

    Returns ``(eligible, skipped, by_block)``: path -> weight, ``(path,
    reason)`` for the rest, and the eligible paths per block in model order.
    Raises ``ValueError`` when no layer of any block qualifies.
    """
    eligible: dict[str, torch.Tensor] = {}
    skipped: list[tuple[str, str]] = []
    by_block: list[list[str]] = []
    for blk in model.blocks:
        by_block.append([])
        for name in LAYERS:
            w = blk.weights.linears[name]
            path = f"{blk.name}.{name}"
            if group_size != -1 and w.shape[-1] % group_size:
                skipped.append((path, f"last dimension {w.shape[-1]} is not a multiple of {group_size}"))
                continue
            eligible[path] = w
            by_block[-1].append(path)
    if not eligible:
        raise ValueError("no layer in any block can be quantized at this group size")
    return eligible, skipped, by_block


def _grids(eligible, scheme: QuantScheme) -> dict[str, torch.Tensor]:
    """Each layer's searched scale grid at one width, without importance
    (mround/pipeline/scoring.py:196-211); empty unless the scheme searches."""
    if scheme.scale_init is not ScaleInit.SEARCHED:
        return {}
    out = {}
    for path, w in eligible.items():
        rows, cols = w.shape
        out[path] = search_scales(w, scheme).view(rows, cols // scheme.group_size)
    return out


def score_widths(model, batches: Sequence[torch.Tensor], widths: Sequence[int], base_scheme: QuantScheme,
                 *, eps: float = DEFAULT_EPS_FP32, gradient_source: str = "own_width",
                 progress: Callable[[ScoringProgress], None] | None = None,
                 keep_activations: bool | None = None) -> SensitivityScores:
    """Score every block layer at every candidate width
    (mround/pipeline/scoring.py:425-583).

    ``batches`` are ``[n, seq_len]`` token-id tensors (one ``seq_len``; the
    first batch's sequence count sizes the engine and a later batch may hold
    fewer). Raises ``ValueError`` for no widths, no batches, an unknown
    ``gradient_source`` or when every layer is skipped.
    """
    if not widths:
        raise ValueError("no candidate widths to score")
    if gradient_source not in GRADIENT_SCHEDULES:
        raise ValueError(f"gradient_source must be 'own_width' or 'widest', got {gradient_source!r}")
    if not batches:
        raise ValueError("no calibration batches to score on")
    started = time.perf_counter()
    eligible, skipped, by_block = eligible_block_layers(model, base_scheme.group_size)
    shapes = {p: (int(w.shape[0]), int(w.shape[1])) for p, w in eligible.items()}
    schemes = {int(b): dataclasses.replace(base_scheme, bits=int(b)) for b in widths}
    order = sorted(schemes)
    dev = next(iter(eligible.values())).device
    batch = max(int(t.shape[0]) for t in batches)
    seq_len = int(batches[0].shape[1])
    lm = CausalLM(model, batch=batch, seq_len=seq_len, device=dev, keep_activations=keep_activations)
    place = placements(lm.shape)
    names = {f"{blk.name}.{n}": n for blk in model.blocks for n in LAYERS}

    spent = {"backward": 0.0, "preparation": 0.0}
    prepared = 0
    last = started

    def report(stage: str, index: int, total: int, left: int = 0) -> None:
        nonlocal last, prepared
        if progress is None:
            return
        torch.cuda.synchronize(dev)
        now = time.perf_counter()
        kind = "backward" if stage == "backward" else "preparation"
        spent[kind] += now - last
        if kind == "preparation":
            prepared += 1
        last = now
        progress(ScoringProgress(stage=stage, index=index, total=total, seconds=now - started,
                                 peak_memory_bytes=int(torch.cuda.max_memory_allocated(dev)),
                                 stage_seconds=spent[kind], preparations_left=left,
                                 preparation_seconds=spent["preparation"] / prepared if prepared else 0.0))

    def accumulate(bits: list[int], grids: list[dict[str, torch.Tensor]], acc: dict[str, torch.Tensor]):
        mode = mode_of(schemes[bits[0]])
        searched = mode == "searched"

        def on_block(b: int, dw: dict[str, torch.Tensor]) -> None:
            for path in by_block[b]:
                p = place[names[path]]
                w = eligible[path]
                if w.dtype not in (torch.float32, torch.bfloat16):
                    w = w.float()
                K.delta_loss_mapped(w, dw[p.operand], group_size=base_scheme.group_size, bits_list=bits,
                                    mode=mode, eps=eps, scores_out=acc[path],
                                    grids=[g[path] for g in grids] if searched else None,
                                    row_block=p.row_block, row_stride=p.row_stride,
                                    row_offset=p.row_offset)
        return on_block

    scores: dict[str, dict[int, float]] = {p: {} for p in eligible}
    if gradient_source == "own_width":
        passes = len(batches) * len(order)
        done = 0
        for built, width in enumerate(order, start=1):
            grids = _grids(eligible, schemes[width])
            lm.set_weights({p: schemes[width] for p in eligible}, eps=eps, grids=grids)
            report("width", built, len(order))
            acc = {p: torch.zeros(1, dtype=torch.float64, device=dev) for p in eligible}
            on_block = accumulate([width], [grids], acc)
            for tokens in batches:
                lm.run(tokens, on_block)
                done += 1
                report("backward", done, passes, len(order) - built)
            for p in eligible:
                scores[p][width] = float(acc[p][0])
    else:
        widest = order[-1]
        all_grids = [_grids(eligible, schemes[b]) for b in order]
        lm.set_weights({p: schemes[widest] for p in eligible}, eps=eps, grids=all_grids[-1])
        report("perturbations", len(order), len(order))
        acc = {p: torch.zeros(len(order), dtype=torch.float64, device=dev) for p in eligible}
        on_block = accumulate(order, all_grids, acc)
        for i, tokens in enumerate(batches, start=1):
            lm.run(tokens, on_block)
            report("backward", i, len(batches))
        for p in eligible:
            vals = acc[p].cpu().tolist()
            scores[p] = {b: float(v) for b, v in zip(order, vals)}
    torch.cuda.synchronize(dev)
    return SensitivityScores(scores=scores, shapes=shapes, skipped=tuple(skipped),
                             seconds=time.perf_counter() - started)
