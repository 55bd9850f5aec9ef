"""Public entry points: quantize a model and write an MLX checkpoint, or plan
a mixed-precision allocation.

The surface of ``mround.api.quantize`` (mround/api.py:366-794) and
``plan_mixed_precision`` (api.py:943-1085) for local checkpoints on one
MI355X: resolve the scheme, load the model onto the GPU, embed the
calibration tokens into the block-0 input stream, tune every block
(``QuantizationRunner``), round the tensors outside the blocks to nearest,
write the MLX checkpoint (packed codes, scales, biases, config, index) and
the run record. With ``average_bits`` a mixed run first scores every block
layer at every candidate width with whole-model causal-LM gradients
(``mround_amd.pipeline.scoring``) and allocates widths exactly under the
budget the average implies (api.py:1471-1695), or checks and costs a given
``plan`` (api.py:1698-1802).
"""

from __future__ import annotations

import dataclasses
import json
import math
import time
import warnings
from collections.abc import Mapping, Sequence
from pathlib import Path
from typing import Any

import torch

from mround_amd.core.quantizer import quantize_codes, quantize_pack
from mround_amd.core.scale_search import search_scales
from mround_amd.exceptions import (ArchitectureError, CalibrationError, SchemeError,
                                   UnsupportedSchemeError)
from mround_amd.formats.mlx_export import (MLX_GROUP_SIZES, QuantizedLayer, export_mlx, narrow_codes,
                                           require_mlx_representable)
from mround_amd.pipeline.block import LAYERS, aligned_length
from mround_amd.pipeline.checkpoint import DecoderModel, block_shape, dense_tensors, load_model
from mround_amd.pipeline.runner import QuantizationRunner, RunSummary
from mround_amd import kernels as K
from mround_amd.planner import memory as M
from mround_amd.planner.allocator import allocate_bits
from mround_amd.planner.timing import predict_run_time
from mround_amd.planner.sensitivity import (SENSITIVITY_SAMPLES, SENSITIVITY_SEQ_LEN, gradient_source_for,
                                            mixed_budget_bits, score_layer_options, scoring_batch_size,
                                            storage_bits)
from mround_amd.schemes import (LOW_BIT_THRESHOLD, QuantScheme, ScaleInit, Symmetry,
                                TuningConfig)

RUN_RECORD = "mround_run.json"


@dataclasses.dataclass(frozen=True)
class Storage:
    """What the checkpoint costs: stored bits over weights (codes plus group
    metadata for quantized tensors, the model dtype for dense ones)."""

    total_bits: int
    parameters: int
    dense_bits_per_weight: float

    @property
    def bits_per_weight(self) -> float:
        return self.total_bits / self.parameters if self.parameters else 0.0

    @property
    def compression(self) -> float:
        return self.dense_bits_per_weight / self.bits_per_weight if self.bits_per_weight else 0.0


@dataclasses.dataclass(frozen=True)
class QuantizeResult:
    """What a run produced (mround/api.py:75-113)."""

    output_dir: Path
    summary: RunSummary
    scheme_by_layer: dict[str, QuantScheme]
    config_path: Path
    storage: Storage
    skipped: tuple[tuple[str, str], ...] = ()
    mixed: dict[str, Any] | None = None
    seconds: Mapping[str, float] = dataclasses.field(default_factory=dict)

    def describe(self) -> str:
        return (f"{len(self.scheme_by_layer)} modules tuned, {len(self.skipped)} left dense, "
                f"{self.storage.bits_per_weight:.2f} bits per weight overall "
                f"({self.storage.compression:.2f}x smaller)")


def default_scale_init(narrowest_width: int, symmetry: Symmetry) -> ScaleInit:
    """Searched below 4 bits on symmetric schemes, observed range otherwise
    (mround/api.py:116-153)."""
    if Symmetry(symmetry) is not Symmetry.SYMMETRIC:
        return ScaleInit.OBSERVED_RANGE
    return ScaleInit.SEARCHED if narrowest_width < LOW_BIT_THRESHOLD else ScaleInit.OBSERVED_RANGE


# Below this share of the block stack a run is refused rather than producing a
# checkpoint mostly at full precision (mround/api.py:156-165).
MIN_BLOCK_COVERAGE = 0.5
_DIMENSIONS_SHOWN = 3


@dataclasses.dataclass(frozen=True)
class Coverage:
    """How much of a block stack a group size reaches (mround/api.py:168-232):
    a layer is groupable only when its input dimension is a multiple of the
    group size; the rest are left at full precision."""

    total: int
    blocked: tuple[tuple[str, int], ...] = ()

    @property
    def representable(self) -> int:
        return self.total - len(self.blocked)

    @property
    def fraction(self) -> float:
        """Share of the block stack that will be quantized (1 when it has no linears)."""
        return 1.0 if self.total == 0 else self.representable / self.total

    def alternatives(self, supported) -> tuple[int, ...]:
        """Which of ``supported`` divide every input dimension that blocked."""
        dims = {d for _, d in self.blocked}
        return tuple(sorted(g for g in supported if all(d % g == 0 for d in dims)))

    def explain(self, group_size: int, supported) -> str:
        dims = sorted({d for _, d in self.blocked})
        shown = ", ".join(str(d) for d in dims[:_DIMENSIONS_SHOWN]) + (", ..." if len(dims) > _DIMENSIONS_SHOWN
                                                                        else "")
        works = self.alternatives(supported)
        remedy = (f"Group sizes that divide every one of them: {', '.join(str(g) for g in works)}."
                  if works else "No supported group size divides all of them.")
        return (f"group size {group_size} can only quantize {self.representable} of {self.total} layers in the "
                f"block stack ({self.fraction:.0%}); the rest would be left at full precision and the checkpoint "
                f"would be far larger than the width asked for. Input dimensions that do not divide: {shown}. "
                f"{remedy}")


def block_coverage(model: DecoderModel | str | Path, group_size: int) -> Coverage:
    """What ``group_size`` can reach in the block stack, from the layers' shapes
    alone (mround/api.py:257-288): a loaded model, or a checkpoint directory
    (only its ``config.json`` is read). Per-channel (-1) reaches everything."""
    if isinstance(model, DecoderModel):
        blocks = [(b.name, {n: tuple(w.shape) for n, w in b.weights.linears.items()}) for b in model.blocks]
    else:
        config = _read_config(model)
        shape = block_shape(config)
        blocks = [(f"model.layers.{i}", {n: shape.linear_shape(n) for n in LAYERS})
                  for i in range(int(config["num_hidden_layers"]))]
    total, blocked = 0, []
    for name, shapes in blocks:
        for layer in LAYERS:
            total += 1
            dim = int(shapes[layer][-1])
            if group_size > 0 and dim % group_size:
                blocked.append((f"{name}.{layer}", dim))
    return Coverage(total=total, blocked=tuple(blocked))


def _require_coverage(model: DecoderModel, scheme: QuantScheme, minimum: float) -> None:
    """Refuse a group size that would leave most of the block stack dense
    (mround/api.py:235-254), before anything is tuned."""
    coverage = block_coverage(model, scheme.group_size)
    if coverage.fraction < minimum:
        raise UnsupportedSchemeError(coverage.explain(scheme.group_size, MLX_GROUP_SIZES))


def _resolve_scheme(*, bits, group_size, symmetry, average_bits, candidate_bits, remainder_bits,
                    scheme, scale_init) -> tuple[QuantScheme, set[int]]:
    """The scheme a run resolves to and every width it can assign: the
    candidates and the remainder's too when mixed (mround/api.py:1253-1288)."""
    widths = {scheme.bits if scheme is not None else bits}
    if average_bits is not None:
        widths.update(int(b) for b in candidate_bits)
        if remainder_bits is not None:
            widths.add(int(remainder_bits))
    resolved = scheme or QuantScheme(
        bits=bits, group_size=group_size, symmetry=symmetry,
        scale_init=default_scale_init(min(widths), symmetry) if scale_init is None else ScaleInit(scale_init))
    return resolved, widths


def _refuse_unusable_plan(plan, average_bits, candidate_bits) -> None:
    """A given plan needs its average and widths on the menu (mround/api.py:311-346)."""
    if plan is None:
        return
    if average_bits is None:
        raise SchemeError("a given plan is a mixed run's allocation; pass average_bits too, which the "
                          "plan is reported against and which sets the remainder's width")
    if not plan:
        raise SchemeError("a given plan must assign a width to every block layer; this one is empty")
    menu = sorted({int(b) for b in candidate_bits})
    off = sorted({(path, int(b)) for path, b in plan.items() if int(b) not in menu})
    if off:
        shown = ", ".join(f"{path} at {b}" for path, b in off[:4])
        more = f" and {len(off) - 4} more" if len(off) > 4 else ""
        raise SchemeError(f"a given plan may assign only widths in candidate_bits={menu}; it has {shown}{more}")


def _remainder_width(average_bits: float, remainder_bits: int | None, base: QuantScheme) -> int:
    """Nearest supported width to the average, ties toward more bits, unless
    given (mround/api.py:1659-1667)."""
    if remainder_bits is None:
        return min(8, max(2, math.floor(average_bits + 0.5)))
    base.with_bits(int(remainder_bits))  # validates
    return int(remainder_bits)


def _dtype_bits(model: DecoderModel) -> int:
    return 16 if model.dtype in (torch.bfloat16, torch.float16) else 32


def _plan_info(shapes, by_layer, widths, base, average_bits, remainder, dtype_bits, cost, budget):
    elements = sum(o * i for o, i in shapes.values())
    metadata = sum(2 * o * base.groups_per_row(i) * dtype_bits for o, i in shapes.values())
    counts = {w: sum(1 for b in by_layer.values() if b == w) for w in widths}
    return {
        "average_bits": average_bits,
        "candidate_bits": list(widths),
        "achieved_code_bits": (cost - metadata) / elements,
        "layers_by_width": {str(w): c for w, c in counts.items()},
        "remainder_bits": remainder,
        "budget_bits": budget,
        "allocated_cost_bits": cost,
        "assignments": {p: int(b) for p, b in sorted(by_layer.items())},
    }


def _given_plan(model: DecoderModel, base: QuantScheme, average_bits: float, candidate_bits, plan,
                *, remainder_bits: int | None) -> tuple[dict[str, QuantScheme], dict[str, Any]]:
    """Check a given plan against the layers a scored one would cover and cost
    it (mround/api.py:1698-1802)."""
    from mround_amd.pipeline.scoring import eligible_block_layers

    widths = sorted({int(b) for b in candidate_bits})
    eligible, _, _ = eligible_block_layers(model, base.group_size)
    unknown = sorted(set(plan) - set(eligible))
    missing = sorted(set(eligible) - set(plan))
    if unknown or missing:
        parts = []
        if unknown:
            parts.append(f"{len(unknown)} the run does not plan over, the first {unknown[0]}")
        if missing:
            parts.append(f"{len(missing)} left out, the first {missing[0]}")
        raise SchemeError("a given plan must name exactly the block layers a scored plan would cover; "
                          "this one names " + " and ".join(parts))
    shapes = {p: (int(w.shape[0]), int(w.shape[1])) for p, w in eligible.items()}
    dtype_bits = _dtype_bits(model)
    by_layer = {p: int(plan[p]) for p in eligible}
    cost = sum(storage_bits(shapes[p], b, base.group_size, dtype_bits=dtype_bits) for p, b in by_layer.items())
    budget = mixed_budget_bits(shapes, average_bits, base.group_size, dtype_bits=dtype_bits)
    remainder = _remainder_width(average_bits, remainder_bits, base)
    info = _plan_info(shapes, by_layer, widths, base, average_bits, remainder, dtype_bits, cost, budget)
    over = "" if cost <= budget else f", {cost - budget} bits over the budget"
    summary = ", ".join(f"{c} layers at {w} bits" for w, c in info["layers_by_width"].items())
    info.update(source="given", describe=f"given plan: {summary}; {info['achieved_code_bits']:.3f} code bits "
                f"per weight against a target of {average_bits:g}{over}, remainder at {remainder} bits")
    return {p: base.with_bits(b) for p, b in by_layer.items()}, info


def _scoring_tokens(calibration, vocab: int, samples: int, sequence: int, *, seed: int, device):
    if isinstance(calibration, torch.Tensor):
        t = calibration.to(device=device, dtype=torch.int64)
        if t.dim() != 2 or t.shape[0] < samples or t.shape[1] < sequence:
            raise CalibrationError(f"scoring draws {samples} sequences of {sequence} tokens from the "
                                   f"calibration ids, which are {tuple(t.shape)}; pass scoring_samples "
                                   "and scoring_seq_len that fit")
        return t[:samples, :sequence]
    return calibration_tokens(vocab, samples, sequence, seed=seed, device=device)


def _plan_mixed(model: DecoderModel, base: QuantScheme, average_bits: float, candidate_bits, calibration,
                *, gradient_source: str = "auto", remainder_bits: int | None = None,
                scoring_samples: int | None = None, scoring_seq_len: int | None = None,
                scoring_batch: int | None = None, seed: int = 0, device="cuda",
                progress=None) -> tuple[dict[str, QuantScheme], dict[str, Any]]:
    """Score, allocate, and return per-layer schemes plus what was decided
    (mround/api.py:1471-1695)."""
    from mround_amd.pipeline.scoring import eligible_block_layers, score_widths

    widths = sorted({int(b) for b in candidate_bits})
    if not widths:
        raise SchemeError("mixed precision needs at least one candidate width")
    for w in widths:
        base.with_bits(w)
    if not widths[0] <= average_bits <= widths[-1]:
        raise SchemeError(f"average_bits={average_bits} is outside the achievable range "
                          f"[{widths[0]}, {widths[-1]}] for candidate_bits={widths}")
    if scoring_batch is not None and int(scoring_batch) < 1:
        raise SchemeError(f"scoring_batch_size must be at least 1, or None; got {scoring_batch}")
    eligible, _, _ = eligible_block_layers(model, base.group_size)
    scored_weights = sum(int(w.numel()) for w in eligible.values())
    requested = gradient_source
    gradient_source = gradient_source_for(requested, scored_weights)
    samples = SENSITIVITY_SAMPLES if scoring_samples is None else int(scoring_samples)
    sequence = SENSITIVITY_SEQ_LEN if scoring_seq_len is None else int(scoring_seq_len)
    batch = (scoring_batch_size(samples, sequence) if scoring_batch is None
             else max(1, min(samples, int(scoring_batch))))
    tokens = _scoring_tokens(calibration, int(model.config["vocab_size"]), samples, sequence, seed=seed,
                             device=device)
    batches = [tokens[i:i + batch] for i in range(0, samples, batch)]
    scored = score_widths(model, batches, widths, base, gradient_source=gradient_source, progress=progress)
    dtype_bits = _dtype_bits(model)
    options = score_layer_options(scored.scores, scored.shapes, base, dtype_bits=dtype_bits)
    budget = mixed_budget_bits(scored.shapes, average_bits, base.group_size, dtype_bits=dtype_bits)
    allocation = allocate_bits(options, budget_bits=budget)
    remainder = _remainder_width(average_bits, remainder_bits, base)
    info = _plan_info(scored.shapes, allocation.by_layer, widths, base, average_bits, remainder, dtype_bits,
                      allocation.total_cost_bits, budget)
    summary = ", ".join(f"{c} layers at {w} bits" for w, c in info["layers_by_width"].items())
    info.update(
        source="scored", predicted_loss=allocation.predicted_loss, scoring_seconds=round(scored.seconds, 1),
        scoring_samples=samples, scoring_seq_len=sequence, scoring_batch_size=batch,
        gradient_source=gradient_source, gradient_source_requested=requested,
        scored_weights=scored_weights,
        describe=(f"planned {summary}; {info['achieved_code_bits']:.3f} code bits per weight against a "
                  f"target of {average_bits:g}, remainder at {remainder} bits, scored {samples}x{sequence} "
                  f"in {scored.seconds:.1f}s with gradients at "
                  f"{'the widest width' if gradient_source == 'widest' else 'each own width'}"
                  + (f", by size at {scored_weights / 1e9:.2f} billion weights" if requested == "auto" else "")))
    return {p: base.with_bits(b) for p, b in allocation.by_layer.items()}, info


def calibration_tokens(vocab: int, n_samples: int, seq_len: int, *, seed: int, device) -> torch.Tensor:
    """Token ids drawn uniformly from the vocabulary (the synthetic calibration of
    the benchmark configurations), ``[n_samples, seq_len]`` int64."""
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randint(0, vocab, (n_samples, seq_len), generator=g, device=device)


def _entrance(model: DecoderModel, tokens: torch.Tensor, batch_size: int) -> list[torch.Tensor]:
    """The block-0 input stream: embedding rows in float32 (``mr_embed_rows``),
    one ``[batch * rows, hidden]`` tensor per batch, ``rows`` being the
    sequence length rounded up to a multiple of 128 and each sequence's rows
    past its tokens zero (padding the block engine keeps out of the loss)."""
    n_seq, length = tokens.shape
    rows = aligned_length(length)
    out = []
    for i in range(0, n_seq, batch_size):
        ids = tokens[i:i + batch_size]
        if rows != length:
            ids = torch.nn.functional.pad(ids, (0, rows - length))  # token 0 at the padding rows
        ids = ids.reshape(-1).to(torch.int32)
        x = torch.empty(ids.numel(), model.embed.shape[1], dtype=torch.float32, device=model.embed.device)
        K.embed_rows(model.embed, ids, x)
        if rows != length:
            x.view(-1, rows, x.shape[1])[:, length:].zero_()
        out.append(x)
    return out


def _round_to_nearest(model: DecoderModel, scheme: QuantScheme, *, dense: bool):
    """Embedding and untied head at round to nearest (mround/api.py:1877-1937)."""
    out, skipped = {}, []
    targets = [("model.embed_tokens", model.embed)]
    if model.lm_head is not None:
        targets.append(("lm_head", model.lm_head))
    for path, w in targets:
        if scheme.group_size != -1 and w.shape[-1] % scheme.group_size:
            skipped.append((path, f"last dimension {w.shape[-1]} is not a multiple of {scheme.group_size}"))
            continue
        if dense:
            skipped.append((path, "dense by request, to match a reference's coverage"))
            continue
        init = search_scales(w, scheme) if scheme.scale_init is ScaleInit.SEARCHED else None
        out[path] = _rtn_layer(w, scheme, init, model.dtype)
    return out, skipped


def _rtn_layer(w: torch.Tensor, scheme: QuantScheme, init_scale, dtype: torch.dtype) -> QuantizedLayer:
    """A layer at round to nearest, straight into MLX's words, scales and biases
    in the checkpoint dtype (``mr_quantize_pack``) where the group size allows;
    otherwise as codes, packed at export."""
    rows, cols = w.shape
    gs = scheme.group_size
    if gs >= 32 and gs & (gs - 1) == 0 and cols % gs == 0 and w.dtype in (torch.bfloat16, torch.float32):
        return QuantizedLayer(None, None, None, scheme, packed=quantize_pack(w, None, scheme, init_scale=init_scale,
                                                                             dtype=dtype))
    codes, scale, zp = quantize_codes(w, None, scheme, init_scale=init_scale, narrow=True)
    return QuantizedLayer(narrow_codes(codes, scheme), scale, zp, scheme)


def _storage(model: DecoderModel, quantized: Mapping[str, QuantizedLayer]) -> Storage:
    dtype_bits = torch.finfo(model.dtype).bits
    total = params = 0
    for name, t in dense_tensors(model).items():
        path = name.removesuffix(".weight")
        n = t.numel()
        params += n
        if name.endswith(".weight") and path in quantized:
            layer = quantized[path]
            groups = layer.groups
            total += n * layer.scheme.bits + 2 * groups * dtype_bits
        else:
            total += n * dtype_bits
    return Storage(total, params, float(dtype_bits))


def _read_config(model: str | Path) -> dict[str, Any]:
    path = Path(model)
    if not (path / "config.json").is_file():
        raise ArchitectureError(f"{path} is not a local checkpoint directory (no config.json); "
                                "hub downloads are not available")
    return json.loads((path / "config.json").read_text())


def _run_shape(config, resolved: QuantScheme, tuning: TuningConfig, *, average_bits, plan, widths,
               gradient_source, scoring_samples, scoring_seq_len, scoring_batch, dense_remainder,
               quantized_inputs, holdout_batches=0, split_precision=False) -> tuple[M.ModelShape, M.RunShape]:
    shape = M.ModelShape.from_config(config)
    mixed = average_bits is not None and plan is None
    samples = SENSITIVITY_SAMPLES if scoring_samples is None else int(scoring_samples)
    sequence = SENSITIVITY_SEQ_LEN if scoring_seq_len is None else int(scoring_seq_len)
    batch = (scoring_batch_size(samples, sequence) if scoring_batch is None
             else max(1, min(samples, int(scoring_batch))))
    source = gradient_source_for(gradient_source, shape.layers * shape.block_weights) if mixed else "own_width"
    run = M.RunShape(n_samples=tuning.n_samples, seq_len=tuning.seq_len, batch_size=tuning.batch_size,
                     group_size=resolved.group_size, searched=resolved.scale_init is ScaleInit.SEARCHED,
                     quantized_inputs=quantized_inputs, mixed=mixed, widths=len(widths),
                     gradient_source=source, scoring_samples=samples, scoring_seq_len=sequence,
                     scoring_batch=batch, dense_remainder=dense_remainder, holdout_batches=holdout_batches,
                     micro_batches=tuning.micro_batches, half=str(config.get("torch_dtype")) == "float16",
                     split=bool(split_precision))
    return shape, run


# Code widths whose block objective one bf16 product cannot resolve: the
# bf16 rounding of the block's activations is as large as the quantization
# error itself (the objective reads about a third high against float64), so
# split precision is on for them unless the caller says otherwise.
SPLIT_PRECISION_WIDTHS = frozenset({8})


def _split_choice(split_precision: bool | None, tuned_widths) -> tuple[bool, str]:
    """Whether the block forward runs in split precision, and why: the
    caller's choice, else on when a tuned width is one of
    ``SPLIT_PRECISION_WIDTHS``. A caller turning it off for such a width is
    warned that the objective will be imprecise."""
    wide = sorted(set(int(w) for w in tuned_widths) & SPLIT_PRECISION_WIDTHS)
    if split_precision is None:
        if wide:
            return True, f"automatic: tuned width {wide[0]} needs the split-precision objective"
        return False, "automatic: no tuned width needs the split-precision objective"
    if not split_precision and wide:
        warnings.warn(f"split_precision=False with {wide[0]}-bit codes: the block objective runs on single "
                      "bf16 products, whose rounding is as large as the quantization error at this width "
                      "(the loss reads about a third high against float64)", stacklevel=3)
    return bool(split_precision), "requested"


def _tuned_widths(resolved: QuantScheme, average_bits, candidate_bits, plan) -> tuple[int, ...]:
    """The code widths the block tunes may run at: the scheme's, the plan's,
    or (a mixed run still to be planned) every candidate."""
    if average_bits is None:
        return (resolved.bits,)
    if plan is not None:
        return tuple(sorted(set(int(v) for v in plan.values())))
    return tuple(candidate_bits)


def predict_memory(model: str | Path, *, bits: int = 4, group_size: int = 64,
                   symmetry: Symmetry = Symmetry.SYMMETRIC, average_bits: float | None = None,
                   candidate_bits: Sequence[int] = (2, 3, 4), sensitivity_gradients: str = "auto",
                   remainder_bits: int | None = None, dense_remainder: bool = False,
                   scoring_samples: int | None = None, scoring_seq_len: int | None = None,
                   scoring_batch_size: int | None = None, scheme: QuantScheme | None = None,
                   tuning: TuningConfig | None = None, scale_init: ScaleInit | str | None = None,
                   quantized_inputs: bool = True, holdout_batches: int = 0,
                   memory_budget: int | None = None, device: str = "cuda",
                   split_precision: bool | None = None) -> M.MemoryCheck:
    """Predict the device memory of the run :func:`quantize` would make, and
    stop (mround/api.py:1088-1192). Reads ``config.json`` and nothing else.
    ``memory_budget`` defaults to 90 % of the device's memory;
    ``split_precision`` follows :func:`quantize`'s rule."""
    config = _read_config(model)
    resolved, widths = _resolve_scheme(bits=bits, group_size=group_size, symmetry=symmetry,
                                       average_bits=average_bits, candidate_bits=candidate_bits,
                                       remainder_bits=remainder_bits, scheme=scheme, scale_init=scale_init)
    if split_precision is None:
        split_precision = _split_choice(None, _tuned_widths(resolved, average_bits, candidate_bits, None))[0]
    tuning = tuning or TuningConfig()
    _check_calibration_sizes(tuning)
    shape, run = _run_shape(config, resolved, tuning, average_bits=average_bits, plan=None,
                            widths=candidate_bits if average_bits is not None else (resolved.bits,),
                            gradient_source=sensitivity_gradients, scoring_samples=scoring_samples,
                            scoring_seq_len=scoring_seq_len, scoring_batch=scoring_batch_size,
                            dense_remainder=dense_remainder, quantized_inputs=quantized_inputs,
                            holdout_batches=holdout_batches, split_precision=split_precision)
    budget = M.default_budget(device) if memory_budget is None else memory_budget
    return M.check_memory(shape, run, budget=budget)


def predict_time(model: str | Path, *, bits: int = 4, group_size: int = 64,
                 symmetry: Symmetry = Symmetry.SYMMETRIC, average_bits: float | None = None,
                 candidate_bits: Sequence[int] = (2, 3, 4), sensitivity_gradients: str = "auto",
                 remainder_bits: int | None = None, scoring_samples: int | None = None,
                 scoring_seq_len: int | None = None, scheme: QuantScheme | None = None,
                 tuning: TuningConfig | None = None, scale_init: ScaleInit | str | None = None,
                 per_layer_recipe: bool = False, holdout_batches: int = 0,
                 split_precision: bool | None = None):
    """Predict the seconds the run :func:`quantize` would make takes on one
    MI355X (``mround_amd.planner.timing``), from ``config.json`` alone
    (mround/cli/main.py:590-624); ``split_precision`` follows
    :func:`quantize`'s rule."""
    config = _read_config(model)
    resolved, widths = _resolve_scheme(bits=bits, group_size=group_size, symmetry=symmetry,
                                       average_bits=average_bits, candidate_bits=candidate_bits,
                                       remainder_bits=remainder_bits, scheme=scheme, scale_init=scale_init)
    if split_precision is None:
        split_precision = _split_choice(None, _tuned_widths(resolved, average_bits, candidate_bits, None))[0]
    tuning = tuning or TuningConfig()
    _check_calibration_sizes(tuning)
    shape, run = _run_shape(config, resolved, tuning, average_bits=average_bits, plan=None,
                            widths=candidate_bits if average_bits is not None else (resolved.bits,),
                            gradient_source=sensitivity_gradients, scoring_samples=scoring_samples,
                            scoring_seq_len=scoring_seq_len, scoring_batch=None, dense_remainder=False,
                            quantized_inputs=True, holdout_batches=holdout_batches,
                            split_precision=split_precision)
    return predict_run_time(shape, run, tuning, resolved.bits,
                            candidate_bits=candidate_bits if average_bits is not None else (),
                            per_layer_recipe=per_layer_recipe, scoring_samples=scoring_samples,
                            scoring_seq_len=scoring_seq_len, gradient_source=sensitivity_gradients)


def _check_calibration_sizes(tuning: TuningConfig) -> None:
    """mround/pipeline/calibration.py:442-447, before anything is predicted or loaded."""
    if tuning.n_samples < 1 or tuning.seq_len < 1 or tuning.batch_size < 1:
        raise CalibrationError(f"n_samples, seq_len, and batch_size must all be positive; got "
                               f"{tuning.n_samples}, {tuning.seq_len}, {tuning.batch_size}")


def _load_tokens(m: DecoderModel, calibration, tuning: TuningConfig, seed: int, device) -> torch.Tensor:
    vocab = int(m.config["vocab_size"])
    if isinstance(calibration, torch.Tensor):
        tokens = calibration.to(device=device, dtype=torch.int64)
        if tokens.dim() != 2:
            raise CalibrationError("calibration token ids must be [n_samples, seq_len]")
        if tokens.numel() and (int(tokens.min()) < 0 or int(tokens.max()) >= vocab):
            raise CalibrationError(f"calibration token ids must lie in [0, {vocab})")
    elif calibration in ("random", "auto"):
        tokens = calibration_tokens(vocab, tuning.n_samples, tuning.seq_len, seed=seed, device=device)
    else:
        raise CalibrationError(f"calibration {calibration!r} needs a text corpus, which is not "
                               "available offline; pass 'random' or a tensor of token ids")
    return tokens


def quantize(model: str | Path, *, output_dir: str | Path, bits: int = 4, group_size: int = 64,
             symmetry: Symmetry = Symmetry.SYMMETRIC, average_bits: float | None = None,
             candidate_bits: Sequence[int] = (2, 3, 4), sensitivity_gradients: str = "auto",
             remainder_bits: int | None = None, dense_remainder: bool = False,
             scoring_samples: int | None = None, scoring_seq_len: int | None = None,
             scoring_batch_size: int | None = None, scheme: QuantScheme | None = None,
             tuning: TuningConfig | None = None, calibration: str | torch.Tensor = "random",
             export_format: str = "mlx", quantized_inputs: bool = True, holdout_batches: int = 0,
             per_layer_recipe: bool = False, plan: Mapping[str, int] | None = None,
             scale_init: ScaleInit | str | None = None, seed: int | None = None,
             memory_budget: int | None = None, memory_check: bool = True,
             min_block_coverage: float = MIN_BLOCK_COVERAGE, split_precision: bool | None = None,
             device: str = "cuda", progress=None, scoring_progress=None) -> QuantizeResult:
    """Quantize the local checkpoint ``model`` into ``output_dir``.

    ``calibration`` is ``"random"`` (``"auto"`` is the same here: token ids
    uniform over the vocabulary, since no text corpus is available offline)
    or a ``[n_samples, seq_len]`` tensor of token ids. ``average_bits``
    engages the planner: a whole-model scoring pass over ``candidate_bits``
    and an exact allocation (or, with ``plan``, the given per-layer widths),
    the block layers tuned at their assigned widths and the remainder at
    ``remainder_bits`` (default: the width nearest the average, ties up).
    The run's device memory is predicted from ``config.json`` before anything
    is loaded (``predict_memory``) and a run past ``memory_budget`` (default
    90 % of the device's memory) is refused with ``MemoryBudgetError`` unless
    ``memory_check`` is off. A group size that reaches less than
    ``min_block_coverage`` of the block stack's linears is refused with
    ``UnsupportedSchemeError`` (``block_coverage``); the layers it cannot
    reach are left dense and reported in ``skipped``. ``split_precision``
    runs the block forward as three bf16 products of hi and lo halves per
    product, the attention's included (the reference's documented remedy for
    the block objective's precision, mround DOCUMENTATION.md:885-925): about
    16 significant bits in place of 8 for about 1.9x the block tune time.
    ``None`` (the default) turns it on when a tuned width is 8 bits, whose
    quantization error single bf16 products cannot resolve, in uniform and
    mixed runs alike (a mixed run still to be planned counts it on for the
    memory and time predictions when 8 is a candidate, and runs it when the
    plan tunes a layer at 8); ``False`` with 8-bit codes warns. The choice
    and its reason are recorded in the run record. Raises the reference's
    exceptions for unrepresentable schemes, bad calibration, unusable plans
    and unsupported architectures.
    """
    started = time.perf_counter()
    if export_format != "mlx":
        raise UnsupportedSchemeError(f"export format {export_format!r} is not supported; only 'mlx'")
    if holdout_batches < 0:
        raise CalibrationError(f"holdout_batches must be zero or more, got {holdout_batches}")
    _refuse_unusable_plan(plan, average_bits, candidate_bits)
    resolved, widths = _resolve_scheme(bits=bits, group_size=group_size, symmetry=symmetry,
                                       average_bits=average_bits, candidate_bits=candidate_bits,
                                       remainder_bits=remainder_bits, scheme=scheme, scale_init=scale_init)
    for w in sorted(widths):
        require_mlx_representable(resolved.with_bits(w))
    tuning = tuning or TuningConfig()
    _check_calibration_sizes(tuning)
    seed = 0 if seed is None else int(seed)
    requested_split = split_precision
    split_precision, split_reason = _split_choice(
        split_precision, _tuned_widths(resolved, average_bits, candidate_bits, plan))
    mshape, rshape = _run_shape(_read_config(model), resolved, tuning, average_bits=average_bits, plan=plan,
                                widths=candidate_bits if average_bits is not None else (resolved.bits,),
                                gradient_source=sensitivity_gradients, scoring_samples=scoring_samples,
                                scoring_seq_len=scoring_seq_len, scoring_batch=scoring_batch_size,
                                dense_remainder=dense_remainder, quantized_inputs=quantized_inputs,
                                holdout_batches=holdout_batches, split_precision=split_precision)
    budget = M.default_budget(device) if memory_budget is None else memory_budget
    memory = M.check_memory(mshape, rshape, budget=budget)
    if memory_check:
        M.require_fits(memory)
    # and how long it will take on one MI355X: said, never enforced (mround/api.py:624-633)
    timing = predict_run_time(mshape, rshape, tuning, resolved.bits,
                              candidate_bits=candidate_bits if average_bits is not None and plan is None else (),
                              per_layer_recipe=per_layer_recipe, scoring_samples=scoring_samples,
                              scoring_seq_len=scoring_seq_len, gradient_source=sensitivity_gradients)
    print(f"  {timing.describe()}", flush=True)
    on_gpu = torch.cuda.is_available() and str(device).startswith("cuda")
    held_before = 0
    if on_gpu:  # the run's own peak: what the process already holds is left out
        torch.cuda.reset_peak_memory_stats(device)
        held_before = torch.cuda.memory_allocated(device)
    t0 = time.perf_counter()
    m = load_model(model, device=device)
    load_s = time.perf_counter() - t0
    _require_coverage(m, resolved, min_block_coverage)
    tokens = _load_tokens(m, calibration, tuning, seed, device)
    if tokens.shape[1] != tuning.seq_len:
        raise CalibrationError(f"calibration sequences have {tokens.shape[1]} tokens, tuning.seq_len "
                               f"is {tuning.seq_len}")
    if tokens.shape[0] % tuning.batch_size:
        raise CalibrationError(f"{tokens.shape[0]} calibration sequences do not split into batches of "
                               f"{tuning.batch_size}")

    schemes_by_layer = None
    mixed = None
    remainder_scheme = resolved
    plan_s = 0.0
    if average_bits is not None:
        tp = time.perf_counter()
        if plan is not None:
            schemes_by_layer, mixed = _given_plan(m, resolved, average_bits, candidate_bits, plan,
                                                  remainder_bits=remainder_bits)
        else:
            schemes_by_layer, mixed = _plan_mixed(
                m, resolved, average_bits, candidate_bits, calibration,
                gradient_source=sensitivity_gradients, remainder_bits=remainder_bits,
                scoring_samples=scoring_samples, scoring_seq_len=scoring_seq_len,
                scoring_batch=scoring_batch_size, seed=seed, device=device, progress=scoring_progress)
        remainder_scheme = resolved.with_bits(int(mixed["remainder_bits"]))
        plan_s = time.perf_counter() - tp
        if requested_split is None:  # the plan decides which widths are tuned
            split_precision, split_reason = _split_choice(
                None, {sch.bits for sch in schemes_by_layer.values()} or {resolved.bits})
    runner = QuantizationRunner(resolved, tuning, progress=progress, quantized_inputs=quantized_inputs,
                                holdout_batches=holdout_batches, per_layer_recipe=per_layer_recipe,
                                split_precision=split_precision)
    entrance = _entrance(m, tokens, tuning.batch_size)
    summary, quantized = runner.run(m.blocks, entrance, scheme_by_layer=schemes_by_layer)
    del entrance
    t1 = time.perf_counter()
    remainder, skipped = _round_to_nearest(m, remainder_scheme, dense=dense_remainder)
    skipped = [(f"{b.name}.{n}", why) for b in summary.blocks for n, why in b.skipped] + skipped
    quantized.update(remainder)
    if not quantized:
        raise ArchitectureError(f"nothing in {model!r} could be quantized at group_size={group_size}")
    t2 = time.perf_counter()
    dense = {k: v for k, v in dense_tensors(m).items() if k.removesuffix(".weight") not in quantized
             or not k.endswith(".weight")}
    dtype_name = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}[m.dtype]
    out = Path(output_dir)
    export_mlx(out, dense_weights=dense, quantized=quantized, config=m.config, dtype=dtype_name)
    t3 = time.perf_counter()
    storage = _storage(m, quantized)
    seconds = {"load": load_s, "plan": plan_s, "blocks": summary.total_seconds, "remainder": t2 - t1,
               "export": t3 - t2, "total": t3 - started}
    record = {
        "model": str(model),
        "scheme": {"bits": resolved.bits, "group_size": resolved.group_size,
                   "symmetry": resolved.symmetry.value, "scale_init": resolved.scale_init.value},
        "tuning": dataclasses.asdict(tuning),
        "calibration": "random" if not isinstance(calibration, torch.Tensor) else "tokens",
        "seed": seed,
        "mixed": mixed,
        "quantized_inputs": quantized_inputs,
        "holdout_batches": holdout_batches,
        "split_precision": bool(split_precision),
        "split_precision_reason": split_reason,
        "blocks": [{"index": b.index, "name": b.name, "initial_loss": b.initial_loss,
                    "final_loss": b.final_loss, "reverted": b.reverted, "seconds": b.seconds,
                    "search_seconds": b.search_seconds} for b in summary.blocks],
        "skipped": skipped,
        "storage": {"bits_per_weight": storage.bits_per_weight, "compression": storage.compression},
        "seconds": seconds,
        "time_check": timing.record(),
        "memory": {**memory.record(),
                   "peak_allocated": int(torch.cuda.max_memory_allocated(device)) - held_before
                   if on_gpu else None},
    }
    config_path = out / RUN_RECORD
    config_path.write_text(json.dumps(record, indent=2) + "\n")
    return QuantizeResult(out, summary, dict(summary.scheme_by_layer), config_path, storage,
                          tuple(skipped), mixed, seconds)


@dataclasses.dataclass(frozen=True)
class RoundToNearestResult:
    """What a round-to-nearest run produced (mround/api.py:798-838)."""

    output_dir: Path
    scheme: QuantScheme
    quantized: tuple[str, ...]
    skipped: tuple[tuple[str, str], ...]
    bits_per_weight: float
    stored_bytes: int
    original_bytes: int

    @property
    def compression(self) -> float:
        return self.original_bytes / max(1, self.stored_bytes)

    def describe(self) -> str:
        return (f"{len(self.quantized)} modules at {self.scheme.bits} bits, {len(self.skipped)} left dense, "
                f"{self.bits_per_weight:.2f} bits per weight overall ({self.compression:.2f}x smaller)")


def quantize_round_to_nearest(model: str | Path, *, output_dir: str | Path, bits: int = 4, group_size: int = 64,
                              symmetry: Symmetry = Symmetry.SYMMETRIC, dense_remainder: bool = False,
                              device: str = "cuda") -> RoundToNearestResult:
    """Quantize every linear at round to nearest with the observed-range scale,
    nothing learned and no calibration, and write the MLX checkpoint: the
    baseline learned rounding has to beat (mround/api.py:841-940). With
    ``dense_remainder`` only the block linears are rounded."""
    scheme = QuantScheme(bits=bits, group_size=group_size, symmetry=symmetry)
    require_mlx_representable(scheme)
    m = load_model(model, device=device)
    quantized: dict[str, QuantizedLayer] = {}
    skipped: list[tuple[str, str]] = []
    for blk in m.blocks:
        for name, w in sorted(blk.weights.linears.items()):
            path = f"{blk.name}.{name}"
            if group_size != -1 and w.shape[-1] % group_size:
                skipped.append((path, f"last dimension {w.shape[-1]} is not a multiple of {group_size}"))
                continue
            quantized[path] = _rtn_layer(w, scheme, None, m.dtype)
    remainder, rem_skipped = _round_to_nearest(m, scheme, dense=dense_remainder)
    quantized.update(remainder)
    skipped.extend(rem_skipped)
    if not quantized:
        raise ArchitectureError(f"nothing in {model!r} could be quantized at group_size={group_size}")
    dense = {k: v for k, v in dense_tensors(m).items() if k.removesuffix(".weight") not in quantized
             or not k.endswith(".weight")}
    dtype_name = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}[m.dtype]
    out = Path(output_dir)
    export_mlx(out, dense_weights=dense, quantized=quantized, config=m.config, dtype=dtype_name)
    storage = _storage(m, quantized)
    original = int(storage.parameters * storage.dense_bits_per_weight) // 8
    return RoundToNearestResult(out, scheme, tuple(sorted(quantized)), tuple(skipped), storage.bits_per_weight,
                                storage.total_bits // 8, original)


def plan_mixed_precision(model: str | Path, average_bits: float, candidate_bits: Sequence[int] = (2, 3, 4),
                         *, bits: int = 4, group_size: int = 64, symmetry: Symmetry = Symmetry.SYMMETRIC,
                         scale_init: ScaleInit | str | None = None, scheme: QuantScheme | None = None,
                         calibration: str | torch.Tensor = "random", sensitivity_gradients: str = "auto",
                         remainder_bits: int | None = None, scoring_samples: int | None = None,
                         scoring_seq_len: int | None = None, scoring_batch_size: int | None = None,
                         seed: int | None = None, device: str = "cuda", progress=None) -> dict[str, Any]:
    """Score and allocate, and stop there: nothing is tuned or written
    (mround/api.py:943-1085). Returns the plan summary, whose
    ``assignments`` map each block layer path to its width."""
    resolved, widths = _resolve_scheme(bits=bits, group_size=group_size, symmetry=symmetry,
                                       average_bits=average_bits, candidate_bits=candidate_bits,
                                       remainder_bits=remainder_bits, scheme=scheme, scale_init=scale_init)
    for w in sorted(widths):
        require_mlx_representable(resolved.with_bits(w))
    if isinstance(calibration, str) and calibration not in ("random", "auto"):
        raise CalibrationError(f"calibration {calibration!r} needs a text corpus, which is not "
                               "available offline; pass 'random' or a tensor of token ids")
    m = load_model(model, device=device)
    _, info = _plan_mixed(m, resolved, average_bits, candidate_bits, calibration,
                          gradient_source=sensitivity_gradients, remainder_bits=remainder_bits,
                          scoring_samples=scoring_samples, scoring_seq_len=scoring_seq_len,
                          scoring_batch=scoring_batch_size, seed=0 if seed is None else int(seed),
                          device=device, progress=progress)
    return info
