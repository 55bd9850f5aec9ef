"""Public entry point: quantize a model and write an MLX checkpoint.

The surface of ``mround.api.quantize`` (mround/api.py:366-794) for local
checkpoints on one MI355X: resolve the scheme, load the model onto the GPU,
embed the calibration tokens into the block-0 input stream, tune every block
(``QuantizationRunner``), round the tensors outside the blocks to nearest,
write the MLX checkpoint (packed codes, scales, biases, config, index) and
the run record. Mixed precision takes a ready ``plan`` (per-layer widths,
e.g. from ``mround_amd.planner.allocator.allocate_bits``); the whole-model
sensitivity pass that would produce one from ``average_bits`` is not part of
this build and is refused with that reason.
"""

from __future__ import annotations

import dataclasses
import json
import time
from collections.abc import Mapping, Sequence
from pathlib import Path
from typing import Any

import torch

from mround_amd.core.quantizer import quantize_codes
from mround_amd.core.scale_search import search_scales
from mround_amd.exceptions import ArchitectureError, CalibrationError, UnsupportedSchemeError
from mround_amd.formats.mlx_export import (QuantizedLayer, export_mlx, narrow_codes,
                                           require_mlx_representable)
from mround_amd.pipeline.checkpoint import DecoderModel, dense_tensors, load_model
from mround_amd.pipeline.runner import QuantizationRunner, RunSummary
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


def _resolve_scheme(*, bits, group_size, symmetry, plan, scheme, scale_init) -> tuple[QuantScheme, set[int]]:
    widths = {scheme.bits if scheme is not None else bits}
    if plan:
        widths.update(int(b) for b in plan.values())
    resolved = scheme or QuantScheme(
        bits=bits, group_size=group_size, symmetry=symmetry,
        scale_init=default_scale_init(min(widths), symmetry) if scale_init is None else ScaleInit(scale_init))
    return resolved, widths


def calibration_tokens(vocab: int, n_samples: int, seq_len: int, *, seed: int, device) -> torch.Tensor:
    """Token ids drawn uniformly from the vocabulary (the synthetic calibration of
    the benchmark configurations), ``[n_samples, seq_len]`` int64."""
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randint(0, vocab, (n_samples, seq_len), generator=g, device=device)


def _entrance(model: DecoderModel, tokens: torch.Tensor, batch_size: int) -> list[torch.Tensor]:
    """The block-0 input stream: embedding rows in float32, one
    ``[batch * seq_len, hidden]`` tensor per batch."""
    return [model.embed[tokens[i:i + batch_size].reshape(-1)].float()
            for i in range(0, tokens.shape[0], batch_size)]


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
        codes, scale, zp = quantize_codes(w, None, scheme, init_scale=init, narrow=True)
        out[path] = QuantizedLayer(narrow_codes(codes, scheme), scale, zp, scheme)
    return out, skipped


def _storage(model: DecoderModel, quantized: Mapping[str, QuantizedLayer]) -> Storage:
    dtype_bits = torch.finfo(model.dtype).bits
    total = params = 0
    for name, t in dense_tensors(model).items():
        path = name.removesuffix(".weight")
        n = t.numel()
        params += n
        if name.endswith(".weight") and path in quantized:
            layer = quantized[path]
            groups = layer.scale.numel()
            total += n * layer.scheme.bits + 2 * groups * dtype_bits
        else:
            total += n * dtype_bits
    return Storage(total, params, float(dtype_bits))


def quantize(model: str | Path, *, output_dir: str | Path, bits: int = 4, group_size: int = 64,
             symmetry: Symmetry = Symmetry.SYMMETRIC, average_bits: float | None = None,
             dense_remainder: bool = False, scheme: QuantScheme | None = None,
             tuning: TuningConfig | None = None, calibration: str | torch.Tensor = "random",
             export_format: str = "mlx", quantized_inputs: bool = True, holdout_batches: int = 0,
             per_layer_recipe: bool = False, plan: Mapping[str, int] | None = None,
             scale_init: ScaleInit | str | None = None, seed: int | None = None,
             device: str = "cuda", progress=None) -> QuantizeResult:
    """Quantize the local checkpoint ``model`` into ``output_dir``.

    ``calibration`` is ``"random"`` (token ids uniform over the vocabulary) or
    a ``[n_samples, seq_len]`` tensor of token ids; ``plan`` maps block layer
    paths to widths. Raises the reference's exceptions for unrepresentable
    schemes, bad calibration and unsupported architectures.
    """
    started = time.perf_counter()
    if export_format != "mlx":
        raise UnsupportedSchemeError(f"export format {export_format!r} is not supported; only 'mlx'")
    if average_bits is not None:
        raise UnsupportedSchemeError(
            "average_bits needs the whole-model sensitivity scoring pass, which this build does not "
            "include; pass plan= (layer path -> width, e.g. from planner.allocator.allocate_bits)")
    resolved, widths = _resolve_scheme(bits=bits, group_size=group_size, symmetry=symmetry, plan=plan,
                                       scheme=scheme, scale_init=scale_init)
    for w in sorted(widths):
        require_mlx_representable(resolved.with_bits(w))
    tuning = tuning or TuningConfig()
    seed = 0 if seed is None else int(seed)
    t0 = time.perf_counter()
    m = load_model(model, device=device)
    load_s = time.perf_counter() - t0

    vocab = int(m.config["vocab_size"])
    if isinstance(calibration, torch.Tensor):
        tokens = calibration.to(device=device, dtype=torch.int64)
        if tokens.dim() != 2:
            raise CalibrationError("calibration token ids must be [n_samples, seq_len]")
        if tokens.numel() and (int(tokens.min()) < 0 or int(tokens.max()) >= vocab):
            raise CalibrationError(f"calibration token ids must lie in [0, {vocab})")
    elif calibration == "random":
        tokens = calibration_tokens(vocab, tuning.n_samples, tuning.seq_len, seed=seed, device=device)
    else:
        raise CalibrationError(f"calibration {calibration!r} needs a text corpus, which is not "
                               "available offline; pass 'random' or a tensor of token ids")
    if tokens.shape[1] != tuning.seq_len:
        raise CalibrationError(f"calibration sequences have {tokens.shape[1]} tokens, tuning.seq_len "
                               f"is {tuning.seq_len}")
    if tokens.shape[0] % tuning.batch_size:
        raise CalibrationError(f"{tokens.shape[0]} calibration sequences do not split into batches of "
                               f"{tuning.batch_size}")

    schemes_by_layer = None
    if plan:
        schemes_by_layer = {p: resolved.with_bits(int(b)) for p, b in plan.items()}
    runner = QuantizationRunner(resolved, tuning, progress=progress, quantized_inputs=quantized_inputs,
                                holdout_batches=holdout_batches, per_layer_recipe=per_layer_recipe)
    entrance = _entrance(m, tokens, tuning.batch_size)
    summary, quantized = runner.run(m.blocks, entrance, scheme_by_layer=schemes_by_layer)
    del entrance
    t1 = time.perf_counter()
    remainder, skipped = _round_to_nearest(m, resolved, dense=dense_remainder)
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
    seconds = {"load": load_s, "blocks": summary.total_seconds, "remainder": t2 - t1, "export": t3 - t2,
               "total": t3 - started}
    record = {
        "model": str(model),
        "scheme": {"bits": resolved.bits, "group_size": resolved.group_size,
                   "symmetry": resolved.symmetry.value, "scale_init": resolved.scale_init.value},
        "tuning": dataclasses.asdict(tuning),
        "calibration": "random" if not isinstance(calibration, torch.Tensor) else "tokens",
        "seed": seed,
        "plan": dict(plan) if plan else None,
        "quantized_inputs": quantized_inputs,
        "holdout_batches": holdout_batches,
        "blocks": [{"index": b.index, "name": b.name, "initial_loss": b.initial_loss,
                    "final_loss": b.final_loss, "reverted": b.reverted, "seconds": b.seconds,
                    "search_seconds": b.search_seconds} for b in summary.blocks],
        "skipped": skipped,
        "storage": {"bits_per_weight": storage.bits_per_weight, "compression": storage.compression},
        "seconds": seconds,
    }
    config_path = out / RUN_RECORD
    config_path.write_text(json.dumps(record, indent=2) + "\n")
    return QuantizeResult(out, summary, dict(summary.scheme_by_layer), config_path, storage,
                          tuple(skipped), None, seconds)
