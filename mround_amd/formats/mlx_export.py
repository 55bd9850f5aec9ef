"""MLX-native checkpoint export (``mround/formats/mlx_export.py:57-425``).

Same tensor names, shapes, dtypes, ``config.json`` quantization block, shard
rule and index as the reference's ``export_mlx``. Codes are packed and the
affine metadata formed on the GPU (``mr_pack_codes``, ``mr_to_affine``); the
files are written with ``safetensors`` (``metadata={"format": "mlx"}``).

MLX reconstructs ``W = scales * q_u + biases`` with ``q_u`` the stored
unsigned code; the bias is formed from the *stored* (rounded) scale, so
symmetric zero stays exactly representable.

Portions follow MRound (Copyright 2026 The MRound Authors, Apache License 2.0);
see NOTICE.
"""

from __future__ import annotations

import dataclasses
import json
import re
from collections.abc import Mapping
from pathlib import Path
from typing import Any

import torch

from mround_amd import kernels as K
from mround_amd.exceptions import ExportError, UnsupportedSchemeError
from mround_amd.formats.packing import pack_codes, packed_width
from mround_amd.schemes import QuantScheme, Symmetry

__all__ = [
    "MLX_GROUP_SIZES",
    "MLX_SUPPORTED_BITS",
    "SHARD_BYTES",
    "QuantizedLayer",
    "export_mlx",
    "narrow_codes",
    "require_mlx_representable",
    "shard_names",
    "to_affine",
]

MLX_SUPPORTED_BITS: frozenset[int] = frozenset({2, 3, 4, 5, 6, 8})
MLX_GROUP_SIZES: frozenset[int] = frozenset({32, 64, 128})
RESERVED_CONFIG_KEYS: frozenset[str] = frozenset({"group_size", "bits", "mode"})
GROUPED_NDIM = 3
SHARD_BYTES = 5 << 30
_WEIGHT_FILE = re.compile(r"model(-\d{5}-of-\d{5})?\.safetensors")
_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


@dataclasses.dataclass(frozen=True)
class QuantizedLayer:
    """One layer's codes, scale, zero point and scheme (``mlx_export.py:89-106``).

    ``packed`` optionally holds the layer already in MLX's layout (uint32 words,
    scales, biases; ``mround_amd.core.quantizer.quantize_pack``), written as is
    when its dtype is the checkpoint's; ``codes``, ``scale`` and
    ``zero_point`` may then be ``None``."""

    codes: torch.Tensor | None
    scale: torch.Tensor | None
    zero_point: torch.Tensor | None
    scheme: QuantScheme
    packed: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None

    @property
    def groups(self) -> int:
        return self.scale.numel() if self.scale is not None else self.packed[1].numel()


def narrow_codes(codes: torch.Tensor, scheme: QuantScheme) -> torch.Tensor:
    """One byte per code, int8 when signed (``mlx_export.py:109-125``)."""
    lo, hi = scheme.code_range
    target = torch.int8 if lo < 0 else torch.uint8
    if (lo < 0 and (lo < -(2**7) or hi > 2**7 - 1)) or (lo >= 0 and hi > 2**8 - 1):
        msg = f"codes in [{lo}, {hi}] do not fit one byte"
        raise UnsupportedSchemeError(msg)
    return codes if codes.dtype == target else codes.to(target)


def _require_mlx_representable(path: str, scheme: QuantScheme) -> None:
    """``mlx_export.py:128-151``."""
    if scheme.bits not in MLX_SUPPORTED_BITS:
        supported = ", ".join(str(b) for b in sorted(MLX_SUPPORTED_BITS))
        msg = (
            f"{path}: MLX quantization accepts bits in {{{supported}}} and "
            f"rejects {scheme.bits}. MRound can pack this width, but no MLX "
            f"consumer can read it, and no other export path exists yet."
        )
        raise UnsupportedSchemeError(msg)
    if scheme.group_size not in MLX_GROUP_SIZES:
        sizes = ", ".join(str(g) for g in sorted(MLX_GROUP_SIZES))
        detail = "per-channel" if scheme.is_per_channel else str(scheme.group_size)
        msg = f"{path}: MLX quantization accepts group sizes {{{sizes}}} and cannot represent {detail}."
        raise UnsupportedSchemeError(msg)


def require_mlx_representable(scheme: QuantScheme, *, path: str = "scheme") -> None:
    _require_mlx_representable(path, scheme)


def to_affine(scale: torch.Tensor, zero_point: torch.Tensor | None, scheme: QuantScheme, *,
              dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor]:
    """``(scales, biases)`` with ``W = scales * q_u + biases`` (``mlx_export.py:159-195``)."""
    s = scale.to(torch.float32).contiguous()
    zp = None if zero_point is None else zero_point.to(torch.float32).contiguous()
    scales = torch.empty(s.shape, dtype=dtype, device=s.device)
    biases = torch.empty(s.shape, dtype=dtype, device=s.device)
    K.to_affine(s, zp, scheme.bits, scales, biases)
    return scales, biases


def _tensors_for_layer(path: str, layer: QuantizedLayer, dtype: torch.dtype) -> dict[str, torch.Tensor]:
    """Packed weight, scales and biases under MLX's names (``mlx_export.py:198-235``)."""
    scheme = layer.scheme
    _require_mlx_representable(path, scheme)
    if layer.packed is not None and (layer.packed[1].dtype == dtype or layer.codes is None):
        packed, scales, biases = layer.packed
        if scales.dtype != dtype:
            msg = f"{path}: packed with {scales.dtype} metadata, the checkpoint is {dtype}"
            raise ExportError(msg)
        return {f"{path}.weight": packed, f"{path}.scales": scales, f"{path}.biases": biases}
    if layer.codes.ndim != GROUPED_NDIM:
        msg = (f"{path}: expected grouped codes shaped (out_features, n_groups, group_size), "
               f"got {tuple(layer.codes.shape)}")
        raise ExportError(msg)
    out_features, n_groups, group_size = layer.codes.shape
    if group_size != scheme.group_size:
        msg = f"{path}: codes are grouped by {group_size} but the scheme says {scheme.group_size}"
        raise ExportError(msg)
    flat = narrow_codes(layer.codes, scheme).reshape(out_features, n_groups * group_size)
    offset = 2 ** (scheme.bits - 1) if scheme.symmetry is Symmetry.SYMMETRIC else 0
    packed = pack_codes(flat, scheme.bits, offset=offset)
    expected = packed_width(n_groups * group_size, scheme.bits)
    if tuple(packed.shape) != (out_features, expected):
        msg = f"{path}: packed to {tuple(packed.shape)}, expected {(out_features, expected)}"
        raise ExportError(msg)
    scales, biases = to_affine(layer.scale, layer.zero_point, scheme, dtype=dtype)
    shape = (out_features, n_groups)
    return {
        f"{path}.weight": packed,
        f"{path}.scales": scales.reshape(shape),
        f"{path}.biases": biases.reshape(shape),
    }


def _nbytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


def _shards(tensors: Mapping[str, torch.Tensor], limit: int) -> list[dict[str, torch.Tensor]]:
    """``mlx_export.py:238-252``: consecutive runs of at most ``limit`` bytes."""
    shards: list[dict[str, torch.Tensor]] = [{}]
    held = 0
    for name, tensor in tensors.items():
        if shards[-1] and held + _nbytes(tensor) > limit:
            shards.append({})
            held = 0
        shards[-1][name] = tensor
        held += _nbytes(tensor)
    return shards


def shard_names(count: int) -> list[str]:
    """``mlx_export.py:255-266``."""
    if count < 1:
        msg = f"a checkpoint has at least one weight file, not {count}"
        raise ExportError(msg)
    if count == 1:
        return ["model.safetensors"]
    return [f"model-{i:05d}-of-{count:05d}.safetensors" for i in range(1, count + 1)]


def _quantization_block(quantized: Mapping[str, QuantizedLayer]) -> dict[str, Any]:
    """``mlx_export.py:269-307``: default scheme plus flat per-path overrides."""
    schemes = [layer.scheme for layer in quantized.values()]
    ordered = sorted(set(schemes), key=lambda s: (s.bits, s.group_size, s.symmetry.value,
                                                  s.scale_init.value))
    default = max(ordered, key=schemes.count)
    block: dict[str, Any] = {"group_size": default.group_size, "bits": default.bits, "mode": "affine"}
    for path, layer in sorted(quantized.items()):
        if layer.scheme == default:
            continue
        if path in RESERVED_CONFIG_KEYS:
            msg = (f"module path {path!r} collides with a quantization setting key, "
                   f"so its per-layer override would be silently ignored")
            raise ExportError(msg)
        block[path] = {"group_size": layer.scheme.group_size, "bits": layer.scheme.bits,
                       "mode": "affine"}
    return block


def export_mlx(output_dir: Path, dense_weights: Mapping[str, torch.Tensor],
               quantized: Mapping[str, QuantizedLayer], config: Mapping[str, Any], *,
               dtype: str = "bfloat16", extra_files: Mapping[str, str] | None = None,
               shard_bytes: int = SHARD_BYTES) -> None:
    """Write a checkpoint mlx-lm loads unmodified (``mlx_export.py:310-425``)."""
    from safetensors.torch import save_file

    output_dir = Path(output_dir)
    if dtype not in _DTYPES:
        known = ", ".join(sorted(_DTYPES))
        msg = f"dtype must be one of {{{known}}}, got {dtype!r}"
        raise ExportError(msg)
    if not quantized:
        raise ExportError("nothing to export: no quantized layers were supplied")
    target = _DTYPES[dtype]
    tensors: dict[str, torch.Tensor] = {k: v.detach().cpu().contiguous() for k, v in dense_weights.items()}
    for path, layer in sorted(quantized.items()):
        collision = f"{path}.weight"
        if collision in dense_weights:
            msg = f"{collision} appears as both a dense and a quantized tensor"
            raise ExportError(msg)
        for name, t in _tensors_for_layer(path, layer, target).items():
            tensors[name] = t.cpu().contiguous()
    merged = dict(config)
    block = _quantization_block(quantized)
    merged["quantization"] = block
    merged["quantization_config"] = block
    shards = _shards(tensors, shard_bytes)
    names = shard_names(len(shards))
    weight_map = {tensor: file for shard, file in zip(shards, names) for tensor in shard}
    try:
        output_dir.mkdir(parents=True, exist_ok=True)
        for shard, file in zip(shards, names):
            save_file(shard, str(output_dir / file), metadata={"format": "mlx"})
        for stale in output_dir.iterdir():
            if _WEIGHT_FILE.fullmatch(stale.name) and stale.name not in names:
                stale.unlink()
        (output_dir / "config.json").write_text(json.dumps(merged, indent=2) + "\n")
        packed_names = {f"{path}.weight" for path in quantized}
        metadata_names = {f"{path}.{kind}" for path in quantized for kind in ("scales", "biases")}
        total_parameters = sum(
            t.numel() * 32 // quantized[name.removesuffix(".weight")].scheme.bits
            if name in packed_names else t.numel()
            for name, t in tensors.items() if name not in metadata_names
        )
        index = {
            "metadata": {"total_size": sum(_nbytes(t) for t in tensors.values()),
                         "total_parameters": total_parameters},
            "weight_map": {name: weight_map[name] for name in sorted(weight_map)},
        }
        (output_dir / "model.safetensors.index.json").write_text(json.dumps(index, indent=2) + "\n")
        for name, content in (extra_files or {}).items():
            (output_dir / name).write_text(content)
    except OSError as exc:
        msg = f"could not write the checkpoint to {output_dir}: {exc}"
        raise ExportError(msg) from exc
