"""Local Hugging Face-layout checkpoints of Qwen2 / Llama decoder models.

Stands in for the reference's mlx-lm loading (mround/pipeline/loader.py:
176-269) on a machine with no hub access: a directory holding
``config.json`` and ``*.safetensors`` is read straight onto the device as
torch tensors (safetensors executes nothing from the file). Also writes
random-initialised checkpoints of a given geometry, the synthetic models the
benchmarks and tests run on.
"""

from __future__ import annotations

import dataclasses
import json
from pathlib import Path
from typing import Any

import torch

from mround_amd.exceptions import ArchitectureError
from mround_amd.pipeline.block import LAYERS, QKV, ROPE_TYPES, BlockShape, BlockWeights
from mround_amd.pipeline.runner import DecoderBlock

SUPPORTED_TYPES = ("qwen2", "llama", "mistral")
_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


@dataclasses.dataclass
class DecoderModel:
    """A decoder-only LM: config, embedding, blocks, final norm, optional head."""

    config: dict[str, Any]
    dtype: torch.dtype
    embed: torch.Tensor
    blocks: list[DecoderBlock]
    norm: torch.Tensor
    lm_head: torch.Tensor | None  # None when tied to the embedding

    @property
    def tied(self) -> bool:
        return self.lm_head is None


def rope_scaling(config: dict[str, Any]) -> tuple:
    """The config's RoPE frequency scaling as sorted (key, value) pairs (empty
    for none). Types the block's rope table does not implement are refused:
    tuning through the unscaled frequencies would fit a different function
    from the model's."""
    raw = config.get("rope_scaling") or config.get("rope_parameters")
    if not raw:
        return ()
    kind = raw.get("rope_type", raw.get("type", "default"))
    if kind not in ROPE_TYPES:
        raise ArchitectureError(f"rope_scaling type {kind!r} is not supported (supported: "
                                f"{', '.join(ROPE_TYPES)})")
    if kind == "default":
        return ()
    need = {"linear": ("factor",),
            "llama3": ("factor", "low_freq_factor", "high_freq_factor", "original_max_position_embeddings")}[kind]
    missing = [k for k in need if k not in raw]
    if missing:
        raise ArchitectureError(f"rope_scaling of type {kind!r} lacks {', '.join(missing)}")
    return tuple(sorted([("rope_type", kind)] + [(k, float(raw[k])) for k in need]))


def rope_theta(config: dict[str, Any]) -> float:
    """RoPE base: the top-level ``rope_theta``, or the one inside
    ``rope_parameters`` (the newer Hugging Face layout), else 10000."""
    theta = config.get("rope_theta")
    if theta is None:
        theta = (config.get("rope_parameters") or {}).get("rope_theta", 10000.0)
    return float(theta)


def block_shape(config: dict[str, Any]) -> BlockShape:
    """The block geometry a config describes."""
    kind = config.get("model_type")
    if kind not in SUPPORTED_TYPES:
        raise ArchitectureError(f"model_type {kind!r} is not a supported decoder "
                                f"({', '.join(SUPPORTED_TYPES)})")
    heads = int(config["num_attention_heads"])
    hidden = int(config["hidden_size"])
    head_dim = int(config.get("head_dim") or hidden // heads)
    bias = kind == "qwen2" or bool(config.get("attention_bias", False))
    return BlockShape(hidden=hidden, n_heads=heads,
                      n_kv_heads=int(config.get("num_key_value_heads") or heads), head_dim=head_dim,
                      intermediate=int(config["intermediate_size"]),
                      norm_eps=float(config.get("rms_norm_eps", 1e-6)),
                      rope_theta=rope_theta(config), attn_bias=bias, rope_scaling=rope_scaling(config))


def _read_tensors(path: Path, device) -> dict[str, torch.Tensor]:
    from safetensors.torch import load_file

    files = sorted(path.glob("*.safetensors"))
    if not files:
        raise ArchitectureError(f"no *.safetensors weights in {path}")
    out: dict[str, torch.Tensor] = {}
    for f in files:
        out.update(load_file(str(f), device=str(device)))
    return out


def load_model(path: str | Path, *, device="cuda") -> DecoderModel:
    """Load a local checkpoint directory onto ``device``."""
    path = Path(path)
    if not (path / "config.json").is_file():
        raise ArchitectureError(f"{path} is not a local checkpoint directory (no config.json); "
                                "hub downloads are not available")
    config = json.loads((path / "config.json").read_text())
    shape = block_shape(config)
    dtype = _DTYPES.get(str(config.get("torch_dtype", "bfloat16")), torch.bfloat16)
    t = _read_tensors(path, device)

    def take(name: str) -> torch.Tensor:
        if name not in t:
            raise ArchitectureError(f"checkpoint has no tensor {name!r}")
        return t.pop(name)

    n_layers = int(config["num_hidden_layers"])
    blocks = []
    for i in range(n_layers):
        pre = f"model.layers.{i}"
        lin = {n: take(f"{pre}.{n}.weight") for n in LAYERS}
        biases = {n: take(f"{pre}.{n}.bias").float() for n in QKV} if shape.attn_bias else {}
        w = BlockWeights(lin, biases, take(f"{pre}.input_layernorm.weight").float(),
                         take(f"{pre}.post_attention_layernorm.weight").float())
        blocks.append(DecoderBlock(i, pre, shape, w))
    embed = take("model.embed_tokens.weight")
    norm = take("model.norm.weight")
    head = None if config.get("tie_word_embeddings", False) else take("lm_head.weight")
    return DecoderModel(config, dtype, embed, blocks, norm, head)


def dense_tensors(model: DecoderModel) -> dict[str, torch.Tensor]:
    """Every tensor of the model by its checkpoint name, in the model dtype
    (norm weights and biases included), for export."""
    out: dict[str, torch.Tensor] = {"model.embed_tokens.weight": model.embed,
                                    "model.norm.weight": model.norm.to(model.dtype)}
    if model.lm_head is not None:
        out["lm_head.weight"] = model.lm_head
    for b in model.blocks:
        for n, w in b.weights.linears.items():
            out[f"{b.name}.{n}.weight"] = w
        for n, bias in b.weights.biases.items():
            out[f"{b.name}.{n}.bias"] = bias.to(model.dtype)
        out[f"{b.name}.input_layernorm.weight"] = b.weights.input_norm.to(model.dtype)
        out[f"{b.name}.post_attention_layernorm.weight"] = b.weights.post_norm.to(model.dtype)
    return out


def write_random_checkpoint(path: str | Path, config: dict[str, Any], *, seed: int = 0,
                            std: float = 0.02, device="cpu") -> Path:
    """A checkpoint of the given config with weights N(0, std) (norm weights 1,
    biases N(0, std)), in ``config['torch_dtype']`` (bfloat16 by default)."""
    from safetensors.torch import save_file

    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    shape = block_shape(config)
    dtype = _DTYPES.get(str(config.get("torch_dtype", "bfloat16")), torch.bfloat16)
    g = torch.Generator(device=device).manual_seed(seed)
    rnd = lambda *s: (torch.randn(*s, generator=g, device=device) * std).to(dtype)
    vocab, h = int(config["vocab_size"]), shape.hidden
    t: dict[str, torch.Tensor] = {"model.embed_tokens.weight": rnd(vocab, h),
                                  "model.norm.weight": torch.ones(h, dtype=dtype, device=device)}
    if not config.get("tie_word_embeddings", False):
        t["lm_head.weight"] = rnd(vocab, h)
    for i in range(int(config["num_hidden_layers"])):
        pre = f"model.layers.{i}"
        for n in LAYERS:
            t[f"{pre}.{n}.weight"] = rnd(*shape.linear_shape(n))
        if shape.attn_bias:
            for n in QKV:
                t[f"{pre}.{n}.bias"] = rnd(shape.linear_shape(n)[0])
        t[f"{pre}.input_layernorm.weight"] = torch.ones(h, dtype=dtype, device=device)
        t[f"{pre}.post_attention_layernorm.weight"] = torch.ones(h, dtype=dtype, device=device)
    save_file({k: v.cpu().contiguous() for k, v in t.items()}, str(path / "model.safetensors"),
              metadata={"format": "pt"})
    cfg = dict(config)
    cfg.setdefault("torch_dtype", "bfloat16")
    (path / "config.json").write_text(json.dumps(cfg, indent=2) + "\n")
    return path
