"""The MLX checkpoint's sharding and index, restating the reference's
expectations (mround tests/unit/test_mlx_formats.py:234-251, 380-470) on
bytes rather than gigabytes: one 4-bit 8 x 64 layer at group size 32 stores
256 bytes of words and 32 bytes each of bf16 scales and biases. The greedy
split, numbering, a tensor past the limit alone in its shard, the index's
weight map and totals, and stale weight files of an earlier export removed
while other files stay."""

from __future__ import annotations

import itertools
import json

import numpy as np
import pytest
import torch
from safetensors.torch import load_file

from mround_amd.core.quantizer import quantize_codes
from mround_amd.exceptions import ExportError
from mround_amd.formats import mlx_export as MX
from mround_amd.schemes import QuantScheme
from tests.helpers import dev

pytestmark = pytest.mark.gpu


def a_layer(bits=4, group_size=32, out_features=8, in_features=64) -> MX.QuantizedLayer:
    w = np.random.default_rng(bits).normal(scale=0.05, size=(out_features, in_features)).astype(np.float32)
    scheme = QuantScheme(bits=bits, group_size=group_size)
    codes, scale, zp = quantize_codes(torch.from_numpy(w).to(dev()), None, scheme, narrow=True)
    return MX.QuantizedLayer(codes, scale, zp, scheme)


def _weight_files(path) -> list[str]:
    return sorted(p.name for p in path.iterdir() if MX._WEIGHT_FILE.fullmatch(p.name))


def _contents(path) -> dict[str, dict[str, torch.Tensor]]:
    return {f: load_file(str(path / f)) for f in _weight_files(path)}


def _nbytes(shard) -> int:
    return sum(t.numel() * t.element_size() for t in shard.values())


def test_past_the_limit_it_is_split_into_numbered_shards(tmp_path):
    layers = {f"model.layers.{i}.mlp.up_proj": a_layer(bits=4) for i in range(5)}
    dense = {"model.embed_tokens.weight": torch.zeros(10, 64, dtype=torch.bfloat16, device=dev())}
    limit = 1000
    MX.export_mlx(tmp_path, dense, layers, config={}, shard_bytes=limit)
    files = _weight_files(tmp_path)
    assert len(files) > 1 and files == MX.shard_names(len(files))
    shards = _contents(tmp_path)
    held, sizes = {}, []
    for f in files:
        shard = shards[f]
        assert shard, f"{f} holds nothing"
        sizes.append(_nbytes(shard))
        assert sizes[-1] <= limit or len(shard) == 1
        for name in shard:
            assert name not in held
            held[name] = f
    assert all(a + b > limit for a, b in itertools.pairwise(sizes))  # greedy
    index = json.loads((tmp_path / "model.safetensors.index.json").read_text())
    assert index["weight_map"] == held
    assert set(held) == {"model.embed_tokens.weight"} | {f"{p}.{k}" for p in layers
                                                        for k in ("weight", "scales", "biases")}
    assert index["metadata"]["total_size"] == sum(sizes)


def test_a_checkpoint_of_exactly_the_limit_stays_one_file(tmp_path):
    layers = {"layers.0.mlp": a_layer(), "layers.1.mlp": a_layer()}
    size = 2 * (256 + 32 + 32)
    MX.export_mlx(tmp_path / "at", {}, layers, config={}, shard_bytes=size)
    MX.export_mlx(tmp_path / "under", {}, layers, config={}, shard_bytes=size - 1)
    assert _weight_files(tmp_path / "at") == ["model.safetensors"]
    index = json.loads((tmp_path / "at" / "model.safetensors.index.json").read_text())
    assert set(index["weight_map"].values()) == {"model.safetensors"}
    assert _weight_files(tmp_path / "under") == MX.shard_names(2)


def test_a_tensor_past_the_limit_fills_a_shard_of_its_own(tmp_path):
    layers = {"layers.0.mlp": a_layer(), "layers.1.mlp": a_layer()}
    MX.export_mlx(tmp_path, {}, layers, config={}, shard_bytes=100)
    shards = _contents(tmp_path)
    assert [sorted(s) for s in shards.values()] == [
        ["layers.0.mlp.weight"], ["layers.0.mlp.biases", "layers.0.mlp.scales"],
        ["layers.1.mlp.weight"], ["layers.1.mlp.biases", "layers.1.mlp.scales"]]


def test_the_names_and_the_limit():
    assert MX.shard_names(1) == ["model.safetensors"]
    assert MX.shard_names(3) == [f"model-0000{i}-of-00003.safetensors" for i in (1, 2, 3)]
    with pytest.raises(ExportError, match="at least one"):
        MX.shard_names(0)
    assert MX.SHARD_BYTES == 5 * 1024**3


def test_an_export_over_an_earlier_one_leaves_none_of_its_weight_files(tmp_path):
    layers = {f"layers.{i}.mlp": a_layer() for i in range(3)}
    (tmp_path / "other.safetensors").write_bytes(b"not a weight file of this export")
    MX.export_mlx(tmp_path, {}, layers, config={}, shard_bytes=300)
    assert _weight_files(tmp_path) == MX.shard_names(5)
    MX.export_mlx(tmp_path, {}, layers, config={}, shard_bytes=700)
    assert _weight_files(tmp_path) == MX.shard_names(2)
    MX.export_mlx(tmp_path, {}, layers, config={})
    assert _weight_files(tmp_path) == ["model.safetensors"]
    MX.export_mlx(tmp_path, {}, layers, config={}, shard_bytes=700)
    assert _weight_files(tmp_path) == MX.shard_names(2)
    assert (tmp_path / "other.safetensors").read_bytes() == b"not a weight file of this export"


def test_index_totals_count_represented_parameters(tmp_path):
    # a packed uint32 word counts 32 / bits parameters; storage counts bytes
    emb = torch.zeros(10, 64, dtype=torch.float16, device=dev())
    MX.export_mlx(tmp_path, {"embed.weight": emb}, {"layers.0.mlp": a_layer(bits=4, group_size=32)}, config={},
                  dtype="float16")
    index = json.loads((tmp_path / "model.safetensors.index.json").read_text())
    assert index["metadata"]["total_parameters"] == 8 * 64 + 10 * 64
    words = 8 * (64 * 4 // 32)
    assert index["metadata"]["total_size"] == words * 4 + (8 * 2 + 8 * 2) * 2 + 640 * 2
