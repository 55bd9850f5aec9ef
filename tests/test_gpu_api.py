"""api.quantize end to end on a random two-block Qwen2 model: the MLX
checkpoint it writes (names, dtypes, config, packing), the round-to-nearest
remainder bit-exact with the oracle, and the CLI."""

from __future__ import annotations

import json
import sys

import numpy as np
import pytest
import torch
from safetensors.torch import load_file

from mround_amd import api
from mround_amd.cli import main
from mround_amd.pipeline.block import LAYERS
from mround_amd.pipeline.checkpoint import load_model, write_random_checkpoint
from mround_amd.schemes import Symmetry, TuningConfig
from oracle import packing as OP
from oracle import quantize as OQ

pytestmark = pytest.mark.gpu

TINY = dict(model_type="qwen2", hidden_size=128, num_attention_heads=2, num_key_value_heads=1,
            intermediate_size=256, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=2,
            vocab_size=512, tie_word_embeddings=True)


def _bf16(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16)


@pytest.mark.parametrize("bits,asym", [(4, True), (2, False)])
def test_quantize_writes_an_mlx_checkpoint(tmp_path, bits, asym):
    print("case api", bits, asym, flush=True, file=sys.stderr)
    src = write_random_checkpoint(tmp_path / "m", TINY, seed=1, std=0.05)
    tuning = TuningConfig(iters=6, batch_size=2, n_samples=4, seq_len=128)
    res = api.quantize(src, output_dir=tmp_path / "q", bits=bits,
                       symmetry=Symmetry.ASYMMETRIC if asym else Symmetry.SYMMETRIC, tuning=tuning, seed=5)
    assert len(res.summary.blocks) == 2
    for b in res.summary.blocks:
        assert b.final_loss <= b.initial_loss
    cfg = json.loads((tmp_path / "q" / "config.json").read_text())
    assert cfg["quantization"] == {"group_size": 64, "bits": bits, "mode": "affine"}
    assert cfg["quantization_config"] == cfg["quantization"]
    t = load_file(str(tmp_path / "q" / "model.safetensors"))
    index = json.loads((tmp_path / "q" / "model.safetensors.index.json").read_text())
    assert set(index["weight_map"]) == set(t)
    for i in range(2):
        for n in LAYERS:
            p = f"model.layers.{i}.{n}"
            assert t[f"{p}.weight"].dtype == torch.uint32
            assert t[f"{p}.scales"].dtype == torch.bfloat16 and t[f"{p}.biases"].dtype == torch.bfloat16
            assert f"{p}.bias" in t or not n.endswith(("q_proj", "k_proj", "v_proj"))
    # the embedding is round to nearest: codes, scales and biases bit-exact with the oracle
    orig = load_model(src, device="cpu")
    emb = orig.embed.float().numpy()
    mode = "asym" if asym else "searched"
    init = None
    if not asym:
        from oracle import scale_search as OS
        init = OS.search_scales_f32(emb, bits, 64).reshape(512, -1, 1)
    _, codes, scale, zp = OQ.fake_quantize(emb, None, None, None, bits=bits, group_size=64, mode=mode,
                                           init_scale=init)
    rows, cols = emb.shape
    q = codes.reshape(rows, cols).astype(np.int64)
    if not asym:
        q = q + 2 ** (bits - 1)
    words = OP.pack_codes(q.astype(np.uint32), bits)
    assert np.array_equal(t["model.embed_tokens.weight"].numpy(), words)
    s_bf = _bf16(scale.reshape(rows, -1))
    assert torch.equal(t["model.embed_tokens.scales"], s_bf)
    zpv = zp.reshape(rows, -1) if asym else np.full((rows, cols // 64), 2 ** (bits - 1), dtype=np.float32)
    want_b = -(s_bf.float() * _bf16(zpv).float())
    assert torch.equal(t["model.embed_tokens.biases"], want_b.to(torch.bfloat16))
    # block layers reconstruct within their quantization error
    w = orig.blocks[0].weights.linears["mlp.up_proj"].float()
    codes = OP.unpack_codes(t["model.layers.0.mlp.up_proj.weight"].numpy(), 128, bits)
    deq = (t["model.layers.0.mlp.up_proj.scales"].float().repeat_interleave(64, 1) * torch.from_numpy(
        codes.astype(np.float32)) + t["model.layers.0.mlp.up_proj.biases"].float().repeat_interleave(64, 1))
    rel = float((deq - w).norm() / w.norm())
    assert rel < (0.2 if bits == 4 else 0.8), rel
    rec = json.loads((tmp_path / "q" / "mround_run.json").read_text())
    assert rec["scheme"]["bits"] == bits and len(rec["blocks"]) == 2
    assert res.storage.bits_per_weight < 16


def test_cli_quantize(tmp_path, capsys):
    src = write_random_checkpoint(tmp_path / "m", TINY, seed=2)
    rc = main(["quantize", str(src), "-o", str(tmp_path / "q"), "--bits", "4", "--asym", "--iters", "4",
               "--samples", "2", "--seq-len", "128", "--batch-size", "2"])
    assert rc == 0
    out = capsys.readouterr().out
    assert "modules tuned" in out and (tmp_path / "q" / "model.safetensors").exists()


@pytest.mark.parametrize("asym,dense", [(True, False), (False, True)])
def test_round_to_nearest_export(tmp_path, asym, dense):
    """Every block linear (and, unless dense, the embedding) at round to nearest
    with the observed-range scale: packed words, scales and biases bit-exact
    with the oracle (mround/api.py:841-940)."""
    print("case rtn", asym, dense, flush=True, file=sys.stderr)
    src = write_random_checkpoint(tmp_path / "m", TINY, seed=4, std=0.05)
    res = api.quantize_round_to_nearest(src, output_dir=tmp_path / "q", bits=3,
                                        symmetry=Symmetry.ASYMMETRIC if asym else Symmetry.SYMMETRIC,
                                        dense_remainder=dense)
    assert len(res.quantized) == 14 + (0 if dense else 1)
    assert ("model.embed_tokens" in dict(res.skipped)) == dense
    assert 3 < res.bits_per_weight < 16 and res.compression > 1
    cfg = json.loads((tmp_path / "q" / "config.json").read_text())
    assert cfg["quantization"]["bits"] == 3
    t = load_file(str(tmp_path / "q" / "model.safetensors"))
    orig = load_model(src, device="cpu")
    w = orig.blocks[1].weights.linears["self_attn.o_proj"].float().numpy()
    mode = "asym" if asym else "sym"
    _, codes, scale, zp = OQ.fake_quantize(w, None, None, None, bits=3, group_size=64, mode=mode)
    rows, cols = w.shape
    q = codes.reshape(rows, cols).astype(np.int64) + (0 if asym else 4)
    assert np.array_equal(t["model.layers.1.self_attn.o_proj.weight"].numpy(), OP.pack_codes(q.astype(np.uint32), 3))
    s_bf = _bf16(scale.reshape(rows, -1))
    assert torch.equal(t["model.layers.1.self_attn.o_proj.scales"], s_bf)
    zpv = zp.reshape(rows, -1) if asym else np.full((rows, cols // 64), 4, dtype=np.float32)
    assert torch.equal(t["model.layers.1.self_attn.o_proj.biases"],
                       (-(s_bf.float() * _bf16(zpv).float())).to(torch.bfloat16))
    if dense:
        assert t["model.embed_tokens.weight"].dtype == torch.bfloat16
