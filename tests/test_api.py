"""Model-level host logic on the CPU: random checkpoints, loading, scheme
resolution and the errors api.quantize raises before any GPU work."""

from __future__ import annotations

import pytest
import torch

from mround_amd import api
from mround_amd.cli import GEOMETRIES, main
from mround_amd.exceptions import ArchitectureError, CalibrationError, SchemeError, UnsupportedSchemeError
from mround_amd.pipeline.checkpoint import block_shape, dense_tensors, load_model, write_random_checkpoint
from mround_amd.schemes import ScaleInit, Symmetry, TuningConfig

TINY = dict(model_type="qwen2", hidden_size=128, num_attention_heads=2, num_key_value_heads=1,
            intermediate_size=256, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=2,
            vocab_size=512, tie_word_embeddings=True)


def test_random_checkpoint_round_trip(tmp_path):
    write_random_checkpoint(tmp_path / "m", TINY, seed=3)
    m = load_model(tmp_path / "m", device="cpu")
    assert m.tied and len(m.blocks) == 2 and m.dtype == torch.bfloat16
    s = m.blocks[0].shape
    assert (s.hidden, s.n_heads, s.n_kv_heads, s.head_dim, s.intermediate) == (128, 2, 1, 64, 256)
    assert s.attn_bias and set(m.blocks[1].weights.biases) == {
        "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"}
    t = dense_tensors(m)
    assert t["model.layers.1.mlp.down_proj.weight"].shape == (128, 256)
    assert t["model.embed_tokens.weight"].shape == (512, 128) and "lm_head.weight" not in t
    again = load_model(tmp_path / "m", device="cpu")
    assert torch.equal(again.blocks[0].weights.linears["mlp.up_proj"], m.blocks[0].weights.linears["mlp.up_proj"])


def test_geometries_are_valid_blocks():
    for name, cfg in GEOMETRIES.items():
        s = block_shape(cfg)
        s.validate(2048)
        assert s.hidden == cfg["hidden_size"]


def test_unknown_architecture_and_missing_checkpoint(tmp_path):
    with pytest.raises(ArchitectureError, match="model_type"):
        block_shape(dict(TINY, model_type="gpt2"))
    with pytest.raises(ArchitectureError, match="config.json"):
        load_model(tmp_path / "nothing", device="cpu")


def test_default_scale_init_rule():
    assert api.default_scale_init(2, Symmetry.SYMMETRIC) is ScaleInit.SEARCHED
    assert api.default_scale_init(4, Symmetry.SYMMETRIC) is ScaleInit.OBSERVED_RANGE
    assert api.default_scale_init(2, Symmetry.ASYMMETRIC) is ScaleInit.OBSERVED_RANGE


def test_quantize_refusals(tmp_path):
    write_random_checkpoint(tmp_path / "m", TINY)
    with pytest.raises(SchemeError, match="pass average_bits too"):
        api.quantize(tmp_path / "m", output_dir=tmp_path / "o", plan={"a": 2}, device="cpu")
    with pytest.raises(SchemeError, match="empty"):
        api.quantize(tmp_path / "m", output_dir=tmp_path / "o", average_bits=3, plan={}, device="cpu")
    with pytest.raises(SchemeError, match="candidate_bits"):
        api.quantize(tmp_path / "m", output_dir=tmp_path / "o", average_bits=3, plan={"a": 5}, device="cpu")
    with pytest.raises(SchemeError, match="outside the achievable range"):
        api.quantize(tmp_path / "m", output_dir=tmp_path / "o", average_bits=4.5, device="cpu",
                     tuning=TuningConfig(n_samples=2, batch_size=2, seq_len=128))
    with pytest.raises(UnsupportedSchemeError):
        api.quantize(tmp_path / "m", output_dir=tmp_path / "o", average_bits=3, candidate_bits=(2, 7),
                     device="cpu")
    with pytest.raises(UnsupportedSchemeError, match="format"):
        api.quantize(tmp_path / "m", output_dir=tmp_path / "o", export_format="gguf", device="cpu")
    with pytest.raises(UnsupportedSchemeError):
        api.quantize(tmp_path / "m", output_dir=tmp_path / "o", bits=7, device="cpu")
    with pytest.raises(CalibrationError, match="corpus"):
        api.quantize(tmp_path / "m", output_dir=tmp_path / "o", calibration="pile-10k", device="cpu")
    with pytest.raises(CalibrationError, match="must all be positive"):
        api.quantize(tmp_path / "m", output_dir=tmp_path / "o", device="cpu",
                     tuning=TuningConfig(n_samples=2, batch_size=2, seq_len=0))


def test_cli_random_model_and_errors(tmp_path, capsys):
    assert main(["random-model", "smollm2-135m", str(tmp_path / "s"), "--layers", "1", "--device", "cpu"]) == 0
    m = load_model(tmp_path / "s", device="cpu")
    assert len(m.blocks) == 1 and m.blocks[0].shape.n_heads == 9
    assert main(["quantize", str(tmp_path / "s"), "-o", str(tmp_path / "o"), "--average-bits", "2.5",
                 "--options", "2,x"]) == 1
    assert "--options must be comma separated" in capsys.readouterr().err
