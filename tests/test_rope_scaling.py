"""RoPE frequency scaling of the block's rope table, pinned against Hugging
Face transformers' own rope initialisation (``ROPE_INIT_FUNCTIONS``) and its
rotary embedding, and the refusal of scaling types the table does not
implement. CPU only."""

from __future__ import annotations

import math

import pytest
import torch
from transformers import LlamaConfig
from transformers import modeling_rope_utils as R
from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

from mround_amd.exceptions import ArchitectureError
from mround_amd.pipeline.block import rope_frequencies, rope_table
from mround_amd.pipeline.checkpoint import block_shape

LLAMA31 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
           "original_max_position_embeddings": 8192}


def _config(scaling, theta=500000.0, head_dim=128):
    return LlamaConfig(hidden_size=32 * head_dim, num_attention_heads=32, num_key_value_heads=8,
                       head_dim=head_dim, intermediate_size=14336, rope_theta=theta, rope_scaling=scaling,
                       max_position_embeddings=131072)


def _ours(cfg_dict):
    s = block_shape({**cfg_dict, "model_type": "llama"})
    return s, rope_frequencies(s.head_dim, s.rope_theta, s.rope_scaling)


@pytest.mark.parametrize("scaling,fn", [(LLAMA31, "llama3"), ({"rope_type": "linear", "factor": 4.0}, "linear"),
                                        (None, "default")])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_frequencies_match_hugging_face(scaling, fn, head_dim):
    cfg = _config(scaling, head_dim=head_dim)
    inv_hf, _ = R.ROPE_INIT_FUNCTIONS[fn](cfg) if fn != "default" else (None, None)
    if inv_hf is None:
        inv_hf = 1.0 / (500000.0 ** (torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim))
    shape, inv = _ours(cfg.to_dict())
    assert shape.rope_theta == 500000.0
    assert torch.allclose(inv, inv_hf.double(), rtol=2e-6, atol=0)
    if fn == "llama3":
        # the rule's three regimes all occur at these settings
        wavelength = 2 * math.pi / inv_hf.double()
        assert (wavelength < 8192 / 4).any() and (wavelength > 8192).any()
        assert ((wavelength >= 2048) & (wavelength <= 8192)).any()


def test_rope_table_matches_the_rotary_embedding():
    cfg = _config(LLAMA31)
    emb = LlamaRotaryEmbedding(cfg)
    S = 4096
    pos = torch.arange(S)[None]
    cos, sin = emb(torch.zeros(1, S, 8, dtype=torch.float32), pos)
    shape, _ = _ours(cfg.to_dict())
    table = rope_table(S, shape.head_dim, shape.rope_theta, "cpu", shape.rope_scaling)
    half = shape.head_dim // 2
    # the embedding repeats the d/2 frequencies over both halves; it forms
    # pos x frequency in float32 (a rounding of up to 4096 x 2^-24 rad here),
    # the table in float64
    assert torch.allclose(table[..., 0], cos[0, :, :half], atol=1e-3)
    assert torch.allclose(table[..., 1], sin[0, :, :half], atol=1e-3)
    assert torch.equal(cos[0, :, :half], cos[0, :, half:])


@pytest.mark.parametrize("kind", ["yarn", "dynamic", "longrope"])
def test_unimplemented_scaling_is_refused(kind):
    cfg = {"model_type": "llama", "hidden_size": 4096, "num_attention_heads": 32, "intermediate_size": 11008,
           "rope_scaling": {"rope_type": kind, "factor": 4.0}}
    with pytest.raises(ArchitectureError, match=kind):
        block_shape(cfg)


def test_old_layout_and_no_scaling():
    cfg = {"model_type": "qwen2", "hidden_size": 896, "num_attention_heads": 14, "intermediate_size": 4864,
           "rope_theta": 1e6, "rope_scaling": None}
    s = block_shape(cfg)
    assert s.rope_theta == 1e6 and s.rope_scaling == ()
    lin = block_shape({**cfg, "rope_scaling": {"type": "linear", "factor": 2.0}})
    assert dict(lin.rope_scaling) == {"rope_type": "linear", "factor": 2.0}
    with pytest.raises(ArchitectureError, match="lacks"):
        block_shape({**cfg, "rope_scaling": {"rope_type": "llama3", "factor": 8.0}})
