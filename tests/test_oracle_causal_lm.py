"""The float64 causal-LM oracle against Hugging Face's whole-model
``Qwen2ForCausalLM`` / ``LlamaForCausalLM`` (loss and every block linear's
weight gradient), and the scoring schedules' invariants."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import block as OB
from oracle import causal_lm as OC


def tiny_model(kind: str, *, layers=2, vocab=96, hidden=64, heads=4, kv=2, head_dim=16, mlp=96,
               tied=True, seed=0) -> OC.Model:
    shape = OB.Shape(hidden=hidden, n_heads=heads, n_kv_heads=kv, head_dim=head_dim, intermediate=mlp,
                     norm_eps=1e-6, rope_theta=1e6 if kind == "qwen2" else 1e4, attn_bias=kind == "qwen2")
    g = torch.Generator().manual_seed(seed)
    rnd = lambda *s, std=0.08: torch.randn(*s, generator=g, dtype=torch.float64) * std
    blocks = []
    for i in range(layers):
        lin = {n: rnd(*shape.linear_shape(n)) for n in OB.LAYERS}
        biases = ({n: rnd(shape.linear_shape(n)[0], std=0.1)
                   for n in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj")}
                  if shape.attn_bias else {})
        norms = (1 + rnd(hidden, std=0.1), 1 + rnd(hidden, std=0.1))
        blocks.append((f"model.layers.{i}", lin, biases, norms))
    return OC.Model(shape=shape, embed=rnd(vocab, hidden, std=0.5), blocks=blocks,
                    norm=1 + rnd(hidden, std=0.1), head=None if tied else rnd(vocab, hidden, std=0.5))


def hf_model(kind: str, m: OC.Model):
    s = m.shape
    common = dict(hidden_size=s.hidden, intermediate_size=s.intermediate, num_attention_heads=s.n_heads,
                  num_key_value_heads=s.n_kv_heads, rms_norm_eps=s.norm_eps, rope_theta=s.rope_theta,
                  num_hidden_layers=len(m.blocks), vocab_size=m.embed.shape[0],
                  tie_word_embeddings=m.head is None)
    if kind == "qwen2":
        from transformers import Qwen2Config, Qwen2ForCausalLM
        cfg = Qwen2Config(**common)
        model = Qwen2ForCausalLM
    else:
        from transformers import LlamaConfig, LlamaForCausalLM
        cfg = LlamaConfig(**common, head_dim=s.head_dim, attention_bias=False, mlp_bias=False)
        model = LlamaForCausalLM
    cfg._attn_implementation = "eager"
    net = model(cfg).double().eval()
    sd = {"model.embed_tokens.weight": m.embed, "model.norm.weight": m.norm}
    for name, lin, biases, norms in m.blocks:
        sd.update({f"{name}.{n}.weight": w for n, w in lin.items()})
        sd.update({f"{name}.{n}.bias": b for n, b in biases.items()})
        sd[f"{name}.input_layernorm.weight"] = norms[0]
        sd[f"{name}.post_attention_layernorm.weight"] = norms[1]
    sd["lm_head.weight"] = m.embed if m.head is None else m.head
    net.load_state_dict(sd, strict=False)
    return net


@pytest.mark.parametrize("kind,tied", [("qwen2", True), ("llama", False)])
def test_loss_and_gradients_match_hugging_face(kind, tied):
    m = tiny_model(kind, tied=tied)
    tokens = torch.randint(0, m.embed.shape[0], (2, 21), generator=torch.Generator().manual_seed(5))
    linears = {f"{name}.{n}": lin[n] for name, lin, *_ in m.blocks for n in OB.LAYERS}
    loss, grads = OC.layer_gradients(m, tokens, linears)

    net = hf_model(kind, m)
    out = net(input_ids=tokens, labels=tokens)
    out.loss.backward()
    # Hugging Face's RMSNorm squares in float32, so the two agree to float32
    # rounding; a missing shift, a wrong head or a dropped norm moves the loss
    # by orders of magnitude more.
    assert loss == pytest.approx(float(out.loss), rel=1e-6)
    params = dict(net.named_parameters())
    for path, g in grads.items():
        theirs = params[f"{path}.weight"].grad
        err = float((g - theirs).norm() / theirs.norm())
        assert err < 1e-5, (path, err)


@pytest.mark.parametrize("mode", ["asym", "sym"])
def test_schedules_agree_at_the_widest_width(mode):
    m = tiny_model("llama", layers=1)
    g = torch.Generator().manual_seed(7)
    batches = [torch.randint(0, m.embed.shape[0], (2, 17), generator=g) for _ in range(2)]
    own = OC.score_widths(m, batches, [2, 4], group_size=16, mode=mode, gradient_source="own_width")
    wide = OC.score_widths(m, batches, [2, 4], group_size=16, mode=mode, gradient_source="widest")
    for p in own:
        assert own[p][4] == pytest.approx(wide[p][4], rel=1e-12)
        assert own[p][2] > 0 and wide[p][2] > 0
        # narrower codes perturb more
        assert wide[p][2] > wide[p][4]


def test_scores_are_sums_over_batches():
    m = tiny_model("qwen2", layers=1)
    g = torch.Generator().manual_seed(8)
    a, b = (torch.randint(0, m.embed.shape[0], (2, 17), generator=g) for _ in range(2))
    both = OC.score_widths(m, [a, b], [3], group_size=16, mode="asym")
    one = OC.score_widths(m, [a], [3], group_size=16, mode="asym")
    two = OC.score_widths(m, [b], [3], group_size=16, mode="asym")
    for p in both:
        assert both[p][3] == pytest.approx(one[p][3] + two[p][3], rel=1e-12)


def test_searched_perturbation_uses_the_grid():
    m = tiny_model("llama", layers=1)
    w = m.blocks[0][1]["mlp.down_proj"].numpy().astype(np.float32)
    rows, cols = w.shape
    grid = np.full((rows, cols // 16), 0.05, dtype=np.float32)
    q = OC.rtn(w, bits=2, group_size=16, mode="searched", init_scale=grid)
    # every reconstruction is a multiple of the grid's scale within the 2-bit code range
    codes = q / 0.05
    assert np.allclose(codes, np.round(codes), atol=1e-4)
    assert codes.min() >= -2 and codes.max() <= 1
