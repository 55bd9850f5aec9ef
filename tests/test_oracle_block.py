"""The float64 block oracle against Hugging Face's decoder layers, and the
tuning loop against the reference's property tests
(``tests/test_reference_tuning.py``: initial parameters are round to nearest,
learning happens, determinism, the revert rule)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import block as OB
from oracle import quantize as OQ


def _weights(shape: OB.Shape, seed: int, *, bias: bool, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    lin = {n: torch.randn(*shape.linear_shape(n), generator=g, dtype=torch.float64).to(dtype) * 0.05
           for n in OB.LAYERS}
    biases = {}
    if bias:
        for n in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"):
            biases[n] = torch.randn(shape.linear_shape(n)[0], generator=g, dtype=torch.float64) * 0.1
    norms = (1 + 0.1 * torch.randn(shape.hidden, generator=g, dtype=torch.float64),
             1 + 0.1 * torch.randn(shape.hidden, generator=g, dtype=torch.float64))
    return lin, biases, norms


def _hf_layer(kind: str, shape: OB.Shape, lin, biases, norms):
    if kind == "qwen2":
        from transformers import Qwen2Config
        from transformers.models.qwen2.modeling_qwen2 import Qwen2DecoderLayer as Layer
        cfg = Qwen2Config(hidden_size=shape.hidden, intermediate_size=shape.intermediate,
                          num_attention_heads=shape.n_heads, num_key_value_heads=shape.n_kv_heads,
                          rms_norm_eps=shape.norm_eps, rope_theta=shape.rope_theta)
    else:
        from transformers import LlamaConfig
        from transformers.models.llama.modeling_llama import LlamaDecoderLayer as Layer
        cfg = LlamaConfig(hidden_size=shape.hidden, intermediate_size=shape.intermediate,
                          num_attention_heads=shape.n_heads, num_key_value_heads=shape.n_kv_heads,
                          rms_norm_eps=shape.norm_eps, rope_theta=shape.rope_theta,
                          head_dim=shape.head_dim, attention_bias=False, mlp_bias=False)
    cfg._attn_implementation = "eager"
    layer = Layer(cfg, 0).double().eval()
    sd = {f"{n}.weight": w for n, w in lin.items()}
    sd.update({f"{n}.bias": b for n, b in biases.items()})
    sd["input_layernorm.weight"] = norms[0]
    sd["post_attention_layernorm.weight"] = norms[1]
    layer.load_state_dict(sd, strict=True)
    return layer


@pytest.mark.parametrize("kind", ["qwen2", "llama"])
def test_block_matches_hugging_face(kind):
    shape = OB.Shape(hidden=64, n_heads=4, n_kv_heads=2, head_dim=16, intermediate=96,
                     norm_eps=1e-6, rope_theta=1e6 if kind == "qwen2" else 1e4,
                     attn_bias=kind == "qwen2")
    lin, biases, norms = _weights(shape, 3, bias=shape.attn_bias)
    B, S = 2, 24
    x = torch.randn(B, S, shape.hidden, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    ours = OB.block_forward(x, lin, biases, norms, shape)
    layer = _hf_layer(kind, shape, lin, biases, norms)
    cos, sin = OB.rope_cos_sin(S, shape.head_dim, shape.rope_theta)
    emb = (torch.cat([cos, cos], -1)[None].expand(B, S, -1), torch.cat([sin, sin], -1)[None].expand(B, S, -1))
    mask = torch.zeros(B, 1, S, S, dtype=torch.float64)
    mask.masked_fill_(~torch.ones(S, S, dtype=torch.bool).tril(), float("-inf"))
    with torch.no_grad():
        theirs = layer(x, attention_mask=mask, position_embeddings=emb)
    if isinstance(theirs, tuple):
        theirs = theirs[0]
    # Hugging Face's RMSNorm squares in float32 whatever the input dtype, so the
    # two agree to float32 rounding; a layout, bias, mask or head-mapping slip
    # moves the output by orders of magnitude more.
    assert torch.allclose(ours, theirs, rtol=0, atol=1e-6), float((ours - theirs).abs().max())


def test_block_is_causal_and_batch_independent():
    shape = OB.Shape(hidden=32, n_heads=2, n_kv_heads=1, head_dim=16, intermediate=64)
    lin, biases, norms = _weights(shape, 5, bias=False)
    x = torch.randn(2, 10, 32, generator=torch.Generator().manual_seed(6), dtype=torch.float64)
    full = OB.block_forward(x, lin, biases, norms, shape)
    prefix = OB.block_forward(x[:, :6], lin, biases, norms, shape)
    single = OB.block_forward(x[1:], lin, biases, norms, shape)
    assert torch.allclose(full[:, :6], prefix, atol=1e-13)
    assert torch.allclose(full[1:], single, atol=1e-13)


TINY = OB.Shape(hidden=64, n_heads=2, n_kv_heads=1, head_dim=32, intermediate=128)


def _tiny_problem(seed=11, n_batches=2, B=2, S=16, bits=2):
    lin, biases, norms = _weights(TINY, seed, bias=False, dtype=torch.float32)
    lin = {n: w.float() for n, w in lin.items()}
    g = torch.Generator().manual_seed(seed + 1)
    inputs = [torch.randn(B, S, TINY.hidden, generator=g) for _ in range(n_batches)]
    targets = [OB.block_forward(x.double(), {n: w.double() for n, w in lin.items()}, biases, norms, TINY)
               for x in inputs]
    return lin, biases, norms, inputs, targets, OB.Scheme(bits=bits, group_size=32)


def test_initial_parameters_are_round_to_nearest():
    lin, _, _, _, _, scheme = _tiny_problem()
    params = OB.init_params(lin, scheme)
    wq = OB.quantized_linears(lin, params, scheme)
    for n, w in lin.items():
        rtn, _, _, _ = OQ.fake_quantize(w.numpy(), None, None, None, bits=2, group_size=32, mode="asym")
        assert np.array_equal(wq[n].float().numpy(), rtn)


@pytest.mark.parametrize("bits", [2, 4])
def test_tuning_learns_and_is_deterministic(bits):
    lin, biases, norms, inputs, targets, scheme = _tiny_problem(bits=bits)
    run = lambda: OB.tune_block(inputs, targets, lin, biases, norms, TINY, scheme, iters=40,
                                lr=1.0 / 40, suppress=bits < 4)
    a = run()
    assert not a["reverted"]
    assert a["final_loss"] < 0.95 * a["initial_loss"], (a["initial_loss"], a["final_loss"])
    b = run()
    assert a["losses"] == b["losses"]
    assert all(torch.equal(x, y) for n in a["params"] for x, y in zip(a["params"][n], b["params"][n]))


def test_no_improvement_reverts_to_round_to_nearest():
    lin, biases, norms, inputs, targets, scheme = _tiny_problem()
    res = OB.tune_block(inputs, targets, lin, biases, norms, TINY, scheme, iters=0, lr=0.0,
                        suppress=True)
    assert res["reverted"] and res["final_loss"] == res["initial_loss"]
    init = OB.init_params(lin, scheme)
    assert all(torch.equal(x, y) for n in init for x, y in zip(init[n], res["params"][n]))


def test_step_gradient_matches_finite_difference_of_surrogate():
    """dL/dalpha of one layer against a central difference of the loss through the
    straight-through surrogate W'(alpha) with the codes held fixed."""
    lin, biases, norms, inputs, targets, scheme = _tiny_problem(bits=4)
    params = OB.init_params(lin, scheme)
    name = "mlp.up_proj"
    loss, grads = OB.step_grads(inputs[0], targets[0], lin, biases, norms, params, TINY, scheme,
                                suppress=False)
    w = lin[name].double().numpy()
    rows, cols = w.shape
    gs = scheme.group_size
    grouped = w.reshape(rows, -1, gs)
    wmax = np.maximum(grouped.max(-1, keepdims=True), 0)
    wmin = np.minimum(grouped.min(-1, keepdims=True), 0)
    q_hi = 2**scheme.bits - 1
    _, codes, _, zp = OQ.fake_quantize(w.astype(np.float32), None, None, None, bits=4, group_size=gs,
                                       mode="asym")
    codes = codes.reshape(grouped.shape).astype(np.float64)
    zp = zp.reshape(rows, -1, 1).astype(np.float64)

    s0 = (wmax - wmin) / q_hi
    raw = np.rint(grouped / s0) + zp
    inside = (raw >= 0) & (raw <= q_hi)
    rtn = OB.quantized_linears(lin, params, scheme)

    def surrogate_loss(alpha):
        # The straight-through surrogate at v = 0 with the codes frozen: inside
        # the clamp the code follows W/s, outside the zero point follows -wmin/s.
        s = (wmax * alpha - wmin) / q_hi
        qdq = s * (codes - zp) + np.where(inside, grouped - s * grouped / s0, wmin - s * wmin / s0)
        wq = dict(rtn)
        wq[name] = torch.from_numpy(qdq.reshape(rows, cols))
        out = OB.block_forward(inputs[0].double(), wq, biases, norms, TINY)
        return OB.batch_loss(out, targets[0].double(), False)[0]

    r, gidx = 3, 1
    h = 1e-6
    alpha_p = np.ones_like(wmax)
    alpha_m = np.ones_like(wmax)
    alpha_p[r, gidx] += h
    alpha_m[r, gidx] -= h
    fd = (surrogate_loss(alpha_p) - surrogate_loss(alpha_m)) / (2 * h)
    got = float(grads[name][1][r, gidx])
    assert abs(got - fd) <= 1e-3 * abs(fd) + 1e-9, (got, fd)
