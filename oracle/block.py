"""float64 CPU decoder block and block-tuning loop (oracle; test infrastructure only).

The block is the one the reference runs through ``block_output``
(``mround/pipeline/blocks.py:578-606``): an mlx-lm 0.31.3 ``qwen2`` / ``llama``
decoder layer. mlx-lm is a third-party dependency absent here; its published
algorithm is restated:

    x1 = rms_norm(x, w_in, eps)                 mx.fast.rms_norm
    q, k, v = x1 Wq^T (+bq), x1 Wk^T (+bk), x1 Wv^T (+bv)
    q, k = rope(q), rope(k)                     mx.fast.rope(traditional=False, base=theta)
    o = softmax(q k^T / sqrt(d) + causal) v     mx.fast.scaled_dot_product_attention,
                                                grouped-query (head h reads kv head h // G)
    h = x + o Wo^T
    out = h + (silu(x2 Wg^T) * (x2 Wu^T)) Wd^T  with x2 = rms_norm(h, w_post, eps)

``tune_block`` restates ``QuantizationRunner._tune`` (``mround/pipeline/runner.py:790-953``):
score every batch with the initial parameters, ``iters`` sign-SGD steps on
cycled batches with the linearly decaying rate, projection after each step,
score again, keep the last parameters unless the score did not improve
(then the initial ones, i.e. round to nearest). Fake quantization and its
straight-through gradient come from ``oracle.quantize`` (float32, the
reference's arithmetic); everything else is float64 autograd.

Pinned by: a cross-check against the Hugging Face ``Qwen2DecoderLayer`` /
``LlamaDecoderLayer`` (same architecture as mlx-lm's), finite differences of
the block loss with respect to a weight, and the reference's property tests
for the tuning loop (initial parameters reproduce round to nearest, learning
happens, the revert rule, determinism).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from oracle import losses as OL
from oracle import quantize as OQ

# The block's linears in the order the reference walks them
# (sorted(named_modules()), mround/pipeline/blocks.py:654-678).
LAYERS = ("mlp.down_proj", "mlp.gate_proj", "mlp.up_proj", "self_attn.k_proj",
          "self_attn.o_proj", "self_attn.q_proj", "self_attn.v_proj")


@dataclass(frozen=True)
class Shape:
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    intermediate: int
    norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    attn_bias: bool = False

    def linear_shape(self, name: str) -> tuple[int, int]:
        h, d = self.hidden, self.head_dim
        return {
            "self_attn.q_proj": (self.n_heads * d, h),
            "self_attn.k_proj": (self.n_kv_heads * d, h),
            "self_attn.v_proj": (self.n_kv_heads * d, h),
            "self_attn.o_proj": (h, self.n_heads * d),
            "mlp.gate_proj": (self.intermediate, h),
            "mlp.up_proj": (self.intermediate, h),
            "mlp.down_proj": (h, self.intermediate),
        }[name]


def rope_cos_sin(seq_len: int, head_dim: int, theta: float):
    """cos and sin of ``pos * theta^(-2i/d)``, ``[S, d/2]`` float64."""
    inv = theta ** (-torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim)
    ang = torch.arange(seq_len, dtype=torch.float64)[:, None] * inv[None, :]
    return torch.cos(ang), torch.sin(ang)


def rms_norm(x, w, eps):
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w


def rope(x, cos, sin):
    """Halves layout (``traditional=False``): x is ``[B, H, S, d]``."""
    half = x.shape[-1] // 2
    a, b = x[..., :half], x[..., half:]
    return torch.cat([a * cos - b * sin, b * cos + a * sin], -1)


def block_forward(x, linears, biases, norms, shape: Shape):
    """``x`` ``[B, S, h]``; ``linears[name]`` ``[out, in]``; ``biases`` for q/k/v
    (or empty); ``norms = (w_in, w_post)``. Returns ``[B, S, h]`` in x's dtype."""
    B, S, _ = x.shape
    d, hq, hkv = shape.head_dim, shape.n_heads, shape.n_kv_heads
    x1 = rms_norm(x, norms[0], shape.norm_eps)

    def proj(name, inp):
        y = inp @ linears[name].transpose(0, 1)
        return y + biases[name] if name in biases else y

    q = proj("self_attn.q_proj", x1).reshape(B, S, hq, d).transpose(1, 2)
    k = proj("self_attn.k_proj", x1).reshape(B, S, hkv, d).transpose(1, 2)
    v = proj("self_attn.v_proj", x1).reshape(B, S, hkv, d).transpose(1, 2)
    cos, sin = rope_cos_sin(S, d, shape.rope_theta)
    cos, sin = cos.to(x.dtype), sin.to(x.dtype)
    q, k = rope(q, cos, sin), rope(k, cos, sin)
    g = hq // hkv
    k = k.repeat_interleave(g, 1)
    v = v.repeat_interleave(g, 1)
    s = (q @ k.transpose(-1, -2)) * (d ** -0.5)
    causal = torch.ones(S, S, dtype=torch.bool).tril()
    s = s.masked_fill(~causal, float("-inf"))
    o = torch.softmax(s, -1) @ v
    o = o.transpose(1, 2).reshape(B, S, hq * d)
    h = x + proj("self_attn.o_proj", o)
    x2 = rms_norm(h, norms[1], shape.norm_eps)
    act = torch.nn.functional.silu(proj("mlp.gate_proj", x2)) * proj("mlp.up_proj", x2)
    return h + proj("mlp.down_proj", act)


# ------------------------------------------------------------------ tuning --

@dataclass(frozen=True)
class Scheme:
    bits: int
    group_size: int
    mode: str = "asym"


class _FakeQuant(torch.autograd.Function):
    """W' = fake_quantize(W; v, alpha, beta) with the reference's straight-through
    gradient for (v, alpha, beta) (``mround/reference/quantize.py:249-522``)."""

    @staticmethod
    def forward(ctx, v, alpha, beta, weight_np, scheme, eps):
        qdq, _, _, _ = OQ.fake_quantize(weight_np, v.numpy(), alpha.numpy(), beta.numpy(),
                                        bits=scheme.bits, group_size=scheme.group_size,
                                        mode=scheme.mode, eps=eps, dtype=np.float32)
        ctx.save_for_backward(v, alpha, beta)
        ctx.weight_np, ctx.scheme, ctx.eps = weight_np, scheme, eps
        return torch.from_numpy(np.ascontiguousarray(qdq)).double()

    @staticmethod
    def backward(ctx, grad):
        v, alpha, beta = ctx.saved_tensors
        s = ctx.scheme
        gv, ga, gb = OQ.quantize_grad(ctx.weight_np, v.numpy(), alpha.numpy(), beta.numpy(),
                                      grad.float().numpy(), bits=s.bits, group_size=s.group_size,
                                      mode=s.mode, eps=ctx.eps, dtype=np.float32)
        as_t = lambda a, like: torch.from_numpy(np.ascontiguousarray(a)).reshape(like.shape)
        return as_t(gv, v), as_t(ga, alpha), as_t(gb, beta), None, None, None


def init_params(weights, scheme: Scheme):
    """v = 0, alpha = beta = 1 per layer (``mround/reference/quantize.py:335-350``):
    ``(v [rows, cols], alpha [rows, groups], beta [rows, groups])`` float32."""
    out = {}
    for name, w in weights.items():
        rows, cols = w.shape
        v, a, b = OQ.init_params(rows, cols, scheme.group_size)
        out[name] = (torch.from_numpy(v.reshape(rows, -1)[:, :cols].copy()),
                     torch.from_numpy(a.reshape(rows, -1).copy()),
                     torch.from_numpy(b.reshape(rows, -1).copy()))
    return out


def quantized_linears(weights, params, scheme: Scheme, eps=1e-8, *, differentiable=False):
    """The block's W' for the given parameters (float64 tensors)."""
    out = {}
    for name, w in weights.items():
        w_np = w.float().numpy()
        v, a, b = params[name]
        if differentiable:
            out[name] = _FakeQuant.apply(v, a, b, w_np, scheme, eps)
        else:
            qdq, _, _, _ = OQ.fake_quantize(w_np, v.numpy(), a.numpy(), b.numpy(), bits=scheme.bits,
                                            group_size=scheme.group_size, mode=scheme.mode, eps=eps)
            out[name] = torch.from_numpy(np.ascontiguousarray(qdq)).double()
    return out


def batch_loss(pred, target, suppress: bool):
    """(loss, dL/dpred) by the block path's rule (``mround/core/losses.py:42-107``)."""
    if suppress:
        loss, grad, _ = OL.outlier_suppressed_loss(pred.numpy(), target.numpy(), dtype=np.float64)
    else:
        loss, grad = OL.reconstruction_loss(pred.numpy(), target.numpy())
    return loss, torch.from_numpy(np.asarray(grad, dtype=np.float64))


def step_grads(x, target, weights, biases, norms, params, shape, scheme, suppress, eps=1e-8):
    """Loss of one batch and its gradient for every layer's (v, alpha, beta)."""
    leaf = {n: tuple(t.clone().requires_grad_(True) for t in p) for n, p in params.items()}
    wq = quantized_linears(weights, leaf, scheme, eps, differentiable=True)
    out = block_forward(x.double(), wq, biases, norms, shape)
    loss, dpred = batch_loss(out.detach(), target.double(), suppress)
    out.backward(dpred)
    return loss, {n: tuple(t.grad for t in p) for n, p in leaf.items()}


def mean_loss(inputs, targets, weights, biases, norms, params, shape, scheme, suppress, eps=1e-8):
    wq = quantized_linears(weights, params, scheme, eps)
    losses = [batch_loss(block_forward(x.double(), wq, biases, norms, shape), t.double(), suppress)[0]
              for x, t in zip(inputs, targets)]
    return sum(losses) / len(losses)


def tune_block(inputs, targets, weights, biases, norms, shape: Shape, scheme: Scheme, *, iters: int,
               lr: float, suppress: bool, eps: float = 1e-8, steps: int | None = None):
    """``QuantizationRunner._tune`` (``mround/pipeline/runner.py:790-953``) without holdout.
    ``steps`` stops after that many steps of the ``iters``-step schedule (the
    final score and the revert rule then apply to the parameters reached)."""
    params = init_params(weights, scheme)
    start = {n: tuple(t.clone() for t in p) for n, p in params.items()}
    initial = mean_loss(inputs, targets, weights, biases, norms, start, shape, scheme, suppress, eps)
    losses = []
    for step in range(iters if steps is None else min(steps, iters)):
        b = step % len(inputs)
        loss, grads = step_grads(inputs[b], targets[b], weights, biases, norms, params, shape,
                                 scheme, suppress, eps)
        losses.append(loss)
        rate = lr * (1.0 - step / iters)  # LinearDecay, mround/core/signsgd.py:23-40
        new = {}
        for n, p in params.items():
            stepped = [OQ.sign_step(t.numpy(), g.numpy().astype(np.float32), rate)
                       for t, g in zip(p, grads[n])]
            new[n] = tuple(torch.from_numpy(np.ascontiguousarray(t))
                           for t in OQ.project_params(*stepped, scheme.mode))
        params = new
    final = mean_loss(inputs, targets, weights, biases, norms, params, shape, scheme, suppress, eps)
    if final >= initial:
        return {"initial_loss": initial, "final_loss": initial, "losses": losses, "params": start,
                "reverted": True}
    return {"initial_loss": initial, "final_loss": final, "losses": losses, "params": params,
            "reverted": False}
