"""float64 CPU causal LM and whole-model DeltaLoss scoring (oracle; test
infrastructure only).

Restates the reference's scoring pass (``mround/pipeline/scoring.py``):

* ``causal_loss`` -- ``_causal_loss`` (scoring.py:183-192): logits of the
  model on ``tokens[:, :-1]``, mean cross-entropy against ``tokens[:, 1:]``;
  the model is an mlx-lm Qwen2 / Llama decoder (embedding, the blocks of
  ``oracle.block.block_forward``, final RMSNorm, tied or untied head);
* ``layer_gradients`` -- the cotangents of the block linears' weights
  (scoring.py:507-514), by float64 autograd, at whatever weights are given;
* ``score_widths`` -- the two schedules, ``own_width`` (scoring.py:269-315)
  and ``widest`` (scoring.py:318-365): each width's perturbation is the
  float32 round-to-nearest reconstruction (``oracle.quantize``, the searched
  grid where given) less the float32 weight, and each batch adds
  ``sum |g * perturbation|`` per layer (scoring.py:238-266).

The oracle runs the unpadded ``seq_len - 1`` positions and each batch at its
own size, so padding in the GPU path is checked rather than mirrored.

Pinned by: the Hugging Face ``Qwen2ForCausalLM`` / ``LlamaForCausalLM``
(transformers) loss and weight gradients at the same float64 weights, and, at
the widest width, the equality of the two schedules (the reference's own
invariant, scoring.py:465-470).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from oracle.block import LAYERS, Shape, block_forward, rms_norm
from oracle.quantize import fake_quantize


@dataclass
class Model:
    """A decoder model in float64 on the CPU. ``blocks[i]`` is ``(name,
    linears, biases, (w_in, w_post))``; ``head`` None means tied."""

    shape: Shape
    embed: torch.Tensor
    blocks: list = field(default_factory=list)
    norm: torch.Tensor | None = None
    head: torch.Tensor | None = None


def causal_loss(model: Model, tokens: torch.Tensor, linears: dict | None = None) -> torch.Tensor:
    """Mean shifted cross-entropy of ``tokens`` ``[B, S]``; ``linears[path]``
    replaces that block linear's weight."""
    linears = linears or {}
    ids, labels = tokens[:, :-1], tokens[:, 1:]
    x = model.embed[ids]
    for name, lin, biases, norms in model.blocks:
        w = {n: linears.get(f"{name}.{n}", lin[n]) for n in LAYERS}
        x = block_forward(x, w, biases, norms, model.shape)
    xn = rms_norm(x, model.norm, model.shape.norm_eps)
    head = model.embed if model.head is None else model.head
    logits = xn @ head.transpose(0, 1)
    return torch.nn.functional.cross_entropy(logits.reshape(-1, logits.shape[-1]), labels.reshape(-1))


def layer_gradients(model: Model, tokens: torch.Tensor, linears: dict[str, torch.Tensor]):
    """``(loss, {path: dL/dW})`` at the given block linear weights (float64)."""
    leaves = {p: w.detach().double().clone().requires_grad_(True) for p, w in linears.items()}
    loss = causal_loss(model, tokens, leaves)
    grads = torch.autograd.grad(loss, list(leaves.values()))
    return float(loss.detach()), dict(zip(leaves, grads))


def rtn(weight32: np.ndarray, *, bits: int, group_size: int, mode: str, eps: float = 1e-8,
        init_scale: np.ndarray | None = None) -> np.ndarray:
    """Round-to-nearest quantize-dequantize in float32 (scoring.py:213-221)."""
    q, _, _, _ = fake_quantize(weight32, None, None, None, bits=bits, group_size=group_size, mode=mode,
                               eps=eps, init_scale=init_scale, dtype=np.float32)
    return q


def score_widths(model: Model, batches, widths, *, group_size: int, mode: str, eps: float = 1e-8,
                 gradient_source: str = "own_width", grids: dict | None = None) -> dict[str, dict[int, float]]:
    """DeltaLoss per block-linear path and width. ``grids[width][path]`` is
    the searched scale grid (searched mode only)."""
    paths = [f"{name}.{n}" for name, *_ in model.blocks for n in LAYERS]
    w32 = {f"{name}.{n}": lin[n].numpy().astype(np.float32) for name, lin, *_ in model.blocks for n in LAYERS}
    order = sorted(int(b) for b in widths)

    def recon(width: int) -> dict[str, np.ndarray]:
        g = (grids or {}).get(width, {})
        return {p: rtn(w32[p], bits=width, group_size=group_size, mode=mode, eps=eps, init_scale=g.get(p))
                for p in paths}

    scores = {p: {} for p in paths}
    if gradient_source == "own_width":
        for width in order:
            q = recon(width)
            acc = dict.fromkeys(paths, 0.0)
            for tokens in batches:
                _, grads = layer_gradients(model, tokens, {p: torch.from_numpy(q[p]) for p in paths})
                for p in paths:
                    pert = (q[p] - w32[p]).astype(np.float64)
                    acc[p] += float(np.abs(grads[p].numpy() * pert).sum())
            for p in paths:
                scores[p][width] = acc[p]
    elif gradient_source == "widest":
        qs = {w: recon(w) for w in order}
        anchor = qs[order[-1]]
        acc = {p: dict.fromkeys(order, 0.0) for p in paths}
        for tokens in batches:
            _, grads = layer_gradients(model, tokens, {p: torch.from_numpy(anchor[p]) for p in paths})
            for p in paths:
                g = grads[p].numpy()
                for w in order:
                    pert = (qs[w][p] - w32[p]).astype(np.float64)
                    acc[p][w] += float(np.abs(g * pert).sum())
        scores = {p: dict(acc[p]) for p in paths}
    else:
        raise ValueError(f"unknown gradient_source {gradient_source!r}")
    return scores
