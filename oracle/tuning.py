"""Single-layer learned rounding on the CPU (oracle; test infrastructure only).

Restates ``mround/reference/tuning.py:85-201``: the layer loss of the weight
difference ``x (W' - W)^T`` against zero (``_layer_loss``, 91-115) and the
loop that measures before each update and keeps the best measured parameters
(``tune_layer``, 118-201), over this oracle's fake quantization, its
straight-through gradients and the sign step with linear decay (the outlier
rule by the MLX path's threshold, as the GPU loop has it). Pinned by the
reference's own tests of the loop (``tests/unit/test_reference_tuning.py``:
tuning reduces the error by more than 5 % at 2-4 bits, step 0 is round to
nearest, the best state is tracked, identical inputs give identical results),
restated in ``tests/test_oracle_tuning.py``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from oracle import losses as OL
from oracle import quantize as OQ
from oracle.optimizer import LinearDecay, resolved_lr


@dataclass
class LayerResult:
    v: np.ndarray
    alpha: np.ndarray
    beta: np.ndarray
    qdq: np.ndarray
    initial_loss: float
    final_loss: float
    losses: list
    best_step: int

    @property
    def improvement(self) -> float:
        return 0.0 if self.initial_loss <= 0.0 else 1.0 - self.final_loss / self.initial_loss


def layer_loss(activations, weight_q, weight, *, suppress: bool):
    """``(loss, dL/dW')`` of ``x (W' - W)^T`` against zero (reference/tuning.py:91-115)."""
    residual = activations @ (weight_q - weight).T
    zero = np.zeros_like(residual)
    if suppress:
        # the threshold rule of the MLX path (mround/core/losses.py:59-107)
        loss, grad_out, _ = OL.outlier_suppressed_loss(residual, zero, dtype=residual.dtype)
    else:
        loss, grad_out = OL.reconstruction_loss(residual, zero)
    return loss, grad_out.T @ activations


def tune_layer(weight, activations, *, bits: int, group_size: int, mode: str, iters: int = 200,
               lr: float | None = None, suppress: bool | None = None, eps: float = 1e-8,
               init_scale=None, dtype=np.float64) -> LayerResult:
    """reference/tuning.py:118-201 in ``dtype`` (float64 by default)."""
    weight = np.asarray(weight, dtype=dtype)
    activations = np.asarray(activations, dtype=dtype)
    if activations.shape[1] != weight.shape[1]:
        raise ValueError(f"activations have {activations.shape[1]} features but the weight "
                         f"expects {weight.shape[1]}")
    if suppress is None:
        suppress = bits < 4
    rows, cols = weight.shape
    v, alpha, beta = OQ.init_params(rows, cols, group_size, dtype=dtype)
    schedule = LinearDecay(resolved_lr(bits, iters, lr), iters)
    kw = dict(bits=bits, group_size=group_size, mode=mode, eps=eps, init_scale=init_scale, dtype=dtype)
    best_loss, best, best_step, losses = math.inf, (v, alpha, beta), 0, []
    for step in range(iters):
        qdq = OQ.fake_quantize(weight, v, alpha, beta, **kw)[0]
        loss, grad_w = layer_loss(activations, qdq, weight, suppress=suppress)
        losses.append(loss)
        if loss < best_loss:
            best_loss, best, best_step = loss, (v.copy(), alpha.copy(), beta.copy()), step
        gv, ga, gb = OQ.quantize_grad(weight, v, alpha, beta, grad_w, **kw)
        rate = schedule(step)
        v, alpha, beta = OQ.project_params(OQ.sign_step(v, gv, rate), OQ.sign_step(alpha, ga, rate),
                                           OQ.sign_step(beta, gb, rate), mode)
    qdq = OQ.fake_quantize(weight, *best, **kw)[0]
    return LayerResult(*best, qdq=qdq, initial_loss=losses[0], final_loss=best_loss, losses=losses,
                       best_step=best_step)
