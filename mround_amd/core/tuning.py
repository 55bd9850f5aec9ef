"""Learned rounding of a single linear layer on the GPU
(``mround/core/tuning.py:63-202``).

The reference's smallest unit of the method: one weight, calibration inputs
for it, and the loop that measures the layer error before each update and
keeps the best measured parameters (the block loop keeps the last ones and
reverts instead). The layer error is the product of the inputs with the
weight *difference*, ``x (W' - W)^T`` against zero, as the reference forms
it: the residual then carries only its own rounding, not that of two large
products subtracted.

Per step: W' by the fake-quant kernel (fp32), the residual and dL/dW' as two
fp32 MFMA GEMMs (``mr_gemm_f32``: ``x (W' - W)^T``, the difference formed as
the operand is loaded, and ``(dL/dr)^T x``, any shape), the loss and dL/dr
by the loss kernels (the outlier rule's threshold on the device), and the
straight-through gradient, sign step and projection in one fused kernel on
``v``, ``alpha`` and ``beta`` in place. The loss is read back once per step,
as the reference evaluates once per step.

Portions follow MRound (Copyright 2026 The MRound Authors, Apache License 2.0);
see NOTICE.
"""

from __future__ import annotations

import dataclasses
import math
from collections.abc import Mapping

import torch

from mround_amd import kernels as K
from mround_amd.core.losses import OUTLIER_FRACTION
from mround_amd.core.quantizer import Params, fake_quantize, init_params
from mround_amd.core.signsgd import LinearDecay, fused_step
from mround_amd.schemes import DEFAULT_EPS_FP32, QuantScheme, TuningConfig

__all__ = ["TuningResult", "round_to_nearest", "tune_layer"]


@dataclasses.dataclass(frozen=True)
class TuningResult:
    """What tuning a single layer achieved (``mround/core/tuning.py:63-89``).

    ``losses[i]`` is measured before update ``i``, so ``losses[0]`` is the
    round-to-nearest error and the parameters left by the final update are
    never measured; ``params`` are those of ``best_step``."""

    params: Params
    qdq: torch.Tensor
    initial_loss: float
    final_loss: float
    losses: list[float]
    best_step: int

    @property
    def improvement(self) -> float:
        """Fractional loss reduction against round to nearest."""
        if self.initial_loss <= 0.0:
            return 0.0
        return 1.0 - (self.final_loss / self.initial_loss)


def round_to_nearest(weight: torch.Tensor, scheme: QuantScheme, *, eps: float = DEFAULT_EPS_FP32,
                     init_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Quantize with no learning (``mround/core/tuning.py:92-102``)."""
    return fake_quantize(weight, init_params(weight, scheme), scheme, eps=eps, init_scale=init_scale)


def tune_layer(weight: torch.Tensor, activations: torch.Tensor, scheme: QuantScheme,
               config: TuningConfig | None = None, *, eps: float = DEFAULT_EPS_FP32,
               init_scale: torch.Tensor | None = None) -> TuningResult:
    """Learn the rounding for one linear layer (``mround/core/tuning.py:105-202``).

    Args:
        weight: ``(out_features, in_features)`` on the device.
        activations: Calibration inputs ``(n_samples, in_features)``.
        scheme: Target representation.
        config: Tuning hyperparameters; ``None`` uses the standard recipe.
        eps: Scale epsilon.
        init_scale: The searched per-group scale of a ``SEARCHED`` scheme.

    Raises:
        ValueError: If the activation width does not match the weight.
    """
    if activations.shape[1] != weight.shape[1]:
        msg = (
            f"activations have {activations.shape[1]} features but the weight "
            f"expects {weight.shape[1]}"
        )
        raise ValueError(msg)
    config = config or TuningConfig()
    suppress = config.resolved_suppress_outliers(scheme.bits)
    dev = weight.device
    x = activations.to(device=dev, dtype=torch.float32).contiguous()
    w32 = weight.to(torch.float32).contiguous()
    rows, cols = weight.shape
    n = x.shape[0]
    elements = n * rows
    params = init_params(weight, scheme)
    schedule = LinearDecay(config.resolved_lr(scheme.bits), config.iters)
    qdq = torch.empty(rows, cols, dtype=torch.float32, device=dev)
    residual = torch.empty(n, rows, dtype=torch.float32, device=dev)
    zero = torch.zeros_like(residual)
    grad_r = torch.empty_like(residual)
    grad_w = torch.empty(rows, cols, dtype=torch.float32, device=dev)
    loss_val = torch.empty(1, dtype=torch.float32, device=dev)
    threshold = torch.empty(1, dtype=torch.float32, device=dev)
    ws = K.loss_workspace(dev, elements)
    k = max(1, int(elements * OUTLIER_FRACTION))

    best_loss, best_params, best_step = math.inf, _copy(params), 0
    losses: list[float] = []
    for step in range(config.iters):
        fake_quantize(weight, params, scheme, eps=eps, init_scale=init_scale, out=qdq)
        K.gemm_f32("nt", x, qdq, residual, M=n, N=rows, K=cols, b_minus=w32)
        if suppress:
            K.loss_outlier(residual, zero, k=k, denom=elements, loss_out=loss_val, threshold_out=threshold,
                           grad_out=grad_r, workspace=ws)
        else:
            K.loss_mse(residual, zero, denom=elements, loss_out=loss_val, grad_out=grad_r, workspace=ws)
        K.gemm_f32("tn", grad_r, x, grad_w, M=rows, N=cols, K=n)
        value = float(loss_val)
        losses.append(value)
        if value < best_loss:
            best_loss, best_params, best_step = value, _copy(params), step
        fused_step(weight, params, grad_w, scheme, schedule(step), eps=eps, init_scale=init_scale)
    final = fake_quantize(weight, best_params, scheme, eps=eps, init_scale=init_scale)
    return TuningResult(params=best_params, qdq=final, initial_loss=losses[0], final_loss=best_loss,
                        losses=losses, best_step=best_step)


def _copy(params: Mapping[str, torch.Tensor]) -> Params:
    return {name: t.clone() for name, t in params.items()}
