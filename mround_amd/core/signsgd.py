"""Signed gradient descent, and the fused backward + step of one layer.

``LinearDecay``, ``total_excursion``, ``sign_update`` and ``SignSGD`` mirror
``mround/core/signsgd.py:36-145``. :func:`fused_step` is the tuning path's
form: the straight-through backward of ``fake_quantize``, the sign step and
the projection of ``mround/core/quantizer.py:430-446`` in one HIP kernel that
reads W, v and dL/dW' once and writes v, alpha and beta in place.

Portions follow MRound (Copyright 2026 The MRound Authors, Apache License 2.0);
see NOTICE.
"""

from __future__ import annotations

from collections.abc import Mapping

import torch

from mround_amd import kernels as K
from mround_amd.core.quantizer import V_BOUND, _geometry, _init_scale_arg, _unpack, mode_of
from mround_amd.schemes import DEFAULT_EPS_FP32, QuantScheme

__all__ = ["LinearDecay", "SignSGD", "fused_step", "sign_update", "total_excursion"]


class LinearDecay:
    """``mround/core/signsgd.py:36-62``: falls linearly to exactly zero."""

    __slots__ = ("initial_lr", "total_steps")

    def __init__(self, initial_lr: float, total_steps: int) -> None:
        if total_steps <= 0:
            msg = f"total_steps must be positive, got {total_steps}"
            raise ValueError(msg)
        self.initial_lr = initial_lr
        self.total_steps = total_steps

    def __call__(self, step: int) -> float:
        if step >= self.total_steps:
            return 0.0
        return self.initial_lr * (1.0 - step / self.total_steps)


def total_excursion(initial_lr: float, total_steps: int) -> float:
    """``mround/core/signsgd.py:65-73``."""
    schedule = LinearDecay(initial_lr, total_steps)
    return sum(schedule(step) for step in range(total_steps))


def sign_update(param: torch.Tensor, grad: torch.Tensor, lr: float) -> torch.Tensor:
    """``mround/core/signsgd.py:76-85``: ``param - lr * sign(grad)``."""
    return param - lr * torch.sign(grad)


class SignSGD:
    """``mround/core/signsgd.py:88-145`` over a flat mapping of named tensors."""

    __slots__ = ("_buffers", "_step", "learning_rate", "momentum")

    def __init__(self, learning_rate: float | LinearDecay, *, momentum: float = 0.0) -> None:
        self.learning_rate = learning_rate
        self.momentum = momentum
        self._step = 0
        self._buffers: dict[str, torch.Tensor] = {}

    @property
    def step_count(self) -> int:
        return self._step

    def current_lr(self) -> float:
        if isinstance(self.learning_rate, LinearDecay):
            return self.learning_rate(self._step)
        return self.learning_rate

    def advance(self) -> float:
        """The rate for this step, then count the step (used by :func:`fused_step`)."""
        lr = self.current_lr()
        self._step += 1
        return lr

    def apply(self, params: Mapping[str, torch.Tensor], grads: Mapping[str, torch.Tensor]) -> dict:
        lr = self.current_lr()
        updated: dict[str, torch.Tensor] = {}
        for name, value in params.items():
            if name not in grads:
                msg = f"no gradient supplied for parameter {name!r}"
                raise KeyError(msg)
            grad = grads[name]
            if self.momentum:
                buf = self._buffers.get(name)
                buf = grad.clone() if buf is None else self.momentum * buf + grad
                self._buffers[name] = buf
                grad = buf
            updated[name] = sign_update(value, grad, lr)
        self._step += 1
        return updated


def fused_step(
    weight: torch.Tensor,
    params: Mapping[str, torch.Tensor],
    grad_qdq: torch.Tensor,
    scheme: QuantScheme,
    lr: float,
    *,
    eps: float = DEFAULT_EPS_FP32,
    init_scale: torch.Tensor | None = None,
) -> None:
    """Backward of ``fake_quantize`` + sign step + projection, in place.

    Equivalent to ``project_params(SignSGD.apply(params, quantize_grad(...)))``
    at momentum 0 with the same ``lr`` (``mround/pipeline/runner.py:926-931``),
    but the parameters are updated in place: the gradients are taken at the
    values on entry.
    """
    rows, _, gs, ng = _geometry(weight, scheme)
    v, alpha, beta = _unpack(params, rows, ng, gs)
    if v.data_ptr() != params["v"].data_ptr():
        raise ValueError("fused_step updates in place: params must be contiguous")
    lo, hi = scheme.coefficient_bounds
    K.fq_backward_signsgd(weight, v, alpha, beta, grad_qdq, bits=scheme.bits,
                          group_size=scheme.group_size, mode=mode_of(scheme), eps=eps, update=True,
                          lr=lr, coef_lo=lo, coef_hi=hi, v_bound=V_BOUND,
                          init_scale=_init_scale_arg(init_scale, rows, ng))
