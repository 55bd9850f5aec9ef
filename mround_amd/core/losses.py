"""Block reconstruction losses on MI355X (``mround/core/losses.py:42-130``).

Each loss returns the scalar as a 0-d float32 device tensor (no host sync) and,
with ``with_grad=True``, also ``dL/dpredicted`` -- the tuning loop needs the
gradient, and the kernel writes it in the same pass that forms the loss.

The outlier rule is the block path's: the threshold is the k-th largest
``|r|`` over the flattened batch, ``k = max(1, int(n * fraction))``, found
exactly on the device by radix select; an error is kept when strictly below
it, and the denominator stays the full element count.
"""

from __future__ import annotations

import torch

from mround_amd import kernels as K

__all__ = [
    "OUTLIER_FRACTION",
    "outlier_suppressed_loss",
    "outlier_threshold",
    "piece_loss",
    "reconstruction_loss",
]

OUTLIER_FRACTION: float = 0.001


def _prep(predicted: torch.Tensor, reference: torch.Tensor):
    if predicted.shape != reference.shape:
        msg = f"predicted {tuple(predicted.shape)} and reference {tuple(reference.shape)} differ"
        raise ValueError(msg)
    return (predicted.to(torch.float32).contiguous(), reference.to(torch.float32).contiguous())


def reconstruction_loss(predicted, reference, *, with_grad: bool = False):
    """``mean((pred - ref)^2)`` in float32 (``mround/core/losses.py:42-56``)."""
    p, r = _prep(predicted, reference)
    loss = torch.empty((), dtype=torch.float32, device=p.device)
    grad = torch.empty_like(p) if with_grad else None
    K.loss_mse(p, r, denom=p.numel(), loss_out=loss, grad_out=grad)
    return (loss, grad) if with_grad else loss


def outlier_threshold(residual: torch.Tensor, *, fraction: float = OUTLIER_FRACTION) -> torch.Tensor:
    """k-th largest ``|residual|`` (``mround/core/losses.py:96-107``), a 0-d tensor."""
    r = residual.to(torch.float32).contiguous()
    n = r.numel()
    k = max(1, int(n * fraction))
    zero = torch.zeros_like(r)
    thr = torch.empty((), dtype=torch.float32, device=r.device)
    loss = torch.empty((), dtype=torch.float32, device=r.device)
    K.loss_outlier(r, zero, k=k, denom=n, loss_out=loss, threshold_out=thr)
    return thr


def outlier_suppressed_loss(predicted, reference, *, fraction: float = OUTLIER_FRACTION,
                            with_grad: bool = False, threshold_out: torch.Tensor | None = None):
    """The outlier rule (``mround/core/losses.py:59-93``)."""
    p, r = _prep(predicted, reference)
    n = p.numel()
    k = max(1, int(n * fraction))
    loss = torch.empty((), dtype=torch.float32, device=p.device)
    thr = threshold_out if threshold_out is not None else torch.empty((), dtype=torch.float32,
                                                                       device=p.device)
    grad = torch.empty_like(p) if with_grad else None
    K.loss_outlier(p, r, k=k, denom=n, loss_out=loss, threshold_out=thr, grad_out=grad)
    return (loss, grad) if with_grad else loss


def piece_loss(predicted, reference, *, elements: int, threshold: torch.Tensor | None = None,
               with_grad: bool = False):
    """A piece's share of the whole batch's loss (``mround/core/losses.py:110-130``)."""
    p, r = _prep(predicted, reference)
    loss = torch.empty((), dtype=torch.float32, device=p.device)
    grad = torch.empty_like(p) if with_grad else None
    if threshold is None:
        K.loss_mse(p, r, denom=elements, loss_out=loss, grad_out=grad)
    else:
        thr = threshold.to(torch.float32).reshape(()).contiguous()
        K.loss_outlier(p, r, k=1, denom=elements, loss_out=loss, threshold_in=thr, grad_out=grad)
    return (loss, grad) if with_grad else loss
