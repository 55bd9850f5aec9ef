"""Block reconstruction losses with their gradients (oracle).

Two selection rules for the outlier loss exist in the reference and both are
restated:

* ``outlier_threshold`` / ``outlier_suppressed_loss``: the block path's rule
  (``mround/core/losses.py:59-107``). The threshold is the k-th largest
  ``|r|`` (``sort(|r|)[n - k]``) and an element is kept when strictly below it,
  so ties at the threshold are all excluded.
* ``outlier_suppressed_loss_exact_k``: the NumPy oracle's rule
  (``mround/reference/losses.py:229-276``), exactly k elements excluded.

The denominator is the full element count (or ``elements`` for a piece,
``mround/core/losses.py:110-130``); the gradient is ``2 r keep / n``.
"""

from __future__ import annotations

import numpy as np

OUTLIER_FRACTION = 0.001


def outlier_k(n: int, fraction: float = OUTLIER_FRACTION) -> int:
    """``k = max(1, int(n * fraction))`` (``mround/core/losses.py:96-107``)."""
    return max(1, int(n * fraction))


def reconstruction_loss(predicted, reference, dtype=np.float64):
    """``mround/reference/losses.py:199-226``: ``(loss, dL/dpredicted)``."""
    r = np.asarray(predicted, dtype=dtype) - np.asarray(reference, dtype=dtype)
    n = r.size
    return float(np.sum(r.astype(np.float64) ** 2) / n), (2.0 * r / n).astype(dtype)


def outlier_threshold(residual, fraction: float = OUTLIER_FRACTION):
    """k-th largest ``|r|`` of the flattened residual (``mround/core/losses.py:96-107``)."""
    flat = np.abs(np.asarray(residual)).reshape(-1)
    n = flat.size
    k = outlier_k(n, fraction)
    return np.sort(flat)[n - k]


def outlier_suppressed_loss(predicted, reference, *, fraction: float = OUTLIER_FRACTION,
                            elements: int | None = None, threshold=None, dtype=np.float32):
    """Threshold rule, ``(loss, grad, threshold)``; ``mround/core/losses.py:59-93``."""
    r = np.asarray(predicted, dtype=dtype) - np.asarray(reference, dtype=dtype)
    n = r.size if elements is None else elements
    thr = outlier_threshold(r, fraction) if threshold is None else threshold
    keep = (np.abs(r) < thr).astype(dtype)
    kept = r * keep
    loss = float(np.sum(kept.astype(np.float64) ** 2) / n)
    grad = (2.0 * kept / n).astype(dtype)
    return loss, grad, thr


def outlier_suppressed_loss_exact_k(predicted, reference, *, fraction: float = OUTLIER_FRACTION):
    """Exactly-k rule of ``mround/reference/losses.py:229-276``, float64."""
    r = np.asarray(predicted, dtype=np.float64) - np.asarray(reference, dtype=np.float64)
    n = r.size
    k = outlier_k(n, fraction)
    flat = np.abs(r).reshape(-1)
    if k >= n:
        keep = np.zeros(n, dtype=bool)
    else:
        keep = np.ones(n, dtype=bool)
        keep[np.argpartition(flat, n - k)[n - k:]] = False
    mask = keep.reshape(r.shape).astype(np.float64)
    kept = r * mask
    return float(np.sum(kept**2) / n), 2.0 * kept * mask / n


def piece_loss(predicted, reference, *, elements: int, threshold=None, dtype=np.float32):
    """``mround/core/losses.py:110-130``: a piece's share of the batch loss."""
    r = np.asarray(predicted, dtype=dtype) - np.asarray(reference, dtype=dtype)
    if threshold is not None:
        r = r * (np.abs(r) < threshold).astype(dtype)
    return float(np.sum(r.astype(np.float64) ** 2) / elements), (2.0 * r / elements).astype(dtype)
