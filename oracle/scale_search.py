"""The v2 candidate-scale grid search (oracle; test infrastructure only).

Restates ``mround/reference/scale_search.py:57-211`` (the reference's NumPy
oracle) and, in float32 with a sequential sum over each group, the
arithmetic the GPU kernel performs. Symmetric schemes only.

Per group: the anchor maps the signed largest-magnitude element onto
``-nmax`` (``nmax = 2^(b-1)``); candidate ``i`` in ``[-half, half] \\ {0}``
replaces ``nmax`` by ``nmax - step * i``; for each, ``inverse = -eff / gmax``,
``codes = clip(rne(inverse * w), -nmax, nmax - 1)``, ``scale = 1 / inverse``
(0 for 0), loss ``sum((scale * codes - w)^2 * importance)``. The anchor is
evaluated first, candidates from the widest range to the narrowest, and a
candidate replaces the best only with a strictly lower loss.

Grid: 2 bits -> step 0.01, half 90 (180 candidates); otherwise
``span = nmax * ratio`` (ratio 0.75), ``step = span / 200 * 2``,
``half = int(span / step)``.

Pinned by the reference's grid table (``tests/unit/test_scale_search.py:54-67``),
a brute-force per-group minimum over the same candidates, and the all-zero
group and anchor-tie rules (tests/test_oracle_scale_search.py).
"""

from __future__ import annotations

import numpy as np

TWO_BIT_HALF_COUNT = 90
TWO_BIT_STEP = 0.01
GRID = 200


def grid_steps(bits: int, ratio: float = 0.75) -> tuple[float, int]:
    """``(step, half_count)`` (``mround/reference/scale_search.py:84-100``)."""
    if bits == 2:
        return TWO_BIT_STEP, TWO_BIT_HALF_COUNT
    nmax = float(2 ** (bits - 1))
    span = nmax * ratio
    step = span / GRID * 2
    return step, int(span / step)


def candidates(bits: int, ratio: float = 0.75) -> list[float]:
    """Effective ranges in evaluation order, anchor first (float64)."""
    nmax = float(2 ** (bits - 1))
    step, half = grid_steps(bits, ratio)
    return [nmax] + [nmax - step * i for i in range(-half, half + 1) if i != 0]


def _reciprocal(x):
    out = np.zeros_like(x)
    np.divide(np.asarray(1.0, dtype=x.dtype), x, out=out, where=x != 0)
    return out


def _anchor(grouped):
    idx = np.argmax(np.abs(grouped), axis=-1)[:, None]
    return np.take_along_axis(grouped, idx, axis=-1)


def search_scales(weight, bits: int, group_size: int, *, importance=None, ratio: float = 0.75):
    """float64, vectorized sums: the reference oracle. Returns ``(n_groups, 1)``."""
    w = np.asarray(weight, dtype=np.float64)
    if w.ndim != 2 or w.shape[1] % group_size:
        raise ValueError("search expects a 2-D weight whose last dimension is a multiple of group_size")
    grouped = w.reshape(-1, group_size)
    nmax = float(2 ** (bits - 1))
    qw = None
    if importance is not None:
        qw = np.tile(np.asarray(importance, dtype=np.float64).reshape(-1), w.shape[0]).reshape(-1, group_size)
    gmax = _anchor(grouped)

    def evaluate(eff):
        inverse = -eff * _reciprocal(gmax)
        codes = np.clip(np.rint(inverse * grouped), -nmax, nmax - 1.0)
        scale = _reciprocal(inverse)
        r = (scale * codes - grouped) ** 2
        if qw is not None:
            r = r * qw
        return scale, r.sum(axis=-1, keepdims=True)

    cands = candidates(bits, ratio)
    best_s, best_l = evaluate(cands[0])
    for eff in cands[1:]:
        s, l = evaluate(eff)
        better = l < best_l
        best_s = np.where(better, s, best_s)
        best_l = np.where(better, l, best_l)
    return best_s


def search_scales_f32(weight, bits: int, group_size: int, *, importance=None, ratio: float = 0.75):
    """The kernel's arithmetic: float32, each group's loss summed element by
    element in column order, candidates rounded from float64 to float32."""
    w = np.asarray(weight, dtype=np.float32)
    grouped = w.reshape(-1, group_size)
    nmax = np.float32(2 ** (bits - 1))
    qw = None
    if importance is not None:
        qw = np.tile(np.asarray(importance, dtype=np.float32).reshape(-1), w.shape[0]).reshape(-1, group_size)
    gmax = _anchor(grouped)
    recip = _reciprocal(gmax)

    def evaluate(eff):
        inverse = np.float32(-eff) * recip
        codes = np.clip(np.rint(inverse * grouped), -nmax, nmax - np.float32(1.0))
        scale = _reciprocal(inverse)
        loss = np.zeros((grouped.shape[0], 1), dtype=np.float32)
        for j in range(group_size):
            r = scale[:, 0] * codes[:, j] - grouped[:, j]
            t = r * r
            if qw is not None:
                t = t * qw[:, j]
            loss[:, 0] = loss[:, 0] + t
        return scale, loss

    cands = [np.float32(c) for c in candidates(bits, ratio)]
    best_s, best_l = evaluate(cands[0])
    for eff in cands[1:]:
        s, l = evaluate(eff)
        better = l < best_l
        best_s = np.where(better, s, best_s)
        best_l = np.where(better, l, best_l)
    return best_s


def weighted_sse(weight, scale, bits: int, group_size: int, importance=None) -> np.ndarray:
    """Per-group reconstruction error of given scales (float64)."""
    grouped = np.asarray(weight, dtype=np.float64).reshape(-1, group_size)
    s = np.asarray(scale, dtype=np.float64).reshape(-1, 1)
    nmax = float(2 ** (bits - 1))
    codes = np.clip(np.rint(grouped * _reciprocal(s)), -nmax, nmax - 1.0)
    r = (s * codes - grouped) ** 2
    if importance is not None:
        r = r * np.tile(np.asarray(importance, dtype=np.float64).reshape(-1),
                        np.asarray(weight).shape[0]).reshape(-1, group_size)
    return r.sum(axis=-1)
