"""Fake quantization, codes and straight-through gradients (oracle).

Restates ``mround/reference/quantize.py`` (regroup 115-153, extremes 156-165,
clamp_magnitude 168-178, symmetric_scale 181-222, asymmetric_scale 225-246,
fake_quantize 249-319, project_params 353-367, quantize_grad 399-522) with the
observed-range / searched split of ``mround/core/quantizer.py:287-398``.

``mode`` is ``"asym"``, ``"sym"`` or ``"searched"`` (symmetric, searched scale).
Arrays are grouped ``(rows, n_groups, group_size)``; per-group quantities are
``(rows, n_groups, 1)``. Passing ``v=None`` is the round-to-nearest path of
``mround/core/quantizer.py:269-284``: no perturbation is added, and the
coefficients are one.
"""

from __future__ import annotations

import numpy as np

V_BOUND = 0.5


def code_range(bits: int, mode: str) -> tuple[int, int]:
    """``mround/schemes.py:159-174``."""
    if mode == "asym":
        return 0, 2**bits - 1
    half = 2 ** (bits - 1)
    return -half, half - 1


def coefficient_bounds(mode: str) -> tuple[float, float]:
    """``mround/schemes.py:176-194``."""
    return (0.5, 1.5) if mode == "searched" else (0.1, 1.0)


def regroup(weight: np.ndarray, group_size: int) -> tuple[np.ndarray, int]:
    """``mround/reference/quantize.py:115-145``: zero padding to whole groups."""
    rows, cols = weight.shape
    if group_size == -1:
        return weight.reshape(rows, 1, cols), 0
    pad = (-cols) % group_size
    if pad:
        weight = np.concatenate([weight, np.zeros((rows, pad), dtype=weight.dtype)], axis=1)
    return weight.reshape(rows, -1, group_size), pad


def ungroup(grouped: np.ndarray, shape: tuple[int, int], pad: int) -> np.ndarray:
    """``mround/reference/quantize.py:148-153``."""
    flat = grouped.reshape(shape[0], -1)
    return flat[:, : shape[1]] if pad else flat


def _extremes(grouped, alpha, beta):
    """``mround/reference/quantize.py:156-165``: zero forced into the range."""
    w_max_raw = np.clip(grouped.max(axis=-1, keepdims=True), 0.0, None)
    w_min_raw = np.clip(grouped.min(axis=-1, keepdims=True), None, 0.0)
    return w_max_raw, w_min_raw, w_max_raw * alpha, w_min_raw * beta


def clamp_magnitude(scale, eps):
    """``mround/reference/quantize.py:168-178``: sign kept, zero counts as positive."""
    sign = np.sign(scale)
    sign = np.where(sign == 0.0, 1.0, sign).astype(scale.dtype)
    return sign * np.maximum(np.abs(scale), eps)


class Quantized:
    """Everything the forward computes, kept for the gradient."""

    __slots__ = ("codes", "inside", "pos_dom", "qdq_grouped", "scale", "w_max_raw",
                 "w_min", "w_min_raw", "zero_point", "base")


def _forward(grouped, v, alpha, beta, bits, mode, eps, init_scale):
    dt = grouped.dtype
    q_min, q_max = code_range(bits, mode)
    out = Quantized()
    if v is None:
        alpha = beta = np.ones((grouped.shape[0], grouped.shape[1], 1), dtype=dt)
    out.pos_dom = None
    out.zero_point = None
    out.base = None
    if mode == "searched":
        if init_scale is None:
            raise ValueError("a SEARCHED scheme needs the searched scale")
        base = np.asarray(init_scale, dtype=dt).reshape(grouped.shape[0], grouped.shape[1], 1)
        out.base = base
        scale = clamp_magnitude(base * beta, eps)
        out.w_max_raw = out.w_min_raw = out.w_min = None
    else:
        if init_scale is not None:
            raise ValueError("init_scale was given but the scheme's scale_init is not SEARCHED")
        w_max_raw, w_min_raw, w_max, w_min = _extremes(grouped, alpha, beta)
        out.w_max_raw, out.w_min_raw, out.w_min = w_max_raw, w_min_raw, w_min
        if mode == "sym":
            # mround/reference/quantize.py:211-222
            maxq = float(2 ** (bits - 1))
            pos_mag, neg_mag = w_max, -w_min
            pos_dom = pos_mag >= neg_mag
            dominant = np.where(pos_dom, pos_mag, neg_mag)
            signed = np.where(pos_dom, -dominant, dominant)
            scale = clamp_magnitude(signed / maxq, eps)
            out.pos_dom = pos_dom
        else:
            # mround/reference/quantize.py:242-246
            maxq = float(2**bits - 1)
            scale = np.maximum((w_max - w_min) / maxq, eps)
            out.zero_point = np.rint(-w_min / scale)
    pre = grouped / scale if v is None else grouped / scale + v
    raw = np.rint(pre)
    if out.zero_point is not None:
        raw = raw + out.zero_point
    out.inside = ((raw >= q_min) & (raw <= q_max)).astype(dt)
    out.codes = np.clip(raw, q_min, q_max)
    out.scale = scale
    if out.zero_point is None:
        out.qdq_grouped = scale * out.codes
    else:
        out.qdq_grouped = scale * (out.codes - out.zero_point)
    return out


def fake_quantize(weight, v, alpha, beta, *, bits, group_size, mode, eps=1e-8,
                  init_scale=None, dtype=np.float32):
    """``(qdq, codes, scale, zero_point)``; ``mround/reference/quantize.py:249-319``.

    ``weight`` is ``(rows, cols)``; ``v`` grouped or ``None`` (round to nearest).
    """
    w = np.asarray(weight, dtype=dtype)
    grouped, pad = regroup(w, group_size)
    if v is not None:
        v = np.asarray(v, dtype=dtype).reshape(grouped.shape)
        alpha = np.asarray(alpha, dtype=dtype).reshape(grouped.shape[0], grouped.shape[1], 1)
        beta = np.asarray(beta, dtype=dtype).reshape(grouped.shape[0], grouped.shape[1], 1)
    res = _forward(grouped, v, alpha, beta, bits, mode, dtype(eps), init_scale)
    return ungroup(res.qdq_grouped, w.shape, pad), res.codes, res.scale, res.zero_point


def quantize_grad(weight, v, alpha, beta, grad_qdq, *, bits, group_size, mode, eps=1e-8,
                  init_scale=None, dtype=np.float32):
    """``(grad_v, grad_alpha, grad_beta)``; ``mround/reference/quantize.py:370-522``."""
    w = np.asarray(weight, dtype=dtype)
    grouped, pad = regroup(w, group_size)
    v = np.asarray(v, dtype=dtype).reshape(grouped.shape)
    alpha = np.asarray(alpha, dtype=dtype).reshape(grouped.shape[0], grouped.shape[1], 1)
    beta = np.asarray(beta, dtype=dtype).reshape(grouped.shape[0], grouped.shape[1], 1)
    g = np.asarray(grad_qdq, dtype=dtype)
    if pad:
        g = np.concatenate([g, np.zeros((w.shape[0], pad), dtype=dtype)], axis=1)
    g = g.reshape(grouped.shape)
    r = _forward(grouped, v, alpha, beta, bits, mode, dtype(eps), init_scale)
    scale, inside, codes = r.scale, r.inside, r.codes

    grad_v = g * scale * inside
    if mode == "searched":
        # mround/reference/quantize.py:388-396
        d_qdq_d_scale = codes - inside * grouped / scale
        grad_scale = (g * d_qdq_d_scale).sum(axis=-1, keepdims=True)
        return grad_v, np.zeros_like(grad_scale), grad_scale * r.base
    if mode == "sym":
        # mround/reference/quantize.py:472-487
        d_qdq_d_scale = codes - inside * grouped / scale
        grad_scale = (g * d_qdq_d_scale).sum(axis=-1, keepdims=True)
        maxq = float(2 ** (bits - 1))
        d_alpha = np.where(r.pos_dom, -r.w_max_raw / maxq, 0.0).astype(dtype)
        d_beta = np.where(r.pos_dom, 0.0, -r.w_min_raw / maxq).astype(dtype)
        return grad_v, grad_scale * d_alpha, grad_scale * d_beta
    # asymmetric: mround/reference/quantize.py:494-520
    zp = r.zero_point
    d_zp_d_scale = r.w_min / (scale * scale)
    d_codes_d_scale = inside * (-grouped / (scale * scale) + d_zp_d_scale)
    d_qdq_d_scale = (codes - zp) + scale * (d_codes_d_scale - d_zp_d_scale)
    grad_scale = (g * d_qdq_d_scale).sum(axis=-1, keepdims=True)
    maxq = float(2**bits - 1)
    direct_beta = (g * (1.0 - inside) * r.w_min_raw).sum(axis=-1, keepdims=True)
    grad_alpha = grad_scale * (r.w_max_raw / maxq)
    grad_beta = grad_scale * (-r.w_min_raw / maxq) + direct_beta
    return grad_v, grad_alpha, grad_beta


def grad_terms(weight, v, alpha, beta, grad_qdq, *, bits, group_size, mode, eps=1e-8,
               init_scale=None, dtype=np.float32):
    """The per-element summands of ``grad_scale`` and of the direct beta term.

    Returned so that a test can bound the summation-order error of a per-group
    sum computed in another order (``sum |term|`` is the error scale).
    """
    w = np.asarray(weight, dtype=dtype)
    grouped, pad = regroup(w, group_size)
    v = np.asarray(v, dtype=dtype).reshape(grouped.shape)
    alpha = np.asarray(alpha, dtype=dtype).reshape(grouped.shape[0], grouped.shape[1], 1)
    beta = np.asarray(beta, dtype=dtype).reshape(grouped.shape[0], grouped.shape[1], 1)
    g = np.asarray(grad_qdq, dtype=dtype)
    if pad:
        g = np.concatenate([g, np.zeros((w.shape[0], pad), dtype=dtype)], axis=1)
    g = g.reshape(grouped.shape)
    r = _forward(grouped, v, alpha, beta, bits, mode, dtype(eps), init_scale)
    if mode == "asym":
        ss = r.scale * r.scale
        d_zp = r.w_min / ss
        dq = (r.codes - r.zero_point) + r.scale * (r.inside * (-grouped / ss + d_zp) - d_zp)
        return g * dq, g * (1.0 - r.inside) * r.w_min_raw
    dq = r.codes - r.inside * grouped / r.scale
    return g * dq, np.zeros_like(g)


def init_params(rows: int, cols: int, group_size: int, dtype=np.float32):
    """``mround/reference/quantize.py:335-350``: v = 0, alpha = beta = 1."""
    gs = cols if group_size == -1 else group_size
    ng = 1 if group_size == -1 else -(-cols // group_size)
    return (np.zeros((rows, ng, gs), dtype=dtype), np.ones((rows, ng, 1), dtype=dtype),
            np.ones((rows, ng, 1), dtype=dtype))


def project_params(v, alpha, beta, mode):
    """``mround/reference/quantize.py:353-367`` (returns new arrays)."""
    lo, hi = coefficient_bounds(mode)
    return np.clip(v, -V_BOUND, V_BOUND), np.clip(alpha, lo, hi), np.clip(beta, lo, hi)


def sign_step(param, grad, lr):
    """``mround/core/signsgd.py:76-85``: ``param - lr * sign(grad)``."""
    return param - lr * np.sign(grad)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16, half to even, returning the 16-bit patterns."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    rounded = np.where(nan, (u >> 16) | 0x40, rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))
