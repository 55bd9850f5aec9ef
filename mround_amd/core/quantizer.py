"""Fake quantization on MI355X, behind the reference's operator signatures.

Mirrors ``mround/core/quantizer.py`` (lines 74-446): the same names, argument
meanings, shapes, validation and error types, with torch tensors on a ROCm
device in place of MLX arrays. The arithmetic runs in the HIP library
(``mr_fq_forward`` / ``mr_fq_backward_signsgd``): one pass over the weight
computes group extremes, scale, zero point, codes and reconstruction.

Layouts (as in the reference): ``params = {"v": (rows, n_groups, gs),
"alpha": (rows, n_groups, 1), "beta": (rows, n_groups, 1)}``, all float32;
codes are grouped ``(rows, n_groups, gs)``; scales and zero points are
``(rows, n_groups, 1)``. ``params=None`` is round-to-nearest.

Weights may be float32, bfloat16 or float16; they are widened to float32
exactly inside the kernel, which is what the reference's tuning path does
(``mround/pipeline/runner.py:337``). The reconstruction is returned in the
weight's dtype unless ``out_dtype`` says otherwise.
"""

from __future__ import annotations

from collections.abc import Mapping

import torch

from mround_amd import kernels as K
from mround_amd.exceptions import SchemeError
from mround_amd.schemes import DEFAULT_EPS_FP32, QuantScheme, ScaleInit, Symmetry

__all__ = [
    "MATRIX_NDIM",
    "V_BOUND",
    "dequantize",
    "fake_quantize",
    "init_params",
    "mode_of",
    "project_params",
    "quantize_codes",
    "quantize_grad",
    "regroup",
    "ungroup",
]

V_BOUND: float = 0.5
MATRIX_NDIM: int = 2

Params = dict[str, torch.Tensor]


def mode_of(scheme: QuantScheme) -> str:
    """The kernel mode of a scheme: ``asym``, ``sym`` or ``searched``."""
    if scheme.scale_init is ScaleInit.SEARCHED:
        return "searched"
    return "sym" if scheme.symmetry is Symmetry.SYMMETRIC else "asym"


def _check_weight(weight: torch.Tensor) -> None:
    if weight.ndim != MATRIX_NDIM:
        msg = f"expected a 2-D weight matrix, got shape {tuple(weight.shape)}"
        raise SchemeError(msg)


def _geometry(weight: torch.Tensor, scheme: QuantScheme) -> tuple[int, int, int, int]:
    rows, cols = weight.shape
    gs = cols if scheme.group_size == -1 else scheme.group_size
    ng = 1 if scheme.group_size == -1 else -(-cols // gs)
    return rows, cols, gs, ng


def regroup(weight: torch.Tensor, group_size: int) -> tuple[torch.Tensor, int]:
    """``mround/core/quantizer.py:152-174``: ``(rows, n_groups, gs)``, zero padded."""
    _check_weight(weight)
    rows, cols = weight.shape
    if group_size == -1:
        return weight.reshape(rows, 1, cols), 0
    pad = (-cols) % group_size
    if pad:
        weight = torch.nn.functional.pad(weight, (0, pad))
    return weight.reshape(rows, -1, group_size), pad


def ungroup(grouped: torch.Tensor, shape: tuple[int, int], pad: int) -> torch.Tensor:
    """``mround/core/quantizer.py:177-182``."""
    flat = grouped.reshape(shape[0], -1)
    return flat[:, : shape[1]] if pad else flat


def _check_init_scale(scheme: QuantScheme, init_scale: torch.Tensor | None) -> None:
    """``mround/core/quantizer.py:198-214``."""
    if scheme.scale_init is ScaleInit.SEARCHED and init_scale is None:
        msg = "a SEARCHED scheme needs the searched scale: pass init_scale from scale_search.search_scales"
        raise ValueError(msg)
    if scheme.scale_init is not ScaleInit.SEARCHED and init_scale is not None:
        msg = "init_scale was given but the scheme's scale_init is not SEARCHED"
        raise ValueError(msg)


def _unpack(params: Mapping[str, torch.Tensor] | None, rows: int, ng: int, gs: int):
    if params is None:
        return None, None, None
    v, alpha, beta = params["v"], params["alpha"], params["beta"]
    for name, t, shape in (("v", v, (rows, ng, gs)), ("alpha", alpha, (rows, ng, 1)),
                           ("beta", beta, (rows, ng, 1))):
        if tuple(t.shape) != shape:
            msg = f"params[{name!r}] has shape {tuple(t.shape)}, expected {shape}"
            raise SchemeError(msg)
    return v.contiguous(), alpha.contiguous(), beta.contiguous()


def _init_scale_arg(init_scale: torch.Tensor | None, rows: int, ng: int) -> torch.Tensor | None:
    if init_scale is None:
        return None
    return init_scale.to(torch.float32).reshape(rows, ng).contiguous()


def fake_quantize(
    weight: torch.Tensor,
    params: Mapping[str, torch.Tensor] | None,
    scheme: QuantScheme,
    *,
    eps: float = DEFAULT_EPS_FP32,
    init_scale: torch.Tensor | None = None,
    out_dtype: torch.dtype | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Quantize and immediately dequantize (``mround/core/quantizer.py:287-347``).

    Returns the reconstruction in the ungrouped ``(rows, cols)`` shape. ``out``
    may supply the destination (its dtype wins over ``out_dtype``).
    """
    _check_weight(weight)
    _check_init_scale(scheme, init_scale)
    rows, cols, gs, ng = _geometry(weight, scheme)
    v, alpha, beta = _unpack(params, rows, ng, gs)
    weight = weight.contiguous()
    if out is None:
        out = torch.empty((rows, cols), dtype=out_dtype or weight.dtype, device=weight.device)
    K.fq_forward(weight, v, alpha, beta, bits=scheme.bits, group_size=scheme.group_size,
                 mode=mode_of(scheme), eps=eps, init_scale=_init_scale_arg(init_scale, rows, ng),
                 wq_out=out)
    return out


def quantize_codes(
    weight: torch.Tensor,
    params: Mapping[str, torch.Tensor] | None,
    scheme: QuantScheme,
    *,
    eps: float = DEFAULT_EPS_FP32,
    init_scale: torch.Tensor | None = None,
    narrow: bool = False,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """``(codes, scale, zero_point)``, grouped (``mround/core/quantizer.py:350-398``).

    Codes come back as float32 integers like the reference's, or, with
    ``narrow=True``, directly in one byte each (int8 signed, uint8 unsigned) as
    ``narrow_codes`` would leave them. ``zero_point`` is ``None`` under
    symmetric schemes.
    """
    _check_weight(weight)
    _check_init_scale(scheme, init_scale)
    rows, cols, gs, ng = _geometry(weight, scheme)
    v, alpha, beta = _unpack(params, rows, ng, gs)
    signed = scheme.symmetry is Symmetry.SYMMETRIC
    dev = weight.device
    codes = torch.empty((rows, ng, gs), dtype=torch.int8 if signed else torch.uint8, device=dev)
    scale = torch.empty((rows, ng, 1), dtype=torch.float32, device=dev)
    zp = None if signed else torch.empty((rows, ng, 1), dtype=torch.float32, device=dev)
    K.fq_forward(weight.contiguous(), v, alpha, beta, bits=scheme.bits, group_size=scheme.group_size,
                 mode=mode_of(scheme), eps=eps, init_scale=_init_scale_arg(init_scale, rows, ng),
                 codes_out=codes, scale_out=scale, zp_out=zp)
    if not narrow:
        codes = codes.to(torch.float32)
    return codes, scale, zp


def quantize_pack(
    weight: torch.Tensor,
    params: Mapping[str, torch.Tensor] | None,
    scheme: QuantScheme,
    *,
    eps: float = DEFAULT_EPS_FP32,
    init_scale: torch.Tensor | None = None,
    dtype: torch.dtype = torch.bfloat16,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(packed, scales, biases)`` in MLX's layout, in one pass over the weight:
    the packed codes of :func:`quantize_codes` (``mround/formats/packing.py:119-163``)
    and the affine metadata of ``to_affine`` (``mround/formats/mlx_export.py:159-195``)
    in ``dtype``, with no one-byte codes in between. The group size must be a
    power of two of at least 32 that divides the row."""
    _check_weight(weight)
    _check_init_scale(scheme, init_scale)
    rows, cols, gs, ng = _geometry(weight, scheme)
    v, alpha, beta = _unpack(params, rows, ng, gs)
    dev = weight.device
    packed = torch.empty((rows, cols * scheme.bits // 32), dtype=torch.uint32, device=dev)
    scales = torch.empty((rows, ng), dtype=dtype, device=dev)
    biases = torch.empty((rows, ng), dtype=dtype, device=dev)
    K.quantize_pack(weight.contiguous(), v, alpha, beta, bits=scheme.bits, group_size=scheme.group_size,
                    mode=mode_of(scheme), eps=eps, init_scale=_init_scale_arg(init_scale, rows, ng),
                    packed_out=packed, scales_out=scales, biases_out=biases)
    return packed, scales, biases


def dequantize(codes, scale, zero_point, shape: tuple[int, int], scheme: QuantScheme) -> torch.Tensor:
    """``mround/core/quantizer.py:401-411``."""
    c = codes.to(torch.float32)
    grouped = scale * c if zero_point is None else scale * (c - zero_point)
    pad = 0 if scheme.group_size == -1 else (-shape[1]) % scheme.group_size
    return ungroup(grouped, shape, pad)


def init_params(weight: torch.Tensor, scheme: QuantScheme) -> Params:
    """``mround/core/quantizer.py:414-427``: v = 0, alpha = beta = 1 (exactly RTN)."""
    _check_weight(weight)
    rows, _, gs, ng = _geometry(weight, scheme)
    dev = weight.device
    return {
        "v": torch.zeros((rows, ng, gs), dtype=torch.float32, device=dev),
        "alpha": torch.ones((rows, ng, 1), dtype=torch.float32, device=dev),
        "beta": torch.ones((rows, ng, 1), dtype=torch.float32, device=dev),
    }


def project_params(params: Mapping[str, torch.Tensor], scheme: QuantScheme) -> Params:
    """``mround/core/quantizer.py:430-446``: a new mapping, clipped to the bounds.

    The fused step (:func:`mround_amd.core.signsgd.fused_step`) projects
    inside the kernel; this form serves callers that update separately.
    """
    lo, hi = scheme.coefficient_bounds
    return {
        "v": params["v"].clamp(-V_BOUND, V_BOUND),
        "alpha": params["alpha"].clamp(lo, hi),
        "beta": params["beta"].clamp(lo, hi),
    }


def quantize_grad(
    weight: torch.Tensor,
    params: Mapping[str, torch.Tensor],
    scheme: QuantScheme,
    grad_qdq: torch.Tensor,
    *,
    eps: float = DEFAULT_EPS_FP32,
    init_scale: torch.Tensor | None = None,
) -> Params:
    """Straight-through gradients of ``v``, ``alpha``, ``beta``.

    The analytic backward of ``fake_quantize`` (the reference gets it from
    MLX autodiff; its oracle is ``mround/reference/quantize.py:399-522``),
    computed by the HIP kernel without applying a step.
    """
    _check_weight(weight)
    _check_init_scale(scheme, init_scale)
    rows, cols, gs, ng = _geometry(weight, scheme)
    v, alpha, beta = _unpack(params, rows, ng, gs)
    if tuple(grad_qdq.shape) != (rows, cols):
        msg = f"grad_qdq has shape {tuple(grad_qdq.shape)}, expected {(rows, cols)}"
        raise SchemeError(msg)
    dev = weight.device
    gv = torch.empty((rows, ng, gs), dtype=torch.float32, device=dev)
    ga = torch.empty((rows, ng, 1), dtype=torch.float32, device=dev)
    gb = torch.empty((rows, ng, 1), dtype=torch.float32, device=dev)
    K.fq_backward_signsgd(weight.contiguous(), v, alpha, beta, grad_qdq.contiguous(), bits=scheme.bits,
                          group_size=scheme.group_size, mode=mode_of(scheme), eps=eps, update=False,
                          init_scale=_init_scale_arg(init_scale, rows, ng), grad_v_out=gv,
                          grad_alpha_out=ga, grad_beta_out=gb)
    return {"v": gv, "alpha": ga, "beta": gb}
