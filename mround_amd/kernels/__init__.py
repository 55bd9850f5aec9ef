"""ctypes binding of ``libmround_hip.so`` -- the package's only compute path.

The reference leaves ``mround/kernels/`` empty as the designated home for
accelerated operators called from ``core`` and ``formats``
(``mround/kernels/__init__.py:3-8``, ``mround/formats/packing.py:28-30``).
Here it is the binding of the HIP library declared in ``include/mround_hip.h``.

Every wrapper takes torch tensors that already live on a ROCm device,
passes raw device pointers and the current HIP stream, and raises
:class:`~mround_amd.exceptions.KernelError` when the library refuses a call.
If the library is missing, :class:`~mround_amd.exceptions.KernelUnavailableError`
is raised; nothing falls back to another implementation.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

from mround_amd.exceptions import KernelError, KernelUnavailableError

__all__ = [
    "MODE",
    "copy_bytes",
    "cross_entropy",
    "delta_loss",
    "delta_loss_mapped",
    "dtype_code",
    "embed_rows",
    "fq_backward_signsgd",
    "fq_forward",
    "lib",
    "lib_path",
    "loss_mse",
    "loss_outlier",
    "loss_workspace",
    "pack_codes",
    "packed_width",
    "quantize_pack",
    "to_affine",
    "unpack_codes",
]

_PKG = Path(__file__).resolve().parent.parent
_LIB_PATH = _PKG / "_lib" / "libmround_hip.so"
_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

MR_OK, MR_EINVAL = 0, -22
MODE = {"asym": 0, "sym": 1, "searched": 2}
_DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_D = ctypes.c_double

_SIGNATURES = {
    "mr_last_error": (ctypes.c_char_p, []),
    "mr_abi_version": (_I, []),
    "mr_fq_forward": (_I, [_P, _I, _P, _P, _P, _P, _L, _L, _I, _I, _I, _F, _P, _I, _P, _P, _P, _P]),
    "mr_fq_backward_signsgd": (_I, [_P, _I, _P, _P, _P, _P, _P, _I, _L, _L, _I, _I, _I, _F, _I, _F,
                                    _F, _F, _F, _P, _P, _P, _P]),
    "mr_pack_codes": (_I, [_P, _I, _I, _L, _L, _I, _P, _P, _P]),
    "mr_quantize_pack": (_I, [_P, _I, _P, _P, _P, _P, _L, _L, _I, _I, _I, _F, _P, _P, _P, _I, _P]),
    "mr_packed_width": (_L, [_L, _I]),
    "mr_unpack_codes": (_I, [_P, _L, _L, _I, _P, _P]),
    "mr_to_affine": (_I, [_P, _P, _L, _I, _I, _P, _P, _P]),
    "mr_loss_workspace_bytes": (ctypes.c_size_t, [_L]),
    "mr_loss_mse": (_I, [_P, _P, _L, _L, _P, _P, _P, _P]),
    "mr_loss_outlier": (_I, [_P, _P, _L, _L, _L, _P, _P, _P, _P, _P, _P]),
    "mr_loss_outlier_noalloc": (_I, [_P, _P, _L, _L, _L, _P, _P, _P, _P, _P]),
    "mr_delta_loss_workspace_bytes": (ctypes.c_size_t, [_L, _L, _I]),
    "mr_delta_loss": (_I, [_P, _I, _P, _L, _L, _I, _P, _I, _I, _F, _P, _P, _P]),
    "mr_copy_bytes": (_I, [_P, _P, ctypes.c_size_t, _P]),
    "mr_gemm_workspace_bytes": (ctypes.c_size_t, [_L, _L, _L]),
    "mr_gemm": (_I, [_I, _L, _L, _L, _P, _L, _P, _L, _P, _I, _L, _P, _P, _L, _P, ctypes.c_size_t, _P]),
    "mr_gemm_f32": (_I, [_I, _L, _L, _L, _P, _L, _P, _P, _L, _P, _L, _P]),
    "mr_gemm_swiglu": (_I, [_L, _L, _L, _P, _L, _P, _L, _P, _L, _P, _L, _P, ctypes.c_size_t, _P]),
    "mr_gemm_swiglu_bwd": (_I, [_L, _L, _L, _P, _L, _P, _L, _P, _L, _P, _L, _P, ctypes.c_size_t, _P]),
    "mr_rmsnorm_fwd": (_I, [_P, _P, _L, _L, _F, _P, _P, _P]),
    "mr_rmsnorm_bwd": (_I, [_P, _P, _P, _P, _P, _L, _L, _P, _P, _P]),
    "mr_rmsnorm_fwd_split": (_I, [_P, _P, _L, _L, _F, _P, _P, _P, _P]),
    "mr_split_bf16": (_I, [_P, _L, _L, _L, _I, _P, _L, _P, _L, _P]),
    "mr_swiglu_split": (_I, [_P, _L, _L, _P, _P, _P, _P]),
    "mr_rope": (_I, [_P, _L, _L, _I, _I, _I, _P, _I, _P]),
    "mr_attn_fwd": (_I, [_P, _L, _I, _I, _I, _I, _I, _F, _P, _L, _P, _P]),
    "mr_attn_fwd_split": (_I, [_P, _P, _L, _I, _I, _I, _I, _I, _F, _P, _L, _P, _L, _P, _P]),
    "mr_rope_split": (_I, [_P, _L, _L, _I, _I, _I, _I, _P, _P, _P, _L, _P]),
    "mr_attn_bwd_workspace_bytes": (ctypes.c_size_t, [_I, _I, _I, _I, _I, _I]),
    "mr_attn_bwd": (_I, [_P, _L, _P, _P, _L, _P, _P, _I, _I, _I, _I, _I, _F, _P, _I, _P, ctypes.c_size_t,
                         _P]),
    "mr_cast_f32_bf16": (_I, [_P, _P, _L, _P]),
    "mr_allocate_bits": (_I, [_I, _P, _P, _P, _L, _L, _P, _P, _P]),
    "mr_search_scales": (_I, [_P, _I, _P, _L, _L, _I, _I, ctypes.c_double, _I, _P, _P]),
    "mr_colsumsq_workspace_bytes": (_L, [_L]),
    "mr_colsumsq": (_I, [_P, _I, _L, _L, _L, _P, _P, _P]),
    "mr_fq_forward_mapped": (_I, [_P, _I, _P, _P, _P, _P, _L, _L, _I, _I, _I, _F, _P, _I, _L, _L,
                                  _L, _P]),
    "mr_fq_backward_signsgd_mapped": (_I, [_P, _I, _P, _P, _P, _P, _P, _I, _L, _L, _I, _I, _I, _F,
                                           _F, _F, _F, _F, _L, _L, _L, _P]),
    "mr_fq_step_requant_mapped": (_I, [_P, _I, _P, _P, _P, _P, _P, _I, _L, _L, _I, _I, _I, _F, _F, _F,
                                       _F, _F, _L, _L, _L, _P, _I, _P]),
    "mr_fq_step_requant_mapped_sched": (_I, [_P, _I, _P, _P, _P, _P, _P, _I, _L, _L, _I, _I, _I, _F,
                                             _P, _I, _P, _F, _F, _F, _L, _L, _L, _P, _I, _P]),
    "mr_counter_add": (_I, [_P, _I, _P]),
    "mr_delta_loss_mapped": (_I, [_P, _I, _P, _L, _L, _I, _P, _I, _I, _F, _P, _L, _L, _L, _P, _P,
                                  _P]),
    "mr_cross_entropy": (_I, [_P, _L, _L, _L, _P, _F, _P, _P, _P, _L, _P]),
    "mr_embed_rows": (_I, [_P, _I, _L, _L, _L, _P, _L, _P, _L, _P]),
}


def lib_path() -> Path:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """The loaded library; raises :class:`KernelUnavailableError` if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not _LIB_PATH.exists():
                raise KernelUnavailableError(
                    f"{_LIB_PATH} is missing: build it with `python -m mround_amd.build` "
                    "(hipcc --offload-arch=gfx950); there is no CPU fallback"
                )
            try:
                handle = ctypes.CDLL(str(_LIB_PATH))
            except OSError as exc:
                raise KernelUnavailableError(f"cannot load {_LIB_PATH}: {exc}") from exc
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def _check(rc: int, name: str) -> None:
    if rc != MR_OK:
        msg = lib().mr_last_error().decode(errors="replace")
        raise KernelError(f"{name} failed ({rc}): {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise KernelError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16") from None


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise KernelError("tensors passed to the HIP library must live on a ROCm device")
    if not t.is_contiguous():
        raise KernelError("tensors passed to the HIP library must be contiguous")
    return t.data_ptr()


def _rows_ptr(t: torch.Tensor | None) -> int | None:
    """A 2-D operand whose rows may be strided (a column range of a wider
    matrix): unit stride along the row, the leading dimension passed apart."""
    if t is None:
        return None
    if not t.is_cuda:
        raise KernelError("tensors passed to the HIP library must live on a ROCm device")
    if t.dim() != 2 or t.stride(1) != 1:
        raise KernelError("a matrix operand must be 2-D with contiguous rows")
    return t.data_ptr()


def _f32(t: torch.Tensor | None, name: str) -> torch.Tensor | None:
    if t is not None and t.dtype != torch.float32:
        raise KernelError(f"{name} must be float32, got {t.dtype}")
    return t


# ---------------------------------------------------------------- quantizer --

def fq_forward(weight, v, alpha, beta, *, bits, group_size, mode, eps, init_scale=None,
               wq_out=None, codes_out=None, scale_out=None, zp_out=None) -> None:
    """``mr_fq_forward``: fills whichever outputs are given."""
    rows, cols = weight.shape
    rc = lib().mr_fq_forward(
        _ptr(weight), dtype_code(weight.dtype), _ptr(_f32(v, "v")), _ptr(_f32(alpha, "alpha")),
        _ptr(_f32(beta, "beta")), _ptr(_f32(init_scale, "init_scale")), rows, cols, group_size,
        bits, MODE[mode], eps, _ptr(wq_out), dtype_code(wq_out.dtype) if wq_out is not None else 0,
        _ptr(codes_out), _ptr(_f32(scale_out, "scale")), _ptr(_f32(zp_out, "zero_point")),
        _stream(weight))
    _check(rc, "mr_fq_forward")


def fq_backward_signsgd(weight, v, alpha, beta, grad_wq, *, bits, group_size, mode, eps,
                        update, lr=0.0, coef_lo=0.0, coef_hi=0.0, v_bound=0.5, init_scale=None,
                        grad_v_out=None, grad_alpha_out=None, grad_beta_out=None) -> None:
    """``mr_fq_backward_signsgd``: gradients and/or the fused sign step."""
    rows, cols = weight.shape
    rc = lib().mr_fq_backward_signsgd(
        _ptr(weight), dtype_code(weight.dtype), _ptr(_f32(v, "v")), _ptr(_f32(alpha, "alpha")),
        _ptr(_f32(beta, "beta")), _ptr(_f32(init_scale, "init_scale")), _ptr(grad_wq),
        dtype_code(grad_wq.dtype), rows, cols, group_size, bits, MODE[mode], eps, int(update), lr,
        coef_lo, coef_hi, v_bound, _ptr(grad_v_out), _ptr(grad_alpha_out), _ptr(grad_beta_out),
        _stream(weight))
    _check(rc, "mr_fq_backward_signsgd")


# ------------------------------------------------------------------ packing --

def packed_width(cols: int, bits: int) -> int:
    w = lib().mr_packed_width(cols, bits)
    if w < 0:
        raise ValueError(lib().mr_last_error().decode())
    return int(w)


def pack_codes(codes, bits: int, *, signed: bool, offset: int, packed_out, range_out=None) -> None:
    rows, cols = codes.shape
    rc = lib().mr_pack_codes(_ptr(codes), int(signed), offset, rows, cols, bits, _ptr(packed_out),
                             _ptr(range_out), _stream(codes))
    _check(rc, "mr_pack_codes")


def quantize_pack(weight, v, alpha, beta, *, bits, group_size, mode, eps, packed_out, scales_out,
                  biases_out, init_scale=None) -> None:
    """``mr_quantize_pack``: MLX words, scales and biases straight from the weight."""
    rows, cols = weight.shape
    if scales_out.dtype != biases_out.dtype:
        raise KernelError("scales and biases share one dtype")
    rc = lib().mr_quantize_pack(
        _ptr(weight), dtype_code(weight.dtype), _ptr(_f32(v, "v")), _ptr(_f32(alpha, "alpha")),
        _ptr(_f32(beta, "beta")), _ptr(_f32(init_scale, "init_scale")), rows, cols, group_size, bits,
        MODE[mode], eps, _ptr(packed_out), _ptr(scales_out), _ptr(biases_out), dtype_code(scales_out.dtype),
        _stream(weight))
    _check(rc, "mr_quantize_pack")


def unpack_codes(packed, rows: int, cols: int, bits: int, codes_out) -> None:
    rc = lib().mr_unpack_codes(_ptr(packed), rows, cols, bits, _ptr(codes_out), _stream(packed))
    _check(rc, "mr_unpack_codes")


def to_affine(scale, zero_point, bits: int, scales_out, biases_out) -> None:
    rc = lib().mr_to_affine(_ptr(_f32(scale, "scale")), _ptr(_f32(zero_point, "zero_point")),
                            scale.numel(), bits, dtype_code(scales_out.dtype), _ptr(scales_out),
                            _ptr(biases_out), _stream(scale))
    _check(rc, "mr_to_affine")


# ------------------------------------------------------------------- losses --

_workspaces: dict[tuple[int, str], torch.Tensor] = {}


def loss_workspace(device: torch.device, n: int) -> torch.Tensor:
    """A cached workspace for the loss kernels on ``device``."""
    nbytes = int(lib().mr_loss_workspace_bytes(n))
    key = (device.index or 0, "loss")
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def loss_mse(pred, target, *, denom, loss_out, grad_out=None, workspace=None) -> None:
    n = pred.numel()
    ws = workspace if workspace is not None else loss_workspace(pred.device, n)
    rc = lib().mr_loss_mse(_ptr(_f32(pred, "pred")), _ptr(_f32(target, "target")), n, denom,
                           _ptr(loss_out), _ptr(grad_out), _ptr(ws), _stream(pred))
    _check(rc, "mr_loss_mse")


def loss_outlier(pred, target, *, k, denom, loss_out, threshold_in=None, threshold_out=None,
                 grad_out=None, workspace=None) -> None:
    n = pred.numel()
    ws = workspace if workspace is not None else loss_workspace(pred.device, n)
    rc = lib().mr_loss_outlier(_ptr(_f32(pred, "pred")), _ptr(_f32(target, "target")), n, k, denom,
                               _ptr(threshold_in), _ptr(threshold_out), _ptr(loss_out),
                               _ptr(grad_out), _ptr(ws), _stream(pred))
    _check(rc, "mr_loss_outlier")


def loss_outlier_noalloc(pred, target, *, k, denom, loss_out, threshold_in=None, threshold_out=None,
                         grad_out=None) -> None:
    """``mr_loss_outlier_noalloc``: the outlier loss on the library's static
    per-GPU workspace (no allocation; overlapping calls on one GPU race)."""
    n = pred.numel()
    rc = lib().mr_loss_outlier_noalloc(_ptr(_f32(pred, "pred")), _ptr(_f32(target, "target")), n, k, denom,
                                       _ptr(threshold_in), _ptr(threshold_out), _ptr(loss_out),
                                       _ptr(grad_out), _stream(pred))
    _check(rc, "mr_loss_outlier_noalloc")


# ------------------------------------------------------------- sensitivity --

def _delta_workspace(weight, n_bits: int, workspace):
    rows, cols = weight.shape
    nbytes = int(lib().mr_delta_loss_workspace_bytes(rows, cols, n_bits))
    if workspace is None:
        key = (weight.device.index or 0, "delta")
        workspace = _workspaces.get(key)
        if workspace is None or workspace.numel() < nbytes:
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=weight.device)
            _workspaces[key] = workspace
    return workspace


def delta_loss(weight, grad, *, group_size, bits_list, mode, eps, scores_out, workspace=None) -> None:
    rows, cols = weight.shape
    n_bits = len(bits_list)
    arr = (ctypes.c_int * n_bits)(*bits_list)
    workspace = _delta_workspace(weight, n_bits, workspace)
    if scores_out.dtype != torch.float64:
        raise KernelError("scores_out must be float64")
    rc = lib().mr_delta_loss(_ptr(weight), dtype_code(weight.dtype), _ptr(_f32(grad, "grad")), rows,
                             cols, group_size, arr, n_bits, MODE[mode], eps, _ptr(scores_out),
                             _ptr(workspace), _stream(weight))
    _check(rc, "mr_delta_loss")


def delta_loss_mapped(weight, grad, *, group_size, bits_list, mode, eps, scores_out, grids=None,
                      row_block=0, row_stride=0, row_offset=0, workspace=None) -> None:
    """``mr_delta_loss_mapped``: ``grad`` is the placed gradient buffer (its rows
    at the placement), ``grids`` one (rows, n_groups) fp32 scale grid per width
    for the searched mode."""
    rows, cols = weight.shape
    n_bits = len(bits_list)
    arr = (ctypes.c_int * n_bits)(*bits_list)
    grid_arr = None
    if grids is not None:
        if len(grids) != n_bits:
            raise KernelError("one scale grid per width")
        grid_arr = (ctypes.c_void_p * n_bits)(*[_ptr(_f32(g, "grid")) for g in grids])
    if grad.shape[1] != cols or not grad.is_contiguous():
        raise KernelError("the placed gradient must be contiguous with the weight's column count")
    last = ((rows - 1) // row_block) * row_stride + row_offset + (rows - 1) % row_block if row_block else rows - 1
    if last >= grad.shape[0]:
        raise KernelError(f"the placement reaches gradient row {last}, past the {grad.shape[0]} rows given")
    if scores_out.dtype != torch.float64:
        raise KernelError("scores_out must be float64")
    workspace = _delta_workspace(weight, n_bits, workspace)
    rc = lib().mr_delta_loss_mapped(
        _ptr(weight), dtype_code(weight.dtype), _ptr(_f32(grad, "grad")), rows, cols, group_size, arr,
        n_bits, MODE[mode], eps, grid_arr, row_block, row_stride, row_offset, _ptr(scores_out),
        _ptr(workspace), _stream(weight))
    _check(rc, "mr_delta_loss_mapped")


# ------------------------------------------------------------- LM head ends --

def cross_entropy(logits, labels, *, V, scale, row_loss, loss_out=None, dlogits=None) -> None:
    """``mr_cross_entropy`` over bf16 logits rows ``[T, >=V]``; int32 labels."""
    if logits.dtype != torch.bfloat16 or (dlogits is not None and dlogits.dtype != torch.bfloat16):
        raise KernelError("cross-entropy logits and their gradient are bf16")
    if labels.dtype != torch.int32:
        raise KernelError("labels must be int32")
    T = logits.shape[0]
    if labels.numel() != T or row_loss.numel() < T:
        raise KernelError("one label and one row loss per logits row")
    rc = lib().mr_cross_entropy(_ptr(logits), logits.stride(0), T, V, _ptr(labels), scale,
                                _ptr(_f32(row_loss, "row_loss")), _ptr(_f32(loss_out, "loss")),
                                _ptr(dlogits), dlogits.stride(0) if dlogits is not None else 0,
                                _stream(logits))
    _check(rc, "mr_cross_entropy")


def embed_rows(table, ids, out) -> None:
    """``mr_embed_rows``: ``out[t] = table[ids[t]]`` as fp32; int32 ids."""
    if ids.dtype != torch.int32:
        raise KernelError("token ids must be int32")
    V, H = table.shape
    T = ids.numel()
    if out.shape[0] < T or out.shape[1] != H:
        raise KernelError(f"embedding output must be [{T}, {H}]")
    rc = lib().mr_embed_rows(_ptr(table), dtype_code(table.dtype), V, H, table.stride(0), _ptr(ids), T,
                             _ptr(_f32(out, "out")), out.stride(0), _stream(table))
    _check(rc, "mr_embed_rows")


# -------------------------------------------------------------------- GEMM --

GEMM_LAYOUT = {"nt": 0, "nn": 1, "tn": 2}


def gemm_workspace_bytes(M: int, N: int, K: int) -> int:
    """``mr_gemm_workspace_bytes``: k-split partials for an M x N x K product
    (N is the product's width: 2N for the SwiGLU pair)."""
    return int(lib().mr_gemm_workspace_bytes(M, N, K))


def _gemm_ws(device: torch.device, M: int, N: int, K: int, workspace):
    """The caller's workspace, or the binding's own per-device one grown to the
    plan's size (the library allocates nothing)."""
    if workspace is not None:
        return workspace
    nbytes = gemm_workspace_bytes(M, N, K)
    if nbytes == 0:
        return None
    key = (device.index or 0, "gemm")
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def _ws_args(ws):
    return (None, 0) if ws is None else (_ptr(ws), ws.numel() * ws.element_size())


def gemm(layout: str, a, b, c, *, M, N, K, bias=None, resid=None, workspace=None) -> None:
    """``mr_gemm``: C = op(A) op(B) (+ bias) (+ resid); leading dims from strides.
    ``workspace``: the k-split partials (a device tensor of at least
    ``gemm_workspace_bytes(M, N, K)`` bytes); None uses the binding's own."""
    ws_ptr, ws_bytes = _ws_args(_gemm_ws(a.device, M, N, K, workspace))
    rc = lib().mr_gemm(GEMM_LAYOUT[layout], M, N, K, _rows_ptr(a), a.stride(0), _rows_ptr(b), b.stride(0),
                       _rows_ptr(c), dtype_code(c.dtype), c.stride(0), _ptr(_f32(bias, "bias")),
                       _rows_ptr(_f32(resid, "resid")), resid.stride(0) if resid is not None else 0,
                       ws_ptr, ws_bytes, _stream(a))
    _check(rc, "mr_gemm")


def gemm_f32(layout: str, a, b, c, *, M, N, K, b_minus=None) -> None:
    """``mr_gemm_f32``: C = op(A) (op(B) - op(b_minus)) in fp32 on the MFMA
    cores, any sizes; leading dimensions from the strides (``b_minus``
    shares ``b``'s)."""
    for name, t in (("a", a), ("b", b), ("c", c)) + ((("b_minus", b_minus),) if b_minus is not None else ()):
        if t.dtype != torch.float32 or t.stride(-1) != 1:
            raise KernelError(f"gemm_f32: {name} must be float32 with unit column stride")
    if b_minus is not None and (b_minus.shape != b.shape or b_minus.stride(0) != b.stride(0)):
        raise KernelError("gemm_f32: b_minus must share b's shape and layout")
    rc = lib().mr_gemm_f32(GEMM_LAYOUT[layout], M, N, K, _rows_ptr(a), a.stride(0), _rows_ptr(b),
                           _rows_ptr(b_minus) if b_minus is not None else None, b.stride(0), _rows_ptr(c),
                           c.stride(0), _stream(a))
    _check(rc, "mr_gemm_f32")


def gemm_swiglu(x, wgu, act, gu=None, *, workspace=None) -> None:
    """``mr_gemm_swiglu`` over the 32-row interleaved gate/up weight ``wgu`` [2N, K]."""
    M, K = x.shape
    N = wgu.shape[0] // 2
    ws_ptr, ws_bytes = _ws_args(_gemm_ws(x.device, M, 2 * N, K, workspace))
    rc = lib().mr_gemm_swiglu(M, N, K, _ptr(x), x.stride(0), _ptr(wgu), wgu.stride(0), _ptr(act),
                              act.stride(0), _ptr(gu), gu.stride(0) if gu is not None else 0,
                              ws_ptr, ws_bytes, _stream(x))
    _check(rc, "mr_gemm_swiglu")


def gemm_swiglu_bwd(dd, wd, gu, dgu, *, workspace=None) -> None:
    """``mr_gemm_swiglu_bwd``: dgu from dact = dd Wd and the saved interleaved gate/up."""
    M, K = dd.shape
    N = wd.shape[1]
    ws_ptr, ws_bytes = _ws_args(_gemm_ws(dd.device, M, N, K, workspace))
    rc = lib().mr_gemm_swiglu_bwd(M, N, K, _ptr(dd), dd.stride(0), _ptr(wd), wd.stride(0), _ptr(gu),
                                  gu.stride(0), _ptr(dgu), dgu.stride(0), ws_ptr, ws_bytes, _stream(dd))
    _check(rc, "mr_gemm_swiglu_bwd")


def rmsnorm_fwd(h, w, eps, y, rstd=None) -> None:
    T, H = h.shape
    rc = lib().mr_rmsnorm_fwd(_ptr(_f32(h, "h")), _ptr(_f32(w, "w")), T, H, eps, _ptr(y),
                              _ptr(_f32(rstd, "rstd")), _stream(h))
    _check(rc, "mr_rmsnorm_fwd")


def rmsnorm_fwd_split(h, w, eps, y_split, y=None, rstd=None) -> None:
    """``mr_rmsnorm_fwd_split``: ``y_split`` [T, 3H] bf16 as [hi | hi | lo]."""
    T, H = h.shape
    if tuple(y_split.shape) != (T, 3 * H):
        raise KernelError(f"y_split must be [{T}, {3 * H}]")
    rc = lib().mr_rmsnorm_fwd_split(_ptr(_f32(h, "h")), _ptr(_f32(w, "w")), T, H, eps, _ptr(y_split), _ptr(y),
                                    _ptr(_f32(rstd, "rstd")), _stream(h))
    _check(rc, "mr_rmsnorm_fwd_split")


SPLIT_ACTIVATION, SPLIT_WEIGHT = 0, 1


def split_bf16(src, dst, *, order, plain=None) -> None:
    """``mr_split_bf16``: fp32 ``src`` [rows, cols] into ``dst`` [rows, >= 3 cols]
    (activation order [hi | hi | lo], weight order [hi | lo | hi]), hi alone
    into ``plain`` when given. Rows may be strided."""
    rows, cols = src.shape
    if dst.shape[0] != rows or (plain is not None and plain.shape[0] != rows):
        raise KernelError("split outputs must have the source's rows")
    rc = lib().mr_split_bf16(_rows_ptr(_f32(src, "src")), src.stride(0), rows, cols, order, _rows_ptr(dst),
                             dst.stride(0), _rows_ptr(plain), plain.stride(0) if plain is not None else 0,
                             _stream(src))
    _check(rc, "mr_split_bf16")


def swiglu_split(gu32, act_split, act, gu) -> None:
    """``mr_swiglu_split``: act from fp32 interleaved gate/up rows, split and plain."""
    T, N2 = gu32.shape
    N = N2 // 2
    if tuple(act_split.shape) != (T, 3 * N) or tuple(act.shape) != (T, N) or tuple(gu.shape) != (T, N2):
        raise KernelError("swiglu_split: act_split [T, 3N], act [T, N], gu [T, 2N]")
    rc = lib().mr_swiglu_split(_ptr(_f32(gu32, "gu32")), T, N, _ptr(act_split), _ptr(act), _ptr(gu),
                               _stream(gu32))
    _check(rc, "mr_swiglu_split")


def rmsnorm_bwd(dy, h, w, rstd, dres, dh_bf16=None, dh_f32=None) -> None:
    T, H = h.shape
    rc = lib().mr_rmsnorm_bwd(_ptr(_f32(dy, "dy")), _ptr(_f32(h, "h")), _ptr(_f32(w, "w")),
                              _ptr(_f32(rstd, "rstd")), _ptr(_f32(dres, "dres")), T, H, _ptr(dh_bf16),
                              _ptr(_f32(dh_f32, "dh")), _stream(h))
    _check(rc, "mr_rmsnorm_bwd")


def rope(x, *, seq_len, n_heads, head_dim, cos_sin, backward=False) -> None:
    T = x.shape[0]
    rc = lib().mr_rope(_ptr(x), x.stride(0), T, seq_len, n_heads, head_dim, _ptr(_f32(cos_sin, "cos_sin")),
                       int(backward), _stream(x))
    _check(rc, "mr_rope")


def attn_fwd(qkv, *, batch, seq_len, n_heads, n_kv_heads, head_dim, scale, out, lse) -> None:
    rc = lib().mr_attn_fwd(_ptr(qkv), qkv.stride(0), batch, seq_len, n_heads, n_kv_heads, head_dim,
                           scale, _ptr(out), out.stride(0), _ptr(_f32(lse, "lse")), _stream(qkv))
    _check(rc, "mr_attn_fwd")


def attn_fwd_split(qkv_hi, qkv_lo, *, batch, seq_len, n_heads, n_kv_heads, head_dim, scale, out, out_split,
                   lse) -> None:
    """``mr_attn_fwd_split``: the attention with q/k/v, probabilities and
    output carried as bf16 hi/lo halves; ``out`` gets the output's hi half,
    ``out_split`` [T, 3 Hq d] its [hi | hi | lo] rows."""
    if qkv_lo.stride(0) != qkv_hi.stride(0) or qkv_lo.shape != qkv_hi.shape:
        raise KernelError("attn_fwd_split: qkv_hi and qkv_lo must share a layout")
    if out_split.shape[0] != out.shape[0] or out_split.shape[1] < 3 * n_heads * head_dim:
        raise KernelError(f"attn_fwd_split: out_split must be [{out.shape[0]}, {3 * n_heads * head_dim}]")
    rc = lib().mr_attn_fwd_split(_ptr(qkv_hi), _ptr(qkv_lo), qkv_hi.stride(0), batch, seq_len, n_heads, n_kv_heads,
                                 head_dim, scale, _ptr(out), out.stride(0), _ptr(out_split), out_split.stride(0),
                                 _ptr(_f32(lse, "lse")), _stream(qkv_hi))
    _check(rc, "mr_attn_fwd_split")


def rope_split(x, hi, lo, *, seq_len, n_rope_heads, head_dim, cos_sin) -> None:
    """``mr_rope_split``: fp32 q/k/v rows ``x`` rotated (the first
    ``n_rope_heads`` heads) and written as bf16 ``hi`` and ``lo`` halves."""
    T, cols = x.shape
    if hi.shape != (T, cols) or lo.shape != (T, cols) or hi.stride(0) != lo.stride(0):
        raise KernelError(f"rope_split: hi and lo must be [{T}, {cols}] with one layout")
    rc = lib().mr_rope_split(_ptr(_f32(x, "x")), x.stride(0), T, seq_len, n_rope_heads, cols // head_dim, head_dim,
                             _ptr(_f32(cos_sin, "cos_sin")), _ptr(hi), _ptr(lo), hi.stride(0), _stream(x))
    _check(rc, "mr_rope_split")


def attn_bwd_workspace_bytes(*, batch, seq_len, n_heads, n_kv_heads, head_dim, hsplit=0) -> int:
    """``mr_attn_bwd_workspace_bytes``: dK/dV partials of the (automatic, 0) head split."""
    return int(lib().mr_attn_bwd_workspace_bytes(batch, seq_len, n_heads, n_kv_heads, head_dim, hsplit))


def attn_bwd(qkv, out, dout, lse, dsum, *, batch, seq_len, n_heads, n_kv_heads, head_dim, scale,
             dqkv, hsplit=0, workspace=None) -> None:
    """``mr_attn_bwd``. ``hsplit`` 0 splits the query heads of a kv head over
    blocks automatically, 1..G forces it; ``workspace`` holds the dK/dV
    partials (None: the binding's own, sized for the split)."""
    if dout.stride(0) != out.stride(0) or dqkv.stride(0) != qkv.stride(0):
        raise KernelError("attention backward: dout/out and dqkv/qkv must share layouts")
    if workspace is None:
        nbytes = attn_bwd_workspace_bytes(batch=batch, seq_len=seq_len, n_heads=n_heads,
                                          n_kv_heads=n_kv_heads, head_dim=head_dim, hsplit=hsplit)
        if nbytes:
            key = (qkv.device.index or 0, "attn")
            workspace = _workspaces.get(key)
            if workspace is None or workspace.numel() < nbytes:
                workspace = torch.empty(nbytes, dtype=torch.uint8, device=qkv.device)
                _workspaces[key] = workspace
    ws_ptr, ws_bytes = _ws_args(workspace)
    rc = lib().mr_attn_bwd(_ptr(qkv), qkv.stride(0), _ptr(out), _ptr(dout), out.stride(0),
                           _ptr(_f32(lse, "lse")), _ptr(_f32(dsum, "dsum")), batch, seq_len, n_heads,
                           n_kv_heads, head_dim, scale, _ptr(dqkv), hsplit, ws_ptr, ws_bytes, _stream(qkv))
    _check(rc, "mr_attn_bwd")


def allocate_bits(n_options, cost_bits, delta_loss, budget_bits: int, max_states: int):
    """``mr_allocate_bits`` on host arrays; returns (choices, loss, cost).

    Infeasible instances raise ``ValueError`` with the library's message."""
    n = len(n_options)
    n_opt = (ctypes.c_int32 * n)(*n_options)
    costs = (ctypes.c_int64 * len(cost_bits))(*cost_bits)
    losses = (ctypes.c_double * len(delta_loss))(*delta_loss)
    choice = (ctypes.c_int32 * n)()
    loss = ctypes.c_double()
    cost = ctypes.c_int64()
    rc = lib().mr_allocate_bits(n, ctypes.cast(n_opt, ctypes.c_void_p), ctypes.cast(costs, ctypes.c_void_p),
                                ctypes.cast(losses, ctypes.c_void_p), int(budget_bits), int(max_states),
                                ctypes.cast(choice, ctypes.c_void_p), ctypes.addressof(loss),
                                ctypes.addressof(cost))
    if rc != 0:
        raise ValueError(lib().mr_last_error().decode())
    return list(choice), loss.value, cost.value


def search_scales(weight, *, bits, group_size, step, half_count, scale_out, importance=None) -> None:
    rows, cols = weight.shape
    rc = lib().mr_search_scales(_ptr(weight), dtype_code(weight.dtype), _ptr(_f32(importance, "importance")),
                                rows, cols, group_size, bits, float(step), int(half_count),
                                _ptr(_f32(scale_out, "scale_out")), _stream(weight))
    _check(rc, "mr_search_scales")


def colsumsq(x, out) -> None:
    """``out += sum(x^2, axis=0)`` for a 2-D fp32/bf16 device tensor."""
    rows, cols = x.shape
    nbytes = int(lib().mr_colsumsq_workspace_bytes(cols))
    key = (x.device.index or 0, "colsumsq")
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
        _workspaces[key] = ws
    if x.stride(1) != 1:
        raise KernelError("colsumsq: rows must be contiguous")
    if not x.is_cuda:
        raise KernelError("tensors passed to the HIP library must live on a ROCm device")
    rc = lib().mr_colsumsq(x.data_ptr(), dtype_code(x.dtype), rows, cols, x.stride(0),
                           _ptr(_f32(out, "out")), _ptr(ws), _stream(x))
    _check(rc, "mr_colsumsq")


def cast_bf16(x, y) -> None:
    rc = lib().mr_cast_f32_bf16(_ptr(_f32(x, "x")), _ptr(y), x.numel(), _stream(x))
    _check(rc, "mr_cast_f32_bf16")


def fq_forward_mapped(weight, v, alpha, beta, *, bits, group_size, mode, eps, wq_out, row_block,
                      row_stride, row_offset, init_scale=None) -> None:
    """``mr_fq_forward_mapped``: W' rows placed inside the larger ``wq_out``."""
    rows, cols = weight.shape
    if wq_out.shape[1] != cols:
        raise KernelError("the placed output must have the weight's column count")
    rc = lib().mr_fq_forward_mapped(
        _ptr(weight), dtype_code(weight.dtype), _ptr(_f32(v, "v")), _ptr(_f32(alpha, "alpha")),
        _ptr(_f32(beta, "beta")), _ptr(_f32(init_scale, "init_scale")), rows, cols, group_size,
        bits, MODE[mode], eps, _ptr(wq_out), dtype_code(wq_out.dtype), row_block, row_stride,
        row_offset, _stream(weight))
    _check(rc, "mr_fq_forward_mapped")


def fq_step_mapped(weight, v, alpha, beta, grad, *, bits, group_size, mode, eps, lr, coef_lo,
                   coef_hi, v_bound, row_block, row_stride, row_offset, init_scale=None) -> None:
    """``mr_fq_backward_signsgd_mapped``: fused step, dL/dW' read from a placed buffer."""
    rows, cols = weight.shape
    if grad.shape[1] != cols:
        raise KernelError("the placed gradient must have the weight's column count")
    rc = lib().mr_fq_backward_signsgd_mapped(
        _ptr(weight), dtype_code(weight.dtype), _ptr(_f32(v, "v")), _ptr(_f32(alpha, "alpha")),
        _ptr(_f32(beta, "beta")), _ptr(_f32(init_scale, "init_scale")), _ptr(grad),
        dtype_code(grad.dtype), rows, cols, group_size, bits, MODE[mode], eps, lr, coef_lo, coef_hi,
        v_bound, row_block, row_stride, row_offset, _stream(weight))
    _check(rc, "mr_fq_backward_signsgd_mapped")


def fq_step_requant_mapped(weight, v, alpha, beta, grad, *, bits, group_size, mode, eps, lr, coef_lo,
                           coef_hi, v_bound, row_block, row_stride, row_offset, wq_out,
                           init_scale=None) -> None:
    """``mr_fq_step_requant_mapped``: the fused step, then the new W' placed in ``wq_out``."""
    rows, cols = weight.shape
    if grad.shape[1] != cols or wq_out.shape[1] != cols:
        raise KernelError("the placed gradient and W' must have the weight's column count")
    rc = lib().mr_fq_step_requant_mapped(
        _ptr(weight), dtype_code(weight.dtype), _ptr(_f32(v, "v")), _ptr(_f32(alpha, "alpha")),
        _ptr(_f32(beta, "beta")), _ptr(_f32(init_scale, "init_scale")), _ptr(grad),
        dtype_code(grad.dtype), rows, cols, group_size, bits, MODE[mode], eps, lr, coef_lo, coef_hi,
        v_bound, row_block, row_stride, row_offset, _ptr(wq_out), dtype_code(wq_out.dtype),
        _stream(weight))
    _check(rc, "mr_fq_step_requant_mapped")


def fq_step_requant_sched(weight, v, alpha, beta, grad, *, bits, group_size, mode, eps, lr_table, step,
                          coef_lo, coef_hi, v_bound, row_block, row_stride, row_offset, wq_out,
                          init_scale=None) -> None:
    """``mr_fq_step_requant_mapped_sched``: the rate is ``lr_table[step[0]]`` on the device."""
    rows, cols = weight.shape
    if grad.shape[1] != cols or wq_out.shape[1] != cols:
        raise KernelError("the placed gradient and W' must have the weight's column count")
    if step.dtype != torch.int32:
        raise KernelError("the step counter is int32")
    rc = lib().mr_fq_step_requant_mapped_sched(
        _ptr(weight), dtype_code(weight.dtype), _ptr(_f32(v, "v")), _ptr(_f32(alpha, "alpha")),
        _ptr(_f32(beta, "beta")), _ptr(_f32(init_scale, "init_scale")), _ptr(grad),
        dtype_code(grad.dtype), rows, cols, group_size, bits, MODE[mode], eps,
        _ptr(_f32(lr_table, "lr_table")), lr_table.numel(), _ptr(step), coef_lo, coef_hi, v_bound,
        row_block, row_stride, row_offset, _ptr(wq_out), dtype_code(wq_out.dtype), _stream(weight))
    _check(rc, "mr_fq_step_requant_mapped_sched")


def counter_add(counter, delta: int = 1) -> None:
    """``mr_counter_add``: ``counter[0] += delta`` on the current stream (int32)."""
    if counter.dtype != torch.int32:
        raise KernelError("the counter is int32")
    _check(lib().mr_counter_add(_ptr(counter), delta, _stream(counter)), "mr_counter_add")


def copy_bytes(src, dst, nbytes: int) -> None:
    rc = lib().mr_copy_bytes(_ptr(src), _ptr(dst), nbytes, _stream(src))
    _check(rc, "mr_copy_bytes")
