"""The 4-wave GEMM kernel (whole 256 x 256 tiles, A in three LDS stages and B
in two, a stage pattern that repeats every 6 k-tiles).

* Every entry position into the 6-k-tile stage pattern (K = 64 KT for KT = 17
  .. 22 covers KT % 6 = 0 .. 5), each layout, fp32 and bf16 outputs, against a
  float32 product of the same bf16 inputs on the GPU within the accumulation
  bound 2 K 2^-23 |A||B| (plus the bf16 output rounding).
* Ragged edges (M and N off the tile) with the bias and residual epilogue.
* The SwiGLU forward and backward epilogues.
* K-split tails (raw partial tiles summed in split order by the reduce kernel).
* Bit-identity with the 8-wave kernel (MR_GEMM_8WAVE=1): both accumulate each
  output over the same k16 steps in the same order with the same MFMA, so every
  layout and epilogue must give the same bits.

At 4096 x 4096 with K > 1024 the dispatcher takes 256 x 256 tiles (one wave of
256), which all run on the 4-wave kernel.
"""

from __future__ import annotations

import os
import sys

import pytest
import torch

from mround_amd import kernels as K
from tests.helpers import dev
from tests.test_gpu_gemm import _gpu_ref, _rand, interleave_gate_up

pytestmark = pytest.mark.gpu


def _operands(layout, M, N, Kd, seed):
    """Device operands in the layout's storage and the [M, K], [K, N] views for the reference."""
    if layout == "nt":
        a, b = _rand(M, Kd, seed=seed).to(dev()), _rand(N, Kd, seed=seed + 1).to(dev())
        return a, b, a, b.t().contiguous()
    if layout == "nn":
        a, b = _rand(M, Kd, seed=seed).to(dev()), _rand(Kd, N, seed=seed + 1).to(dev())
        return a, b, a, b
    a, b = _rand(Kd, M, seed=seed).to(dev()), _rand(Kd, N, seed=seed + 1).to(dev())
    return a, b, a.t().contiguous(), b


class _EightWave:
    """Every launch inside the block runs on the 8-wave kernel."""

    def __enter__(self):
        os.environ["MR_GEMM_8WAVE"] = "1"

    def __exit__(self, *exc):
        del os.environ["MR_GEMM_8WAVE"]


@pytest.mark.parametrize("layout", ["nt", "nn", "tn"])
@pytest.mark.parametrize("kt", [17, 18, 19, 20, 21, 22])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_4wave_phases(layout, kt, out):
    M, N, Kd = 4096, 4096, 64 * kt
    print("case gemm4 phase", layout, kt % 6, (M, N, Kd), out, flush=True, file=sys.stderr)
    a, b, a_ref, b_ref = _operands(layout, M, N, Kd, seed=100 + kt)
    ref, bound = _gpu_ref(a_ref, b_ref)
    c = torch.full((M, N), 7.0, dtype=out, device=dev())
    K.gemm(layout, a, b, c, M=M, N=N, K=Kd)
    tol = bound + (ref.abs() * 2.0**-8 if out == torch.bfloat16 else 0)
    assert bool(torch.all((c.float() - ref).abs() <= tol))
    c8 = torch.full((M, N), 5.0, dtype=out, device=dev())
    with _EightWave():
        K.gemm(layout, a, b, c8, M=M, N=N, K=Kd)
    assert torch.equal(c, c8), "4-wave and 8-wave kernels differ"


@pytest.mark.parametrize("layout", ["nt", "nn", "tn"])
def test_4wave_ragged_bias_residual(layout):
    # 17 x 17 tiles, the last tile row and column cut (M = 4216, N = 4104);
    # the residual epilogue keeps every tile on the large-tile kernel
    M, N, Kd = 4216, 4104, 64 * 19
    print("case gemm4 ragged", layout, (M, N, Kd), flush=True, file=sys.stderr)
    a, b, a_ref, b_ref = _operands(layout, M, N, Kd, seed=140)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(142)).to(dev())
    resid = torch.randn(M, N, generator=torch.Generator().manual_seed(143)).to(dev())
    prod, bound = _gpu_ref(a_ref, b_ref)
    ref = resid + (prod + bias)
    c = torch.empty(M, N, device=dev())
    K.gemm(layout, a, b, c, M=M, N=N, K=Kd, bias=bias, resid=resid)
    assert bool(torch.all((c - ref).abs() <= bound + ref.abs() * 2.0**-22))
    c8 = torch.empty(M, N, device=dev())
    with _EightWave():
        K.gemm(layout, a, b, c8, M=M, N=N, K=Kd, bias=bias, resid=resid)
    assert torch.equal(c, c8), "4-wave and 8-wave kernels differ"


@pytest.mark.parametrize("kt", [18, 20])
def test_4wave_swiglu(kt):
    M, n, Kd = 4096, 2048, 64 * kt
    print("case gemm4 swiglu", (M, n, Kd), flush=True, file=sys.stderr)
    x = _rand(M, Kd, seed=150).to(dev())
    wg, wu = _rand(n, Kd, seed=151), _rand(n, Kd, seed=152)
    g, tg = _gpu_ref(x, wg.to(dev()).t().contiguous())
    u, tu = _gpu_ref(x, wu.to(dev()).t().contiguous())
    wgu = interleave_gate_up(wg, wu).to(dev())
    act = torch.empty(M, n, dtype=torch.bfloat16, device=dev())
    gu = torch.empty(M, 2 * n, dtype=torch.bfloat16, device=dev())
    K.gemm_swiglu(x, wgu, act, gu)
    gu_c = gu.float().reshape(M, n // 32, 2, 32)
    assert bool(torch.all((gu_c[:, :, 0, :].reshape(M, n) - g).abs() <= tg + g.abs() * 2.0**-8))
    assert bool(torch.all((gu_c[:, :, 1, :].reshape(M, n) - u).abs() <= tu + u.abs() * 2.0**-8))
    act_ref = torch.nn.functional.silu(g) * u
    tol = 1.1 * tg * u.abs() + tu * torch.nn.functional.silu(g).abs() + act_ref.abs() * 2.0**-7 + 1e-6
    assert bool(torch.all((act.float() - act_ref).abs() <= tol))
    act8, gu8 = torch.empty_like(act), torch.empty_like(gu)
    with _EightWave():
        K.gemm_swiglu(x, wgu, act8, gu8)
    assert torch.equal(act, act8) and torch.equal(gu, gu8), "4-wave and 8-wave kernels differ"


@pytest.mark.parametrize("kt", [19, 22])
def test_4wave_swiglu_backward(kt):
    # dact = dd Wd (NN: dd [M, K], Wd [K, n]), then dgate, dup from the saved gate/up
    M, n, Kd = 4096, 4096, 64 * kt
    print("case gemm4 swiglu backward", (M, n, Kd), flush=True, file=sys.stderr)
    dd = _rand(M, Kd, seed=160).to(dev())
    wd = _rand(Kd, n, seed=161).to(dev())
    gu = (torch.randn(M, 2 * n, generator=torch.Generator().manual_seed(162)) * 2).to(torch.bfloat16).to(dev())
    dgu = torch.empty(M, 2 * n, dtype=torch.bfloat16, device=dev())
    K.gemm_swiglu_bwd(dd, wd, gu, dgu)
    dact, bound = _gpu_ref(dd, wd)
    gu_c = gu.float().reshape(M, n // 32, 2, 32)
    g, u = gu_c[:, :, 0, :].reshape(M, n), gu_c[:, :, 1, :].reshape(M, n)
    sg = torch.sigmoid(g)
    dg_ref = dact * u * sg * (1 + g * (1 - sg))
    du_ref = dact * g * sg
    got = dgu.float().reshape(M, n // 32, 2, 32)
    got_g, got_u = got[:, :, 0, :].reshape(M, n), got[:, :, 1, :].reshape(M, n)
    # dact's accumulation bound through the smooth factors (|d silu| <= 1.1), the
    # bf16 output rounding and the hardware reciprocal in the sigmoid
    tol_g = bound * (u.abs() * 1.1) + dg_ref.abs() * 2.0**-7 + 1e-6
    tol_u = bound * (g.abs() * sg) + du_ref.abs() * 2.0**-7 + 1e-6
    assert bool(torch.all((got_g - dg_ref).abs() <= tol_g))
    assert bool(torch.all((got_u - du_ref).abs() <= tol_u))
    dgu8 = torch.empty_like(dgu)
    with _EightWave():
        K.gemm_swiglu_bwd(dd, wd, gu, dgu8)
    assert torch.equal(dgu, dgu8), "4-wave and 8-wave kernels differ"


@pytest.mark.parametrize("layout", ["nt", "nn", "tn"])
@pytest.mark.parametrize("mnk", [(4096, 4352, 6144), (904, 696, 6400)])
def test_4wave_k_split(layout, mnk):
    # 4096 x 4352: one whole wave of 256 tiles and 16 past it, cut along K;
    # 904 x 696 (12 tiles, under one wave, long K): the whole grid cut along K.
    # The split blocks run on the 4-wave kernel and write raw partial tiles
    # that the reduce kernel sums in split order, as the 8-wave kernel's do.
    M, N, Kd = mnk
    print("case gemm4 k-split", layout, mnk, flush=True, file=sys.stderr)
    a, b, a_ref, b_ref = _operands(layout, M, N, Kd, seed=170)
    ref, bound = _gpu_ref(a_ref, b_ref)
    ws = torch.empty(max(K.gemm_workspace_bytes(M, N, Kd), 16), dtype=torch.uint8, device=dev())
    assert K.gemm_workspace_bytes(M, N, Kd) > 0, "this shape is expected to split"
    c = torch.full((M, N), 7.0, device=dev())
    K.gemm(layout, a, b, c, M=M, N=N, K=Kd, workspace=ws)
    assert bool(torch.all((c - ref).abs() <= bound))
    c8 = torch.full((M, N), 5.0, device=dev())
    with _EightWave():
        K.gemm(layout, a, b, c8, M=M, N=N, K=Kd, workspace=ws)
    assert torch.equal(c, c8), "4-wave and 8-wave kernels differ"
