"""GPU parity of the MFMA GEMMs against a float64 CPU product of the same bf16 inputs.

The inputs are bf16 (exact in fp32), the products are exact in fp32, and the
only error is fp32 accumulation: |C - ref| <= K * 2^-23 * (|A| |B|) elementwise.
bf16 outputs add one rounding (2^-8 relative).
"""

from __future__ import annotations

import sys

import pytest
import torch

from mround_amd import kernels as K
from tests.helpers import dev

pytestmark = pytest.mark.gpu


def _rand(*shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(torch.bfloat16)


def _bound(a64, b64, k):
    return (a64.abs() @ b64.abs()) * (k * 2.0**-23) + 1e-30


@pytest.mark.parametrize("layout", ["nt", "nn", "tn"])
@pytest.mark.parametrize("mnk", [(256, 256, 64), (200, 136, 128), (1024, 512, 320), (8, 8, 64),
                                 (576, 192, 576), (4096, 576, 1536), (512, 768, 896)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_gemm_layouts(layout, mnk, out):
    M, N, Kd = mnk
    print("case gemm", layout, mnk, out, flush=True, file=sys.stderr)
    if layout == "nt":
        a, b = _rand(M, Kd, seed=1), _rand(N, Kd, seed=2)
        a64, b64 = a.double(), b.double().t()
    elif layout == "nn":
        a, b = _rand(M, Kd, seed=3), _rand(Kd, N, seed=4)
        a64, b64 = a.double(), b.double()
    else:
        a, b = _rand(Kd, M, seed=5), _rand(Kd, N, seed=6)
        a64, b64 = a.double().t(), b.double()
    ref = a64 @ b64
    c = torch.empty(M, N, dtype=out, device=dev())
    K.gemm(layout, a.to(dev()), b.to(dev()), c, M=M, N=N, K=Kd)
    got = c.double().cpu()
    tol = _bound(a64, b64, Kd)
    if out == torch.bfloat16:
        tol = tol + ref.abs() * 2.0**-8
    assert torch.all((got - ref).abs() <= tol), float(((got - ref).abs() / tol).max())


# Large tiles: 4096 x 4096 is exactly one wave of 256 x 256 tiles (one launch).
# 4352 x 4096 leaves a partial wave with a short K (not split); 256 x 384 and
# 200 x 136 are small tiles over a long K (not split either). The k-split of
# large tiles is covered below and by the SwiGLU and residual cases.
@pytest.mark.parametrize("mnk", [(4096, 4096, 64), (4352, 4096, 640), (256, 384, 6144), (200, 136, 6208)])
@pytest.mark.parametrize("layout", ["nt", "nn", "tn"])
def test_gemm_large_tiles_and_split_tail(mnk, layout):
    M, N, Kd = mnk
    print("case gemm large", layout, mnk, flush=True, file=sys.stderr)
    if layout == "nt":
        a, b = _rand(M, Kd, seed=21), _rand(N, Kd, seed=22)
        a64, b64 = a.double(), b.double().t()
    elif layout == "nn":
        a, b = _rand(M, Kd, seed=25), _rand(Kd, N, seed=26)
        a64, b64 = a.double(), b.double()
    else:
        a, b = _rand(Kd, M, seed=23), _rand(Kd, N, seed=24)
        a64, b64 = a.double().t(), b.double()
    ref = a64 @ b64
    c = torch.empty(M, N, device=dev())
    K.gemm(layout, a.to(dev()), b.to(dev()), c, M=M, N=N, K=Kd)
    assert torch.all((c.double().cpu() - ref).abs() <= _bound(a64, b64, Kd))


# The k-split tail of large tiles: 4096 x 4352 (or 4352 x 4096) x 6144 has 272
# tiles of 256 x 256; the 16 past the wave are cut along K and their partials
# summed in order by the reduce kernel, which also applies the epilogue.
# References: float32 PyTorch products of the same bf16 inputs on the GPU
# (their own accumulation error is within the K 2^-23 |A||B| bound used).
SPLIT_M, SPLIT_N, SPLIT_K = 4096, 4352, 6144


def _gpu_ref(a, b):
    """float32 product and the bound 2 K 2^-23 |A||B| (a: [M, K], b: [K, N], on the GPU)."""
    ref = a.float() @ b.float()
    bound = (a.float().abs() @ b.float().abs()) * (2 * a.shape[1] * 2.0**-23) + 1e-30
    return ref, bound


@pytest.mark.parametrize("layout", ["nt", "nn", "tn"])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_gemm_split_tail_large_tiles(layout, out):
    M, N, Kd = (SPLIT_N, SPLIT_M, SPLIT_K) if layout == "tn" else (SPLIT_M, SPLIT_N, SPLIT_K)
    print("case gemm split", layout, (M, N, Kd), out, flush=True, file=sys.stderr)
    if layout == "nt":
        a, b = _rand(M, Kd, seed=27).to(dev()), _rand(N, Kd, seed=28).to(dev())
        ref, bound = _gpu_ref(a, b.t().contiguous())
    elif layout == "nn":
        a, b = _rand(M, Kd, seed=29).to(dev()), _rand(Kd, N, seed=30).to(dev())
        ref, bound = _gpu_ref(a, b)
    else:
        a, b = _rand(Kd, M, seed=31).to(dev()), _rand(Kd, N, seed=32).to(dev())
        ref, bound = _gpu_ref(a.t().contiguous(), b)
    c = torch.empty(M, N, dtype=out, device=dev())
    K.gemm(layout, a, b, c, M=M, N=N, K=Kd)
    tol = bound + (ref.abs() * 2.0**-8 if out == torch.bfloat16 else 0)
    assert bool(torch.all((c.float() - ref).abs() <= tol))


def test_gemm_split_tail_bias_residual():
    M, N, Kd = SPLIT_M, SPLIT_N, SPLIT_K
    a, b = _rand(M, Kd, seed=33).to(dev()), _rand(N, Kd, seed=34).to(dev())
    bias = torch.randn(N, generator=torch.Generator().manual_seed(35)).to(dev())
    resid = torch.randn(M, N, generator=torch.Generator().manual_seed(36)).to(dev())
    prod, bound = _gpu_ref(a, b.t().contiguous())
    ref = resid + (prod + bias)
    c = torch.empty(M, N, device=dev())
    K.gemm("nt", a, b, c, M=M, N=N, K=Kd, bias=bias, resid=resid)
    assert bool(torch.all((c - ref).abs() <= bound + ref.abs() * 2.0**-22))


def test_swiglu_split_tail():
    M, N, Kd = SPLIT_M, SPLIT_N // 2, SPLIT_K
    x = _rand(M, Kd, seed=37).to(dev())
    wg, wu = _rand(N, Kd, seed=38), _rand(N, Kd, seed=39)
    g, tg = _gpu_ref(x, wg.to(dev()).t().contiguous())
    u, tu = _gpu_ref(x, wu.to(dev()).t().contiguous())
    act = torch.empty(M, N, dtype=torch.bfloat16, device=dev())
    gu = torch.empty(M, 2 * N, dtype=torch.bfloat16, device=dev())
    K.gemm_swiglu(x, interleave_gate_up(wg, wu).to(dev()), act, gu)
    gu_c = gu.float().reshape(M, N // 32, 2, 32)
    got_g, got_u = gu_c[:, :, 0, :].reshape(M, N), gu_c[:, :, 1, :].reshape(M, N)
    assert bool(torch.all((got_g - g).abs() <= tg + g.abs() * 2.0**-8))
    assert bool(torch.all((got_u - u).abs() <= tu + u.abs() * 2.0**-8))
    act_ref = torch.nn.functional.silu(g) * u
    tol = 1.1 * tg * u.abs() + tu * torch.nn.functional.silu(g).abs() + act_ref.abs() * 2.0**-7 + 1e-6
    assert bool(torch.all((act.float() - act_ref).abs() <= tol))


# Under one wave of large tiles with a long K (at least 96 steps of 64) the whole
# grid is cut along K: ragged 296 x 200 (2 tiles) and 904 x 696 (12 tiles).
@pytest.mark.parametrize("layout", ["nt", "nn", "tn"])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mn", [(296, 200), (904, 696)])
def test_gemm_small_grid_long_k(layout, out, mn):
    M, N = mn
    Kd = 6400
    print("case gemm small grid", layout, (M, N, Kd), out, flush=True, file=sys.stderr)
    if layout == "nt":
        a, b = _rand(M, Kd, seed=41).to(dev()), _rand(N, Kd, seed=42).to(dev())
        ref, bound = _gpu_ref(a, b.t().contiguous())
    elif layout == "nn":
        a, b = _rand(M, Kd, seed=43).to(dev()), _rand(Kd, N, seed=44).to(dev())
        ref, bound = _gpu_ref(a, b)
    else:
        a, b = _rand(Kd, M, seed=45).to(dev()), _rand(Kd, N, seed=46).to(dev())
        ref, bound = _gpu_ref(a.t().contiguous(), b)
    c = torch.full((M, N), 7.0, dtype=out, device=dev())
    K.gemm(layout, a, b, c, M=M, N=N, K=Kd)
    tol = bound + (ref.abs() * 2.0**-8 if out == torch.bfloat16 else 0)
    assert bool(torch.all((c.float() - ref).abs() <= tol))


# 17 x 16 = 272 large tiles: one whole wave and a last wave of 16, which runs
# as quarter tiles; with M = 4160 the lower quarters of the last tile row lie
# wholly past the edge, and N = 4056 cuts the last tile column.
@pytest.mark.parametrize("layout", ["nt", "nn", "tn"])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_gemm_quarter_tile_tail(layout, out):
    M, N, Kd = 4160, 4056, 192
    print("case gemm quarter-tile tail", layout, out, flush=True, file=sys.stderr)
    if layout == "nt":
        a, b = _rand(M, Kd, seed=53).to(dev()), _rand(N, Kd, seed=54).to(dev())
        ref, bound = _gpu_ref(a, b.t().contiguous())
    elif layout == "nn":
        a, b = _rand(M, Kd, seed=55).to(dev()), _rand(Kd, N, seed=56).to(dev())
        ref, bound = _gpu_ref(a, b)
    else:
        a, b = _rand(Kd, M, seed=57).to(dev()), _rand(Kd, N, seed=58).to(dev())
        ref, bound = _gpu_ref(a.t().contiguous(), b)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(59)).to(dev())
    c = torch.full((M, N), 7.0, dtype=out, device=dev())
    K.gemm(layout, a, b, c, M=M, N=N, K=Kd, bias=bias)
    ref = ref + bias
    tol = bound + ref.abs() * (2.0**-8 if out == torch.bfloat16 else 2.0**-23)
    assert bool(torch.all((c.float() - ref).abs() <= tol))


def test_gemm_small_grid_bias_residual_and_swiglu():
    M, N, Kd = 328, 256, 6144
    print("case gemm small grid epilogues", flush=True, file=sys.stderr)
    a, b = _rand(M, Kd, seed=47).to(dev()), _rand(N, Kd, seed=48).to(dev())
    bias = torch.randn(N, generator=torch.Generator().manual_seed(49)).to(dev())
    resid = torch.randn(M, N, generator=torch.Generator().manual_seed(50)).to(dev())
    prod, bound = _gpu_ref(a, b.t().contiguous())
    ref = resid + (prod + bias)
    c = torch.empty(M, N, device=dev())
    K.gemm("nt", a, b, c, M=M, N=N, K=Kd, bias=bias, resid=resid)
    assert bool(torch.all((c - ref).abs() <= bound + ref.abs() * 2.0**-22))
    n = N // 2
    wg, wu = _rand(n, Kd, seed=51), _rand(n, Kd, seed=52)
    g, tg = _gpu_ref(a, wg.to(dev()).t().contiguous())
    u, tu = _gpu_ref(a, wu.to(dev()).t().contiguous())
    act = torch.empty(M, n, dtype=torch.bfloat16, device=dev())
    gu = torch.empty(M, 2 * n, dtype=torch.bfloat16, device=dev())
    K.gemm_swiglu(a, interleave_gate_up(wg, wu).to(dev()), act, gu)
    gu_c = gu.float().reshape(M, n // 32, 2, 32)
    assert bool(torch.all((gu_c[:, :, 0, :].reshape(M, n) - g).abs() <= tg + g.abs() * 2.0**-8))
    assert bool(torch.all((gu_c[:, :, 1, :].reshape(M, n) - u).abs() <= tu + u.abs() * 2.0**-8))
    act_ref = torch.nn.functional.silu(g) * u
    tol = 1.1 * tg * u.abs() + tu * torch.nn.functional.silu(g).abs() + act_ref.abs() * 2.0**-7 + 1e-6
    assert bool(torch.all((act.float() - act_ref).abs() <= tol))


def test_gemm_bias_and_residual():
    M, N, Kd = 304, 264, 128
    a, b = _rand(M, Kd, seed=7), _rand(N, Kd, seed=8)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(9))
    resid = torch.randn(M, N, generator=torch.Generator().manual_seed(10))
    ref = resid.double() + (a.double() @ b.double().t() + bias.double())
    c = torch.empty(M, N, device=dev())
    K.gemm("nt", a.to(dev()), b.to(dev()), c, M=M, N=N, K=Kd, bias=bias.to(dev()),
           resid=resid.to(dev()))
    tol = _bound(a.double(), b.double().t(), Kd) + ref.abs() * 2.0**-23 * 4
    assert torch.all((c.double().cpu() - ref).abs() <= tol)


def interleave_gate_up(wg, wu):
    """Rows 64b..64b+31 = gate rows 32b.., rows 64b+32.. = the matching up rows."""
    n, k = wg.shape
    return torch.stack([wg.reshape(n // 32, 32, k), wu.reshape(n // 32, 32, k)], 1).reshape(2 * n, k)


@pytest.mark.parametrize("mnk", [(512, 256, 128), (200, 96, 64), (4096, 1536, 576), (1024, 4864, 896)])
def test_swiglu(mnk):
    M, N, Kd = mnk
    x, wg, wu = _rand(M, Kd, seed=11), _rand(N, Kd, seed=12), _rand(N, Kd, seed=13)
    g = x.double() @ wg.double().t()
    u = x.double() @ wu.double().t()
    act_ref = torch.nn.functional.silu(g) * u
    act = torch.empty(M, N, dtype=torch.bfloat16, device=dev())
    gu = torch.empty(M, 2 * N, dtype=torch.bfloat16, device=dev())
    K.gemm_swiglu(x.to(dev()), interleave_gate_up(wg, wu).to(dev()), act, gu)
    tg = _bound(x.double(), wg.double().t(), Kd)
    tu = _bound(x.double(), wu.double().t(), Kd)
    gu_c = gu.double().cpu().reshape(M, N // 32, 2, 32)
    got_g = gu_c[:, :, 0, :].reshape(M, N)
    got_u = gu_c[:, :, 1, :].reshape(M, N)
    assert torch.all((got_g - g).abs() <= tg + g.abs() * 2.0**-8)
    assert torch.all((got_u - u).abs() <= tu + u.abs() * 2.0**-8)
    # act from fp32 g, u: silu' <= 1.1, plus the bf16 rounding of act and the fast exp
    tol = (1.1 * tg * u.abs() + tu * torch.nn.functional.silu(g).abs() + act_ref.abs() * 2.0**-7
           + 1e-6)
    assert torch.all((act.double().cpu() - act_ref).abs() <= tol)


@pytest.mark.parametrize("mnk", [(200, 96, 64), (1000, 2400, 576), (4096, 4096, 1152), (4216, 4128, 1216)])
def test_swiglu_copy_bitwise_and_act_only(mnk):
    # The gate/up copy is the bf16 rounding of the fp32 product over the
    # interleaved weight, which the plain fp32 GEMM computes with the same
    # k16 steps in the same order: equal bits. Without the copy, act is
    # unchanged. Shapes: the 8-wave 128 x 128 and 256 x 256 kernels, and the
    # 4-wave kernel with whole and cut edge tiles.
    M, N, Kd = mnk
    print("case swiglu copy", mnk, flush=True, file=sys.stderr)
    x = _rand(M, Kd, seed=61).to(dev())
    wgu = interleave_gate_up(_rand(N, Kd, seed=62), _rand(N, Kd, seed=63)).to(dev())
    prod = torch.empty(M, 2 * N, device=dev())
    K.gemm("nt", x, wgu, prod, M=M, N=2 * N, K=Kd)
    act = torch.full((M, N), 3.0, dtype=torch.bfloat16, device=dev())
    gu = torch.full((M, 2 * N), 3.0, dtype=torch.bfloat16, device=dev())
    K.gemm_swiglu(x, wgu, act, gu)
    assert torch.equal(gu, prod.to(torch.bfloat16))
    act2 = torch.full((M, N), 5.0, dtype=torch.bfloat16, device=dev())
    K.gemm_swiglu(x, wgu, act2)
    assert torch.equal(act, act2)
    pc = prod.reshape(M, N // 32, 2, 32)
    g, u = pc[:, :, 0, :].reshape(M, N), pc[:, :, 1, :].reshape(M, N)
    act_ref = torch.nn.functional.silu(g) * u
    # the fast exp and the bf16 rounding of act
    assert bool(torch.all((act.float() - act_ref).abs() <= act_ref.abs() * 2.0**-7 + 1e-6))


def test_nn_over_interleaved_pair_equals_sum():
    """dx = dgu Wgu over the interleaved K = 2N equals dgate Wg + dup Wu."""
    M, N, Kd = 256, 192, 128
    dg, du = _rand(M, N, seed=14), _rand(M, N, seed=15)
    wg, wu = _rand(N, Kd, seed=16), _rand(N, Kd, seed=17)
    dgu = torch.stack([dg.reshape(M, N // 32, 32), du.reshape(M, N // 32, 32)], 2).reshape(M, 2 * N)
    wgu = interleave_gate_up(wg, wu)
    ref = dg.double() @ wg.double() + du.double() @ wu.double()
    c = torch.empty(M, Kd, device=dev())
    K.gemm("nn", dgu.to(dev()), wgu.to(dev()), c, M=M, N=Kd, K=2 * N)
    tol = _bound(dgu.double(), wgu.double(), 2 * N)
    assert torch.all((c.double().cpu() - ref).abs() <= tol)


def test_gemm_rejects_bad_shapes():
    a = torch.zeros(10, 64, dtype=torch.bfloat16, device=dev())
    b = torch.zeros(16, 64, dtype=torch.bfloat16, device=dev())
    c = torch.zeros(10, 16, device=dev())
    with pytest.raises(Exception, match="multiples of 8"):
        K.gemm("nt", a, b, c, M=10, N=16, K=64)


# The residual epilogue on every layout, with the output written over the
# residual itself (the accumulation of weight gradients over the pieces of a
# batch): short K on large tiles, and a long K whose remainder wave is cut
# along K (the reduce kernel adds the residual).
@pytest.mark.parametrize("layout", ["nt", "nn", "tn"])
@pytest.mark.parametrize("mnk", [(304, 264, 128), (4352, 4096, 6144)])
@pytest.mark.parametrize("inplace", [False, True])
def test_gemm_residual_every_layout(layout, mnk, inplace):
    M, N, Kd = mnk
    print("case gemm residual", layout, mnk, inplace, flush=True, file=sys.stderr)
    if layout == "nt":
        a, b = _rand(M, Kd, seed=61).to(dev()), _rand(N, Kd, seed=62).to(dev())
        prod, bound = _gpu_ref(a, b.t().contiguous())
    elif layout == "nn":
        a, b = _rand(M, Kd, seed=63).to(dev()), _rand(Kd, N, seed=64).to(dev())
        prod, bound = _gpu_ref(a, b)
    else:
        a, b = _rand(Kd, M, seed=65).to(dev()), _rand(Kd, N, seed=66).to(dev())
        prod, bound = _gpu_ref(a.t().contiguous(), b)
    resid = torch.randn(M, N, generator=torch.Generator().manual_seed(67)).to(dev())
    ref = resid + prod
    c = resid if inplace else torch.full((M, N), 7.0, device=dev())
    if Kd >= 6144:
        assert K.gemm_workspace_bytes(M, N, Kd) > 0  # the k-split path
    K.gemm(layout, a, b, c, M=M, N=N, K=Kd, resid=resid)
    assert bool(torch.all((c - ref).abs() <= bound + ref.abs() * 2.0**-22))


# ------------------------------------------------------------------ fp32 GEMM --
# mr_gemm_f32, the single-layer loop's products: fp32 products and
# accumulation, any sizes, B - B2 formed as the operand is loaded. Bound: the
# float64 product of the same fp32 operands within (K + 4) 2^-23 of the sum of
# magnitudes (fp32 accumulation, the subtraction's own rounding, a factor 2
# of margin); columns past N and rows past M untouched.
@pytest.mark.parametrize("layout", ["nt", "nn", "tn"])
@pytest.mark.parametrize("mnk", [(128, 16, 64), (300, 77, 130), (1, 1, 1), (513, 257, 1000), (64, 2048, 33)])
@pytest.mark.parametrize("minus", [False, True])
def test_gemm_f32(layout, mnk, minus):
    M, N, Kd = mnk
    print("case gemm f32", layout, mnk, minus, flush=True, file=sys.stderr)
    g = torch.Generator().manual_seed(71)
    a = torch.randn(M, Kd, generator=g)
    b = torch.randn(N, Kd, generator=g)
    b2 = torch.randn(N, Kd, generator=g) * 0.5 if minus else None
    bm = b - b2 if minus else b
    want = a.double() @ bm.double().T
    mags = a.double().abs() @ (b.double().abs() + (b2.double().abs() if minus else 0)).T
    # the operands in the layout's memory order
    A = a if layout != "tn" else a.T.contiguous()
    B = b if layout == "nt" else b.T.contiguous()
    B2 = None if not minus else (b2 if layout == "nt" else b2.T.contiguous())
    c = torch.full((M + 3, N + 5), 7.0, device=dev())
    K.gemm_f32(layout, A.to(dev()), B.to(dev()), c[:M, :N], M=M, N=N, K=Kd,
               b_minus=None if B2 is None else B2.to(dev()))
    got = c.double().cpu()
    assert torch.all((got[:M, :N] - want).abs() <= (Kd + 4) * 2.0**-23 * mags + 1e-30)
    assert torch.all(got[M:] == 7.0) and torch.all(got[:, N:] == 7.0)
    # deterministic
    c2 = torch.empty(M, N, device=dev())
    K.gemm_f32(layout, A.to(dev()), B.to(dev()), c2, M=M, N=N, K=Kd, b_minus=None if B2 is None else B2.to(dev()))
    assert torch.equal(c2.cpu(), c[:M, :N].cpu())
