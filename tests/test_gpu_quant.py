"""GPU parity of fake-quant forward, codes, STE backward and the fused step.

Each case runs the HIP path through the C ABI (``mround_amd.kernels``) and the
float32 oracle on the same seeded inputs. Codes, scales, zero points and
reconstructions must be bit-identical; the per-element gradient of v and the
updated v must be bit-identical; the per-group gradient sums differ only by
summation order, so they must agree within 4 fp32 ulps of ``sum |term|``
(the order-independent error scale), and the updated coefficients must agree
wherever the gradient's sign is unambiguous at that scale.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from mround_amd.core import quantizer as QZ
from mround_amd.core import signsgd as SG
from mround_amd.schemes import QuantScheme
from oracle import quantize as Q
from tests.helpers import dev, oracle_fq, params, to_np, weight

pytestmark = pytest.mark.gpu

SCHEMES = {
    "asym": dict(symmetry="asym"),
    "sym": dict(symmetry="sym"),
    "searched": dict(symmetry="sym", scale_init="searched"),
}

SHAPES = [  # (rows, cols, group_size): fast path, per-channel, padded, odd
    (48, 256, 64), (40, 384, 32), (32, 512, 128), (24, 96, 8), (16, 200, -1), (12, 100, 32),
    (8, 4096, -1), (10, 72, 24),
]


def _scheme(mode, bits, gs):
    return QuantScheme(bits=bits, group_size=gs, **SCHEMES[mode])


def _init_scale(rows, cols, gs, seed=5):
    ng = 1 if gs == -1 else -(-cols // gs)
    g = torch.Generator().manual_seed(seed)
    return -(torch.rand(rows, ng, 1, generator=g) * 0.01 + 0.002)


def _note(*case):
    print("case", *case, flush=True, file=sys.stderr)


@pytest.mark.parametrize("mode", ["asym", "sym", "searched"])
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_forward_bit_exact(mode, bits, shape, wdtype):
    rows, cols, gs = shape
    _note("fwd", mode, bits, shape, wdtype)
    w = weight(rows, cols, seed=bits + rows, dtype=wdtype)
    v, a, b = params(rows, cols, gs, seed=bits, coef_jitter=0.3)
    init = _init_scale(rows, cols, gs) if mode == "searched" else None
    scheme = _scheme(mode, bits, gs)
    wn = to_np(w)
    for use_params in (True, False):
        p = {"v": v.to(dev()), "alpha": a.to(dev()), "beta": b.to(dev())} if use_params else None
        init_d = init.to(dev()) if init is not None else None
        got32 = QZ.fake_quantize(w.to(dev()), p, scheme, init_scale=init_d, out_dtype=torch.float32)
        got16 = QZ.fake_quantize(w.to(dev()), p, scheme, init_scale=init_d, out_dtype=torch.bfloat16)
        codes, scale, zp = QZ.quantize_codes(w.to(dev()), p, scheme, init_scale=init_d, narrow=True)
        ref_q, ref_c, ref_s, ref_zp = oracle_fq(wn, v if use_params else None, a, b, bits, gs, mode,
                                                None if init is None else init.numpy())
        assert np.array_equal(to_np(got32), ref_q), "fp32 reconstruction differs"
        assert np.array_equal(to_np(got16), Q.round_to_bf16(ref_q)), "bf16 reconstruction differs"
        assert np.array_equal(to_np(codes).astype(np.int64), ref_c.astype(np.int64)), "codes differ"
        assert np.array_equal(to_np(scale), ref_s), "scales differ"
        if mode == "asym":
            assert np.array_equal(to_np(zp), ref_zp), "zero points differ"
        else:
            assert zp is None


def _grad_tolerance(w, v, a, b, g, bits, gs, mode, init):
    ts, td = Q.grad_terms(w, v, a, b, g, bits=bits, group_size=gs, mode=mode,
                          init_scale=init, dtype=np.float32)
    scale_s = np.abs(ts.astype(np.float64)).sum(-1, keepdims=True)
    scale_d = np.abs(td.astype(np.float64)).sum(-1, keepdims=True)
    return scale_s, scale_d


@pytest.mark.parametrize("mode", ["asym", "sym", "searched"])
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
def test_backward_and_fused_step(mode, bits, shape, gdtype):
    rows, cols, gs = shape
    _note("bwd", mode, bits, shape, gdtype)
    w = weight(rows, cols, seed=3 * bits + cols, dtype=torch.bfloat16)
    v, a, b = params(rows, cols, gs, seed=bits + 7, vrange=0.45, coef_jitter=0.4)
    g = (torch.randn(rows, cols, generator=torch.Generator().manual_seed(bits)) * 1e-3).to(gdtype)
    init = _init_scale(rows, cols, gs) if mode == "searched" else None
    scheme = _scheme(mode, bits, gs)
    wn, gn = to_np(w), to_np(g)
    init_np = None if init is None else init.numpy()
    ref_gv, ref_ga, ref_gb = Q.quantize_grad(wn, v.numpy(), a.numpy(), b.numpy(), gn, bits=bits,
                                             group_size=gs, mode=mode, init_scale=init_np,
                                             dtype=np.float32)
    p = {"v": v.to(dev()), "alpha": a.to(dev()), "beta": b.to(dev())}
    init_d = None if init is None else init.to(dev())
    got = QZ.quantize_grad(w.to(dev()), p, scheme, g.to(dev()), init_scale=init_d)
    assert np.array_equal(to_np(got["v"]), ref_gv), "grad v differs"
    ss, sd = _grad_tolerance(wn, v.numpy(), a.numpy(), b.numpy(), gn, bits, gs, mode, init_np)
    eps32 = np.finfo(np.float32).eps
    # Summation-order error bound: each lane sums its share of the group in
    # order, then a butterfly (fast path) or wave reduction (generic path);
    # |ds/dcoef| <= 1 for these weights.
    gs_eff = cols if gs == -1 else gs
    tol = (gs_eff / 64 + 16) * eps32 * (ss + sd) + 1e-30
    ga, gb = to_np(got["alpha"]), to_np(got["beta"])
    assert np.all(np.abs(ga - ref_ga) <= tol), "grad alpha differs"
    assert np.all(np.abs(gb - ref_gb) <= tol), "grad beta differs"

    lr = 0.005
    SG.fused_step(w.to(dev()), p, g.to(dev()), scheme, lr, init_scale=init_d)
    lo, hi = scheme.coefficient_bounds
    ref_v = np.clip(v.numpy() - np.float32(lr) * np.sign(ref_gv), -0.5, 0.5)
    assert np.array_equal(to_np(p["v"]), ref_v), "updated v differs"
    for name, ref_grad, base in (("alpha", ref_ga, a.numpy()), ("beta", ref_gb, b.numpy())):
        ref_new = np.clip(base - np.float32(lr) * np.sign(ref_grad), lo, hi)
        clear = np.abs(ref_grad) > tol
        assert np.array_equal(to_np(p[name])[clear], ref_new[clear]), f"updated {name} differs"


def test_fused_step_equals_separate_update():
    """fused_step == project(SignSGD.apply(quantize_grad)) on the device."""
    rows, cols, gs = 64, 512, 64
    scheme = QuantScheme(bits=2, group_size=gs, symmetry="asym")
    w = weight(rows, cols, seed=11).to(dev())
    v, a, b = params(rows, cols, gs, seed=12, coef_jitter=0.2)
    p = {"v": v.to(dev()), "alpha": a.to(dev()), "beta": b.to(dev())}
    g = (torch.randn(rows, cols, generator=torch.Generator().manual_seed(13)) * 1e-3).to(dev())
    grads = QZ.quantize_grad(w, p, scheme, g)
    opt = SG.SignSGD(SG.LinearDecay(0.005, 200))
    separate = QZ.project_params(opt.apply(p, grads), scheme)
    SG.fused_step(w, p, g, scheme, 0.005)
    for k in ("v", "alpha", "beta"):
        assert torch.equal(separate[k], p[k]), k


def test_full_size_rows_sampled():
    """The 18944 x 3584 bf16 microbench matrix: sampled rows match the oracle bit for bit."""
    rows, cols, gs, bits = 18944, 3584, 64, 2
    w = weight(rows, cols, seed=0)
    v, a, b = params(rows, cols, gs, seed=2)
    scheme = QuantScheme(bits=bits, group_size=gs, symmetry="asym")
    p = {"v": v.to(dev()), "alpha": a.to(dev()), "beta": b.to(dev())}
    got = QZ.fake_quantize(w.to(dev()), p, scheme)
    sel = np.r_[0:64, 9000:9064, rows - 64:rows]
    ref = oracle_fq(to_np(w)[sel], v[sel], a[sel], b[sel], bits, gs, "asym")[0]
    assert np.array_equal(to_np(got)[sel], Q.round_to_bf16(ref))


def test_zero_rows_and_validation():
    scheme = QuantScheme(bits=4, group_size=64, symmetry="asym")
    w = torch.zeros(0, 128, dtype=torch.bfloat16, device=dev())
    assert QZ.fake_quantize(w, None, scheme).shape == (0, 128)
    with pytest.raises(ValueError, match="searched scale"):
        QZ.fake_quantize(torch.zeros(4, 64, device=dev()), None,
                         QuantScheme(bits=4, group_size=64, scale_init="searched"))


@pytest.mark.parametrize("shape", [(64, 512, 64), (96, 256, 32), (32, 200, -1), (16, 4, -1)])
def test_mapped_placement(shape):
    """W' rows placed in a stacked / interleaved buffer, gradients read back the same way."""
    from mround_amd import kernels as K

    rows, cols, gs = shape
    scheme = QuantScheme(bits=2, group_size=gs, symmetry="asym")
    w = weight(rows, cols, seed=rows).to(dev())
    v, a, b = params(rows, cols, gs, seed=3, coef_jitter=0.2)
    ref = QZ.fake_quantize(w, {"v": v.to(dev()), "alpha": a.to(dev()), "beta": b.to(dev())}, scheme)
    big = torch.zeros(2 * rows + 64, cols, dtype=torch.bfloat16, device=dev())
    for blk, stride, off in ((rows, 0, 17), (32, 64, 32), (32, 64, 0)):
        if blk == 32 and rows % 32:
            continue
        big.zero_()
        K.fq_forward_mapped(w, v.to(dev()), a.to(dev()), b.to(dev()), bits=2, group_size=gs,
                            mode="asym", eps=1e-8, wq_out=big, row_block=blk, row_stride=stride,
                            row_offset=off)
        idx = torch.tensor([(r // blk) * stride + off + r % blk for r in range(rows)])
        assert torch.equal(big[idx.to(dev())], ref)
        # the fused step reading g from the same placement equals the plain one
        g = torch.randn(rows, cols, generator=torch.Generator().manual_seed(5)).to(dev()) * 1e-3
        gbig = torch.zeros(2 * rows + 64, cols, device=dev())
        gbig[idx.to(dev())] = g
        p1 = {"v": v.clone().to(dev()), "alpha": a.clone().to(dev()), "beta": b.clone().to(dev())}
        p2 = {k: t.clone() for k, t in p1.items()}
        SG.fused_step(w, p1, g, scheme, 0.005)
        K.fq_step_mapped(w, p2["v"], p2["alpha"], p2["beta"], gbig, bits=2, group_size=gs,
                         mode="asym", eps=1e-8, lr=0.005, coef_lo=0.1, coef_hi=1.0, v_bound=0.5,
                         row_block=blk, row_stride=stride, row_offset=off)
        for k in p1:
            assert torch.equal(p1[k], p2[k]), k


@pytest.mark.parametrize("shape", [(64, 512, 64), (96, 256, 32), (32, 200, -1)])
@pytest.mark.parametrize("mode", ["asym", "sym", "searched"])
def test_step_requant_writes_the_next_forward(shape, mode):
    """The fused step that also writes W' leaves the parameters exactly as the
    plain fused step does, and its W' (placed) is bit-identical to the forward
    of the updated parameters; rows outside the placement are untouched."""
    from mround_amd import kernels as K

    rows, cols, gs = shape
    print("case step requant", shape, mode, flush=True, file=sys.stderr)
    w = weight(rows, cols, seed=rows + 1).to(dev())
    v, a, b = params(rows, cols, gs, seed=4, coef_jitter=0.2)
    ng = 1 if gs == -1 else cols // gs
    init = None
    if mode == "searched":
        init = (torch.rand(rows, ng, generator=torch.Generator().manual_seed(6)) * 0.02 + 0.005).to(dev())
    lo, hi = (0.5, 1.5) if mode == "searched" else (0.1, 1.0)
    g = torch.randn(rows, cols, generator=torch.Generator().manual_seed(7)).to(dev()) * 1e-3
    for blk, stride, off in ((rows, 0, 17), (32, 64, 32)):
        if blk == 32 and rows % 32:
            continue
        idx = torch.tensor([(r // blk) * stride + off + r % blk for r in range(rows)]).to(dev())
        gbig = torch.zeros(2 * rows + 64, cols, device=dev())
        gbig[idx] = g
        p1 = [t.clone().to(dev()).contiguous() for t in (v.reshape(rows, -1), a.reshape(rows, ng),
                                                          b.reshape(rows, ng))]
        p2 = [t.clone() for t in p1]
        common = dict(bits=2, group_size=gs, mode=mode, eps=1e-8, lr=0.005, coef_lo=lo, coef_hi=hi,
                      v_bound=0.5, row_block=blk, row_stride=stride, row_offset=off, init_scale=init)
        K.fq_step_mapped(w, *p1, gbig, **common)
        wbig = torch.full((2 * rows + 64, cols), 7.0, dtype=torch.bfloat16, device=dev())
        K.fq_step_requant_mapped(w, *p2, gbig, wq_out=wbig, **common)
        for x, y in zip(p1, p2):
            assert torch.equal(x, y)
        ref = torch.zeros_like(wbig)
        K.fq_forward_mapped(w, *p1, bits=2, group_size=gs, mode=mode, eps=1e-8, wq_out=ref, row_block=blk,
                            row_stride=stride, row_offset=off, init_scale=init)
        assert torch.equal(wbig[idx], ref[idx])
        mask = torch.ones(wbig.shape[0], dtype=torch.bool, device=dev())
        mask[idx] = False
        assert bool((wbig[mask] == 7.0).all())
