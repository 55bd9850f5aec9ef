"""GPU parity of packing, affine metadata, losses and DeltaLoss.

Packed words, unpacked codes and affine metadata must be bit-identical to the
oracle; the outlier threshold must equal the k-th largest |r| exactly (it is
a selection, not an approximation); losses agree within 1e-6 relative (fp64
sums on both sides, fp32 terms) and gradients bit for bit; DeltaLoss within
1e-9 relative of the fp64 sum of the oracle's fp32 terms.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from mround_amd import kernels as K
from mround_amd.core import losses as LS
from mround_amd.core import quantizer as QZ
from mround_amd.formats import mlx_export as MX
from mround_amd.formats import packing as PK
from mround_amd.schemes import QuantScheme
from oracle import losses as OL
from oracle import packing as OP
from oracle import quantize as Q
from oracle import sensitivity as OS
from tests.helpers import dev, to_np, weight

pytestmark = pytest.mark.gpu


def _note(*case):
    print("case", *case, flush=True, file=sys.stderr)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("shape", [(17, 128), (64, 3584), (3, 32), (5, 4096)])
def test_pack_unpack_bit_exact(bits, shape):
    _note("pack", bits, shape)
    rows, cols = shape
    codes = np.random.default_rng(bits * 1000 + cols).integers(0, 2**bits, size=shape).astype(np.uint8)
    packed = PK.pack_codes(torch.from_numpy(codes).to(dev()), bits)
    ref = OP.pack_codes(codes.astype(np.int64), bits)
    assert np.array_equal(to_np(packed.view(torch.int32)).view(np.uint32), ref)
    assert np.array_equal(ref, OP.mlx_style_pack(codes, bits))
    back = PK.unpack_codes(packed, cols, bits)
    assert np.array_equal(to_np(back), codes)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_pack_even_widths_short_rows(bits):
    per = 32 // bits
    cols = per * 3  # not a multiple of 32: word-per-lane kernel
    codes = np.random.default_rng(bits).integers(0, 2**bits, size=(7, cols)).astype(np.uint8)
    packed = PK.pack_codes(torch.from_numpy(codes).to(dev()), bits)
    ref = OP.pack_codes(codes.astype(np.int64), bits)
    assert np.array_equal(to_np(packed.view(torch.int32)).view(np.uint32), ref)
    assert np.array_equal(to_np(PK.unpack_codes(packed, cols, bits)), codes)


def test_pack_known_answer_and_range_errors():
    codes = torch.arange(8, dtype=torch.uint8, device=dev()).reshape(1, 8)
    assert int(PK.pack_codes(codes, 4).view(torch.int32)[0, 0]) == 0x76543210
    bad = torch.tensor([[0, 16, 3, 4, 5, 6, 7, 8]], dtype=torch.uint8, device=dev())
    with pytest.raises(ValueError, match=r"codes must lie in \[0, 15\] at 4 bits, got \[0, 16\]"):
        PK.pack_codes(bad, 4)
    signed = torch.tensor([[-9] + [0] * 31], dtype=torch.int8, device=dev())
    with pytest.raises(ValueError, match="codes must lie in"):
        PK.pack_codes(signed, 4, offset=8)
    with pytest.raises(ValueError, match="expected 8 words per row"):
        PK.unpack_codes(torch.zeros(2, 3, dtype=torch.uint32, device=dev()), 64, 4)


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("symmetry", ["asym", "sym"])
@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_export_tensors_bit_exact(bits, symmetry, dtype):
    _note("export", bits, symmetry, dtype)
    scheme = QuantScheme(bits=bits, group_size=64, symmetry=symmetry)
    w = weight(32, 512, seed=bits)
    codes, scale, zp = QZ.quantize_codes(w.to(dev()), None, scheme, narrow=True)
    layer = MX.QuantizedLayer(codes, scale, zp, scheme)
    td = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}[dtype]
    tensors = MX._tensors_for_layer("m.q", layer, td)
    flat = to_np(codes).astype(np.int64).reshape(32, 512)
    if symmetry == "sym":
        flat = flat + 2 ** (bits - 1)
    ref_packed = OP.pack_codes(flat, bits)
    got_packed = to_np(tensors["m.q.weight"].view(torch.int32)).view(np.uint32)
    assert np.array_equal(got_packed, ref_packed)
    ref_s, ref_b = OP.to_affine(to_np(scale).reshape(32, 8),
                                None if zp is None else to_np(zp).reshape(32, 8), bits, dtype)
    assert np.array_equal(tensors["m.q.scales"].float().cpu().numpy(), ref_s)
    assert np.array_equal(tensors["m.q.biases"].float().cpu().numpy(), ref_b)
    if symmetry == "sym":
        s = tensors["m.q.scales"].float()
        assert torch.all(s * 2 ** (bits - 1) + tensors["m.q.biases"].float() == 0)


# ------------------------------------------------------- fused quantize+pack --

QP_SCHEMES = {"asym": dict(symmetry="asym"), "sym": dict(symmetry="sym"),
              "searched": dict(symmetry="sym", scale_init="searched")}


@pytest.mark.parametrize("mode", ["asym", "sym", "searched"])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("learned", [False, True])
def test_quantize_pack_equals_the_separate_chain(mode, bits, gs, learned):
    """mr_quantize_pack against quantize_codes -> pack_codes -> to_affine on the
    same weight and parameters: words, scales and biases identical, in every
    output dtype."""
    rows, cols = 40, 512
    print("case quantize_pack", mode, bits, gs, learned, flush=True, file=sys.stderr)
    scheme = QuantScheme(bits=bits, group_size=gs, **QP_SCHEMES[mode])
    w = weight(rows, cols, seed=bits * gs, std=0.05).to(dev())
    params = None
    if learned:
        g = torch.Generator().manual_seed(bits + gs)
        params = {"v": ((torch.rand(rows, cols // gs, gs, generator=g) - 0.5) * 0.9).to(dev()),
                  "alpha": (1 - 0.4 * torch.rand(rows, cols // gs, 1, generator=g)).to(dev()),
                  "beta": (1 - 0.4 * torch.rand(rows, cols // gs, 1, generator=g)).to(dev())}
    init = None
    if mode == "searched":
        init = -(torch.rand(rows, cols // gs, 1, generator=torch.Generator().manual_seed(9)) * 0.01 + 0.002).to(dev())
    codes, scale, zp = QZ.quantize_codes(w, params, scheme, init_scale=init, narrow=True)
    off = 0 if mode == "asym" else 2 ** (bits - 1)
    want_words = PK.pack_codes(codes.reshape(rows, cols), bits, offset=off)
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        words, scales, biases = QZ.quantize_pack(w, params, scheme, init_scale=init, dtype=dtype)
        assert torch.equal(words.view(torch.int32), want_words.view(torch.int32)), dtype
        ws, wb = MX.to_affine(scale, zp, scheme, dtype=dtype)
        assert torch.equal(scales, ws.reshape(rows, -1)) and torch.equal(biases, wb.reshape(rows, -1)), dtype


def test_quantize_pack_against_the_oracle():
    """Round to nearest at 3 bits (words straddle): the oracle's codes packed by
    the oracle, and the oracle's affine metadata."""
    rows, cols, gs, bits = 64, 1024, 64, 3
    w = weight(rows, cols, seed=77)
    scheme = QuantScheme(bits=bits, group_size=gs, symmetry="asym")
    words, scales, biases = QZ.quantize_pack(w.to(dev()), None, scheme, dtype=torch.bfloat16)
    _, c, s, z = Q.fake_quantize(to_np(w), None, None, None, bits=bits, group_size=gs, mode="asym")
    assert np.array_equal(words.view(torch.int32).cpu().numpy().view(np.uint32),
                          OP.pack_codes(c.reshape(rows, cols).astype(np.int64), bits))
    ws, wb = OP.to_affine(s.reshape(rows, -1), z.reshape(rows, -1), bits, "bfloat16")
    assert np.array_equal(scales.float().cpu().numpy(), ws) and np.array_equal(biases.float().cpu().numpy(), wb)


def test_quantize_pack_refuses_what_it_cannot_pack():
    w = weight(8, 96, seed=1).to(dev())
    with pytest.raises(Exception, match="power-of-two group size"):
        QZ.quantize_pack(w, None, QuantScheme(bits=4, group_size=48, symmetry="asym"))
    with pytest.raises(Exception, match="power-of-two group size"):
        QZ.quantize_pack(weight(8, 80, seed=1).to(dev()), None, QuantScheme(bits=4, group_size=16, symmetry="asym"))


@pytest.mark.parametrize("n", [1000, 4096, 2_359_296, 3 * 1024 + 1])
def test_mse_loss_and_grad(n):
    _note("mse", n)
    gen = torch.Generator().manual_seed(n)
    pred = torch.randn(n, generator=gen)
    ref = torch.randn(n, generator=gen)
    loss, grad = LS.reconstruction_loss(pred.to(dev()), ref.to(dev()), with_grad=True)
    r = (pred - ref).numpy()
    expect = float(np.sum(r.astype(np.float64) ** 2) / n)
    assert float(loss) == pytest.approx(expect, rel=1e-6)
    np.testing.assert_array_equal(to_np(grad), r * np.float32(2.0 / n))


@pytest.mark.parametrize("n", [2000, 2001, 4097, 1 << 20, 2_359_296, 58_720_256 // 8])
def test_outlier_threshold_exact(n):
    _note("outlier", n)
    gen = torch.Generator().manual_seed(n + 1)
    pred = torch.randn(n, generator=gen) * 0.1
    pred[: n // 500] *= 50.0
    ref = torch.zeros(n)
    thr = torch.empty((), device=dev())
    loss, grad = LS.outlier_suppressed_loss(pred.to(dev()), ref.to(dev()), with_grad=True,
                                            threshold_out=thr)
    r = pred.numpy()
    ref_loss, ref_grad, ref_thr = OL.outlier_suppressed_loss(r, np.zeros_like(r))
    assert float(thr) == float(ref_thr)
    assert float(loss) == pytest.approx(ref_loss, rel=1e-6)
    keep = np.abs(r) < ref_thr
    np.testing.assert_array_equal(to_np(grad), np.where(keep, r, 0).astype(np.float32) * np.float32(2.0 / n))


@pytest.mark.parametrize("n", [4096, 4099, 1 << 20])
def test_outlier_threshold_constant_residual(n):
    """Every residual equal: the k-th largest is that value and every element
    is tied with it, so the loss and gradient are zero."""
    _note("outlier constant", n)
    pred = torch.full((n,), 0.75)
    thr = torch.empty((), device=dev())
    loss, grad = LS.outlier_suppressed_loss(pred.to(dev()), torch.zeros(n, device=dev()),
                                            with_grad=True, threshold_out=thr)
    assert float(thr) == 0.75
    assert float(loss) == 0.0
    assert not torch.any(grad.cpu())


def test_outlier_ties_all_excluded_and_pieces():
    pred = torch.tensor([1.0, 5.0, 5.0, 2.0] + [0.5] * 996)
    thr = torch.empty((), device=dev())
    loss, grad = LS.outlier_suppressed_loss(pred.to(dev()), torch.zeros(1000, device=dev()),
                                            with_grad=True, threshold_out=thr)
    assert float(thr) == 5.0
    g = grad.cpu()
    assert g[1] == 0 and g[2] == 0 and g[0] != 0
    # pieces with the batch threshold sum to the batch loss
    parts = sum(float(LS.piece_loss(pred[i:i + 250].to(dev()), torch.zeros(250, device=dev()),
                                    elements=1000, threshold=thr)) for i in range(0, 1000, 250))
    assert parts == pytest.approx(float(loss), rel=1e-6)


@pytest.mark.parametrize("mode", ["asym", "sym"])
@pytest.mark.parametrize("shape", [(64, 512, 64), (896, 896, 64), (128, 1024, 32), (32, 256, 128)])
def test_delta_loss(mode, shape):
    _note("delta", mode, shape)
    rows, cols, gs = shape
    w = weight(rows, cols, seed=rows)
    g = torch.randn(rows, cols, generator=torch.Generator().manual_seed(cols)) * 1e-2
    scores = torch.zeros(3, dtype=torch.float64, device=dev())
    K.delta_loss(w.to(dev()), g.to(dev()), group_size=gs, bits_list=[2, 3, 4], mode=mode, eps=1e-8,
                 scores_out=scores)
    K.delta_loss(w.to(dev()), g.to(dev()), group_size=gs, bits_list=[2, 3, 4], mode=mode, eps=1e-8,
                 scores_out=scores)  # accumulates
    for i, bits in enumerate((2, 3, 4)):
        terms = OS.delta_terms_f32(to_np(w), g.numpy(), bits=bits, group_size=gs, mode=mode)
        expect = 2 * float(np.sum(terms.astype(np.float64)))
        assert float(scores[i]) == pytest.approx(expect, rel=1e-9)
        # and against the float64 definition (fp32 perturbation vs fp64 product): close
        q, *_ = __import__("oracle.quantize", fromlist=["x"]).fake_quantize(
            to_np(w), None, None, None, bits=bits, group_size=gs, mode=mode)
        assert float(scores[i]) == pytest.approx(2 * OS.delta_loss(to_np(w), q, g.numpy()), rel=1e-5)


def test_copy_kernel():
    src = torch.randint(0, 255, (1 << 20,), dtype=torch.uint8, device=dev())
    dst = torch.empty_like(src)
    K.copy_bytes(src, dst, src.numel())
    assert torch.equal(src, dst)
