"""GPU scale search and importance against the oracle, and the searched
block tune end to end (symmetric 2-bit, commit bit-exact with the oracle)."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from mround_amd import kernels as K
from mround_amd.core.scale_search import SearchGrid, search_scales
from mround_amd.pipeline.block import LAYERS, BlockShape, BlockWeights
from mround_amd.pipeline.runner import DecoderBlock, QuantizationRunner
from mround_amd.schemes import QuantScheme, ScaleInit, Symmetry, TuningConfig
from oracle import quantize as OQ
from oracle import scale_search as OS
from tests.helpers import dev, weight

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("with_imp", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_search_bit_exact_with_the_float32_oracle(bits, gs, with_imp, dtype):
    print("case search", bits, gs, with_imp, dtype, flush=True, file=sys.stderr)
    w = weight(96, 512, seed=bits * 7 + gs, dtype=dtype)
    w[3, :gs] = 0  # an all-zero group
    w[5, :4] = torch.tensor([0.5, -0.5, 0.25, 0.5], dtype=dtype)  # magnitude ties: first wins
    imp = (torch.rand(512, generator=torch.Generator().manual_seed(gs)) * 10 + 0.1) if with_imp else None
    scheme = QuantScheme(bits=bits, group_size=gs, symmetry=Symmetry.SYMMETRIC,
                         scale_init=ScaleInit.SEARCHED)
    got = search_scales(w.to(dev()), scheme, importance=None if imp is None else imp.to(dev())).cpu().numpy()
    want = OS.search_scales_f32(w.float().numpy(), bits, gs, importance=None if imp is None else imp.numpy())
    assert got.shape == want.shape
    assert np.array_equal(got, want)
    assert got.reshape(96, -1)[3, 0] == 0.0
    ref64 = OS.search_scales(w.float().numpy(), bits, gs, importance=None if imp is None else imp.numpy())
    assert np.isclose(got, ref64, rtol=1e-6, atol=0).mean() >= 0.98


def test_search_grid_matches_oracle():
    for bits in (2, 3, 4, 5, 8):
        assert SearchGrid().steps(bits) == OS.grid_steps(bits)


def test_search_rejects():
    w = torch.zeros(4, 64, device=dev())
    with pytest.raises(ValueError, match="symmetric"):
        search_scales(w, QuantScheme(bits=2, group_size=64, symmetry=Symmetry.ASYMMETRIC))
    with pytest.raises(ValueError, match="channels"):
        search_scales(w, QuantScheme(bits=2, group_size=64), importance=torch.ones(32, device=dev()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_colsumsq(dtype):
    x = torch.randn(3000, 700, generator=torch.Generator().manual_seed(1)).to(dtype)
    out = torch.full((700,), 2.0, device=dev())
    K.colsumsq(x.to(dev()), out)
    want = 2.0 + (x.double() ** 2).sum(0)
    assert torch.allclose(out.double().cpu(), want, rtol=1e-5, atol=0)
    xs = x.to(dev())[:, 50:650]
    out2 = torch.zeros(600, device=dev())
    K.colsumsq(xs, out2)
    assert torch.allclose(out2.double().cpu(), (x[:, 50:650].double() ** 2).sum(0), rtol=1e-5)


def test_searched_block_tune_commits_bit_exact():
    shape = BlockShape(hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, intermediate=256, attn_bias=True)
    B, S = 2, 128
    w = BlockWeights.random(shape, dtype=torch.bfloat16, device=dev(), seed=4, std=0.05)
    g = torch.Generator().manual_seed(9)
    inputs = [torch.randn(B * S, 128, generator=g).to(dev()) for _ in range(2)]
    scheme = QuantScheme(bits=2, group_size=64, symmetry=Symmetry.SYMMETRIC, scale_init=ScaleInit.SEARCHED)
    runner = QuantizationRunner(scheme, TuningConfig(iters=8, batch_size=B, n_samples=2 * B, seq_len=S,
                                                     lr=0.005))
    originals = {n: t.clone() for n, t in w.linears.items()}
    # targets from the original block
    eng = runner.engine(shape, B * S, torch.device(dev()))
    eng.set_block(w)
    eng.load_dense(w.linears)
    targets = []
    for x in inputs:
        t = torch.empty_like(x)
        eng.forward(x, t, save=False)
        targets.append(t)
    captured = {}
    orig_commit = runner._commit

    def spy(blk, layer):
        captured[layer.name] = (layer.v.cpu().clone(), layer.alpha.cpu().clone(), layer.beta.cpu().clone(),
                                layer.init_scale.cpu().clone())
        return orig_commit(blk, layer)

    runner._commit = spy
    block = DecoderBlock(0, "b", shape, w)
    res, layers = runner.quantize_block(block, inputs, targets, path_prefix="b")
    assert res.search_seconds > 0
    assert res.final_loss <= res.initial_loss
    for n in LAYERS:
        v, a, b, init = captured[n]
        rows, cols = originals[n].shape
        wq, codes, scale, _ = OQ.fake_quantize(originals[n].float().cpu().numpy(), v.numpy(), a.numpy(),
                                               b.numpy(), bits=2, group_size=64, mode="searched",
                                               init_scale=init.numpy().reshape(rows, -1, 1))
        q = layers[f"b.{n}"]
        assert q.codes.dtype == torch.int8
        assert np.array_equal(q.codes.cpu().numpy().astype(np.float32), codes.reshape(q.codes.shape))
        assert np.array_equal(q.scale.cpu().numpy(), scale.reshape(q.scale.shape))
        assert np.array_equal(block.weights.linears[n].float().cpu().numpy(),
                              OQ.round_to_bf16(wq.astype(np.float32)))
