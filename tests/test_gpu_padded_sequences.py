"""Sequences whose length is not a multiple of the attention tile (128): the
block loop runs each sequence on ``aligned_length(seq_len)`` rows, the rows
past ``seq_len`` being padding at the sequence's end. The reference tunes on
sequences of any ``seq_len`` (``TuningConfig.seq_len``, mround/schemes.py:266;
``calibration.py:442`` asks only for seq_len >= 1), so the padded run must be
the run on the ``seq_len``-token sequences:

* padding never reaches a token row, the loss or a gradient: whatever
  finite values the padding rows hold, the loss, the outlier threshold and
  every dL/dW' are bit-identical (causal attention keeps later rows out of
  earlier ones, and the padding rows' residuals are zero, so their gradient
  terms are exact zeros: 0 times a finite activation; an inf or NaN padding
  row would make them NaN, and the API pads with token 0's embedding, which
  is finite);
* the loss and dL/dW' match the float64 oracle run on the unpadded
  ``seq_len``-token sequences, within the bars of the unpadded block tests
  (loss 1e-2 relative, dL/dW' 5e-2 normwise with under 1e-2 of the gradient
  mass of the wrong sign);
* a tune's step losses follow the oracle's tune of the unpadded sequences
  within 1e-2, with the same revert decision;
* a step in pieces equals the whole-batch step, as without padding;
* ``api.quantize`` runs end to end at such a length.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from mround_amd import api
from mround_amd.pipeline.block import LAYERS, BlockShape, BlockWeights, aligned_length, placements, unplace
from mround_amd.pipeline.checkpoint import write_random_checkpoint
from mround_amd.pipeline.runner import DecoderBlock, QuantizationRunner
from mround_amd.schemes import QuantScheme, Symmetry, TuningConfig
from oracle import block as OB
from oracle import quantize as OQ
from tests.helpers import dev

pytestmark = pytest.mark.gpu

SHAPE = BlockShape(hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, intermediate=256, rope_theta=1e6,
                   attn_bias=True)
D128 = BlockShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, attn_bias=True)


def _case(*a):
    print("case", *a, flush=True, file=sys.stderr)


def _oshape(s: BlockShape) -> OB.Shape:
    return OB.Shape(hidden=s.hidden, n_heads=s.n_heads, n_kv_heads=s.n_kv_heads, head_dim=s.head_dim,
                    intermediate=s.intermediate, norm_eps=s.norm_eps, rope_theta=s.rope_theta,
                    attn_bias=s.attn_bias)


def _weights(shape, seed):
    w = BlockWeights.random(shape, dtype=torch.bfloat16, device="cpu", seed=seed, std=0.05)
    g = torch.Generator().manual_seed(seed + 100)
    w.input_norm = 1 + 0.1 * torch.randn(shape.hidden, generator=g)
    w.post_norm = 1 + 0.1 * torch.randn(shape.hidden, generator=g)
    if shape.attn_bias:
        w.biases = {n: torch.randn(shape.linear_shape(n)[0], generator=g) * 0.1 for n in w.biases}
    return w


def _dev(w):
    return BlockWeights({n: t.to(dev()) for n, t in w.linears.items()},
                        {n: t.to(dev()) for n, t in w.biases.items()}, w.input_norm.to(dev()),
                        w.post_norm.to(dev()))


def _oracle(shape, w, x, linears=None):
    """Block output of ``x`` ``[B, L, h]`` (unpadded) in float64."""
    lin = {n: (linears or w.linears)[n].double() for n in LAYERS}
    biases = {n: b.double() for n, b in w.biases.items()}
    norms = (w.input_norm.double(), w.post_norm.double())
    return OB.block_forward(x.double(), lin, biases, norms, _oshape(shape))


def _pad(t: torch.Tensor, rows: int, fill: torch.Tensor | None = None) -> torch.Tensor:
    """``[B, L, h]`` -> ``[B * rows, h]``, the rows past L from ``fill`` (or zero)."""
    B, L, h = t.shape
    out = torch.zeros(B, rows, h, dtype=torch.float32)
    out[:, :L] = t.float()
    if fill is not None:
        out[:, L:] = fill
    return out.reshape(B * rows, h)


def _rtn_bf16(w: torch.Tensor) -> torch.Tensor:
    qdq, _, _, _ = OQ.fake_quantize(w.float().numpy(), None, None, None, bits=2, group_size=64, mode="asym")
    return torch.from_numpy(np.ascontiguousarray(qdq)).to(torch.bfloat16)


def test_aligned_length():
    assert [aligned_length(n) for n in (1, 127, 128, 129, 200, 2048, 2049)] == [128, 128, 128, 256, 256,
                                                                              2048, 2176]


def _engine_step(shape, w, wq, x, t, real, suppress, pieces=1):
    """(loss, threshold, {operand: dL/dW'}) of one step through the runner's
    step at ``real`` tokens per padded sequence."""
    B = x.shape[0] // aligned_length(real)
    runner = QuantizationRunner(QuantScheme(bits=2, group_size=64, symmetry=Symmetry.ASYMMETRIC),
                                TuningConfig(iters=2, batch_size=B, n_samples=B, seq_len=real,
                                             micro_batches=pieces))
    eng = runner.engine(shape, x.shape[0], dev())
    assert eng.seq_len == aligned_length(real) and eng.real_len == real
    eng.set_block(_dev(w))
    eng.load_dense({n: t_.to(dev()) for n, t_ in wq.items()})
    loss = torch.zeros(1, device=dev())
    xd, td = x.to(dev()), t.to(dev())
    runner._gradients(eng, xd, td, torch.empty_like(xd), suppress, loss)
    torch.cuda.synchronize()
    return float(loss), float(eng.threshold), {k: v.clone() for k, v in eng.dw.items()}


@pytest.mark.parametrize("suppress", [False, True])
@pytest.mark.parametrize("real", [200, 129])
def test_padding_rows_reach_no_loss_or_gradient(real, suppress):
    _case("padding invariance", real, suppress)
    B, rows = 2, aligned_length(real)
    w = _weights(SHAPE, seed=7)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(B, real, SHAPE.hidden, generator=g)
    with torch.no_grad():
        t = _oracle(SHAPE, w, x).float()
    wq = {n: (w.linears[n].float() * 1.01).to(torch.bfloat16) for n in LAYERS}
    base = _engine_step(SHAPE, w, wq, _pad(x, rows), _pad(t, rows), real, suppress)
    noise = 3 * torch.randn(B, rows - real, SHAPE.hidden, generator=g)
    other = _engine_step(SHAPE, w, wq, _pad(x, rows, noise), _pad(t, rows, -noise), real, suppress)
    assert other[0] == base[0]
    if suppress:
        assert other[1] == base[1]
    for k in base[2]:
        assert torch.equal(other[2][k], base[2][k]), k
    # in pieces: the whole batch's threshold, the loss to the order of additions
    split = _engine_step(SHAPE, w, wq, _pad(x, rows, noise), _pad(t, rows), real, suppress, pieces=2)
    if suppress:
        assert split[1] == base[1]
    assert split[0] == pytest.approx(base[0], rel=1e-6)
    for k in base[2]:
        assert float((split[2][k] - base[2][k]).norm() / base[2][k].norm()) < 1e-5, k


@pytest.mark.parametrize(("shape", "real"), [(SHAPE, 200), (D128, 300)])
def test_padded_step_matches_the_oracle_on_the_unpadded_sequences(shape, real):
    """Mean squared error and dL/dW' at the first tuning step (W' = 2-bit
    round to nearest, in bf16) against float64 autodiff through the oracle
    block on the ``real``-token sequences."""
    _case("padded step vs oracle", shape.hidden, real)
    B, rows = 2, aligned_length(real)
    w = _weights(shape, seed=9)
    g = torch.Generator().manual_seed(10)
    x = torch.randn(B, real, shape.hidden, generator=g)
    with torch.no_grad():
        t = _oracle(shape, w, x)
    wq = {n: _rtn_bf16(w.linears[n]) for n in LAYERS}
    lin = {n: wq[n].double().requires_grad_(True) for n in LAYERS}
    loss = ((_oracle(shape, w, x, linears=lin) - t) ** 2).mean()
    loss.backward()
    ref = float(loss.detach())
    fill = torch.randn(B, rows - real, shape.hidden, generator=g)
    got, _, dw = _engine_step(shape, w, wq, _pad(x, rows, fill), _pad(t, rows), real, suppress=False)
    print(f"  loss gpu {got:.6e} oracle {ref:.6e}", file=sys.stderr)
    assert abs(got - ref) <= 1e-2 * ref
    place = placements(shape)
    for n in LAYERS:
        r = lin[n].grad
        d = unplace(dw[place[n].operand], r.shape[0], place[n]).double().cpu()
        rel = float((d - r).norm() / r.norm())
        flipped = float(r.abs()[torch.sign(d) != torch.sign(r)].sum() / r.abs().sum())
        print(f"  {n}: rel err {rel:.2e}, flipped mass {flipped:.2e}", file=sys.stderr)
        assert rel < 5e-2, n
        assert flipped < 1e-2, n


def test_padded_tune_follows_the_oracle_tune():
    """12 steps at rate 1/200, 2 bits (outlier rule on), two batches of two
    200-token sequences, against the oracle's tune of the same sequences."""
    _case("padded tune")
    iters, lr, real, B = 12, 0.005, 200, 2
    rows = aligned_length(real)
    w = _weights(SHAPE, seed=3)
    g = torch.Generator().manual_seed(5)
    xs = [torch.randn(B, real, SHAPE.hidden, generator=g) for _ in range(2)]
    with torch.no_grad():
        ts = [_oracle(SHAPE, w, x).float() for x in xs]
    scheme = QuantScheme(bits=2, group_size=64, symmetry=Symmetry.ASYMMETRIC)
    runner = QuantizationRunner(scheme, TuningConfig(iters=iters, batch_size=B, n_samples=2 * B, seq_len=real,
                                                     lr=lr))
    block = DecoderBlock(0, "model.layers.0", SHAPE, _dev(w))
    res, _ = runner.quantize_block(block, [_pad(x, rows).to(dev()) for x in xs],
                                   [_pad(t, rows).to(dev()) for t in ts], path_prefix=block.name)
    lin32 = {n: w.linears[n].float() for n in LAYERS}
    biases = {n: b.double() for n, b in w.biases.items()}
    norms = (w.input_norm.double(), w.post_norm.double())
    ob = OB.tune_block(xs, ts, lin32, biases, norms, _oshape(SHAPE), OB.Scheme(2, 64), iters=iters, lr=lr,
                       suppress=True)
    print("  gpu", res.initial_loss, res.final_loss, res.step_losses, file=sys.stderr)
    print("  cpu", ob["initial_loss"], ob["final_loss"], ob["losses"], file=sys.stderr)
    assert abs(res.initial_loss - ob["initial_loss"]) <= 1e-2 * ob["initial_loss"]
    for a, b in zip(res.step_losses, ob["losses"]):
        assert abs(a - b) <= 1e-2 * b
    assert res.reverted == ob["reverted"]
    assert abs(res.final_loss - ob["final_loss"]) <= 1e-2 * ob["final_loss"]


def test_a_tune_does_not_see_the_padding():
    """A whole block tune (searched symmetric scales, whose search weighs the
    layers' inputs, 2 bits with the outlier rule, steps replayed as graphs)
    is bit-identical whatever finite values the padding rows of its inputs
    and targets hold."""
    _case("padded tune invariance")
    iters, real, B = 6, 200, 2
    rows = aligned_length(real)
    w = _weights(SHAPE, seed=4)
    g = torch.Generator().manual_seed(6)
    xs = [torch.randn(B, real, SHAPE.hidden, generator=g) for _ in range(2)]
    with torch.no_grad():
        ts = [_oracle(SHAPE, w, x).float() for x in xs]
    scheme = QuantScheme(bits=2, group_size=64, symmetry=Symmetry.SYMMETRIC, scale_init="searched")
    out = []
    for fill in (None, 2.0):
        pads = [None if fill is None else fill * torch.randn(B, rows - real, SHAPE.hidden, generator=g)
                for _ in range(4)]
        runner = QuantizationRunner(scheme, TuningConfig(iters=iters, batch_size=B, n_samples=2 * B, seq_len=real,
                                                         lr=0.005))
        block = DecoderBlock(0, "b", SHAPE, _dev(w))
        res, layers = runner.quantize_block(block, [_pad(x, rows, p).to(dev()) for x, p in zip(xs, pads)],
                                            [_pad(t, rows, p).to(dev()) for t, p in zip(ts, pads[2:])])
        torch.cuda.synchronize()
        out.append((res, {k: (v.codes.cpu(), v.scale.cpu()) for k, v in layers.items()}))
    (r0, c0), (r1, c1) = out
    assert r0.initial_loss == r1.initial_loss and r0.final_loss == r1.final_loss
    assert r0.step_losses == r1.step_losses and r0.reverted == r1.reverted
    for k in c0:
        assert torch.equal(c0[k][0], c1[k][0]) and torch.equal(c0[k][1], c1[k][1]), k


TINY = dict(model_type="qwen2", hidden_size=128, num_attention_heads=2, num_key_value_heads=1,
            intermediate_size=256, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=2,
            vocab_size=512, tie_word_embeddings=True)


@pytest.mark.parametrize("symmetry", [Symmetry.ASYMMETRIC, Symmetry.SYMMETRIC])
def test_quantize_at_a_length_off_the_tile(tmp_path, symmetry):
    _case("api seq_len 200", symmetry)
    src = write_random_checkpoint(tmp_path / "m", TINY, seed=1, std=0.05)
    tuning = TuningConfig(iters=6, batch_size=2, n_samples=4, seq_len=200)
    res = api.quantize(src, output_dir=tmp_path / "q", bits=4, symmetry=symmetry, tuning=tuning, seed=5)
    assert len(res.summary.blocks) == 2
    for b in res.summary.blocks:
        assert 0 < b.final_loss <= b.initial_loss
        assert all(l == l and l > 0 for l in b.step_losses)
