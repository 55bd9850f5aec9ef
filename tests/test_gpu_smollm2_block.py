"""The SmolLM2-135M-shaped block workload at its full size: one decoder block
(hidden 576, 9 query / 3 kv heads x 64, SwiGLU 1536, RMSNorm eps 1e-5, RoPE
theta 1e4, no linear biases, fp32 weights N(0, 0.02) seed 0, norm weights 1),
8 x 512 hidden states N(0, 1) (seed 1) with channels 7, 111, 333 and 500
scaled x20, 4-bit asymmetric gs64, 200 sign-SGD steps at lr 5e-3 and batch 8
(one batch; no outlier rule at 4 bits).

Against the float64 oracle on the same inputs and targets (the original
block's output): the initial loss and the first three steps' losses within
the 1e-2 bf16 bar. At the full 200 steps, properties the tune must have: the loss
falls, the block is not reverted, two runs commit identical codes, and every
code lies in the 4-bit range. The GPU wall clock of the tune and the CPU
oracle's time per step (float32 PyTorch block forward and backward plus the
NumPy fake quantization and its gradient, on this host's cores) are printed.
"""

from __future__ import annotations

import os
import sys
import time

import numpy as np
import pytest
import torch

from mround_amd.pipeline.block import LAYERS, BlockShape, BlockWeights
from mround_amd.pipeline.runner import DecoderBlock, QuantizationRunner
from mround_amd.schemes import QuantScheme, Symmetry, TuningConfig
from oracle import block as OB
from tests.helpers import dev

pytestmark = pytest.mark.gpu

SHAPE = BlockShape(hidden=576, n_heads=9, n_kv_heads=3, head_dim=64, intermediate=1536, norm_eps=1e-5,
                   rope_theta=1e4, attn_bias=False)
OUTLIER_CHANNELS = (7, 111, 333, 500)
B, S, ITERS, LR = 8, 512, 200, 5e-3


def _oshape() -> OB.Shape:
    s = SHAPE
    return OB.Shape(hidden=s.hidden, n_heads=s.n_heads, n_kv_heads=s.n_kv_heads, head_dim=s.head_dim,
                    intermediate=s.intermediate, norm_eps=s.norm_eps, rope_theta=s.rope_theta)


def _workload():
    w = BlockWeights.random(SHAPE, dtype=torch.float32, device="cpu", seed=0, std=0.02)
    x = torch.randn(B, S, SHAPE.hidden, generator=torch.Generator().manual_seed(1))
    x[..., list(OUTLIER_CHANNELS)] *= 20.0
    lin = {n: w.linears[n].double() for n in LAYERS}
    norms = (w.input_norm.double(), w.post_norm.double())
    with torch.no_grad():
        target = OB.block_forward(x.double(), lin, {}, norms, _oshape())
    return w, x, target


def _gpu_tune(w, x, target):
    scheme = QuantScheme(bits=4, group_size=64, symmetry=Symmetry.ASYMMETRIC)
    tuning = TuningConfig(iters=ITERS, batch_size=B, n_samples=B, seq_len=S, lr=LR)
    runner = QuantizationRunner(scheme, tuning)
    wd = BlockWeights({n: t.to(dev()) for n, t in w.linears.items()}, {}, w.input_norm.to(dev()),
                      w.post_norm.to(dev()))
    block = DecoderBlock(0, "model.layers.0", SHAPE, wd)
    inputs = [x.reshape(B * S, -1).float().to(dev())]
    targets = [target.reshape(B * S, -1).float().to(dev())]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    res, layers = runner.quantize_block(block, inputs, targets, path_prefix=block.name)
    torch.cuda.synchronize()
    return res, layers, time.perf_counter() - t0


def test_smollm2_block_tune_at_full_size():
    print("case smollm2 block tune", flush=True, file=sys.stderr)
    w, x, target = _workload()
    res, layers, secs = _gpu_tune(w, x, target)
    print(f"  gpu: {secs:.3f} s for the tune, loss {res.initial_loss:.6g} -> {res.final_loss:.6g}",
          file=sys.stderr)
    # the first steps against the oracle (same inputs, targets and schedule)
    lin32 = {n: w.linears[n].float() for n in LAYERS}
    norms = (w.input_norm.double(), w.post_norm.double())
    t0 = time.perf_counter()
    ob = OB.tune_block([x], [target], lin32, {}, norms, _oshape(), OB.Scheme(4, 64), iters=ITERS, lr=LR,
                       suppress=False, steps=3)
    print(f"  oracle (float64, 3 steps): {time.perf_counter() - t0:.1f} s; losses {ob['losses']}, "
          f"gpu {res.step_losses[:3]}", file=sys.stderr)
    assert abs(res.initial_loss - ob["initial_loss"]) <= 1e-2 * ob["initial_loss"]
    for a, b in zip(res.step_losses[:3], ob["losses"]):
        assert abs(a - b) <= 1e-2 * b
    # properties of the full tune
    assert not res.reverted and res.final_loss < 0.9 * res.initial_loss
    losses = np.asarray(res.step_losses)
    assert losses[-20:].mean() < losses[:20].mean()
    res2, layers2, _ = _gpu_tune(w, x, target)
    for path, q in layers.items():
        assert torch.equal(q.codes, layers2[path].codes), path
        assert int(q.codes.max()) <= 15
    assert res2.final_loss == res.final_loss


def test_smollm2_cpu_oracle_step_time():
    """The CPU restatement's cost of one tuning step at this size (float32
    block forward and backward in PyTorch, NumPy fake quantization and STE
    gradient of the seven layers), the baseline the GPU tune is compared with."""
    w, x, target = _workload()
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    scheme = OB.Scheme(4, 64)
    lin = {n: w.linears[n] for n in LAYERS}
    params = OB.init_params(lin, scheme)
    norms = (w.input_norm.float(), w.post_norm.float())
    xs, ts = x.float(), target.float()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        leaf = {n: tuple(t.clone().requires_grad_(True) for t in p) for n, p in params.items()}
        wq = OB.quantized_linears(lin, leaf, scheme, differentiable=True)
        out = OB.block_forward(xs, {n: t.float() for n, t in wq.items()}, {}, norms, _oshape())
        loss = ((out - ts) ** 2).mean()
        loss.backward()
        times.append(time.perf_counter() - t0)
    step = sorted(times)[1]
    print(f"  cpu oracle: {step:.2f} s per step on {threads} threads; x {ITERS} steps + 2 scoring passes "
          f"= {step * (ITERS + 1):.0f} s per block", file=sys.stderr)
    assert step > 0
