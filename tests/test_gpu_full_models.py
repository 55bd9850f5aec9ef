"""Whole-model runs at the benchmark configurations' full sizes, through
``api.quantize`` on random-init checkpoints (bf16 N(0, 0.02), seed 0).

* Qwen2.5-0.5B shape (24 blocks, hidden 896, 14 / 2 heads x 64, SwiGLU 4864,
  vocab 151936, tied): 4-bit asymmetric gs64, 128 x 2048 uniform token ids,
  200 steps per block at batch 8. Run twice: identical codes, scales and
  per-block losses.
* Qwen2.5-3B shape (36 blocks, hidden 2048, 16 / 2 heads x 128, SwiGLU
  11008): the mixed 2.5-bit average over {2, 3, 4}, asymmetric gs64: the
  whole-model scoring pass (128 x 1024 tokens), the exact allocation, then the
  tune on 128 x 2048 tokens. The plan stays within the 2.5-bit budget (and
  within 0.01 bit of it) and every layer is tuned and committed at its
  planned width.

Both: every block's final loss is below its initial one or the block was
reverted (the revert rule), codes lie in their width's range, and for the
first and last blocks the committed codes, scales, zero points and bf16
reconstruction equal, bit for bit, the float32 oracle's forward of the final
(v, alpha, beta) on sampled rows.
"""

from __future__ import annotations

import json
import sys

import numpy as np
import pytest
import torch

from mround_amd import api
from mround_amd.cli import GEOMETRIES
from mround_amd.pipeline.block import LAYERS
from mround_amd.pipeline.checkpoint import write_random_checkpoint
from mround_amd.pipeline.runner import QuantizationRunner
from mround_amd.schemes import Symmetry, TuningConfig
from oracle import quantize as OQ
from tests.test_gpu_configs import layer_rows

pytestmark = pytest.mark.gpu


def _spy_commits(monkeypatch, blocks):
    """Record, for the given block indices, each layer's original rows, final
    parameters and committed codes, scale, zero point and reconstruction on
    the sampled rows (the last commit of a layer wins: a revert re-commits)."""
    seen = {}
    commit = QuantizationRunner._commit

    def spy(self, block, layer):
        q = commit(self, block, layer)
        if block.index in blocks:
            sel = layer_rows(layer.weight.shape[0])
            cpu = lambda t: t[sel].float().cpu().numpy().copy()
            seen[(block.index, layer.name)] = dict(
                w=cpu(layer.weight), v=cpu(layer.v), a=cpu(layer.alpha), b=cpu(layer.beta),
                bits=layer.scheme.bits, codes=q.codes[sel].cpu().numpy().copy(), scale=cpu(q.scale),
                zp=cpu(q.zero_point), recon=cpu(block.weights.linears[layer.name]))
        return q

    monkeypatch.setattr(QuantizationRunner, "_commit", spy)
    return seen


def _check_commits(seen):
    assert seen
    for (index, name), c in seen.items():
        ref_q, ref_c, ref_s, ref_z = OQ.fake_quantize(c["w"], c["v"], c["a"], c["b"], bits=c["bits"],
                                                      group_size=64, mode="asym", dtype=np.float32)
        assert np.array_equal(c["codes"].astype(np.float32), ref_c.reshape(c["codes"].shape)), (index, name)
        assert np.array_equal(c["scale"].reshape(-1), ref_s.reshape(-1)), (index, name)
        assert np.array_equal(c["zp"].reshape(-1), ref_z.reshape(-1)), (index, name)
        assert np.array_equal(c["recon"], OQ.round_to_bf16(ref_q)), (index, name)


def _check_blocks(res):
    """The revert rule (a reverted block reports its initial score) and learning."""
    for b in res.summary.blocks:
        assert np.isfinite(b.initial_loss) and np.isfinite(b.final_loss)
        if b.reverted:
            assert b.final_loss == b.initial_loss, b
        else:
            assert b.final_loss < b.initial_loss, b
    improved = sum(1 for b in res.summary.blocks if not b.reverted)
    assert improved >= len(res.summary.blocks) - 2


def test_qwen25_05b_full_model_4bit(tmp_path, monkeypatch):
    print("case full model 0.5b", flush=True, file=sys.stderr)
    cfg = GEOMETRIES["qwen2.5-0.5b"]
    src = write_random_checkpoint(tmp_path / "m", cfg, seed=0, device="cuda")
    tuning = TuningConfig(iters=200, batch_size=8, n_samples=128, seq_len=2048)
    runs = []
    for i in range(2):
        seen = _spy_commits(monkeypatch, {0, 23})
        res = api.quantize(src, output_dir=tmp_path / f"q{i}", bits=4, symmetry=Symmetry.ASYMMETRIC,
                           tuning=tuning, seed=4)
        print(f"  run {i}: {res.seconds['total']:.1f} s, blocks {res.seconds['blocks']:.1f} s", file=sys.stderr)
        assert len(res.summary.blocks) == 24
        _check_blocks(res)
        _check_commits(seen)
        for c in seen.values():
            assert int(c["codes"].max()) <= 15
        runs.append((res, seen))
        monkeypatch.undo()
    (r0, s0), (r1, s1) = runs
    assert [b.final_loss for b in r0.summary.blocks] == [b.final_loss for b in r1.summary.blocks]
    assert [b.step_losses for b in r0.summary.blocks] == [b.step_losses for b in r1.summary.blocks]
    for k in s0:
        assert np.array_equal(s0[k]["codes"], s1[k]["codes"]) and np.array_equal(s0[k]["scale"], s1[k]["scale"])
    # the two checkpoints hold identical tensors
    from safetensors.torch import load_file

    t0 = load_file(str(tmp_path / "q0" / "model.safetensors"))
    t1 = load_file(str(tmp_path / "q1" / "model.safetensors"))
    assert t0.keys() == t1.keys()
    for k in t0:
        assert torch.equal(t0[k], t1[k]), k


def test_qwen25_3b_mixed_2p5_bits(tmp_path, monkeypatch):
    print("case full model 3b mixed", flush=True, file=sys.stderr)
    cfg = GEOMETRIES["qwen2.5-3b"]
    src = write_random_checkpoint(tmp_path / "m", cfg, seed=0, device="cuda")
    seen = _spy_commits(monkeypatch, {0, 35})
    tuning = TuningConfig(iters=200, batch_size=8, n_samples=128, seq_len=2048)
    res = api.quantize(src, output_dir=tmp_path / "q", symmetry=Symmetry.ASYMMETRIC, average_bits=2.5,
                       candidate_bits=(2, 3, 4), tuning=tuning, seed=5)
    print(f"  {res.seconds['total']:.1f} s; {res.mixed['describe']}", file=sys.stderr)
    assert len(res.summary.blocks) == 36
    plan = res.mixed["assignments"]
    assert len(plan) == 36 * len(LAYERS)
    assert 2.49 <= res.mixed["achieved_code_bits"] <= 2.5
    assert res.mixed["allocated_cost_bits"] <= res.mixed["budget_bits"]
    assert set(plan.values()) <= {2, 3, 4} and len(set(plan.values())) > 1
    for path, bits in plan.items():
        assert res.scheme_by_layer[path].bits == bits, path
    _check_blocks(res)
    _check_commits(seen)
    for (index, name), c in seen.items():
        assert c["bits"] == plan[f"model.layers.{index}.{name}"]
        assert int(c["codes"].max()) <= 2 ** c["bits"] - 1
    cfg_out = json.loads((tmp_path / "q" / "config.json").read_text())
    assert cfg_out["quantization"]["bits"] in (2, 3, 4)
    for path, bits in plan.items():
        if bits != cfg_out["quantization"]["bits"]:
            assert cfg_out["quantization"][path]["bits"] == bits, path
