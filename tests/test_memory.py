"""The device-memory prediction: the geometry's weight counts against the
figures of the benchmark configurations, the block and causal-LM engines'
formulas against the buffers the engines actually allocate (built on the CPU),
and the budget refusals of the API and the CLI."""

from __future__ import annotations

import pytest
import torch

from mround_amd import api
from mround_amd.cli import GEOMETRIES, main
from mround_amd.exceptions import ArchitectureError, MemoryBudgetError
from mround_amd.pipeline.block import BlockEngine, aligned_length
from mround_amd.pipeline.causal_lm import CausalLM
from mround_amd.pipeline.checkpoint import block_shape, load_model, write_random_checkpoint
from mround_amd.planner import memory as M
from mround_amd.schemes import TuningConfig

TINY = dict(model_type="qwen2", hidden_size=128, num_attention_heads=2, num_key_value_heads=1,
            intermediate_size=256, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=2,
            vocab_size=250, tie_word_embeddings=True)


def _bytes(*objs) -> int:
    """Bytes of the distinct tensor storages the objects' attributes hold
    (directly or in dicts, lists and tuples)."""
    seen, total = set(), 0

    def visit(v):
        nonlocal total
        if isinstance(v, torch.Tensor):
            key = (v.untyped_storage().data_ptr(), v.untyped_storage().nbytes())
            if key not in seen and v.untyped_storage().nbytes():
                seen.add(key)
                total += v.untyped_storage().nbytes()
        elif isinstance(v, dict):
            for x in v.values():
                visit(x)
        elif isinstance(v, (list, tuple)):
            for x in v:
                visit(x)

    for obj in objs:
        for v in vars(obj).values():
            visit(v)
    return total


@pytest.mark.parametrize("geo,weights", [("qwen2.5-7b", 233_046_016), ("qwen2.5-3b", 77_070_336),
                                         ("qwen2.5-0.5b", 14_909_440), ("smollm2-135m", 3_538_944)])
def test_block_weights_match_the_configurations(geo, weights):
    assert M.ModelShape.from_config(GEOMETRIES[geo]).block_weights == weights


@pytest.mark.parametrize("geo", ["qwen2.5-0.5b", "smollm2-135m"])
def test_engine_formula_is_the_engine(geo):
    cfg = GEOMETRIES[geo]
    eng = BlockEngine(block_shape(cfg), batch=2, seq_len=256, device="cpu")
    assert _bytes(eng) == M.engine_bytes(M.ModelShape.from_config(cfg), 512, 256)
    assert sum(t.nbytes for t in eng.new_activations().values()) == \
        M.activation_bytes(M.ModelShape.from_config(cfg), 512)


def test_scoring_formula_is_the_causal_lm(tmp_path):
    write_random_checkpoint(tmp_path / "m", TINY)
    model = load_model(tmp_path / "m", device="cpu")
    lm = CausalLM(model, batch=2, seq_len=200, device="cpu", keep_activations=True)
    m = M.ModelShape.from_config(TINY)
    run = M.RunShape(n_samples=2, seq_len=128, batch_size=2, group_size=64, mixed=True, widths=2,
                     scoring_samples=4, scoring_seq_len=200, scoring_batch=2)
    pred = M.predict_memory(m, run)
    formula = pred.stages["scoring"] - pred.stages["load"] - 4 * 200 * 8 - 2 * 128 * 8
    # what the engine object owns (the blocks' norms and biases it points at are the model's),
    # and the input-gradient buffer appears at the first backward
    owned = _bytes(lm, lm.eng) + lm.tokens * m.hidden * 4
    shared = sum(p.untyped_storage().nbytes() for t in lm.params for p in t if p is not None)
    assert abs((owned - shared) - formula) <= 0.005 * formula, (owned - shared, formula)


def test_blocks_stage_counts_the_calibration_streams():
    """With quantized inputs the runner holds the reference stream, the
    quantized stream and the spare its advance writes into (not with held-out
    batches, whose final score is taken apart); without, the inputs and the
    targets."""
    m = M.ModelShape.from_config({**GEOMETRIES["qwen2.5-7b"], "vocab_size": 152064})
    one = 128 * 2048 * m.hidden * 4

    def blocks(**kw):
        return M.predict_memory(m, M.RunShape(n_samples=128, seq_len=2048, batch_size=8, group_size=64,
                                              **kw)).stages["blocks"]

    with_q = blocks()
    assert with_q - blocks(quantized_inputs=False) == one
    assert with_q - blocks(holdout_batches=1) == one
    assert with_q - blocks(half=True) == one
    assert blocks(quantized_inputs=False) == blocks(quantized_inputs=False, holdout_batches=2)


def test_a_length_off_the_tile_counts_padded_rows():
    """Sequences of 200 tokens run on 256 rows each: the streams and the
    engine are those of 256-token sequences, the calibration token ids those
    of 200; the engine the runner builds for them is the formula's."""
    m = M.ModelShape.from_config(GEOMETRIES["qwen2.5-0.5b"])
    run = lambda L: M.RunShape(n_samples=8, seq_len=L, batch_size=4, group_size=64)  # noqa: E731
    padded, aligned = M.predict_memory(m, run(200)), M.predict_memory(m, run(256))
    assert aligned.stages["blocks"] - padded.stages["blocks"] == 8 * (256 - 200) * 8
    assert M.aligned_rows(200) == aligned_length(200) == 256 and M.aligned_rows(256) == 256
    eng = BlockEngine(block_shape(GEOMETRIES["smollm2-135m"]), batch=2, seq_len=aligned_length(200),
                      device="cpu", real_len=200)
    assert _bytes(eng) == M.engine_bytes(M.ModelShape.from_config(GEOMETRIES["smollm2-135m"]), 512, 256)


def test_split_engine_formula_is_the_engine():
    """Split precision adds fp32 and split W', the split normalized inputs and
    SwiGLU output and the fp32 gate/up pair (and the workspace of the 3K
    products) to the engine; the prediction counts exactly what it allocates,
    and the blocks stage holds two streams (the final score apart)."""
    cfg = GEOMETRIES["smollm2-135m"]
    m = M.ModelShape.from_config(cfg)
    eng = BlockEngine(block_shape(cfg), batch=2, seq_len=256, device="cpu", split=True)
    assert _bytes(eng) == M.engine_bytes(m, 512, 256, split=True)
    assert M.engine_bytes(m, 512, 256, split=True) - M.engine_bytes(m, 512, 256) >= M.split_bytes(m, 512)
    run = M.RunShape(n_samples=8, seq_len=256, batch_size=2, group_size=64, split=True)
    assert run.streams == 2


def test_engine_refuses_more_tokens_than_rows():
    with pytest.raises(ArchitectureError):
        BlockEngine(block_shape(GEOMETRIES["smollm2-135m"]), batch=1, seq_len=128, device="cpu", real_len=129)
    with pytest.raises(ArchitectureError):
        BlockEngine(block_shape(GEOMETRIES["smollm2-135m"]), batch=1, seq_len=200, device="cpu")


def test_micro_batches_shrink_the_engine():
    """Steps in pieces hold the engine at the largest piece (8 sequences in 3
    pieces: 3), the rest of the blocks stage unchanged."""
    m = M.ModelShape.from_config(GEOMETRIES["qwen2.5-0.5b"])
    whole = M.RunShape(n_samples=16, seq_len=2048, batch_size=8, group_size=64)
    pieces = M.RunShape(n_samples=16, seq_len=2048, batch_size=8, group_size=64, micro_batches=3)
    assert pieces.piece_sequences == 3
    drop = M.predict_memory(m, whole).stages["blocks"] - M.predict_memory(m, pieces).stages["blocks"]
    assert drop == M.engine_bytes(m, 8 * 2048, 2048) - M.engine_bytes(m, 3 * 2048, 2048) > 0


def test_api_refuses_a_run_past_the_budget(tmp_path):
    write_random_checkpoint(tmp_path / "m", TINY)
    check = api.predict_memory(tmp_path / "m", memory_budget=10 ** 12, device="cpu")
    assert check.fits and check.prediction.peak > 0 and "blocks" in check.describe()
    small = api.predict_memory(tmp_path / "m", memory_budget=1000, device="cpu")
    assert not small.fits and "calibration streams" in small.explain()
    with pytest.raises(MemoryBudgetError, match="predicted peak"):
        api.quantize(tmp_path / "m", output_dir=tmp_path / "o", memory_budget=1000, device="cpu")
    with pytest.raises(ValueError, match="positive"):
        api.predict_memory(tmp_path / "m", memory_budget=-5, device="cpu")
    mixed = api.predict_memory(tmp_path / "m", average_bits=3, candidate_bits=(2, 4), device="cpu",
                               memory_budget=10 ** 12)
    assert "scoring" in mixed.prediction.stages


def test_cli_dry_run(tmp_path, capsys):
    write_random_checkpoint(tmp_path / "m", TINY)
    assert main(["quantize", str(tmp_path / "m"), "-o", str(tmp_path / "o"), "--dry-run",
                 "--memory-budget", "1000"]) == 0
    out = capsys.readouterr().out
    assert "predicted peak" in out and "time: predicted" in out and "MI355X" in out
    assert main(["quantize", str(tmp_path / "m"), "-o", str(tmp_path / "o"), "--dry-run",
                 "--memory-budget", "0.000001"]) == 1
    # split precision and a sequence length off the 128-row tile: accepted, and
    # the prediction grows with both
    assert main(["quantize", str(tmp_path / "m"), "-o", str(tmp_path / "o"), "--dry-run", "--memory-budget",
                 "1000", "--split-precision", "--seq-len", "200", "--samples", "8", "--batch-size", "4"]) == 0
    peaks = [api.predict_memory(tmp_path / "m", tuning=TuningConfig(n_samples=8, batch_size=4, seq_len=seq),
                                split_precision=split, memory_budget=1 << 40, device="cpu").prediction.peak
             for split, seq in ((False, 128), (True, 128), (True, 200))]
    assert peaks[0] < peaks[1] < peaks[2], peaks


def test_engine_workspaces_cover_every_piece():
    """An engine of 8 sequences of the 7B geometry also runs pieces of fewer
    (``set_sequences``): at 7 the dK/dV grid falls under the size that needs
    no head split and the library plans 117,440,512 bytes of partials, where
    8 sequences plan none. The engine's workspaces are the largest over
    every piece size, so no piece's launch falls back to an allocation of
    the binding's own."""
    from mround_amd import kernels as K
    from mround_amd.pipeline.block import BlockShape, gemm_problems, workspace_bytes

    s = BlockShape(hidden=3584, n_heads=28, n_kv_heads=4, head_dim=128, intermediate=18944, attn_bias=True)
    q = dict(seq_len=2048, n_heads=28, n_kv_heads=4, head_dim=128)
    assert K.attn_bwd_workspace_bytes(batch=8, **q) == 0
    assert K.attn_bwd_workspace_bytes(batch=7, **q) == 117_440_512
    gemm, attn = workspace_bytes(s, 8, 2048)
    for n in range(1, 9):
        assert attn >= K.attn_bwd_workspace_bytes(batch=n, **q)
        assert gemm >= max(K.gemm_workspace_bytes(M, N, Kd) for M, N, Kd in gemm_problems(s, n * 2048))
    assert attn == max(K.attn_bwd_workspace_bytes(batch=n, **q) for n in range(1, 9))


def test_split_precision_follows_the_tuned_widths(tmp_path):
    """Split precision defaults on when a tuned width is 8 bits, in uniform
    runs and in mixed runs whose candidates (or given plan) include 8, and
    off otherwise; the predictions count it the same way; turning it off for
    8-bit codes warns."""
    import warnings

    write_random_checkpoint(tmp_path / "m", TINY)
    t = TuningConfig(n_samples=8, batch_size=4, seq_len=128)
    peak = lambda **kw: api.predict_memory(tmp_path / "m", tuning=t, memory_budget=1 << 40, device="cpu",
                                           **kw).prediction.peak
    assert peak(bits=8) == peak(bits=8, split_precision=True) > peak(bits=8, split_precision=False)
    assert peak(bits=4) == peak(bits=4, split_precision=False) < peak(bits=4, split_precision=True)
    assert (peak(average_bits=5, candidate_bits=(4, 8)) ==
            peak(average_bits=5, candidate_bits=(4, 8), split_precision=True))
    assert (peak(average_bits=3, candidate_bits=(2, 4)) ==
            peak(average_bits=3, candidate_bits=(2, 4), split_precision=False))
    secs = lambda **kw: api.predict_time(tmp_path / "m", tuning=t, **kw).total
    assert secs(bits=8) == secs(bits=8, split_precision=True) > secs(bits=8, split_precision=False)
    assert api._split_choice(None, (8,))[0] and not api._split_choice(None, (2, 3, 4))[0]
    assert api._split_choice(True, (4,)) == (True, "requested")
    with pytest.warns(UserWarning, match="8-bit codes"):
        assert api._split_choice(False, (4, 8)) == (False, "requested")
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        api._split_choice(False, (2, 4))
    scheme = api.QuantScheme(bits=4, group_size=64)
    assert api._tuned_widths(scheme, None, (2, 3, 4), None) == (4,)
    assert api._tuned_widths(scheme, 3.0, (2, 3, 4), None) == (2, 3, 4)
    assert api._tuned_widths(scheme, 3.0, (2, 3, 4, 8), {"a": 2, "b": 8}) == (2, 8)
