"""The device-memory prediction against the peak a run actually allocates
(``torch.cuda.max_memory_allocated``: every device buffer of the run, the
library's workspaces included, is a torch allocation)."""

from __future__ import annotations

import json
import sys

import pytest

from mround_amd import api
from mround_amd.pipeline.checkpoint import write_random_checkpoint
from mround_amd.schemes import Symmetry, TuningConfig

pytestmark = pytest.mark.gpu

SMALL = dict(model_type="qwen2", hidden_size=512, num_attention_heads=8, num_key_value_heads=2,
             intermediate_size=1536, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=3,
             vocab_size=4096, tie_word_embeddings=True)


# (mixed, quantized_inputs, holdout_batches, seq_len): the block loop holds
# three calibration streams with quantized inputs and the fused advance, two
# without quantized inputs (inputs, targets) or with held-out batches; 200
# tokens run on sequences padded to 256 rows.
CASES = [(False, True, 0, 256), (True, True, 0, 256), (False, False, 0, 256), (False, True, 1, 256),
         (False, True, 0, 200)]


@pytest.mark.parametrize("mixed,quantized_inputs,holdout,seq_len", CASES)
def test_prediction_bounds_the_measured_peak(tmp_path, mixed, quantized_inputs, holdout, seq_len):
    print("case memory", mixed, quantized_inputs, holdout, seq_len, flush=True, file=sys.stderr)
    src = write_random_checkpoint(tmp_path / "m", SMALL, seed=1)
    tuning = TuningConfig(iters=2, batch_size=4, n_samples=8, seq_len=seq_len)
    kw = dict(average_bits=3.0, candidate_bits=(2, 4), scoring_samples=8, scoring_seq_len=257) if mixed else {}
    res = api.quantize(src, output_dir=tmp_path / "q", bits=4, symmetry=Symmetry.ASYMMETRIC, tuning=tuning,
                       seed=2, quantized_inputs=quantized_inputs, holdout_batches=holdout, **kw)
    rec = json.loads(res.config_path.read_text())["memory"]
    predicted = rec["peak"]
    measured = rec["peak_allocated"]
    print(f"  predicted {predicted} measured {measured} ({measured / predicted:.3f}) in {rec['peak_stage']}",
          file=sys.stderr)
    assert rec["peak_stage"] == ("scoring" if mixed else "blocks")
    assert 0.85 * predicted <= measured <= 1.05 * predicted
