"""How long a quantization run will take on one MI355X, worked out before it
starts (the counterpart of ``mround/planner/timing.py:1-338``).

The reference fits a power law of the block's weights to its runs on one
Mac; this rule is fitted to runs on one MI355X, and its form follows what
the GPU spends its time on. Its constants come from
``mround_amd.planner.timing_runs`` (random-init checkpoints of SmolLM2-135M,
Qwen2.5-0.5B, 1.5B, 3B and 7B shapes: the outlier rule on and off, pieces,
the scale search, other batches and calibration sets, the mixed scoring pass
at both gradient sources), refitted by ``timing_runs.fit``, and
``tests/test_timing.py`` holds the rule to every recorded run.

**A step** (one sign-SGD step of a block: forward, backward, the fused
update of every layer) takes

    a + b * T * W + c * A

with T the step's tokens, W the block's weights and A the attention
forward's flops (4 * batch * seq_len^2 / 2 * heads * head_dim, causal): the
GEMMs' 6 T W flops run at 6 / b = 1.25 PFLOP/s, the attention at
c^-1 per forward flop (forward and backward, with the norms and rotations
that scale with the sequences), and a is what a step pays whatever its size
(launches, the losses, the fake-quant of every layer). The outlier rule adds
its select over the T x hidden loss elements. A step in p pieces pays the
fixed part p - 1 more times and, under the outlier rule, one more forward of
the whole batch for the batch-wide threshold.

**A block** is its search (symmetric codes below 4 bits), its initial score
and final score (a forward over every calibration batch each; the final one
also advances the stream), its steps and its commit. **Between blocks** the
targets pass is one more forward over the calibration batches. **A mixed
run's scoring pass** is a fixed part, a part per block and per block weight,
and the head (vocabulary x hidden, twice if untied), times 2.74 with a
backward at each width (``own_width``); it scales with the scoring tokens
(measured at 128 x 1024).

Every run records the prediction beside what it measured.

Portions follow MRound (Copyright 2026 The MRound Authors, Apache License 2.0);
see NOTICE.
"""

from __future__ import annotations

import dataclasses
from collections.abc import Collection
from typing import Any

from mround_amd.planner.memory import ModelShape, RunShape, aligned_rows
from mround_amd.planner.sensitivity import SENSITIVITY_SAMPLES, SENSITIVITY_SEQ_LEN, gradient_source_for

__all__ = ["MACHINE", "RULE_VERSION", "SPREAD", "TimePrediction", "predict_run_time", "predict_time"]

RULE_VERSION = "2026-12-02.3"
MACHINE = "one AMD Instinct MI355X"

# Recorded over predicted seconds of the measurement runs (block loop and
# scoring pass), lowest and highest, and of the single-block tunes measured
# apart in bf16 and split precision (the 0.5B-shaped block: 1.075 and 1.10).
SPREAD = (0.83, 1.10)

# Fitted constants (seconds), timing_runs.fit.
_STEP = (6.231e-04, 4.364e-15, 1.049e-14)       # fixed, per token x block weight, per attention flop
_OUTLIER = 0.0                                  # per loss element (tokens x hidden)
_FORWARD = (1.691e-04, 1.358e-15, 3.585e-15)     # one forward over a batch: the same three terms
_PIECE = 6.668e-04                               # a step's every piece past the first
_FORWARD_PIECE = 1.411e-04                       # a forward's every piece past the first
_SEARCH = (1.433e-02, 4.461e-10)                 # per block: fixed, per block weight
_COMMIT = 5.0e-4                                # per block
_SCORING = (9.884e-02, 3.352e-02, 8.995e-10, 1.236e-10)  # fixed, per block, per block weight, per head weight
_OWN_WIDTH = 2.76
_SCORING_TOKENS = SENSITIVITY_SAMPLES * SENSITIVITY_SEQ_LEN

def _duration(seconds: float) -> str:
    """``seconds`` spoken the way a progress line says it: whole seconds under a
    minute ("45s"), minutes and seconds under 59.5 minutes ("7m14s"), hours and
    minutes from there on ("4h28m")."""
    if seconds < 3570:
        mins, secs = divmod(round(seconds), 60)
        return f"{mins}m{secs:02d}s" if mins else f"{secs}s"
    hours, mins = divmod(round(seconds / 60), 60)
    return f"{hours}h{mins:02d}m"


@dataclasses.dataclass(frozen=True)
class TimePrediction:
    """The seconds a run is predicted to record (``mround/planner/timing.py:139-206``).

    ``stages``: ``scoring`` (a mixed run's scoring pass), ``blocks`` (every
    block's own tuning as its result reports it: search, scores, steps,
    commit) and ``between_blocks`` (the targets pass of every block).
    """

    stages: dict[str, float]
    block: float
    blocks: int
    iters: int
    outlier_rule: bool
    pieces: int
    searched: bool
    scoring_source: str | None = None
    scoring_tokens: int | None = None

    @property
    def total(self) -> float:
        return sum(self.stages.values())

    def describe(self) -> str:
        scoring = self.stages.get("scoring", 0.0)
        parts = f"the scoring pass {_duration(scoring)} and " if scoring else ""
        return (f"time: predicted {_duration(self.total)} on {MACHINE} ({parts}{self.blocks} blocks of "
                f"{self.block:.2f}s), where the measured runs took {SPREAD[0]:.2f} to {SPREAD[1]:.2f} "
                f"times the rule")

    def record(self) -> dict[str, Any]:
        return {"rule": RULE_VERSION, "machine": MACHINE, "seconds": round(self.total, 2),
                "by_stage_seconds": {k: round(v, 2) for k, v in self.stages.items()},
                "block_seconds": round(self.block, 3), "blocks": self.blocks, "iters": self.iters,
                "outlier_rule": self.outlier_rule, "pieces": self.pieces, "searched": self.searched,
                "scoring_source": self.scoring_source, "scoring_tokens": self.scoring_tokens,
                "spread": list(SPREAD)}


def _work(model: ModelShape, batch: int, seq_len: int) -> tuple[float, float]:
    """(tokens x block weights, attention forward flops) of one batch, over the
    rows the engine runs (sequences padded to the attention tile)."""
    seq_len = aligned_rows(seq_len)
    tokens = batch * seq_len
    attention = 4.0 * batch * seq_len * seq_len / 2 * model.heads * model.head_dim
    return tokens * model.block_weights, attention


# Split precision's measured cost over its extra GEMM work: 7B-, 3B- and
# 0.5B-shaped block tunes (2-bit, 200 steps, 16 batches of 8 x 2048) ran
# 7.92, 2.96 and 0.84 s against 4.22, 1.63 and 0.52 s in bf16; the extra
# GEMM work alone predicts about 0.6 of the difference (the rest is the split
# operands' writes, the fp32 gate/up pair and W' made in fp32 each step).
# Scaled by 1.75 the rule puts the three at 0.93, 0.98 and 1.10 of it (bf16:
# 1.01, 1.02 and 1.075).
_SPLIT_EXTRA = 1.75


def split_forward_factor(model: ModelShape) -> float:
    """How much more GEMM work the forward does in split precision: 3x for
    every product but the attention output projection's 2x."""
    o = model.hidden * model.heads * model.head_dim
    return (3.0 * model.block_weights - o) / model.block_weights


def predict_time(model: ModelShape, run: RunShape, *, iters: int, outlier_rule: bool,
                 scoring_tokens: int | None = None, scoring_source: str | None = None) -> TimePrediction:
    """Predict the seconds a run records on one MI355X (``mround/planner/timing.py:209-282``).

    Raises:
        ValueError: If ``iters`` is not a positive number of steps.
    """
    if iters <= 0:
        raise ValueError(f"a run takes a positive number of steps, got {iters}")
    pieces = max(1, min(int(run.micro_batches), int(run.batch_size)))
    tw, att = _work(model, run.batch_size, run.seq_len)
    tw_forward = tw_step = tw
    if getattr(run, "split", False):
        # split precision: the forward's products over 3K (the attention
        # output projection over 2K, weighted by its share of the weights),
        # the backward's unchanged; the extra work's cost scaled by what the
        # split operands' own passes add (_SPLIT_EXTRA)
        f = split_forward_factor(model)
        tw_forward = tw * (1.0 + _SPLIT_EXTRA * (f - 1.0))
        tw_step = tw * (1.0 + _SPLIT_EXTRA * (f - 1.0) / 3.0)
    forward = _FORWARD[0] + _FORWARD[1] * tw_forward + _FORWARD[2] * att + (pieces - 1) * _FORWARD_PIECE
    step = _STEP[0] + _STEP[1] * tw_step + _STEP[2] * att + (pieces - 1) * _PIECE
    if outlier_rule:
        step += _OUTLIER * run.batch_size * aligned_rows(run.seq_len) * model.hidden
        if pieces > 1:
            step += forward
    batches = max(1, run.n_samples // run.batch_size)
    block = iters * step + 2 * batches * forward + _COMMIT
    if run.searched:
        block += _SEARCH[0] + _SEARCH[1] * model.block_weights
    stages: dict[str, float] = {}
    tokens = source = None
    if run.mixed:
        tokens = _SCORING_TOKENS if scoring_tokens is None else int(scoring_tokens)
        source = "own_width" if scoring_source == "own_width" else "widest"
        head = model.vocab * model.hidden * (1 if model.tied else 2)
        seconds = (_SCORING[0] + _SCORING[1] * model.layers + _SCORING[2] * model.layers * model.block_weights
                   + _SCORING[3] * head) * tokens / _SCORING_TOKENS
        stages["scoring"] = seconds * (_OWN_WIDTH if source == "own_width" else 1.0)
    stages["blocks"] = block * model.layers
    stages["between_blocks"] = batches * forward * model.layers
    return TimePrediction(stages=stages, block=block, blocks=model.layers, iters=iters, outlier_rule=outlier_rule,
                          pieces=pieces, searched=run.searched, scoring_source=source, scoring_tokens=tokens)


def predict_run_time(model: ModelShape, run: RunShape, tuning, bits: int, *,
                     candidate_bits: Collection[int] = (), per_layer_recipe: bool = False,
                     scoring_samples: int | None = None, scoring_seq_len: int | None = None,
                     gradient_source: str = "auto") -> TimePrediction:
    """:func:`predict_time` with the run's settings resolved as the run resolves
    them (``mround/planner/timing.py:285-338``): the outlier rule from the
    base width, or the narrowest candidate with a per-layer recipe; the
    scoring budget's defaults; the scoring gradients by size."""
    widths = sorted(int(w) for w in candidate_bits)
    base = widths[0] if per_layer_recipe and widths else bits
    tokens = source = None
    if run.mixed:
        tokens = ((SENSITIVITY_SAMPLES if scoring_samples is None else int(scoring_samples))
                  * (SENSITIVITY_SEQ_LEN if scoring_seq_len is None else int(scoring_seq_len)))
        source = gradient_source_for(gradient_source, model.layers * model.block_weights)
    return predict_time(model, run, iters=tuning.iters, outlier_rule=tuning.resolved_suppress_outliers(base),
                        scoring_tokens=tokens, scoring_source=source)
