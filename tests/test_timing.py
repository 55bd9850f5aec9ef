"""The MI355X time rule against the runs it was fitted to
(``mround/planner/timing.py`` is the reference's rule for its Mac;
``tests/unit/test_time_rule.py`` holds that rule to the reference's runs).

``tests/golden/mi355x_timing_runs.json`` holds the records of
``python -m mround_amd.planner.timing_runs`` on one MI355X: model shapes from
SmolLM2-135M to Qwen2.5-7B, the outlier rule on and off, pieces, the scale
search, other batches and calibration sets, the mixed scoring pass at both
gradient sources. The rule must put every run's block loop and scoring pass
inside its stated spread, and refitting the records must give back its
constants.
"""

from __future__ import annotations

import json
from pathlib import Path

import pytest

from mround_amd.planner import timing as TM
from mround_amd.planner.memory import ModelShape, RunShape
from mround_amd.planner.timing_runs import fit
from mround_amd.schemes import TuningConfig

RUNS = json.loads((Path(__file__).parent / "golden" / "mi355x_timing_runs.json").read_text())["runs"]


def _predict(r):
    model = ModelShape.from_config(r["config"])
    run = RunShape(n_samples=r["n_samples"], seq_len=r["seq_len"], batch_size=r["batch_size"], group_size=64,
                   searched=r["searched"], mixed=r["scoring_seconds"] is not None,
                   micro_batches=r["micro_batches"])
    return TM.predict_time(model, run, iters=r["iters"], outlier_rule=r["outlier_rule"],
                           scoring_source=r.get("scoring_source"))


@pytest.mark.parametrize("r", RUNS, ids=lambda r: f"{r['model']}-L{r['config']['num_hidden_layers']}-"
                         + "-".join(f"{k}{v}" for k, v in r["settings"].items()))
def test_every_run_inside_the_spread(r):
    p = _predict(r)
    loop = r["seconds"]["blocks"] / (p.stages["blocks"] + p.stages["between_blocks"])
    assert TM.SPREAD[0] <= loop <= TM.SPREAD[1], loop
    if r["scoring_seconds"] is not None:
        scoring = r["seconds"]["plan"] / p.stages["scoring"]
        assert TM.SPREAD[0] <= scoring <= TM.SPREAD[1], scoring


def test_every_run_but_the_smallest_shape_within_seven_percent():
    """SmolLM2-135M's small steps run under the rule's fixed part (0.83-0.87):
    the rest of the shapes sit within 7 %."""
    for r in RUNS:
        if r["model"] == "smollm2-135m":
            continue
        p = _predict(r)
        ratio = r["seconds"]["blocks"] / (p.stages["blocks"] + p.stages["between_blocks"])
        assert abs(ratio - 1.0) <= 0.07, (r["model"], r["settings"], ratio)


def test_refit_gives_the_constants():
    c = fit(RUNS)
    pairs = [(c["step"], TM._STEP), (c["forward"], TM._FORWARD), (c["search"], TM._SEARCH),
             (c["scoring"], TM._SCORING), ([c["outlier"], c["piece"], c["forward_piece"], c["own_width"]],
                                           [TM._OUTLIER, TM._PIECE, TM._FORWARD_PIECE, TM._OWN_WIDTH])]
    for got, want in pairs:
        for g, w in zip(got, want):
            assert g == pytest.approx(w, rel=2e-3), (got, want)


def _shape(name):
    from mround_amd.planner.timing_runs import SHAPES

    return ModelShape.from_config(SHAPES[name])


def test_stages_and_record():
    model = _shape("qwen2.5-7b")
    run = RunShape(n_samples=128, seq_len=2048, batch_size=8, group_size=64, mixed=True)
    p = TM.predict_run_time(model, run, TuningConfig(), 2, candidate_bits=(2, 3, 4))
    assert set(p.stages) == {"scoring", "blocks", "between_blocks"}
    assert p.blocks == 28 and p.iters == 200 and p.outlier_rule and p.pieces == 1
    assert p.scoring_source == "own_width" and p.scoring_tokens == 128 * 1024  # 6.5 B weights: own width
    assert p.total == pytest.approx(sum(p.stages.values()))
    rec = p.record()
    assert rec["rule"] == TM.RULE_VERSION and rec["spread"] == list(TM.SPREAD)
    assert "MI355X" in p.describe()
    # a 7B block: about 4.2 s (the bench measures 4.15-4.2)
    assert 3.9 < p.block < 4.5


def test_scaling():
    model = _shape("qwen2.5-3b")
    base = RunShape(n_samples=128, seq_len=2048, batch_size=8, group_size=64)
    p = TM.predict_time(model, base, iters=200, outlier_rule=False)
    # more steps cost more, linearly
    p2 = TM.predict_time(model, base, iters=400, outlier_rule=False)
    p3 = TM.predict_time(model, base, iters=600, outlier_rule=False)
    assert p3.block - p2.block == pytest.approx(p2.block - p.block)
    # pieces and the search add; the outlier rule never takes away (with the
    # one-pass outlier loss its fitted extra cost is zero, inside the scatter)
    for run in (RunShape(128, 2048, 8, 64, micro_batches=4), RunShape(128, 2048, 8, 64, searched=True)):
        assert TM.predict_time(model, run, iters=200, outlier_rule=False).block > p.block
    assert TM.predict_time(model, base, iters=200, outlier_rule=True).block >= p.block
    # half the calibration set: the passes halve, the steps do not
    half = TM.predict_time(model, RunShape(64, 2048, 8, 64), iters=200, outlier_rule=False)
    assert half.stages["between_blocks"] == pytest.approx(p.stages["between_blocks"] / 2)
    assert p.block > half.block > 0.9 * p.block
    # the own-width scoring pass costs more than the widest's
    mixed = RunShape(128, 2048, 8, 64, mixed=True)
    w = TM.predict_time(model, mixed, iters=200, outlier_rule=False, scoring_source="widest")
    o = TM.predict_time(model, mixed, iters=200, outlier_rule=False, scoring_source="own_width")
    assert o.stages["scoring"] == pytest.approx(TM._OWN_WIDTH * w.stages["scoring"])


SPLIT_RUNS = json.loads((Path(__file__).parent / "golden" / "mi355x_split_runs.json").read_text())["runs"]


@pytest.mark.parametrize("r", SPLIT_RUNS, ids=lambda r: r["model"])
def test_split_precision_runs_inside_the_spread(r):
    """Block tunes measured in bf16 and in split precision (2-bit, 200 steps,
    16 batches of 8 x 2048, outlier rule on): both inside the rule's spread."""
    model = ModelShape.from_config({**r["config"], "num_hidden_layers": 1, "vocab_size": 151936,
                                    "tie_word_embeddings": True})
    for split, key in ((False, "bf16_seconds"), (True, "split_seconds")):
        run = RunShape(n_samples=128, seq_len=2048, batch_size=8, group_size=64, split=split)
        ratio = r[key] / TM.predict_time(model, run, iters=200, outlier_rule=True).block
        assert TM.SPREAD[0] <= ratio <= TM.SPREAD[1], (key, ratio)


def test_split_precision_costs_more():
    model = _shape("qwen2.5-3b")
    plain = TM.predict_time(model, RunShape(128, 2048, 8, 64), iters=200, outlier_rule=False)
    split = TM.predict_time(model, RunShape(128, 2048, 8, 64, split=True), iters=200, outlier_rule=False)
    assert 1.4 * plain.block < split.block < 2.2 * plain.block
    assert 2.8 < TM.split_forward_factor(model) < 3.0


def test_refuses_no_steps():
    with pytest.raises(ValueError):
        TM.predict_time(_shape("qwen2.5-0.5b"), RunShape(128, 2048, 8, 64), iters=0, outlier_rule=False)


def test_api_reads_the_config_alone(tmp_path):
    """``api.predict_time`` from ``config.json``: the 7B shape's 28 blocks."""
    from mround_amd import api
    from mround_amd.planner.timing_runs import SHAPES

    (tmp_path / "config.json").write_text(json.dumps(SHAPES["qwen2.5-7b"]))
    p = api.predict_time(tmp_path, bits=2)
    assert p.blocks == 28 and p.outlier_rule and "scoring" not in p.stages
    assert 28 * 3.9 < p.stages["blocks"] < 28 * 4.5
    mixed = api.predict_time(tmp_path, average_bits=2.5)
    assert mixed.scoring_source == "own_width" and mixed.stages["scoring"] > 0
