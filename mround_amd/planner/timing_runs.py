"""The measurement runs the MI355X time rule (``mround_amd.planner.timing``)
is fitted to, and checked against.

``python -m mround_amd.planner.timing_runs OUT.json`` quantizes random-init
checkpoints of the benchmark model shapes, a few blocks each, at the standard
recipe (200 steps of 8 sequences of 2048 tokens, 128 calibration sequences),
and writes one record per run: the model shape, the run's settings and the
seconds each stage took, per block and in total. Random weights and uniform
token ids cost the same as real ones (every kernel's work is fixed by the
shapes), so these are the seconds a real run of the same shapes takes.

The runs vary what the rule depends on: the block's weights (SmolLM2-135M to
Qwen2.5-7B), the outlier rule (2 bits on, 4 bits off), pieces
(``micro_batches``), the symmetric scale search, the step count, and the
mixed-precision scoring pass. It takes a few minutes on one MI355X.
"""

from __future__ import annotations

import argparse
import json
import sys
import tempfile
import time
from pathlib import Path

# Shapes of the models the rule covers (Hugging Face configuration keys).
SHAPES = {
    "smollm2-135m": dict(model_type="llama", hidden_size=576, num_attention_heads=9, num_key_value_heads=3,
                         head_dim=64, intermediate_size=1536, rms_norm_eps=1e-5, rope_theta=10000.0,
                         num_hidden_layers=30, vocab_size=49152, tie_word_embeddings=True),
    "qwen2.5-0.5b": dict(model_type="qwen2", hidden_size=896, num_attention_heads=14, num_key_value_heads=2,
                         intermediate_size=4864, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=24,
                         vocab_size=151936, tie_word_embeddings=True),
    "qwen2.5-1.5b": dict(model_type="qwen2", hidden_size=1536, num_attention_heads=12, num_key_value_heads=2,
                         intermediate_size=8960, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=28,
                         vocab_size=151936, tie_word_embeddings=True),
    "qwen2.5-3b": dict(model_type="qwen2", hidden_size=2048, num_attention_heads=16, num_key_value_heads=2,
                       intermediate_size=11008, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=36,
                       vocab_size=151936, tie_word_embeddings=True),
    "qwen2.5-7b": dict(model_type="qwen2", hidden_size=3584, num_attention_heads=28, num_key_value_heads=4,
                       intermediate_size=18944, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=28,
                       vocab_size=152064, tie_word_embeddings=False),
}

# (shape, blocks, settings): the runs the rule is fitted to.
RUNS = [
    ("smollm2-135m", 3, dict(bits=4)),
    ("smollm2-135m", 3, dict(bits=2)),
    ("qwen2.5-0.5b", 3, dict(bits=4)),
    ("qwen2.5-0.5b", 3, dict(bits=2)),
    ("qwen2.5-0.5b", 3, dict(bits=2, micro_batches=4)),
    ("qwen2.5-0.5b", 3, dict(bits=2, symmetric=True)),
    ("qwen2.5-0.5b", 3, dict(bits=4, iters=50)),
    ("qwen2.5-0.5b", 3, dict(average_bits=2.5)),
    ("qwen2.5-1.5b", 2, dict(bits=4)),
    ("qwen2.5-1.5b", 2, dict(bits=2)),
    ("qwen2.5-3b", 2, dict(bits=4)),
    ("qwen2.5-3b", 2, dict(bits=2)),
    ("qwen2.5-3b", 2, dict(bits=2, micro_batches=4)),
    ("qwen2.5-3b", 2, dict(average_bits=2.5)),
    ("qwen2.5-7b", 2, dict(bits=4)),
    ("qwen2.5-7b", 2, dict(bits=2)),
    # pieces, search, other batches and calibration sets, longer scoring models
    ("qwen2.5-1.5b", 2, dict(bits=2, micro_batches=2)),
    ("qwen2.5-7b", 2, dict(bits=2, micro_batches=4)),
    ("qwen2.5-1.5b", 2, dict(bits=2, symmetric=True)),
    ("qwen2.5-7b", 2, dict(bits=2, symmetric=True)),
    ("qwen2.5-3b", 2, dict(bits=4, batch_size=4)),
    ("qwen2.5-0.5b", 3, dict(bits=4, n_samples=64)),
    ("qwen2.5-0.5b", 24, dict(average_bits=2.5)),
    ("qwen2.5-3b", 8, dict(average_bits=2.5)),
    ("qwen2.5-7b", 2, dict(average_bits=2.5)),
    ("qwen2.5-0.5b", 24, dict(average_bits=2.5, own_width=True)),
    ("qwen2.5-3b", 8, dict(average_bits=2.5, own_width=True)),
]


def run_one(root: Path, name: str, blocks: int, settings: dict, seed: int = 0) -> dict:
    import torch

    from mround_amd import api
    from mround_amd.pipeline.checkpoint import write_random_checkpoint
    from mround_amd.schemes import Symmetry, TuningConfig

    config = dict(SHAPES[name], num_hidden_layers=blocks)
    src = write_random_checkpoint(root / f"{name}-{blocks}", config, seed=seed, device="cuda")
    tuning = TuningConfig(iters=settings.get("iters", 200), batch_size=settings.get("batch_size", 8),
                          n_samples=settings.get("n_samples", 128), seq_len=2048,
                          micro_batches=settings.get("micro_batches", 1))
    kwargs = dict(symmetry=Symmetry.SYMMETRIC if settings.get("symmetric") else Symmetry.ASYMMETRIC,
                  tuning=tuning, seed=seed)
    if "average_bits" in settings:
        kwargs.update(average_bits=settings["average_bits"], candidate_bits=(2, 3, 4),
                      sensitivity_gradients="own_width" if settings.get("own_width") else "auto")
    else:
        kwargs.update(bits=settings["bits"])
    torch.cuda.synchronize()
    res = api.quantize(src, output_dir=root / "out", **kwargs)
    base_bits = settings.get("bits", 4)  # a mixed run's block loop takes the rule from the base width
    scoring = res.mixed or {}
    return {
        "model": name, "config": config, "settings": settings, "iters": tuning.iters,
        "batch_size": tuning.batch_size, "n_samples": tuning.n_samples, "seq_len": tuning.seq_len,
        "micro_batches": tuning.micro_batches, "searched": bool(settings.get("symmetric")) and base_bits < 4,
        "outlier_rule": tuning.resolved_suppress_outliers(base_bits),
        "seconds": {k: round(v, 4) for k, v in res.seconds.items()},
        "scoring_seconds": scoring.get("scoring_seconds"),
        "scoring_source": scoring.get("gradient_source"),
        "blocks": [{"seconds": round(b.seconds, 4), "search_seconds": round(b.search_seconds, 4),
                    "stages": {k: round(v, 4) for k, v in b.stage_seconds.items()}}
                   for b in res.summary.blocks],
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("out", help="JSON file for the records")
    ap.add_argument("--first", type=int, default=0, help="start at this entry of RUNS")
    ap.add_argument("--count", type=int, default=0, help="run this many entries (0: to the end)")
    args = ap.parse_args(argv)
    records = []
    with tempfile.TemporaryDirectory() as tmp:
        root = Path(tmp)
        # one small run first, so that library loading and first launches stay out of the records
        run_one(root, "smollm2-135m", 1, dict(bits=4, iters=5))
        last = args.first + args.count if args.count > 0 else len(RUNS)
        for name, blocks, settings in RUNS[args.first:last]:
            t0 = time.perf_counter()
            rec = run_one(root, name, blocks, settings)
            records.append(rec)
            print(f"{name} x{blocks} {settings}: loop {rec['seconds']['blocks']:.2f} s "
                  f"({time.perf_counter() - t0:.1f} s with set-up)", flush=True)
    Path(args.out).write_text(json.dumps({"runs": records}, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())


# ---------------------------------------------------------------------- fit --

def _features(record: dict) -> dict:
    """Per-run quantities the rule reads: block weights W, tokens per step T,
    the attention forward's flops per step A, hidden h, batches per pass."""
    c = record["config"]
    h, heads, kv = c["hidden_size"], c["num_attention_heads"], c["num_key_value_heads"]
    d = c.get("head_dim") or h // heads
    w = (heads * d * h * 2 + kv * d * h * 2 + 3 * c["intermediate_size"] * h)
    b, s = record["batch_size"], record["seq_len"]
    return dict(W=w, T=b * s, A=4.0 * b * s * s / 2 * heads * d, h=h, nb=record["n_samples"] // b,
                L=c["num_hidden_layers"], Vh=c["vocab_size"] * h * (1 if c.get("tie_word_embeddings") else 2))


def fit(records: list[dict]) -> dict:
    """Least-squares constants of the rule from the records (the last block of
    each run, past the first block's warm-up)."""
    import numpy as np

    rows = []
    for r in records:
        f = _features(r)
        st = r["blocks"][-1]["stages"]
        rows.append((r, f, st))
    std = [(r, f, st) for r, f, st in rows if r["micro_batches"] == 1]
    # a step: fixed + GEMM work (tokens x weights) + attention; outlier rule additive per loss element
    x = np.array([[1.0, f["T"] * f["W"] / 1e12, f["A"] / 1e12] for r, f, st in std if not r["outlier_rule"]])
    y = np.array([st["tune"] / r["iters"] for r, f, st in std if not r["outlier_rule"]])
    step = np.linalg.lstsq(x, y, rcond=None)[0]
    t_step = lambda f: step[0] + step[1] * f["T"] * f["W"] / 1e12 + step[2] * f["A"] / 1e12
    out = [(st["tune"] / r["iters"] - t_step(f)) / (f["T"] * f["h"]) for r, f, st in std if r["outlier_rule"]]
    # (a cost, so not below zero: with the one-pass outlier loss the rule's
    # extra cost is inside the runs' scatter and the median can come out
    # negative)
    outlier = max(0.0, float(np.median(out)))
    # one forward pass over a batch (the score, targets and advance passes)
    x = np.array([[1.0, f["T"] * f["W"] / 1e12, f["A"] / 1e12] for r, f, st in std])
    y = np.array([st["score"] / f["nb"] for r, f, st in std])
    fwd = np.linalg.lstsq(x, y, rcond=None)[0]
    t_fwd = lambda f: fwd[0] + fwd[1] * f["T"] * f["W"] / 1e12 + fwd[2] * f["A"] / 1e12
    # pieces: each piece past the first costs a fixed part; the outlier rule adds a forward of the batch
    pcs = [(r, f, st) for r, f, st in rows if r["micro_batches"] > 1]
    num = sum(st["tune"] / r["iters"] - t_step(f) - (t_fwd(f) if r["outlier_rule"] else 0.0)
              - outlier * f["T"] * f["h"] * r["outlier_rule"] for r, f, st in pcs)
    piece = num / sum(r["micro_batches"] - 1 for r, f, st in pcs)
    fpiece = sum(st["score"] / f["nb"] - t_fwd(f) for r, f, st in pcs) / sum(r["micro_batches"] - 1
                                                                              for r, f, st in pcs)
    # the scale search per block, the commit per block
    srch = [(f["W"], r["blocks"][-1]["search_seconds"]) for r, f, st in rows if r["searched"]]
    search = np.polyfit([w for w, _ in srch], [t for _, t in srch], 1)[::-1]
    commit = float(np.median([st["commit"] for r, f, st in rows]))
    # the mixed scoring pass at the widest width: fixed + per block + per block weight + the head
    mix = [(r, f) for r, f, st in rows if r["scoring_seconds"] is not None]
    wide = [(r, f) for r, f in mix if r["scoring_source"] == "widest"]
    x = np.array([[1.0, f["L"], f["L"] * f["W"] / 1e9, f["Vh"] / 1e9] for r, f in wide])
    y = np.array([r["seconds"]["plan"] for r, f in wide])
    scoring = np.linalg.lstsq(x, y, rcond=None)[0]
    pred = lambda f: scoring @ np.array([1.0, f["L"], f["L"] * f["W"] / 1e9, f["Vh"] / 1e9])
    own = [r["seconds"]["plan"] / pred(f) for r, f in mix if r["scoring_source"] == "own_width"]
    # in seconds per unit (the features above are in 1e12 and 1e9 units)
    return {"step": [float(step[0]), float(step[1]) / 1e12, float(step[2]) / 1e12], "outlier": outlier,
            "forward": [float(fwd[0]), float(fwd[1]) / 1e12, float(fwd[2]) / 1e12],
            "piece": float(piece), "forward_piece": float(fpiece), "search": [float(v) for v in search],
            "commit": commit,
            "scoring": [float(scoring[0]), float(scoring[1]), float(scoring[2]) / 1e9, float(scoring[3]) / 1e9],
            "own_width": float(np.mean(own))}
