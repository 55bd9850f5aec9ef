"""Command line: ``python -m mround_amd quantize MODEL -o OUT ...`` (the
``mround quantize`` subcommand of mround/cli/main.py:66-200, for local
checkpoints), ``plan`` (``mround.api.plan_mixed_precision``, api.py:943-1085:
score and allocate only), and ``random-model`` to write a random-initialised
checkpoint of a named geometry."""

from __future__ import annotations

import argparse
import json
import sys

GEOMETRIES = {
    # the benchmark configurations' model shapes
    "smollm2-135m": dict(model_type="llama", hidden_size=576, num_attention_heads=9, num_key_value_heads=3,
                         head_dim=64, intermediate_size=1536, rms_norm_eps=1e-5, rope_theta=10000.0,
                         num_hidden_layers=30, vocab_size=49152, tie_word_embeddings=True),
    "qwen2.5-0.5b": dict(model_type="qwen2", hidden_size=896, num_attention_heads=14, num_key_value_heads=2,
                         intermediate_size=4864, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=24,
                         vocab_size=151936, tie_word_embeddings=True),
    "qwen2.5-3b": dict(model_type="qwen2", hidden_size=2048, num_attention_heads=16, num_key_value_heads=2,
                       intermediate_size=11008, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=36,
                       vocab_size=151936, tie_word_embeddings=True),
    "qwen2.5-7b": dict(model_type="qwen2", hidden_size=3584, num_attention_heads=28, num_key_value_heads=4,
                       intermediate_size=18944, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=28,
                       vocab_size=152064, tie_word_embeddings=False),
}


def _parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(prog="mround_amd", description="SignRound v2 quantization on MI355X")
    sub = p.add_subparsers(dest="command", required=True)
    q = sub.add_parser("quantize", help="quantize a local checkpoint into an MLX checkpoint")
    q.add_argument("model", help="local checkpoint directory (config.json + *.safetensors)")
    q.add_argument("-o", "--output-dir", required=True)
    q.add_argument("-b", "--bits", type=int, default=4)
    q.add_argument("-g", "--group-size", type=int, default=64)
    q.add_argument("--asym", action="store_true", help="asymmetric codes with a zero point")
    q.add_argument("--average-bits", type=float, default=None)
    q.add_argument("--options", default="2,3,4",
                   help="candidate widths for --average-bits, comma separated (default: 2,3,4)")
    q.add_argument("--remainder-bits", type=int, default=None,
                   help="width for the tensors outside the block stack (default: nearest the average)")
    q.add_argument("--plan", default=None, help="JSON file mapping layer paths to widths")
    q.add_argument("--format", default="mlx")
    q.add_argument("--iters", type=int, default=None)
    q.add_argument("--samples", type=int, default=None)
    q.add_argument("--seq-len", type=int, default=None)
    q.add_argument("--batch-size", type=int, default=None)
    q.add_argument("--lr", type=float, default=None)
    q.add_argument("--calibration", default="random")
    q.add_argument("--seed", type=int, default=None)
    q.add_argument("--micro-batches", type=int, default=None,
                   help="run each step's batch in this many pieces, summing their gradients (default: 1)")
    q.add_argument("--allow-dense", action="store_true",
                   help="proceed even when the group size reaches under half of the block stack's layers")
    q.add_argument("--split-precision", action=argparse.BooleanOptionalAction, default=None,
                   help="run the block forward as three bf16 products of hi and lo halves per product "
                        "(about 16-bit operands, about 1.9x the tune time; default: on when a tuned width "
                        "is 8 bits)")
    q.add_argument("--memory-budget", type=float, default=None,
                   help="GB the run may use on the device (default: 90 %% of its memory)")
    q.add_argument("--skip-memory-check", action="store_true",
                   help="run even when the prediction exceeds the budget")
    q.add_argument("--dry-run", action="store_true",
                   help="predict the run's peak device memory against the budget and stop; "
                        "exits 0 when it fits, 1 when the run would be refused")
    pl = sub.add_parser("plan", help="score and allocate a mixed-precision plan; nothing is tuned")
    pl.add_argument("model", help="local checkpoint directory (config.json + *.safetensors)")
    pl.add_argument("--average-bits", type=float, required=True)
    pl.add_argument("--options", default="2,3,4", help="candidate widths, comma separated")
    pl.add_argument("-b", "--bits", type=int, default=4)
    pl.add_argument("-g", "--group-size", type=int, default=64)
    pl.add_argument("--asym", action="store_true")
    pl.add_argument("--remainder-bits", type=int, default=None)
    pl.add_argument("--gradients", default="auto", help="auto, own_width or widest")
    pl.add_argument("--scoring-samples", type=int, default=None)
    pl.add_argument("--scoring-seq-len", type=int, default=None)
    pl.add_argument("--scoring-batch-size", type=int, default=None)
    pl.add_argument("--seed", type=int, default=None)
    pl.add_argument("--write", default=None, help="write the per-layer widths as JSON (for --plan)")
    r = sub.add_parser("random-model", help="write a random-initialised checkpoint")
    r.add_argument("geometry", choices=sorted(GEOMETRIES))
    r.add_argument("output_dir")
    r.add_argument("--layers", type=int, default=None, help="override the layer count")
    r.add_argument("--seed", type=int, default=0)
    r.add_argument("--device", default="cuda")
    return p


def _widths(options: str) -> tuple[int, ...]:
    """``--options`` as candidate widths (mround/cli/main.py:439-451)."""
    try:
        return tuple(int(piece) for piece in options.split(",") if piece.strip())
    except ValueError:
        raise ValueError(f"--options must be comma separated integers, not {options!r}") from None


def _tuning(args):
    from mround_amd.schemes import TuningConfig

    kw = {}
    for field, val in (("iters", args.iters), ("n_samples", args.samples), ("seq_len", args.seq_len),
                       ("batch_size", args.batch_size), ("lr", args.lr),
                       ("micro_batches", getattr(args, "micro_batches", None))):
        if val is not None:
            kw[field] = val
    return TuningConfig(**kw)


def main(argv=None) -> int:
    args = _parser().parse_args(argv)
    from mround_amd.exceptions import MRoundError

    try:
        if args.command == "random-model":
            from mround_amd.pipeline.checkpoint import write_random_checkpoint

            cfg = dict(GEOMETRIES[args.geometry])
            if args.layers is not None:
                cfg["num_hidden_layers"] = args.layers
            path = write_random_checkpoint(args.output_dir, cfg, seed=args.seed, device=args.device)
            print(f"wrote {path}")
            return 0
        from mround_amd import api
        from mround_amd.schemes import Symmetry

        if args.command == "plan":
            info = api.plan_mixed_precision(
                args.model, args.average_bits, _widths(args.options), bits=args.bits,
                group_size=args.group_size, symmetry=Symmetry.ASYMMETRIC if args.asym else Symmetry.SYMMETRIC,
                sensitivity_gradients=args.gradients, remainder_bits=args.remainder_bits,
                scoring_samples=args.scoring_samples, scoring_seq_len=args.scoring_seq_len,
                scoring_batch_size=args.scoring_batch_size, seed=args.seed,
                progress=lambda step: print(step.describe(), flush=True))
            print(f"  {info['describe']}")
            if args.write:
                with open(args.write, "w") as f:
                    json.dump(info["assignments"], f, indent=1)
                print(f"  wrote {args.write}")
            return 0

        budget = None if args.memory_budget is None else int(args.memory_budget * 1e9)
        if args.dry_run:
            check = api.predict_memory(
                args.model, bits=args.bits, group_size=args.group_size,
                symmetry=Symmetry.ASYMMETRIC if args.asym else Symmetry.SYMMETRIC,
                average_bits=args.average_bits, candidate_bits=_widths(args.options),
                remainder_bits=args.remainder_bits, tuning=_tuning(args), memory_budget=budget,
                split_precision=args.split_precision)
            print(f"  {check.explain()}")
            timing = api.predict_time(
                args.model, bits=args.bits, group_size=args.group_size,
                symmetry=Symmetry.ASYMMETRIC if args.asym else Symmetry.SYMMETRIC,
                average_bits=args.average_bits, candidate_bits=_widths(args.options),
                remainder_bits=args.remainder_bits, tuning=_tuning(args),
                split_precision=args.split_precision)
            print(f"  {timing.describe()}")
            return 0 if check.fits else 1
        plan = None
        if args.plan:
            with open(args.plan) as f:
                plan = {k: int(v) for k, v in json.load(f).items()}
        result = api.quantize(args.model, output_dir=args.output_dir, bits=args.bits,
                              group_size=args.group_size,
                              symmetry=Symmetry.ASYMMETRIC if args.asym else Symmetry.SYMMETRIC,
                              average_bits=args.average_bits, candidate_bits=_widths(args.options),
                              remainder_bits=args.remainder_bits, plan=plan, tuning=_tuning(args),
                              calibration=args.calibration, export_format=args.format,
                              min_block_coverage=0.0 if args.allow_dense else api.MIN_BLOCK_COVERAGE,
                              split_precision=args.split_precision, seed=args.seed, memory_budget=budget,
                              memory_check=not args.skip_memory_check,
                              progress=lambda b: print(f"  block {b.index}: loss {b.initial_loss:.4g} -> "
                                                       f"{b.final_loss:.4g} in {b.seconds:.2f} s", flush=True),
                              scoring_progress=lambda step: print(step.describe(), flush=True))
    except (MRoundError, ValueError) as exc:
        print(f"mround: {exc}", file=sys.stderr)
        return 1
    if result.mixed:
        print(f"  {result.mixed['describe']}")
    print(f"  {result.describe()}")
    for path, reason in result.skipped:
        print(f"  left dense  {path}: {reason}")
    print(f"  wrote {result.output_dir}")
    return 0
