"""Benchmark of the SignRound v2 tuning path on one MI355X.

Default workload -- the fake-quant kernel microbench: one bf16 weight of
18944 x 3584 (a Qwen2.5-7B gate/up projection) drawn N(0, 0.02) with 0.1 % of
entries scaled x10; v ~ U(-0.5, 0.5), alpha = beta = 1, dL/dW' ~ N(0, 1)
fp32; 2-bit asymmetric, group size 64. One step is one pass of the path over
the matrix: fake-quant forward (bf16 W' out), straight-through backward fused
with the sign-SGD step, then codes + MLX uint32 packing. Inputs are resident
in HBM before the timed region.

Printed as one JSON line:
  value      achieved HBM GB/s of the fake-quant forward (algorithmic bytes:
             read W 2 B + v 4 B, write W' 2 B per weight, alpha/beta 8 B per
             group) over the K timed steps, step-to-step wall clock;
  roofline   the forward kernel's average launch duration -- K back-to-back
             launches between two HIP events on the launch stream -- against
             8 TB/s;
  kernels    the same for the backward + update (14.25 B/weight at gs 64) and
             the packing kernel (1 + b/8 B/weight);
  sweep      (--sweep) every bits x group size of the microbench;
  cpu_baseline  the NumPy float32 oracle's forward on a bounded sample of rows
             of the same matrix, single-threaded.

``--gpus N`` with N > 1 exits: this build runs on one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROWS, COLS = 18944, 3584
HBM_PEAK_GBPS = 8000.0


def _inputs(torch, dev, gs):
    gen = torch.Generator().manual_seed(0)
    w = torch.randn(ROWS, COLS, generator=gen) * 0.02
    n_out = int(round(0.001 * ROWS * COLS))
    idx = torch.randperm(ROWS * COLS, generator=torch.Generator().manual_seed(1))[:n_out]
    w.view(-1)[idx] *= 10.0
    w = w.to(torch.bfloat16)
    ng = COLS // gs
    v = (torch.rand(ROWS, ng, gs, generator=torch.Generator().manual_seed(2)) - 0.5)
    g = torch.randn(ROWS, COLS, generator=torch.Generator().manual_seed(3))
    return (w.to(dev), v.to(dev), torch.ones(ROWS, ng, 1, device=dev),
            torch.ones(ROWS, ng, 1, device=dev), g.to(dev), w)


def fwd_bytes(n, gs):
    return n * (2 + 4 + 2) + (n // gs) * 8


def bwd_bytes(n, gs):
    return n * (2 + 4 + 4 + 4) + (n // gs) * 16


def pack_bytes(n, bits):
    return n * (1 + bits / 8)


def run_config(torch, K, dev, bits, gs, steps, warmup):
    """Times one (bits, gs) configuration; returns per-kernel averages in ms."""
    w, v, a, b, g, _ = _inputs(torch, dev, gs)
    n = ROWS * COLS
    wq = torch.empty(ROWS, COLS, dtype=torch.bfloat16, device=dev)
    codes = torch.empty(ROWS, COLS, dtype=torch.uint8, device=dev)
    scale = torch.empty(ROWS, COLS // gs, dtype=torch.float32, device=dev)
    zp = torch.empty_like(scale)
    words = K.packed_width(COLS, bits)
    packed = torch.empty(ROWS, words, dtype=torch.uint32, device=dev)

    def fwd():
        K.fq_forward(w, v, a, b, bits=bits, group_size=gs, mode="asym", eps=1e-8, wq_out=wq)

    def bwd():
        K.fq_backward_signsgd(w, v, a, b, g, bits=bits, group_size=gs, mode="asym", eps=1e-8,
                              update=True, lr=0.005, coef_lo=0.1, coef_hi=1.0, v_bound=0.5)

    def codes_k():
        K.fq_forward(w, v, a, b, bits=bits, group_size=gs, mode="asym", eps=1e-8, codes_out=codes,
                     scale_out=scale, zp_out=zp)

    def pack():
        K.pack_codes(codes, bits, signed=False, offset=0, packed_out=packed)

    stream = torch.cuda.current_stream(dev)
    for _ in range(warmup):
        fwd(); bwd(); codes_k(); pack()
    torch.cuda.synchronize(dev)

    # Each kernel's average launch duration: `steps` back-to-back launches on
    # the launch stream between two HIP events.
    avg = {}
    t0 = time.perf_counter()
    for name, fn in (("fwd", fwd), ("bwd", bwd), ("codes", codes_k), ("pack", pack)):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(stream)
        for _ in range(steps):
            fn()
        e.record(stream)
        e.synchronize()
        avg[name] = s.elapsed_time(e) / steps
    wall = time.perf_counter() - t0
    return {
        "bits": bits,
        "group_size": gs,
        "wall_s": wall,
        "ms": avg,
        "gbps": {
            "fwd": fwd_bytes(n, gs) / (avg["fwd"] * 1e-3) / 1e9,
            "bwd_update": bwd_bytes(n, gs) / (avg["bwd"] * 1e-3) / 1e9,
            "pack": pack_bytes(n, bits) / (avg["pack"] * 1e-3) / 1e9,
        },
    }


def time_forward_steps(torch, K, dev, bits, gs, steps, warmup):
    """Step-to-step wall clock of K forward passes (the value)."""
    w, v, a, b, _, _ = _inputs(torch, dev, gs)
    wq = torch.empty(ROWS, COLS, dtype=torch.bfloat16, device=dev)
    for _ in range(warmup):
        K.fq_forward(w, v, a, b, bits=bits, group_size=gs, mode="asym", eps=1e-8, wq_out=wq)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        K.fq_forward(w, v, a, b, bits=bits, group_size=gs, mode="asym", eps=1e-8, wq_out=wq)
    torch.cuda.synchronize(dev)
    return (time.perf_counter() - t0) / steps


def cpu_baseline(bits, gs, rows_sample=ROWS, reps=5):
    """The oracle's float32 forward on ``rows_sample`` rows, single-threaded NumPy."""
    import numpy as np
    import torch

    from oracle.quantize import fake_quantize

    gen = torch.Generator().manual_seed(0)
    w = (torch.randn(ROWS, COLS, generator=gen) * 0.02)[:rows_sample].to(torch.bfloat16).float().numpy()
    v = (torch.rand(ROWS, COLS // gs, gs, generator=torch.Generator().manual_seed(2)) - 0.5)[:rows_sample].numpy()
    a = np.ones((rows_sample, COLS // gs, 1), dtype=np.float32)
    fake_quantize(w, v, a, a, bits=bits, group_size=gs, mode="asym")  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fake_quantize(w, v, a, a, bits=bits, group_size=gs, mode="asym")
        times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    n = rows_sample * COLS
    return {
        "value": fwd_bytes(n, gs) / t / 1e9,
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"oracle.quantize.fake_quantize (NumPy float32) on {rows_sample} of {ROWS} rows "
                   f"x {COLS}, {bits}-bit asym gs{gs}, median of {reps} after 1 warm-up: "
                   f"{t:.3f} s per pass"),
        "cpu": _cpu_model(),
    }


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--bits", type=int, default=2)
    ap.add_argument("--group-size", type=int, default=64)
    ap.add_argument("--sweep", action="store_true", help="also time every bits x group size")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-kernels", action="store_true",
                    help="only launch the forward and a copy of known size (for counter runs)")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU; multi-GPU runs are not part of it "
              "(how the path would shard is described in DESIGN.md)", file=sys.stderr)
        return 2

    import torch

    from mround_amd import kernels as K

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    K.lib()  # fail loudly if the HIP library is missing
    dev = torch.device("cuda:0")

    if args.profile_kernels:
        w, v, a, b, _, _ = _inputs(torch, dev, args.group_size)
        wq = torch.empty(ROWS, COLS, dtype=torch.bfloat16, device=dev)
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            K.fq_forward(w, v, a, b, bits=args.bits, group_size=args.group_size, mode="asym",
                         eps=1e-8, wq_out=wq)
            K.copy_bytes(src, dst, src.numel())
        torch.cuda.synchronize(dev)
        print(json.dumps({"profile_kernels": True, "steps": args.steps}))
        return 0

    print(f"bench: timing {args.bits}-bit gs{args.group_size}", file=sys.stderr, flush=True)
    sec_per_step = time_forward_steps(torch, K, dev, args.bits, args.group_size, args.steps,
                                      args.warmup)
    main_cfg = run_config(torch, K, dev, args.bits, args.group_size, args.steps, args.warmup)
    n = ROWS * COLS
    value = fwd_bytes(n, args.group_size) / sec_per_step / 1e9
    fwd_ms = main_cfg["ms"]["fwd"]
    achieved = fwd_bytes(n, args.group_size) / (fwd_ms * 1e-3) / 1e9
    sweep = []
    if args.sweep:
        for bits in (2, 3, 4, 8):
            for gs in (32, 64, 128):
                print(f"bench: sweep {bits}-bit gs{gs}", file=sys.stderr, flush=True)
                r = run_config(torch, K, dev, bits, gs, max(5, args.steps // 2), 2)
                sweep.append({"bits": bits, "group_size": gs,
                              "gbps": {k: round(x, 1) for k, x in r["gbps"].items()},
                              "ms": {k: round(x, 4) for k, x in r["ms"].items()}})
    cpu = None
    if not args.no_cpu_baseline:
        print("bench: cpu baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.bits, args.group_size)
    line = {
        "metric": "sec per decoder-block tune (7B shape, 2-bit); fake-quant HBM GB/s",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec_per_step * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": (f"fake-quant forward, {ROWS}x{COLS} bf16 weight (7B gate/up shape), "
                         f"{args.bits}-bit asym gs{args.group_size}, v U(-0.5,0.5), alpha=beta=1"),
            "weight_dtype": "bf16",
            "output_dtype": "bf16",
            "bits": args.bits,
            "group_size": args.group_size,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "kernel": "fq_fwd_fast<bf16,bf16,asym,v>",
            "bytes_per_launch": fwd_bytes(n, args.group_size),
            "avg_launch_ms": round(fwd_ms, 5),
        },
        "kernels": {
            "fwd": {"ms": round(fwd_ms, 5), "gbps": round(main_cfg["gbps"]["fwd"], 1)},
            "bwd_update": {"ms": round(main_cfg["ms"]["bwd"], 5),
                           "gbps": round(main_cfg["gbps"]["bwd_update"], 1),
                           "bytes": bwd_bytes(n, args.group_size)},
            "codes": {"ms": round(main_cfg["ms"]["codes"], 5)},
            "pack": {"ms": round(main_cfg["ms"]["pack"], 5),
                     "gbps": round(main_cfg["gbps"]["pack"], 1),
                     "bytes": pack_bytes(n, args.bits)},
        },
        "cpu_baseline": cpu,
    }
    if sweep:
        line["sweep"] = sweep
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
