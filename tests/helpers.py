"""Shared helpers for the parity tests (seeded inputs, tensor conversion)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import quantize as Q


def dev():
    return torch.device("cuda:0")


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach()
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.cpu().numpy()


def weight(rows, cols, *, seed=0, dtype=torch.bfloat16, std=0.02, outliers=0.001):
    """N(0, std) with a fraction of entries scaled by 10 (the microbench recipe)."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(rows, cols, generator=g) * std
    n_out = int(round(outliers * rows * cols))
    if n_out:
        idx = torch.randperm(rows * cols, generator=torch.Generator().manual_seed(seed + 1))[:n_out]
        w.view(-1)[idx] *= 10.0
    return w.to(dtype)


def params(rows, cols, gs, *, seed=2, vrange=0.5, coef_jitter=0.0):
    ng = 1 if gs == -1 else -(-cols // gs)
    g_ = cols if gs == -1 else gs
    gen = torch.Generator().manual_seed(seed)
    v = (torch.rand(rows, ng, g_, generator=gen) * 2 - 1) * vrange
    a = torch.ones(rows, ng, 1)
    b = torch.ones(rows, ng, 1)
    if coef_jitter:
        a = a * (1 - torch.rand(rows, ng, 1, generator=gen) * coef_jitter)
        b = b * (1 - torch.rand(rows, ng, 1, generator=gen) * coef_jitter)
    return v, a, b


def oracle_fq(w_np, v, a, b, bits, gs, mode, init_scale=None):
    return Q.fake_quantize(w_np, None if v is None else v.numpy(), None if a is None else a.numpy(),
                           None if b is None else b.numpy(), bits=bits, group_size=gs, mode=mode,
                           init_scale=init_scale, dtype=np.float32)
