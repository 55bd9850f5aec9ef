"""GPU DeltaLoss accumulation over batches against the float64 oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mround_amd.planner.sensitivity import DeltaLossAccumulator
from mround_amd.schemes import QuantScheme, Symmetry
from oracle import sensitivity as OS
from tests.helpers import dev, weight

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("sym", [False, True])
def test_delta_loss_accumulates_over_batches(sym):
    scheme = QuantScheme(bits=4, group_size=64,
                         symmetry=Symmetry.SYMMETRIC if sym else Symmetry.ASYMMETRIC)
    widths = (2, 3, 4)
    acc = DeltaLossAccumulator(widths, scheme)
    w = weight(384, 512, seed=5, dtype=torch.bfloat16)
    want = np.zeros(len(widths))
    for b in range(3):
        g = torch.randn(384, 512, generator=torch.Generator().manual_seed(10 + b))
        acc.add("mlp.up_proj", w.to(dev()), g.to(dev()))
        for i, bits in enumerate(widths):
            want[i] += OS.delta_terms_f32(w.float().numpy(), g.numpy(), bits=bits, group_size=64,
                                          mode="sym" if sym else "asym").astype(np.float64).sum()
    got = acc.scores()["mlp.up_proj"]
    for i, bits in enumerate(widths):
        assert got[bits] == pytest.approx(want[i], rel=1e-9)
