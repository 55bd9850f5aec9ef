"""The single-layer loop on the GPU (``mround_amd.core.tuning``) against the
oracle's (``oracle/tuning.py``, itself pinned by the reference's tests of
its loop) on the reference's synthetic layers.

With the oracle in float32 the fake quantization is the same function bit for
bit, so the round-to-nearest error agrees to the order of summation (1e-5);
the step losses then follow the oracle's (within 1e-4 over all 200 steps,
the same best step: the gradients' signs agree throughout on these layers).
The properties the reference tests hold for any implementation: more than 5 %
better than round to nearest at 2-4 bits, the best measured state returned
with its reconstruction, parameters inside their bounds, determinism.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from mround_amd.core.quantizer import fake_quantize
from mround_amd.core.tuning import round_to_nearest, tune_layer
from mround_amd.schemes import QuantScheme, Symmetry, TuningConfig
from oracle import tuning as OT
from tests.helpers import dev

pytestmark = pytest.mark.gpu


def synthetic_layer(seed: int, out_features: int = 16, in_features: int = 64, n_samples: int = 128):
    """test_reference_tuning.py:25-40."""
    gen = np.random.default_rng(seed)
    weight = gen.normal(scale=0.05, size=(out_features, in_features))
    basis = gen.normal(size=(in_features, in_features))
    covariance = basis @ basis.T / in_features
    activations = gen.multivariate_normal(np.zeros(in_features), covariance, size=n_samples)
    return weight, activations


def _dev(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(dev())


@pytest.mark.parametrize(("bits", "symmetry"), [(2, Symmetry.SYMMETRIC), (3, Symmetry.ASYMMETRIC),
                                                (4, Symmetry.SYMMETRIC), (2, Symmetry.ASYMMETRIC)])
def test_follows_the_oracle(bits, symmetry):
    print("case layer tune", bits, symmetry, flush=True, file=sys.stderr)
    w, x = synthetic_layer(100 + bits)
    w32, x32 = w.astype(np.float32), x.astype(np.float32)
    mode = "sym" if symmetry is Symmetry.SYMMETRIC else "asym"
    scheme = QuantScheme(bits=bits, group_size=32, symmetry=symmetry)
    got = tune_layer(_dev(w32), _dev(x32), scheme, TuningConfig(iters=200))
    ref = OT.tune_layer(w32, x32, bits=bits, group_size=32, mode=mode, iters=200, dtype=np.float32)
    print("  gpu", got.initial_loss, got.final_loss, got.best_step, file=sys.stderr)
    print("  cpu", ref.initial_loss, ref.final_loss, ref.best_step, file=sys.stderr)
    assert got.initial_loss == pytest.approx(ref.initial_loss, rel=1e-5)
    # measured: every one of the 200 step losses within 2e-7 of the oracle's,
    # the same best step
    for a, b in zip(got.losses, ref.losses):
        assert a == pytest.approx(b, rel=1e-4)
    assert got.best_step == ref.best_step
    assert got.improvement > 0.05 and ref.improvement > 0.05
    # the returned reconstruction is the best parameters' fake quantization
    again = fake_quantize(_dev(w32), got.params, scheme)
    assert torch.equal(again, got.qdq.to(again.dtype))
    assert got.losses[got.best_step] == got.final_loss == min(got.losses)


def test_initial_loss_is_round_to_nearest():
    w, x = synthetic_layer(11)
    wd, xd = _dev(w), _dev(x)
    scheme = QuantScheme(bits=3, group_size=32)
    r = tune_layer(wd, xd, scheme, TuningConfig(iters=10))
    rtn = round_to_nearest(wd, scheme).float()
    residual = (xd @ (rtn - wd).T).double()
    # 3 bits: the outlier rule; compare against the oracle's loss of the same residual
    loss, _ = OT.layer_loss(x.astype(np.float64), rtn.double().cpu().numpy(), w, suppress=True)
    assert r.initial_loss == pytest.approx(loss, rel=1e-4)
    assert r.losses[0] == r.initial_loss and residual.abs().max() > 0


def test_bounds_determinism_and_a_large_layer():
    w, x = synthetic_layer(9)
    scheme = QuantScheme(bits=2, group_size=32, symmetry=Symmetry.ASYMMETRIC)
    a = tune_layer(_dev(w), _dev(x), scheme, TuningConfig(iters=100))
    b = tune_layer(_dev(w), _dev(x), scheme, TuningConfig(iters=100))
    assert a.losses == b.losses and torch.equal(a.params["v"], b.params["v"])
    assert float(a.params["v"].abs().max()) <= 0.5
    lo, hi = scheme.coefficient_bounds
    for name in ("alpha", "beta"):
        assert lo <= float(a.params[name].min()) and float(a.params[name].max()) <= hi
    # a 4096 x 4096 layer with 512 inputs, bf16 weight: learns
    g = torch.Generator(device=dev()).manual_seed(0)
    wl = (torch.randn(4096, 4096, generator=g, device=dev()) * 0.02).to(torch.bfloat16)
    xl = torch.randn(512, 4096, generator=g, device=dev())
    r = tune_layer(wl, xl, QuantScheme(bits=2, group_size=64, symmetry=Symmetry.ASYMMETRIC), TuningConfig(iters=50))
    print("  4096 x 4096:", r.initial_loss, r.final_loss, file=sys.stderr)
    assert r.final_loss < r.initial_loss


def test_mismatched_width_is_rejected():
    w, x = synthetic_layer(1)
    with pytest.raises(ValueError, match="features"):
        tune_layer(_dev(w), _dev(x[:, :32]), QuantScheme(bits=2, group_size=32), TuningConfig(iters=2))
