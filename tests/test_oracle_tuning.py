"""The oracle's single-layer loop against the reference's own tests of its loop
(``tests/unit/test_reference_tuning.py``), restated on the same synthetic
layers: correlated activations, group size 32, 200 steps."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import quantize as OQ
from oracle import tuning as OT


def synthetic_layer(seed: int, out_features: int = 16, in_features: int = 64, n_samples: int = 128):
    """A weight and activations correlated across features (test_reference_tuning.py:25-40)."""
    gen = np.random.default_rng(seed)
    weight = gen.normal(scale=0.05, size=(out_features, in_features))
    basis = gen.normal(size=(in_features, in_features))
    covariance = basis @ basis.T / in_features
    activations = gen.multivariate_normal(np.zeros(in_features), covariance, size=n_samples)
    return weight, activations


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_improvement_is_material(bits):
    w, x = synthetic_layer(100 + bits)
    r = OT.tune_layer(w, x, bits=bits, group_size=32, mode="sym", iters=200)
    assert r.final_loss < r.initial_loss and r.improvement > 0.05, r.improvement


def test_the_advantage_grows_as_bits_get_scarcer():
    w, x = synthetic_layer(7)
    imp = {b: OT.tune_layer(w, x, bits=b, group_size=32, mode="sym", iters=200).improvement for b in (2, 4)}
    assert imp[2] > imp[4]


@pytest.mark.parametrize("mode", ["sym", "asym"])
def test_initial_loss_is_round_to_nearest(mode):
    w, x = synthetic_layer(11)
    r = OT.tune_layer(w, x, bits=3, group_size=32, mode=mode, iters=20)
    rtn = OQ.fake_quantize(w, None, None, None, bits=3, group_size=32, mode=mode, dtype=np.float64)[0]
    loss, _ = OT.layer_loss(x, rtn, w, suppress=True)
    assert r.initial_loss == pytest.approx(loss, rel=1e-12)
    assert r.losses[0] == r.initial_loss


def test_best_state_is_tracked():
    w, x = synthetic_layer(5)
    r = OT.tune_layer(w, x, bits=2, group_size=32, mode="sym", iters=200)
    assert r.final_loss == min(r.losses) and r.losses[r.best_step] == r.final_loss
    qdq = OQ.fake_quantize(w, r.v, r.alpha, r.beta, bits=2, group_size=32, mode="sym", dtype=np.float64)[0]
    assert np.array_equal(qdq, r.qdq)
    loss, _ = OT.layer_loss(x, qdq, w, suppress=True)
    assert loss == pytest.approx(r.final_loss, rel=1e-12)


def test_bounds_and_determinism():
    w, x = synthetic_layer(9)
    a = OT.tune_layer(w, x, bits=2, group_size=32, mode="asym", iters=100)
    b = OT.tune_layer(w, x, bits=2, group_size=32, mode="asym", iters=100)
    assert a.losses == b.losses and np.array_equal(a.v, b.v)
    assert np.abs(a.v).max() <= 0.5
    assert 0.1 <= a.alpha.min() and a.alpha.max() <= 1.0 and 0.1 <= a.beta.min() and a.beta.max() <= 1.0


def test_mismatched_width_is_rejected():
    w, x = synthetic_layer(1)
    with pytest.raises(ValueError, match="features"):
        OT.tune_layer(w, x[:, :32], bits=2, group_size=32, mode="sym", iters=2)
