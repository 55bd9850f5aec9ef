"""Mixed-precision planner: the native exact allocator against exhaustive
search, the reference's greedy-defeating instance, a Python restatement of the
reference's dynamic programme (tie order and thinning), and the storage-cost
known answers (tests/unit/test_allocator.py, tests/unit/test_sensitivity.py)."""

from __future__ import annotations

import itertools
import random

import pytest

from mround_amd.planner.allocator import LayerOption, allocate_bits
from mround_amd.planner.sensitivity import (
    groups_per_row, mixed_budget_bits, score_layer_options, storage_bits)
from mround_amd.schemes import QuantScheme
from oracle import allocator as OA


def _instance(seed, n_layers, *, ties=False):
    rng = random.Random(seed)
    opts = {}
    for i in range(n_layers):
        widths = sorted(rng.sample([2, 3, 4, 5, 6, 8], rng.randint(2, 4)))
        size = rng.randint(4, 40)
        cands = []
        for b in widths:
            loss = float(rng.randint(0, 6)) if ties else rng.uniform(0.0, 10.0) / b
            cands.append(LayerOption(bits=b, cost_bits=size * b + rng.randint(0, 3), delta_loss=loss))
        opts[f"layer{i}"] = cands
    return opts


def _brute(options, budget):
    names = list(options)
    best = None
    for combo in itertools.product(*(options[n] for n in names)):
        cost = sum(o.cost_bits for o in combo)
        if cost <= budget:
            loss = sum(o.delta_loss for o in combo)
            if best is None or loss < best:
                best = loss
    return best


def _as_lists(options):
    return [[(o.bits, o.cost_bits, o.delta_loss) for o in v] for v in options.values()]


@pytest.mark.parametrize("seed", range(24))
def test_matches_exhaustive_search(seed):
    options = _instance(seed, n_layers=2 + seed % 5)
    lo = sum(min(o.cost_bits for o in v) for v in options.values())
    hi = sum(max(o.cost_bits for o in v) for v in options.values())
    budget = (lo + hi) // 2
    res = allocate_bits(options, budget_bits=budget)
    assert res.predicted_loss == pytest.approx(_brute(options, budget), rel=1e-12)
    assert res.total_cost_bits <= budget
    chosen = {n: next(o for o in options[n] if o.bits == b) for n, b in res.by_layer.items()}
    assert res.total_cost_bits == sum(o.cost_bits for o in chosen.values())


@pytest.mark.parametrize("seed", range(40))
@pytest.mark.parametrize("max_states", [None, 1, 2, 5])
def test_same_choice_as_the_reference_programme(seed, max_states):
    """Tie order and thinning: identical widths, loss and cost, including
    instances built with many exact ties."""
    options = _instance(seed, n_layers=3 + seed % 9, ties=seed % 2 == 0)
    lo = sum(min(o.cost_bits for o in v) for v in options.values())
    budget = int(lo * 1.4)
    want = OA.allocate(_as_lists(options), budget, max_states)
    if want is None:
        with pytest.raises(ValueError):
            allocate_bits(options, budget_bits=budget, max_states=max_states)
        return
    res = allocate_bits(options, budget_bits=budget, max_states=max_states)
    assert res.predicted_loss == want[0]
    assert res.total_cost_bits == want[1]
    assert tuple(res.by_layer.values()) == want[2]


def test_beats_greedy_on_the_reference_instance():
    # greedy: a=2 (10.0) + b=8 (8.5) = 18.5 at cost 11; exact: a=4 (3.0) + b=2 (10.0) = 13.0 at 15
    options = {"a": [LayerOption(2, 5, 10.0), LayerOption(4, 10, 3.0)],
               "b": [LayerOption(2, 5, 10.0), LayerOption(8, 6, 8.5)]}
    res = allocate_bits(options, budget_bits=15)
    assert res.predicted_loss == 13.0 and res.by_layer == {"a": 4, "b": 2}
    assert res.total_cost_bits == 15


def test_budget_edges_and_errors():
    options = _instance(7, 4)
    lo = sum(min(o.cost_bits for o in v) for v in options.values())
    hi = sum(max(o.cost_bits for o in v) for v in options.values())
    assert allocate_bits(options, budget_bits=lo).total_cost_bits == lo
    best = allocate_bits(options, budget_bits=hi)
    for n, b in best.by_layer.items():
        assert min(o.delta_loss for o in options[n]) == next(o.delta_loss for o in options[n] if o.bits == b)
    with pytest.raises(ValueError, match="infeasible"):
        allocate_bits(options, budget_bits=lo - 1)
    with pytest.raises(ValueError, match="no layers"):
        allocate_bits({}, budget_bits=10)
    with pytest.raises(ValueError, match="no candidate"):
        allocate_bits({"a": []}, budget_bits=10)
    with pytest.raises(ValueError, match="max_states"):
        allocate_bits(options, budget_bits=hi, max_states=0)
    with pytest.raises(ValueError, match="non-negative"):
        LayerOption(2, 5, -1.0)
    losses = [allocate_bits(options, budget_bits=int(lo * f)).predicted_loss for f in (1.0, 1.2, 1.5, 2.0)]
    assert losses == sorted(losses, reverse=True)


def test_large_instance_is_fast_and_exact_against_the_programme():
    """60 layers x 3 widths at realistic cost spreads, native against the programme."""
    import time
    rng = random.Random(3)
    options = {}
    for i in range(60):
        rows, cols = rng.choice([(2048, 2048), (256, 2048), (11008, 2048), (2048, 11008)])
        options[f"l{i}"] = [LayerOption(b, storage_bits((rows, cols), b, 64) // 4096,
                                        rng.uniform(0, 1) / b ** 2) for b in (2, 3, 4)]
    budget = sum(o[1].cost_bits for o in options.values())
    t0 = time.perf_counter()
    res = allocate_bits(options, budget_bits=budget)
    dt = time.perf_counter() - t0
    want = OA.allocate(_as_lists(options), budget)
    assert res.predicted_loss == want[0] and tuple(res.by_layer.values()) == want[2]
    assert dt < 10.0


def test_storage_known_answers():
    assert storage_bits((8, 128), 4, 64) == 8 * 128 * 4 + 2 * (8 * 2) * 16
    assert storage_bits((8, 128), 4, 64) / (8 * 128) == 4.5
    assert storage_bits((4, 64), 2, 64) / (4 * 64) == 2.5
    assert storage_bits((4, 64), 4, -1) == 4 * 64 * 4 + 2 * 4 * 16
    assert groups_per_row(64, -1) == 1 and groups_per_row(64, 32) == 2
    with pytest.raises(ValueError, match="stays dense"):
        storage_bits((4, 100), 4, 64)
    with pytest.raises(ValueError, match="positive"):
        storage_bits((0, 64), 4, 64)
    shapes = {"a": (4, 64), "b": (8, 128)}
    for width in (2, 3, 4, 8):
        assert mixed_budget_bits(shapes, float(width), 64) == sum(
            storage_bits(s, width, 64) for s in shapes.values())
    assert mixed_budget_bits(shapes, 2.0, 64) < mixed_budget_bits(shapes, 2.5, 64) < \
        mixed_budget_bits(shapes, 3.0, 64)
    with pytest.raises(ValueError, match="no layers"):
        mixed_budget_bits({}, 3.0, 64)


def test_score_layer_options_feeds_the_allocator():
    shapes = {"a": (4, 64), "b": (8, 128)}
    scheme = QuantScheme(bits=4, group_size=64)
    opts = score_layer_options({n: {2: 1.0, 4: 0.5} for n in shapes}, shapes, scheme)
    budget = mixed_budget_bits(shapes, 4.0, 64)
    alloc = allocate_bits(opts, budget_bits=budget)
    assert alloc.by_layer == {"a": 4, "b": 4} and alloc.average_bits == 4.0
    with pytest.raises(ValueError, match="same layers"):
        score_layer_options({"a": {2: 1.0}}, shapes, scheme)
    with pytest.raises(ValueError, match="same scoring passes"):
        score_layer_options({"a": {2: 1.0}, "b": {4: 1.0}}, shapes, scheme)
    with pytest.raises(ValueError, match="invalid score"):
        score_layer_options({"a": {2: float("nan")}, "b": {2: 1.0}}, shapes, scheme)
