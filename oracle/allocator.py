"""Exact mixed-precision allocation (oracle; test infrastructure only).

A pure-Python restatement of the dynamic programme of
``mround/planner/allocator.py:98-241``: exact cumulative costs, states walked
in ascending cost and options in order, strict improvement at an equal cost,
Pareto pruning (ascending cost, strictly falling loss), optional thinning at
evenly spaced ranks (``round`` = half to even), final pick by (loss, cost).
Returns ``(loss, cost, widths)`` with ``widths`` in layer order.

Pinned by exhaustive search on small instances and the reference's
greedy-defeating instance (tests/test_planner.py).
"""

from __future__ import annotations


def allocate(options, budget_bits, max_states=None):
    """``options``: list over layers of lists of ``(bits, cost_bits, delta_loss)``."""
    frontier = {0: (0.0, ())}
    for layer in options:
        nxt = {}
        for cost, (loss, path) in frontier.items():
            for bits, c, d in layer:
                new_cost = cost + c
                if new_cost > budget_bits:
                    continue
                new_loss = loss + d
                old = nxt.get(new_cost)
                if old is None or new_loss < old[0]:
                    nxt[new_cost] = (new_loss, (*path, bits))
        if not nxt:
            return None
        kept, best = {}, float("inf")
        for cost in sorted(nxt):
            if nxt[cost][0] < best:
                kept[cost] = nxt[cost]
                best = nxt[cost][0]
        if max_states is not None and len(kept) > max_states:
            costs = sorted(kept)
            if max_states == 1:
                chosen = [costs[0]]
            else:
                step = (len(costs) - 1) / (max_states - 1)
                chosen = sorted({costs[round(i * step)] for i in range(max_states)})
            kept = {c: kept[c] for c in chosen}
        frontier = kept
    cost, (loss, path) = min(frontier.items(), key=lambda it: (it[1][0], it[0]))
    return loss, cost, path
