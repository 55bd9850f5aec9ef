"""Mixed-precision bit allocation (mround/planner/allocator.py).

Pick one bit width per layer, minimizing total predicted loss under a budget
on total storage: a multiple-choice knapsack solved exactly by dynamic
programming over exact cumulative costs with Pareto pruning. The search runs
in native code (``mr_allocate_bits`` in ``libmround_hip.so``, host only); this
module keeps the reference's types, validation and messages.

Portions follow MRound (Copyright 2026 The MRound Authors, Apache License 2.0);
see NOTICE.
"""

from __future__ import annotations

import dataclasses
import math

from mround_amd import kernels as K

__all__ = ["Allocation", "LayerOption", "allocate_bits"]


@dataclasses.dataclass(frozen=True, slots=True)
class LayerOption:
    """One candidate bit width for one layer (mround/planner/allocator.py:30-71).

    ``cost_bits`` counts packed codes and the group metadata; ``delta_loss``
    is the predicted loss increase (finite, non-negative); ``elements`` the
    layer's weight count when known (makes ``Allocation.average_bits`` exact).
    """

    bits: int
    cost_bits: int
    delta_loss: float
    elements: int | None = None

    def __post_init__(self) -> None:
        if self.cost_bits < 0:
            raise ValueError(f"cost_bits must be non-negative, got {self.cost_bits}")
        if not math.isfinite(self.delta_loss) or self.delta_loss < 0.0:
            raise ValueError(f"delta_loss must be finite and non-negative, got {self.delta_loss}")
        if self.elements is not None and self.elements <= 0:
            raise ValueError(f"elements must be positive when given, got {self.elements}")


@dataclasses.dataclass(frozen=True, slots=True)
class Allocation:
    """The chosen width per layer, its storage, predicted loss and
    element-weighted average width (mround/planner/allocator.py:74-89)."""

    by_layer: dict[str, int]
    total_cost_bits: int
    predicted_loss: float
    average_bits: float


def _validate(options: dict[str, list[LayerOption]]) -> None:
    if not options:
        raise ValueError("no layers to allocate")
    for name, candidates in options.items():
        if not candidates:
            raise ValueError(f"layer {name!r} has no candidate bit widths")


def _average_bits(options: dict[str, list[LayerOption]], by_layer: dict[str, int]) -> float:
    """Element-weighted mean code width; the element count is inferred from
    the cost when an option does not carry it (mround/planner/allocator.py:244-272)."""
    total_bits = 0.0
    total_elements = 0.0
    for name, bits in by_layer.items():
        option = next(o for o in options[name] if o.bits == bits)
        if option.elements is not None:
            elements = float(option.elements)
            total_bits += bits * elements
        else:
            elements = option.cost_bits / bits if bits else 0.0
            total_bits += option.cost_bits
        total_elements += elements
    return total_bits / total_elements if total_elements else 0.0


def allocate_bits(options: dict[str, list[LayerOption]], *, budget_bits: int,
                  max_states: int | None = None) -> Allocation:
    """Exact optimum of the allocation (approximate only with ``max_states``).

    Raises ``ValueError`` if a layer has no options, ``max_states`` is not
    positive, or the budget cannot be met by every layer's cheapest option.
    """
    _validate(options)
    if max_states is not None and max_states < 1:
        raise ValueError(f"max_states must be positive or None, got {max_states}")
    names = list(options)
    cheapest = sum(min(o.cost_bits for o in options[n]) for n in names)
    if cheapest > budget_bits:
        raise ValueError(f"budget of {budget_bits} bits is infeasible: the cheapest possible "
                         f"allocation costs {cheapest} bits")
    n_options = [len(options[n]) for n in names]
    costs = [o.cost_bits for n in names for o in options[n]]
    losses = [o.delta_loss for n in names for o in options[n]]
    choice, loss, cost = K.allocate_bits(n_options, costs, losses, budget_bits, max_states or 0)
    by_layer = {n: options[n][c].bits for n, c in zip(names, choice)}
    return Allocation(by_layer=by_layer, total_cost_bits=cost, predicted_loss=loss,
                      average_bits=_average_bits(options, by_layer))
