"""Quantization schemes and tuning configuration.

Restates the contract of the reference's ``mround/schemes.py`` (lines 36-337):
the supported widths, the code ranges, the clipping-coefficient bounds, the
learning-rate rule and the outlier switch. The names, defaults, validation and
error messages follow the reference so that code written against it reads the
same here. The enums derive from ``str`` because this package runs on Python
3.10, which has no ``enum.StrEnum``.

Portions follow MRound (Copyright 2026 The MRound Authors, Apache License 2.0);
see NOTICE.
"""

from __future__ import annotations

import dataclasses
from enum import Enum

from mround_amd.exceptions import SchemeError

__all__ = [
    "DEFAULT_EPS_FP32",
    "DEFAULT_EPS_LOW_PRECISION",
    "LONG_BUDGET_ITERS",
    "LOW_BIT_THRESHOLD",
    "SUPPORTED_BITS",
    "QuantScheme",
    "ScaleInit",
    "Symmetry",
    "TuningConfig",
]

# mround/schemes.py:39 -- widths the packing layout supports.
SUPPORTED_BITS: frozenset[int] = frozenset({2, 3, 4, 5, 6, 7, 8})
# mround/schemes.py:46 -- below this width the outlier rule switches on.
LOW_BIT_THRESHOLD: int = 4
# mround/schemes.py:52 -- from this budget a narrow width starts at twice the rate.
LONG_BUDGET_ITERS: int = 1000
# mround/schemes.py:55-56 -- scale epsilon.
DEFAULT_EPS_FP32: float = 1e-8
DEFAULT_EPS_LOW_PRECISION: float = 1e-5


class Symmetry(str, Enum):
    """Signed (``sym``) or unsigned (``asym``) code range (mround/schemes.py:59-71)."""

    SYMMETRIC = "sym"
    ASYMMETRIC = "asym"

    def __str__(self) -> str:
        return self.value


class ScaleInit(str, Enum):
    """Observed-range or searched initial scale (mround/schemes.py:74-87)."""

    OBSERVED_RANGE = "observed_range"
    SEARCHED = "searched"

    def __str__(self) -> str:
        return self.value


@dataclasses.dataclass(frozen=True)
class QuantScheme:
    """How one layer's weights are quantized (mround/schemes.py:90-211).

    ``group_size`` of ``-1`` means one group per output channel.
    """

    bits: int = 4
    group_size: int = 64
    symmetry: Symmetry = Symmetry.SYMMETRIC
    scale_init: ScaleInit = ScaleInit.OBSERVED_RANGE

    def __post_init__(self) -> None:
        object.__setattr__(self, "symmetry", Symmetry(self.symmetry))
        object.__setattr__(self, "scale_init", ScaleInit(self.scale_init))
        if self.bits not in SUPPORTED_BITS:
            supported = ", ".join(str(b) for b in sorted(SUPPORTED_BITS))
            msg = f"bits must be one of {{{supported}}}, got {self.bits}"
            raise SchemeError(msg)
        if self.group_size != -1 and self.group_size <= 0:
            msg = f"group_size must be positive or -1 (per-channel), got {self.group_size}"
            raise SchemeError(msg)
        if self.scale_init is ScaleInit.SEARCHED and self.symmetry is not Symmetry.SYMMETRIC:
            msg = (
                "the searched scale initialization is defined for symmetric "
                "schemes only; the reference implementation refuses the "
                "asymmetric combination as well"
            )
            raise SchemeError(msg)

    @property
    def is_per_channel(self) -> bool:
        return self.group_size == -1

    @property
    def packs_evenly(self) -> bool:
        return 32 % self.bits == 0

    @property
    def code_range(self) -> tuple[int, int]:
        """Inclusive code range before the storage offset (mround/schemes.py:159-174)."""
        if self.symmetry is Symmetry.SYMMETRIC:
            half = 2 ** (self.bits - 1)
            return (-half, half - 1)
        return (0, 2**self.bits - 1)

    @property
    def coefficient_bounds(self) -> tuple[float, float]:
        """Clip-coefficient bounds (mround/schemes.py:176-194)."""
        if self.scale_init is ScaleInit.SEARCHED:
            return (0.5, 1.5)
        return (0.1, 1.0)

    def groups_per_row(self, in_features: int) -> int:
        """Scales per output channel (mround/schemes.py:196-207)."""
        if self.is_per_channel:
            return 1
        if in_features % self.group_size != 0:
            msg = f"in_features={in_features} is not divisible by group_size={self.group_size}"
            raise SchemeError(msg)
        return in_features // self.group_size

    def with_bits(self, bits: int) -> QuantScheme:
        return dataclasses.replace(self, bits=bits)


@dataclasses.dataclass(frozen=True)
class TuningConfig:
    """How the learned rounding is optimized (mround/schemes.py:214-337)."""

    iters: int = 200
    batch_size: int = 8
    n_samples: int = 128
    seq_len: int = 2048
    lr: float | None = None
    minmax_lr: float | None = None
    gradient_accumulate_steps: int = 1
    suppress_outliers: bool | None = None
    micro_batches: int = 1

    def __post_init__(self) -> None:
        if self.iters <= 0:
            msg = f"iters must be positive, got {self.iters}"
            raise SchemeError(msg)
        if self.batch_size <= 0:
            msg = f"batch_size must be positive, got {self.batch_size}"
            raise SchemeError(msg)
        if self.n_samples < self.batch_size:
            msg = f"n_samples={self.n_samples} is smaller than batch_size={self.batch_size}"
            raise SchemeError(msg)
        if self.minmax_lr is not None:
            msg = (
                "minmax_lr is not implemented: the clipping coefficients share lr in "
                "every tuning loop. Pass None, or set lr for all parameters at once"
            )
            raise SchemeError(msg)
        if self.gradient_accumulate_steps != 1:
            msg = (
                "gradient_accumulate_steps other than 1 is not implemented, got "
                f"{self.gradient_accumulate_steps}; micro_batches splits a step's "
                "batch without changing it"
            )
            raise SchemeError(msg)
        if not 1 <= self.micro_batches <= self.batch_size:
            msg = (
                f"micro_batches must be between 1 and batch_size={self.batch_size}, "
                f"got {self.micro_batches}"
            )
            raise SchemeError(msg)

    def resolved_lr(self, bits: int) -> float:
        """``c / iters``, c = 2 below 4 bits at >= 1000 steps else 1 (mround/schemes.py:307-322)."""
        if self.lr is not None:
            return self.lr
        doubled = bits < LOW_BIT_THRESHOLD and self.iters >= LONG_BUDGET_ITERS
        return (2.0 if doubled else 1.0) / self.iters

    def resolved_minmax_lr(self, bits: int) -> float:
        if self.minmax_lr is not None:
            return self.minmax_lr
        return self.resolved_lr(bits)

    def resolved_suppress_outliers(self, bits: int) -> bool:
        """Outlier rule on below 4 bits unless set (mround/schemes.py:330-337)."""
        if self.suppress_outliers is not None:
            return self.suppress_outliers
        return bits < LOW_BIT_THRESHOLD
