"""Error types, mirroring the reference hierarchy (mround/exceptions.py:24-78).

Every refusal the package makes deliberately is an :class:`MRoundError`.
:class:`SchemeError` is also a :class:`ValueError`, as in the reference, so a
caller checking argument values catches it the ordinary way.

:class:`KernelError` is this package's addition: the HIP library reported a
failure (a bad argument caught by the C ABI, or a HIP runtime error). It is
raised instead of falling back to any other implementation.

Portions follow MRound (Copyright 2026 The MRound Authors, Apache License 2.0);
see NOTICE.
"""

from __future__ import annotations

__all__ = [
    "ArchitectureError",
    "CalibrationError",
    "ExportError",
    "KernelError",
    "KernelUnavailableError",
    "MRoundError",
    "MemoryBudgetError",
    "PlatformError",
    "SchemeError",
    "UnsupportedSchemeError",
]


class MRoundError(Exception):
    """Base class for every error raised deliberately (mround/exceptions.py:24)."""


class PlatformError(MRoundError):
    """The host cannot run this operation (no ROCm GPU, wrong architecture)."""


class SchemeError(MRoundError, ValueError):
    """A quantization scheme is malformed or inapplicable (mround/exceptions.py:37)."""


class UnsupportedSchemeError(SchemeError):
    """A target format cannot represent the scheme (mround/exceptions.py:47)."""


class CalibrationError(MRoundError):
    """Calibration data is missing, malformed, or inconsistent (mround/exceptions.py:55)."""


class ArchitectureError(MRoundError):
    """The model's structure could not be interpreted (mround/exceptions.py:59)."""


class ExportError(MRoundError):
    """A checkpoint could not be written (mround/exceptions.py:67)."""


class MemoryBudgetError(MRoundError):
    """A run is predicted to need more memory than it may use (mround/exceptions.py:71)."""


class KernelError(MRoundError):
    """The HIP library refused a call or the HIP runtime reported an error."""


class KernelUnavailableError(PlatformError):
    """The compiled HIP library is missing or cannot be loaded.

    Raised loudly: no operation on the tuning path has a CPU substitute.
    """
