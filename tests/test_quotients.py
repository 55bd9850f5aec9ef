"""The fast kernels' correctly rounded quotients, checked exhaustively.

The fake-quant kernels divide each bfloat16 weight by its group's float32
scale with a reciprocal and one fused correction, and divide by maxq the same
way (``mround_amd/csrc/mr_quant.hip``: ``quotients``, ``div_maxq``); the
reference divides in float32 (``mround/reference/quantize.py:156-246``). Both
forms must give the IEEE quotient bit for bit. ``quotient_check.c`` runs the
same sequence on the host's fused multiply-add over every significand pair
the identity depends on (2^30 weight/scale pairs, every float32 numerator for
each maxq) plus signed zeros and negative scales. A copy built without the
correction step must fail, so the check can tell.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).with_name("quotient_check.c")


def _build(tmp_path: Path, *defines: str) -> Path:
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = tmp_path / ("qc" + "".join(d.lower() for d in defines))
    flags = ["-O2", "-ffp-contract=off"]
    probe = subprocess.run([cc, "-march=native", "-E", "-x", "c", "/dev/null"], capture_output=True)
    if probe.returncode == 0:
        flags.append("-march=native")
    cmd = [cc, *flags, *(f"-D{d}" for d in defines), str(SRC), "-o", str(exe), "-lm"]
    subprocess.run(cmd, check=True, capture_output=True)
    return exe


def test_fast_quotients_equal_ieee_division_exhaustively(tmp_path):
    out = subprocess.run([str(_build(tmp_path))], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout[-2000:]
    assert out.stdout.startswith("ok "), out.stdout
    assert int(out.stdout.split()[1]) == (1 << 30) + 8 * 9 * 2 + 16 * 2 * (1 << 23)


def test_the_check_catches_a_dropped_correction(tmp_path):
    out = subprocess.run([str(_build(tmp_path, "DROP_CORRECTION"))], capture_output=True, text=True,
                         timeout=600)
    assert out.returncode == 1 and "mismatches" in out.stdout, out.stdout[-2000:]


def _fast_div(d: int) -> tuple[int, int]:
    """``FastDiv::make`` of ``mround_amd/csrc/mr_quant.hip``: (m, p) with
    floor(n * m / 2^p) == n // d for 0 <= n < 2^31."""
    ceil_log2 = 0
    while (1 << ceil_log2) < d:
        ceil_log2 += 1
    p = 31 + ceil_log2
    return ((1 << p) + d - 1) // d, p


def test_row_placement_divider_constants():
    """The fused step finds a chunk's row and its placement block by multiply
    and shift; the constants must fit 32 bits and divide exactly over the
    31-bit range, checked against integer division at the edges (multiples
    of d and their neighbours, 2^31 - 1) for small, power-of-two-adjacent and
    random divisors."""
    import random

    rnd = random.Random(0)
    divisors = list(range(1, 1025)) + [(1 << k) + o for k in range(10, 31) for o in (-1, 0, 1)]
    divisors += [(1 << 31) - 1] + [rnd.randrange(1, 1 << 31) for _ in range(500)]
    for d in divisors:
        m, p = _fast_div(d)
        assert m < 1 << 32, d
        top = (1 << 31) - 1
        ns = {0, 1, d - 1, d, d + 1, top, top - 1, (top // d) * d, (top // d) * d - 1}
        ns |= {rnd.randrange(0, 1 << 31) for _ in range(50)}
        for n in ns:
            if 0 <= n <= top:
                assert (n * m) >> p == n // d, (n, d)
