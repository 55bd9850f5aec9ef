"""The C ABI without a GPU: the library loads, exports every declared entry
point, and refuses bad arguments on the host before launching anything."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mround_hip.h"


@pytest.fixture(scope="module")
def lib():
    from mround_amd import kernels as K

    if not K.lib_path().exists():
        from mround_amd import build

        build.build(verbose=False)
    return K.lib()


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(mr_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(lib):
    names = declared_symbols()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"


def test_abi_version(lib):
    assert lib.mr_abi_version() == 1


@pytest.mark.parametrize(("cols", "bits", "words"), [(64, 2, 4), (64, 4, 8), (64, 8, 16), (64, 3, 6),
                                                     (4096, 5, 640), (16, 2, 1)])
def test_packed_width(lib, cols, bits, words):
    assert lib.mr_packed_width(cols, bits) == words


def test_packed_width_errors(lib):
    assert lib.mr_packed_width(48, 3) == -22
    assert b"multiple of 32" in lib.mr_last_error()
    assert lib.mr_packed_width(64, 9) == -22
    assert lib.mr_packed_width(6, 4) == -22


def test_host_validation_refuses_before_launch(lib):
    P = ctypes.c_void_p
    # null weight
    rc = lib.mr_fq_forward(None, 1, None, None, None, None, 4, 64, 64, 4, 0, 1e-8, P(16), 0,
                           None, None, None, None)
    assert rc == -22 and b"weight pointer is null" in lib.mr_last_error()
    # bad bits
    rc = lib.mr_fq_forward(P(16), 1, None, None, None, None, 4, 64, 64, 9, 0, 1e-8, P(16), 0,
                           None, None, None, None)
    assert rc == -22 and b"bits" in lib.mr_last_error()
    # searched mode without init_scale
    rc = lib.mr_fq_forward(P(16), 1, None, None, None, None, 4, 64, 64, 4, 2, 1e-8, P(16), 0,
                           None, None, None, None)
    assert rc == -22 and b"init_scale" in lib.mr_last_error()
    # v without alpha
    rc = lib.mr_fq_forward(P(16), 1, P(16), None, None, None, 4, 64, 64, 4, 0, 1e-8, P(16), 0,
                           None, None, None, None)
    assert rc == -22
    # backward without params
    rc = lib.mr_fq_backward_signsgd(P(16), 1, None, None, None, None, P(16), 0, 4, 64, 64, 2, 0,
                                    1e-8, 1, 0.005, 0.1, 1.0, 0.5, None, None, None, None)
    assert rc == -22
    # loss with an out-of-range rank
    rc = lib.mr_loss_outlier(P(16), P(16), 100, 0, 100, None, None, P(16), None, P(16), None)
    assert rc == -22 and b"rank" in lib.mr_last_error()
    # DeltaLoss with too many widths
    arr = (ctypes.c_int * 9)(*range(9))
    rc = lib.mr_delta_loss(P(16), 1, P(16), 4, 64, 64, arr, 9, 0, 1e-8, P(16), P(16), None)
    assert rc == -22
    # GEMM outputs are written in 16-byte row pieces: C, resid and the SwiGLU
    # outputs must be 16-byte aligned with 16-byte rows
    MR_F32, MR_BF16 = 0, 1
    rc = lib.mr_gemm(0, 64, 64, 64, P(256), 64, P(256), 64, P(264), MR_F32, 64, None, None, 0, None)
    assert rc == -22 and b"16-byte" in lib.mr_last_error()
    rc = lib.mr_gemm(0, 64, 64, 64, P(256), 64, P(256), 64, P(256), MR_BF16, 68, None, None, 0, None)
    assert rc == -22 and b"16-byte" in lib.mr_last_error()
    rc = lib.mr_gemm(0, 64, 64, 64, P(256), 64, P(256), 64, P(256), MR_F32, 64, None, P(256), 66, None)
    assert rc == -22 and b"16-byte" in lib.mr_last_error()
    rc = lib.mr_gemm_swiglu(64, 64, 64, P(256), 64, P(256), 64, P(256), 68, None, 0, None)
    assert rc == -22 and b"16-byte" in lib.mr_last_error()


def test_workspace_sizes(lib):
    assert lib.mr_loss_workspace_bytes(1 << 26) > 0
    assert lib.mr_delta_loss_workspace_bytes(3584, 18944, 3) > 0
