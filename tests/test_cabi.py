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
    assert lib.mr_abi_version() == 2


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
    # a gradient written over the residual's inputs, which the select reads again
    for grad in (P(1 << 20), P((2 << 20) + 384)):
        rc = lib.mr_loss_outlier(P(1 << 20), P(2 << 20), 100, 1, 100, None, None, P(3 << 20), grad, P(4 << 20),
                                 None)
        assert rc == -22 and b"overlap" in lib.mr_last_error()
    # DeltaLoss with too many widths
    arr = (ctypes.c_int * 9)(*range(9))
    rc = lib.mr_delta_loss(P(16), 1, P(16), 4, 64, 64, arr, 9, 0, 1e-8, P(16), P(16), None)
    assert rc == -22
    # GEMM outputs are written in 16-byte row pieces: C, resid and the SwiGLU
    # outputs must be 16-byte aligned with 16-byte rows
    MR_F32, MR_BF16 = 0, 1
    rc = lib.mr_gemm(0, 64, 64, 64, P(256), 64, P(256), 64, P(264), MR_F32, 64, None, None, 0, None, 0,
                     None)
    assert rc == -22 and b"16-byte" in lib.mr_last_error()
    rc = lib.mr_gemm(0, 64, 64, 64, P(256), 64, P(256), 64, P(256), MR_BF16, 68, None, None, 0, None, 0,
                     None)
    assert rc == -22 and b"16-byte" in lib.mr_last_error()
    rc = lib.mr_gemm(0, 64, 64, 64, P(256), 64, P(256), 64, P(256), MR_F32, 64, None, P(256), 66, None, 0,
                     None)
    assert rc == -22 and b"16-byte" in lib.mr_last_error()
    rc = lib.mr_gemm_swiglu(64, 64, 64, P(256), 64, P(256), 64, P(256), 68, None, 0, None, 0, None)
    assert rc == -22 and b"16-byte" in lib.mr_last_error()
    # the SwiGLU backward reads gu and writes dgu as 16-byte pieces
    for gu, ldgu, dgu in ((P(264), 128, P(256)), (P(256), 128, P(264)), (P(256), 132, P(256))):
        rc = lib.mr_gemm_swiglu_bwd(64, 64, 64, P(256), 64, P(256), 64, gu, ldgu, dgu, ldgu, None, 0, None)
        assert rc == -22 and b"16-byte" in lib.mr_last_error()
    # outputs and the k-split workspace against the operands (64 x 64 x 64, fp32 C: 16 KB)
    A, B_, C = P(1 << 20), P(2 << 20), P(3 << 20)
    for c, ws, resid in ((A, None, None), (P((2 << 20) + 8000), None, None), (C, P((3 << 20) + 1024), None),
                         (C, A, None), (C, None, P((3 << 20) + 256))):
        rc = lib.mr_gemm(0, 64, 64, 64, A, 64, B_, 64, c, MR_F32, 64, None, resid, 64, ws, 4096 if ws else 0,
                         None)
        assert rc == -22 and b"overlap" in lib.mr_last_error(), (c, ws, resid)
    rc = lib.mr_gemm_swiglu(64, 64, 64, A, 64, B_, 64, P(3 << 20), 64, P((3 << 20) + 4096), 128, None, 0, None)
    assert rc == -22 and b"overlap" in lib.mr_last_error()
    rc = lib.mr_gemm_swiglu_bwd(64, 64, 64, A, 64, B_, 64, P(3 << 20), 128, P((3 << 20) + 512), 128, None, 0,
                                None)
    assert rc == -22 and b"overlap" in lib.mr_last_error()
    # a misaligned k-split workspace
    rc = lib.mr_gemm(0, 64, 64, 64, A, 64, B_, 64, C, MR_F32, 64, None, None, 0, P((4 << 20) + 8), 1024, None)
    assert rc == -22 and b"workspace must be 16-byte aligned" in lib.mr_last_error()


def test_split_entry_points_refuse_bad_arguments(lib):
    P = ctypes.c_void_p
    rc = lib.mr_split_bf16(P(256), 64, 4, 64, 2, P(256), 192, None, 0, None)
    assert rc == -22 and b"order" in lib.mr_last_error()
    rc = lib.mr_split_bf16(P(256), 64, 4, 64, 0, P(256), 128, None, 0, None)  # ld_dst < 3 cols
    assert rc == -22 and b"ld_dst" in lib.mr_last_error()
    rc = lib.mr_split_bf16(P(264), 64, 4, 64, 0, P(256), 192, None, 0, None)
    assert rc == -22 and b"aligned" in lib.mr_last_error()
    rc = lib.mr_split_bf16(None, 64, 4, 64, 0, P(256), 192, None, 0, None)
    assert rc == -22 and b"null" in lib.mr_last_error()
    rc = lib.mr_rmsnorm_fwd_split(P(256), P(256), 4, 66, 1e-6, P(256), None, None, None)
    assert rc == -22 and b"multiple of 4" in lib.mr_last_error()
    rc = lib.mr_swiglu_split(P(256), 4, 48, P(256), P(256), P(256), None)
    assert rc == -22 and b"multiple of 32" in lib.mr_last_error()
    rc = lib.mr_swiglu_split(P(256), 4, 64, P(256), None, P(256), None)
    assert rc == -22 and b"null" in lib.mr_last_error()
    # nothing to do is not an error
    assert lib.mr_split_bf16(None, 0, 0, 0, 0, None, 0, None, 0, None) == 0


def test_workspace_sizes(lib):
    assert lib.mr_loss_workspace_bytes(1 << 26) > 0
    assert lib.mr_delta_loss_workspace_bytes(3584, 18944, 3) > 0


# (M, N, K) of the Qwen2.5-7B block's products at 8 x 2048 tokens whose
# 256 x 256 tiles leave a partial last wave with a long K: the remainder is
# cut along K into partial tiles of 256 KiB.
@pytest.mark.parametrize(("M", "N", "K"), [(16384, 3584, 18944), (16384, 3584, 37888),
                                           (3584, 18944, 16384), (37888, 3584, 16384)])
def test_gemm_workspace_split_shapes(lib, M, N, K):
    tiles = ((M + 255) // 256) * ((N + 255) // 256)
    nbytes = lib.mr_gemm_workspace_bytes(M, N, K)
    tile = 256 * 256 * 4
    assert 0 < nbytes <= 128 << 20 and nbytes % tile == 0
    assert (nbytes // tile) % (tiles % 256) == 0  # whole splits of every remainder tile


@pytest.mark.parametrize(("M", "N", "K"), [(16384, 4608, 3584), (16384, 37888, 3584), (16384, 3584, 3584),
                                           (16384, 4096, 18944), (64, 64, 64)])
def test_gemm_workspace_unsplit_shapes(lib, M, N, K):
    # a short K (under 96 steps of 64) or whole waves of tiles: no partials
    assert lib.mr_gemm_workspace_bytes(M, N, K) == 0


def test_attention_workspace_follows_the_head_split(lib):
    T = 8 * 2048
    # 7B: 4 kv heads x 8 x 16 key blocks = 512 blocks, no split
    assert lib.mr_attn_bwd_workspace_bytes(8, 2048, 28, 4, 128, 0) == 0
    # 0.5B: 2 kv heads (256 blocks) split the 7 query heads of a group in two
    assert lib.mr_attn_bwd_workspace_bytes(8, 2048, 14, 2, 64, 0) == 2 * T * 2 * 2 * 64 * 4
    # a forced split sizes its partials; 1 needs none
    assert lib.mr_attn_bwd_workspace_bytes(8, 2048, 28, 4, 128, 7) == 7 * T * 2 * 4 * 128 * 4
    assert lib.mr_attn_bwd_workspace_bytes(8, 2048, 28, 4, 128, 1) == 0


def test_attention_backward_refuses_a_bad_split(lib):
    P = ctypes.c_void_p
    # (distinct, non-overlapping buffers: qkv, out, dout, lse, dsum, dqkv)
    args = (P(1 << 30), 2304, P(2 << 30), P(3 << 30), 1792, P(4 << 30), P(5 << 30), 1, 256, 14, 2, 128, 0.1,
            P(6 << 30))
    # more blocks per kv head than the group has query heads
    assert lib.mr_attn_bwd(*args, 8, None, 0, None) == -22
    assert b"hsplit" in lib.mr_last_error()
    # a forced split without room for its partials
    assert lib.mr_attn_bwd(*args, 2, P(256), 1024, None) == -22
    assert b"workspace" in lib.mr_last_error()


def test_attention_refuses_outputs_that_overlap_inputs(lib):
    P = ctypes.c_void_p
    T, ld, ldo = 256, 2304, 1792  # one sequence of 256, 14 / 2 heads of 128
    qkv, out, dout, lse, dsum, dqkv = (P(k << 30) for k in range(1, 7))
    last_row = (T - 1) * ld * 2  # byte offset of qkv's last row

    def bwd(**kw):
        a = dict(qkv=qkv, out=out, dout=dout, dsum=dsum, dqkv=dqkv)
        a.update(kw)
        return lib.mr_attn_bwd(a["qkv"], ld, a["out"], a["dout"], ldo, lse, a["dsum"], 1, T, 14, 2, 128, 0.1,
                               a["dqkv"], 1, None, 0, None)

    for kw in (dict(dqkv=qkv), dict(dqkv=P((1 << 30) + last_row)), dict(dqkv=out), dict(dqkv=dout),
               dict(dsum=qkv), dict(dsum=out), dict(dsum=dout), dict(dsum=dqkv)):
        assert bwd(**kw) == -22, kw
        assert b"overlap" in lib.mr_last_error()
    # the forward's output against qkv: inside it, and starting in its last 16 bytes
    assert lib.mr_attn_fwd(qkv, ld, 1, T, 14, 2, 128, 0.1, P((1 << 30) + 4096), ldo, lse, None) == -22
    assert b"overlap" in lib.mr_last_error()
    end = (1 << 30) + last_row + (14 + 4) * 128 * 2
    assert lib.mr_attn_fwd(qkv, ld, 1, T, 14, 2, 128, 0.1, P(end - 16), ldo, lse, None) == -22
    # the split forward: its two outputs against the hi and lo halves and each other
    hi, lo, o, osp = P(1 << 30), P(2 << 30), P(3 << 30), P(4 << 30)
    for a in ((hi, lo, hi, osp), (hi, lo, o, lo), (hi, lo, o, o)):
        assert lib.mr_attn_fwd_split(a[0], a[1], ld, 1, T, 14, 2, 128, 0.1, a[2], ldo, a[3], 3 * 14 * 128,
                                     lse, None) == -22, a
        assert b"overlap" in lib.mr_last_error()
