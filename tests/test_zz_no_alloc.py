"""The allocation-free outlier loss (``mr_loss_outlier_noalloc``) through the
C ABI against ``mr_loss_outlier`` with a caller workspace: the same kernels
over the library's static per-GPU scratch, so loss, threshold and gradient
are bit-identical. Two calls in a row, the second smaller, show that the
scratch left by one call does not leak into the next."""

from __future__ import annotations

import ctypes
import sys

import pytest
import torch

from mround_amd import kernels as K
from tests.helpers import dev

pytestmark = pytest.mark.gpu


def _inputs(n, seed):
    g = torch.Generator().manual_seed(seed)
    target = torch.randn(n, generator=g)
    pred = target + torch.randn(n, generator=g) * 0.1
    # a few large residuals and an exact tie at the largest magnitude
    idx = torch.randperm(n, generator=g)[:max(4, n // 500)]
    pred[idx] += torch.randn(idx.numel(), generator=g) * 5
    pred[idx[0]] = target[idx[0]] + 9.0
    pred[idx[1]] = target[idx[1]] - 9.0
    return pred.to(dev()), target.to(dev())


def _via_workspace(pred, target, k, denom):
    lib = K.lib()
    loss = torch.empty(1, device=dev())
    thr = torch.empty(1, device=dev())
    grad = torch.empty_like(pred)
    ws = torch.empty(int(lib.mr_loss_workspace_bytes(pred.numel())), dtype=torch.uint8, device=dev())
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.mr_loss_outlier(pred.data_ptr(), target.data_ptr(), pred.numel(), k, denom, None,
                             thr.data_ptr(), loss.data_ptr(), grad.data_ptr(), ws.data_ptr(), stream)
    assert rc == 0, lib.mr_last_error()
    return loss, thr, grad


def _via_scratch(pred, target, k, denom):
    lib = K.lib()
    loss = torch.empty(1, device=dev())
    thr = torch.empty(1, device=dev())
    grad = torch.empty_like(pred)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.mr_loss_outlier_noalloc(pred.data_ptr(), target.data_ptr(), pred.numel(), k, denom, None,
                                     thr.data_ptr(), loss.data_ptr(), grad.data_ptr(), stream)
    assert rc == 0, lib.mr_last_error()
    return loss, thr, grad


@pytest.mark.parametrize("sizes", [(1 << 20, 40_000), (3 * 2048 * 576 + 4, 4099)])
def test_noalloc_outlier_loss_matches_the_workspace_form(sizes):
    # the second call is smaller (and, in the second case, not a multiple of 4)
    for call, n in enumerate(sizes):
        print("case noalloc loss", call, n, flush=True, file=sys.stderr)
        pred, target = _inputs(n, seed=40 + call)
        k = max(1, int(n * 0.001))
        want = _via_workspace(pred, target, k, n)
        got = _via_scratch(pred, target, k, n)
        torch.cuda.synchronize()
        for w, g, name in zip(want, got, ("loss", "threshold", "gradient")):
            assert torch.equal(w, g), f"{name} differs on call {call} (n={n})"
        # the threshold is the k-th largest |r| (exact)
        r = (pred - target).abs().cpu()
        assert float(got[1]) == float(torch.topk(r, k).values[-1])


def test_noalloc_outlier_loss_with_a_given_threshold():
    n = 1 << 16
    pred, target = _inputs(n, seed=50)
    thr = torch.tensor([0.25], device=dev())
    lib = K.lib()
    out = []
    for fn in ("ws", "scratch"):
        loss = torch.empty(1, device=dev())
        grad = torch.empty_like(pred)
        stream = torch.cuda.current_stream().cuda_stream
        if fn == "ws":
            ws = torch.empty(int(lib.mr_loss_workspace_bytes(n)), dtype=torch.uint8, device=dev())
            rc = lib.mr_loss_outlier(pred.data_ptr(), target.data_ptr(), n, 1, n, thr.data_ptr(), None,
                                     loss.data_ptr(), grad.data_ptr(), ws.data_ptr(), stream)
        else:
            rc = lib.mr_loss_outlier_noalloc(pred.data_ptr(), target.data_ptr(), n, 1, n, thr.data_ptr(),
                                             None, loss.data_ptr(), grad.data_ptr(), stream)
        assert rc == 0, lib.mr_last_error()
        out.append((loss, grad))
    torch.cuda.synchronize()
    assert torch.equal(out[0][0], out[1][0]) and torch.equal(out[0][1], out[1][1])


def test_noalloc_outlier_loss_refuses_bad_arguments():
    lib = K.lib()
    P = ctypes.c_void_p
    # rank outside [1, n], and more elements than the 32-bit histograms count
    assert lib.mr_loss_outlier_noalloc(P(256), P(256), 100, 0, 100, None, None, P(256), None, None) == -22
    assert b"rank" in lib.mr_last_error()
    assert lib.mr_loss_outlier_noalloc(P(256), P(256), 1 << 33, 5, 1 << 33, None, None, P(256), None,
                                       None) == -22
    assert b"elements" in lib.mr_last_error()
    assert lib.mr_loss_outlier_noalloc(None, P(256), 100, 1, 100, None, None, P(256), None, None) == -22
