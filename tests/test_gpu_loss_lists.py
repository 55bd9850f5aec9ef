"""The outlier loss's one-pass form against the float64 restatement.

``mr_loss_outlier`` guesses the threshold's top bits from a sample (every 37th
run of 64 elements), then one pass writes the gradient, the sum over elements under the guess and
per-wave lists of the rest; the exact threshold, the exclusion and the kept
candidates' share come from the lists when they cover the selected top-bits
bin (no list overflowed, guess at or below the bin), and from passes over
every element otherwise. Each case below reads which way the call went from
the workspace, so both are exercised, and checks the result against the
definition (mround/core/losses.py:42-107): threshold = the k-th largest |r|
(exact), gradient = 2 r / n where |r| < threshold else 0 (bitwise), loss =
sum of the kept fp32 squares in float64 over n (within one fp32 rounding).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from mround_amd import kernels as K
from tests.helpers import dev

pytestmark = pytest.mark.gpu

# Workspace layout (mr_loss.hip): 1024 fp64 partials, 2^15 + 2^16 histogram
# bins, then the select state.
_STATE = 8 * 1024 + 4 * (1 << 15) + 4 * (1 << 16)


def _lists_served(ws: torch.Tensor) -> bool:
    st = ws[_STATE:_STATE + 32].cpu().numpy().view(np.uint32)
    digit, key, overflow, guess = int(st[0]), int(st[2]), int(st[3]), int(st[4])
    return overflow == 0 and guess <= (digit << 16) and key <= 0x7F800000


def _check(pred, target, k, *, with_grad=True, ws=None):
    n = pred.numel()
    ws = ws if ws is not None else torch.zeros(int(K.lib().mr_loss_workspace_bytes(n)), dtype=torch.uint8,
                                               device=dev())
    loss = torch.empty(1, device=dev())
    thr = torch.empty(1, device=dev())
    grad = torch.full_like(pred, 7.0) if with_grad else None
    K.loss_outlier(pred, target, k=k, denom=n, loss_out=loss, threshold_out=thr, grad_out=grad, workspace=ws)
    torch.cuda.synchronize()
    r = pred - target
    a = r.abs()
    kth = torch.topk(a, k).values[-1]
    assert float(thr) == float(kth), "threshold is not the k-th largest |r|"
    kept = a < kth
    rk = torch.where(kept, r, torch.zeros_like(r))
    want = float(((rk * rk).double()).sum() / n)
    assert float(loss) == pytest.approx(want, rel=2e-7, abs=0.0)
    if with_grad:
        gs = torch.tensor(2.0 / n, dtype=torch.float32, device=dev())
        assert torch.equal(grad, rk * gs), "gradient differs from 2 r / n over the kept elements"
    return _lists_served(ws), float(loss), float(thr), grad


def _gauss_with_tail(n, seed, every=1000, big=3.0):
    g = torch.Generator(device=dev()).manual_seed(seed)
    target = torch.randn(n, generator=g, device=dev())
    pred = target + torch.randn(n, generator=g, device=dev()) * 0.05
    pred[::every] += big
    return pred, target


@pytest.mark.parametrize("n", [8 * 2048 * 3584, 1_000_003, 1 << 20])
def test_lists_serve_the_common_case(n):
    # the 7B batch, a length that is not a multiple of 4 (scalar loop), a small one
    print("case loss lists common", n, flush=True, file=sys.stderr)
    pred, target = _gauss_with_tail(n, seed=11)
    served, *_ = _check(pred, target, max(1, int(n * 0.001)))
    assert served, "the candidate lists were expected to cover the threshold"


def test_lists_without_gradient_and_equal_bits_whatever_came_before():
    n = 4 << 20
    print("case loss lists history", n, flush=True, file=sys.stderr)
    k = n // 1000
    pred, target = _gauss_with_tail(n, seed=12)
    ws = torch.zeros(int(K.lib().mr_loss_workspace_bytes(n)), dtype=torch.uint8, device=dev())
    served, loss0, thr0, grad0 = _check(pred, target, k, ws=ws)
    assert served
    # other data through the same workspace, then the first again: same bits
    other, tgt2 = _gauss_with_tail(n, seed=13, big=40.0)
    _check(other, tgt2, k, ws=ws)
    _, loss1, thr1, grad1 = _check(pred, target, k, ws=ws)
    assert (loss1, thr1) == (loss0, thr0) and torch.equal(grad0, grad1)
    served, loss2, thr2, _ = _check(pred, target, k, with_grad=False, ws=ws)
    assert served and (loss2, thr2) == (loss0, thr0)


def test_overflowing_lists_fall_back():
    # every |r| is 1 except k / 2 elements of 2: the threshold is 1, the guess
    # too, every element is a candidate and the lists overflow; every element
    # ties at or lies above the threshold, so nothing is kept
    n = 1 << 22
    k = n // 1000
    print("case loss lists overflow", n, flush=True, file=sys.stderr)
    g = torch.Generator(device=dev()).manual_seed(14)
    target = torch.zeros(n, device=dev())
    pred = torch.where(torch.rand(n, generator=g, device=dev()) < 0.5, -1.0, 1.0)
    idx = torch.randperm(n, generator=g, device=dev())[:k // 2]
    pred[idx] *= 2.0
    served, loss, thr, grad = _check(pred, target, k)
    assert not served, "the lists should have overflowed"
    assert loss == 0.0 and thr == 1.0 and not bool(grad.any())


def test_guess_above_the_threshold_falls_back():
    # the first 300 sampled elements (runs of 64 from every 37th run) hold
    # the largest residuals, so the guess lands far above the true k-th
    # largest: the lists miss its bin
    n = 4_000_000
    k = n // 1000
    print("case loss lists high guess", n, flush=True, file=sys.stderr)
    pred, target = _gauss_with_tail(n, seed=15, every=n)  # one tail element only
    j = torch.arange(300, device=dev())
    pred[(j // 64) * (64 * 37) + j % 64] += 10.0
    served, *_ = _check(pred, target, k)
    assert not served, "the guess was expected to miss the threshold's bin"


def test_sparse_heavy_tail_and_nan_threshold():
    n = 1 << 21
    k = 50
    print("case loss lists nan", n, flush=True, file=sys.stderr)
    pred, target = _gauss_with_tail(n, seed=16, every=97, big=-6.0)
    served, *_ = _check(pred, target, k)
    assert served
    # a NaN among the k largest makes the threshold NaN: nothing is kept
    pred[123] = float("nan")
    loss = torch.empty(1, device=dev())
    thr = torch.empty(1, device=dev())
    grad = torch.full_like(pred, 7.0)
    ws = torch.zeros(int(K.lib().mr_loss_workspace_bytes(n)), dtype=torch.uint8, device=dev())
    K.loss_outlier(pred, target, k=1, denom=n, loss_out=loss, threshold_out=thr, grad_out=grad, workspace=ws)
    torch.cuda.synchronize()
    assert torch.isnan(thr).item() and float(loss) == 0.0 and not bool(grad.any())
    assert not _lists_served(ws)
