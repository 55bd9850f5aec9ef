"""Pins the oracle's optimizer, losses, packing and sensitivity.

Known answers follow the reference's tests: optimizer and losses
(``tests/unit/test_reference_optimizer.py:23-280``; the threshold semantics of
``tests/unit/test_mlx_parity.py:443-509``), packing
(``tests/unit/test_reference_packing.py:80-244``) and DeltaLoss / storage
(``tests/unit/test_sensitivity.py:42-224``).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import losses as L
from oracle import optimizer as O
from oracle import packing as P
from oracle import sensitivity as S


def rng(seed=0):
    return np.random.default_rng(seed)


# ---- optimizer --------------------------------------------------------------

def test_every_nonzero_gradient_moves_exactly_lr():
    p = np.zeros(5)
    g = np.array([3.0, -1e-9, 0.0, 100.0, -7.0])
    out = O.sign_update(p, g, 0.01)
    np.testing.assert_array_equal(out, [-0.01, 0.01, 0.0, -0.01, 0.01])


def test_update_invariant_to_loss_scaling():
    g = rng().normal(size=20)
    p = rng(1).normal(size=20)
    assert np.array_equal(O.sign_update(p, g, 0.1), O.sign_update(p, g * 1e6, 0.1))


def test_schedule_reaches_zero_and_excursion():
    sched = O.LinearDecay(0.005, 200)
    assert sched(0) == 0.005 and sched(200) == 0.0 and sched(500) == 0.0
    # c = 1: excursion 0.5 * (1 + 1/iters) (test_mlx_parity.py:443-448)
    assert O.total_excursion(1.0 / 200, 200) == pytest.approx(0.5 * (1 + 1 / 200))


def test_lr_rule():
    assert O.resolved_lr(2, 200) == 0.005
    assert O.resolved_lr(4, 200) == 0.005
    assert O.resolved_lr(2, 1000) == 0.002
    assert O.resolved_lr(4, 1000) == 0.001


def test_signsgd_steps_the_schedule():
    opt = O.SignSGD(O.LinearDecay(1.0, 4))
    p = {"x": np.zeros(1)}
    for _ in range(4):
        p = opt.apply(p, {"x": np.ones(1)})
    assert p["x"][0] == pytest.approx(-(1.0 + 0.75 + 0.5 + 0.25))
    with pytest.raises(KeyError):
        opt.apply({"y": np.zeros(1)}, {})


# ---- losses -----------------------------------------------------------------

def test_selection_is_global_not_per_row():
    """``tests/unit/test_reference_optimizer.py:200-221``: (990 + 1000) * 0.01**2 / 2000."""
    pred = np.full((2, 1000), 0.01)
    pred[0, :5] = 100.0
    pred[0, 5:10] = 0.02
    ref = np.zeros_like(pred)
    loss, grad = L.outlier_suppressed_loss_exact_k(pred, ref, fraction=0.005)
    assert np.allclose(grad[0, :10], 0.0) and np.all(grad[1] != 0.0)
    assert loss == pytest.approx((990 + 1000) * 0.01**2 / 2000)
    loss_t, grad_t, thr = L.outlier_suppressed_loss(pred, ref, fraction=0.005, dtype=np.float64)
    assert thr == 0.02 and np.allclose(grad_t[0, :10], 0.0)
    assert loss_t == pytest.approx((990 + 1000) * 0.01**2 / 2000)


def test_denominator_is_full_count_and_k_at_least_one():
    pred = np.array([[1.0, 2.0, 3.0, 100.0]])
    loss, _ = L.outlier_suppressed_loss_exact_k(pred, np.zeros_like(pred))
    assert loss == pytest.approx((1 + 4 + 9) / 4)
    assert L.outlier_k(10) == 1 and L.outlier_k(58_720_256) == 58_720


def test_threshold_rule_excludes_all_ties():
    pred = np.array([1.0, 5.0, 5.0, 2.0] + [0.5] * 996)
    loss, grad, thr = L.outlier_suppressed_loss(pred, np.zeros_like(pred), dtype=np.float64)
    assert thr == 5.0
    assert grad[1] == 0.0 and grad[2] == 0.0  # both tied elements excluded (k = 1)
    exact, _ = L.outlier_suppressed_loss_exact_k(pred, np.zeros_like(pred))
    assert exact > loss


def test_loss_gradients_by_finite_differences():
    pred = rng(3).normal(size=(4, 50))
    ref = rng(4).normal(size=(4, 50))
    _, g = L.reconstruction_loss(pred, ref)
    _, gk, thr = L.outlier_suppressed_loss(pred, ref, dtype=np.float64)
    for fn, grad in ((lambda p: L.reconstruction_loss(p, ref)[0], g),
                     (lambda p: L.outlier_suppressed_loss(p, ref, threshold=thr, dtype=np.float64)[0], gk)):
        num = np.zeros_like(pred)
        for idx in np.ndindex(pred.shape):
            a, b = pred.copy(), pred.copy()
            a[idx] += 1e-6
            b[idx] -= 1e-6
            num[idx] = (fn(a) - fn(b)) / 2e-6
        smooth = np.abs(np.abs(pred - ref) - thr) > 1e-5  # the element at the threshold is a kink
        np.testing.assert_allclose(grad[smooth], num[smooth], atol=1e-7)


def test_pieces_sum_to_the_batch():
    pred = rng(5).normal(size=(8, 30))
    ref = rng(6).normal(size=(8, 30))
    whole, _, thr = L.outlier_suppressed_loss(pred, ref, dtype=np.float64)
    parts = sum(L.piece_loss(pred[i:i + 2], ref[i:i + 2], elements=pred.size, threshold=thr,
                             dtype=np.float64)[0] for i in range(0, 8, 2))
    assert parts == pytest.approx(whole, rel=1e-12)


# ---- packing ----------------------------------------------------------------

def test_four_bit_known_answer():
    assert P.pack_codes(np.arange(8).reshape(1, 8), 4)[0, 0] == 0x76543210


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_element_zero_lsb_and_next_field(bits):
    per = 32 // bits
    c = np.zeros((1, per), dtype=np.int64)
    c[0, 0] = 1
    assert P.pack_codes(c, bits)[0, 0] == 1
    c[0, 0], c[0, 1] = 0, 1
    assert P.pack_codes(c, bits)[0, 0] == 1 << bits


@pytest.mark.parametrize("bits", [3, 5, 6, 7])
def test_stream_positions_including_straddlers(bits):
    for element in range(32):
        c = np.zeros((1, 32), dtype=np.int64)
        c[0, element] = 2**bits - 1
        stream = 0
        for i, word in enumerate(P.pack_codes(c, bits)[0]):
            stream |= int(word) << (32 * i)
        assert stream == (2**bits - 1) << (element * bits)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_matches_independent_construction(bits):
    c = rng(bits).integers(0, 2**bits, size=(8, 128), dtype=np.uint32)
    assert np.array_equal(P.pack_codes(c, bits), P.mlx_style_pack(c, bits))


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 7, 8])
def test_round_trip_and_width(bits):
    c = rng(bits + 10).integers(0, 2**bits, size=(5, 96))
    packed = P.pack_codes(c, bits)
    assert packed.shape == (5, 96 * bits // 32)
    assert np.array_equal(P.unpack_codes(packed, 96, bits), c)


def test_validation_messages():
    with pytest.raises(ValueError, match=r"codes must lie in \[0, 15\]"):
        P.pack_codes(np.array([[0, 16, 3, 4, 5, 6, 7, 8]]), 4)
    with pytest.raises(ValueError, match="2-D code matrix"):
        P.pack_codes(np.zeros(8, dtype=np.int64), 4)
    with pytest.raises(ValueError, match="expected 8 words per row"):
        P.unpack_codes(np.zeros((2, 3), dtype=np.uint32), 64, 4)


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_symmetric_zero_exactly_representable(bits):
    """``scales * 2**(bits-1) + biases == 0`` in the stored dtype (test_mlx_formats.py:114-127)."""
    s = rng(bits).normal(scale=0.01, size=(64,)).astype(np.float32)
    for dtype in ("bfloat16", "float16", "float32"):
        scales, biases = P.to_affine(s, None, bits, dtype)
        assert np.all(scales * np.float32(2 ** (bits - 1)) + biases == 0.0)


def test_affine_reproduces_reconstruction_in_float32():
    from oracle.quantize import fake_quantize

    w = rng(1).normal(size=(4, 128)).astype(np.float32)
    qdq, codes, s, zp = fake_quantize(w, None, None, None, bits=4, group_size=64, mode="asym")
    scales, biases = P.to_affine(s.reshape(4, 2), zp.reshape(4, 2), 4, "float32")
    rebuilt = (scales[:, :, None] * codes.reshape(4, 2, 64) + biases[:, :, None]).reshape(4, 128)
    np.testing.assert_allclose(rebuilt, qdq, atol=1e-6)


# ---- sensitivity ------------------------------------------------------------

def test_delta_loss_hand_values():
    """``tests/unit/test_sensitivity.py:42-62`` style: abs before the sum."""
    w = np.array([1.0, 2.0, 3.0])
    q = np.array([1.5, 1.5, 3.0])
    g = np.array([1.0, 1.0, 7.0])
    assert S.delta_loss(w, q, g) == pytest.approx(1.0)
    assert S.delta_loss([0.0, 0.0], [0.3, -0.6], [3.0, 2.0]) == pytest.approx(0.9 + 1.2)


def test_storage_bits():
    assert S.storage_bits((64, 128), 4, 64) / (64 * 128) == pytest.approx(4.5)
    assert S.storage_bits((64, 128), 2, 64) / (64 * 128) == pytest.approx(2.5)


def test_integer_average_budget_equals_uniform():
    shapes = {"a": (64, 128), "b": (32, 256)}
    assert S.mixed_budget_bits(shapes, 3, 64) == sum(S.storage_bits(s, 3, 64) for s in shapes.values())
