"""Pins the oracle's quantizer to the reference's known answers.

Hand-computed cases and structural properties follow the reference's
``tests/unit/test_reference_quantize.py`` (ties 45-53, sign convention 97-126,
zero point 162-174, RTN 206-218, clamp boundary 466-506, searched forward
521-531). The gradients are checked against central finite differences of the
straight-through surrogate -- the forward with each rounding residual and the
clamp mask frozen at the base point -- which is the function whose exact
gradient the estimator computes (the reference's method at 253-435); the
surrogate is written here independently of the hand-derived formulas.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import quantize as Q


def rng(seed=0):
    return np.random.default_rng(seed)


@pytest.mark.parametrize(("value", "expected"),
                         [(0.5, 0.0), (1.5, 2.0), (2.5, 2.0), (3.5, 4.0), (-0.5, -0.0), (-1.5, -2.0)])
def test_rounding_ties_to_even(value, expected):
    assert np.rint(np.float32(value)) == expected


def test_half_plus_one_ulp_rounds_up():
    x = np.nextafter(np.float32(0.5), np.float32(1.0))
    assert np.rint(x) == 1.0


def fq(w, v=None, a=None, b=None, **kw):
    return Q.fake_quantize(w, v, a, b, **kw)


class TestSymmetricSign:
    def test_negative_scale_when_positive_dominates(self):
        _, _, s, _ = fq(np.array([[1.0, -0.6, 0.2]]), bits=4, group_size=-1, mode="sym", dtype=np.float64)
        assert s[0, 0, 0] < 0

    def test_positive_scale_when_negative_dominates(self):
        _, _, s, _ = fq(np.array([[0.6, -1.0, 0.2]]), bits=4, group_size=-1, mode="sym", dtype=np.float64)
        assert s[0, 0, 0] > 0

    @pytest.mark.parametrize("bits", [2, 3, 4, 8])
    @pytest.mark.parametrize("sign", [1.0, -1.0])
    def test_dominant_extreme_exact_and_on_extra_code(self, bits, sign):
        w = np.array([[sign, -0.37 * sign, 0.1 * sign]])
        qdq, codes, _, _ = fq(w, bits=bits, group_size=-1, mode="sym", dtype=np.float64)
        assert qdq[0, 0] == pytest.approx(sign, abs=1e-12)
        assert codes[0, 0, 0] == -(2 ** (bits - 1))

    def test_all_zero_group(self):
        qdq, _, s, _ = fq(np.zeros((2, 8)), bits=4, group_size=-1, mode="sym", dtype=np.float64)
        assert np.all(qdq == 0.0) and np.all(s == 1e-8)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("mode", ["sym", "asym"])
def test_codes_stay_in_range(bits, mode):
    w = rng(bits).normal(scale=3.0, size=(6, 64))
    v, a, b = Q.init_params(6, 64, 16, np.float64)
    v = rng(1).uniform(-0.5, 0.5, size=v.shape)
    _, codes, _, _ = fq(w, v, a, b, bits=bits, group_size=16, mode=mode, dtype=np.float64)
    lo, hi = Q.code_range(bits, mode)
    assert codes.min() >= lo and codes.max() <= hi


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_asymmetric_zero_point_representable(bits):
    for w in (np.array([[-2.0, -1.5, -1.0]]), np.array([[1.0, 1.5, 2.0]]), np.array([[-1.0, 0.0, 1.0]])):
        _, _, _, zp = fq(w, bits=bits, group_size=-1, mode="asym", dtype=np.float64)
        assert 0 <= zp[0, 0, 0] <= 2**bits - 1


def test_padding_round_trips():
    w = rng().normal(size=(4, 100))
    g, pad = Q.regroup(w, 32)
    assert g.shape == (4, 4, 32) and pad == 28
    assert np.array_equal(Q.ungroup(g, w.shape, pad), w)


@pytest.mark.parametrize("mode", ["sym", "asym"])
def test_init_params_reproduce_rtn(mode):
    w = rng(9).normal(size=(4, 64)).astype(np.float32)
    v, a, b = Q.init_params(4, 64, 32)
    with_params = fq(w, v, a, b, bits=4, group_size=32, mode=mode)[0]
    rtn = fq(w, bits=4, group_size=32, mode=mode)[0]
    assert np.array_equal(with_params, rtn)


def test_more_bits_and_smaller_groups_reconstruct_better():
    w = rng(7).normal(size=(8, 256))
    err = lambda b, g: float(np.mean((fq(w, bits=b, group_size=g, mode="sym", dtype=np.float64)[0] - w) ** 2))
    assert err(4, 32) < err(2, 32) and err(4, 32) < err(4, 256)


def test_clamp_boundary_fixture():
    """``tests/unit/test_reference_quantize.py:466-506``."""
    w = np.array([[1.0, 0.9, 0.5, -0.3]])
    v, a, b = Q.init_params(1, 4, -1, np.float64)
    _, codes, _, _ = fq(w, v, a, b, bits=2, group_size=-1, mode="sym", dtype=np.float64)
    assert codes.ravel().tolist() == [-2.0, -2.0, -1.0, 1.0]
    gv, _, _ = Q.quantize_grad(w, v, a, b, np.ones_like(w), bits=2, group_size=-1, mode="sym",
                               dtype=np.float64)
    assert np.all(gv != 0.0)
    v2 = v - 1.0
    gv2, _, _ = Q.quantize_grad(w, v2, a, b, np.ones_like(w), bits=2, group_size=-1, mode="sym",
                                dtype=np.float64)
    _, _, s, _ = fq(w, v2, a, b, bits=2, group_size=-1, mode="sym", dtype=np.float64)
    raw = np.rint(w / s.reshape(1, 1) + v2.reshape(1, -1))
    assert np.any(raw < -2)
    assert np.all(gv2.ravel()[(raw < -2).ravel()] == 0.0)


def test_searched_forward_known_answer():
    """``tests/unit/test_reference_quantize.py:521-531``."""
    w = np.array([[0.9, -0.3, 0.2, 0.1]])
    v, a, b = Q.init_params(1, 4, 4, np.float64)
    qdq, codes, _, _ = fq(w, v, a, b, bits=3, group_size=4, mode="searched",
                          init_scale=np.array([[-0.25]]), dtype=np.float64)
    assert codes.ravel().tolist() == [-4.0, 1.0, -1.0, 0.0]
    np.testing.assert_allclose(qdq, [[1.0, -0.25, 0.25, 0.0]])


def test_searched_alpha_inert_and_beta_folds_into_scale():
    w = np.array([[0.9, -0.3, 0.2, 0.1]])
    v, a, b = Q.init_params(1, 4, 4, np.float64)
    base = np.array([[-0.25]])
    x = fq(w, v, a * 0.7, b, bits=3, group_size=4, mode="searched", init_scale=base, dtype=np.float64)
    y = fq(w, v, a, b, bits=3, group_size=4, mode="searched", init_scale=base, dtype=np.float64)
    assert np.array_equal(x[0], y[0])
    z = fq(w, v, a, b * 0.5, bits=3, group_size=4, mode="searched", init_scale=base, dtype=np.float64)
    u = fq(w, v, a, b, bits=3, group_size=4, mode="searched", init_scale=base * 0.5, dtype=np.float64)
    assert np.array_equal(z[1], u[1])


def test_only_dominant_side_gets_coefficient_gradient():
    w = np.array([[1.0, -0.4, 0.2, 0.05]])
    v, a, b = Q.init_params(1, 4, -1, np.float64)
    _, ga, gb = Q.quantize_grad(w, v, a, b, np.ones_like(w), bits=4, group_size=-1, mode="sym",
                                dtype=np.float64)
    assert gb[0, 0, 0] == 0.0 and ga[0, 0, 0] != 0.0


# ---- finite differences of the straight-through surrogate ----------------

def _surrogate(w, v, a, b, frozen, bits, gs, mode, eps=1e-8):
    """The forward with rounding residuals and the clamp mask frozen."""
    g, pad = Q.regroup(w, gs)
    if mode == "searched":
        s = frozen["base"] * b
        x = g / s + v + frozen["res"]
        c = np.where(frozen["mask"], x, frozen["bound"])
        out = s * c
    else:
        hi_raw = np.maximum(g.max(-1, keepdims=True), 0.0)
        lo_raw = np.minimum(g.min(-1, keepdims=True), 0.0)
        hi, lo = hi_raw * a, lo_raw * b
        if mode == "sym":
            m = float(2 ** (bits - 1))
            s = np.where(frozen["pos"], -hi, -lo) / m
            x = g / s + v + frozen["res"]
            c = np.where(frozen["mask"], x, frozen["bound"])
            out = s * c
        else:
            s = np.maximum((hi - lo) / float(2**bits - 1), eps)
            zp = -lo / s + frozen["zres"]
            x = g / s + v + frozen["res"] + zp
            c = np.where(frozen["mask"], x, frozen["bound"])
            out = s * (c - zp)
    return Q.ungroup(out, w.shape, pad)


def _freeze(w, v, a, b, bits, gs, mode, init_scale):
    g, _ = Q.regroup(w, gs)
    _, codes, s, zp = Q.fake_quantize(w, v, a, b, bits=bits, group_size=gs, mode=mode,
                                      init_scale=init_scale, dtype=np.float64)
    pre = g / s + v
    res = np.rint(pre) - pre
    raw = np.rint(pre) + (zp if zp is not None else 0.0)
    lo, hi = Q.code_range(bits, mode)
    fr = {"res": res, "mask": (raw >= lo) & (raw <= hi), "bound": np.clip(raw, lo, hi)}
    if mode == "asym":
        lo_c = np.minimum(g.min(-1, keepdims=True), 0.0) * b
        fr["zres"] = zp - (-lo_c / s)
    if mode == "sym":
        hi_c = np.maximum(g.max(-1, keepdims=True), 0.0) * a
        lo_c = np.minimum(g.min(-1, keepdims=True), 0.0) * b
        fr["pos"] = hi_c >= -lo_c
    if mode == "searched":
        fr["base"] = np.asarray(init_scale, dtype=np.float64).reshape(s.shape)
    return fr


@pytest.mark.parametrize("mode,bits", [(m, b) for m in ("sym", "asym") for b in (2, 4, 8)]
                         + [("searched", 2), ("searched", 3), ("searched", 4)])
def test_gradients_match_finite_differences(mode, bits):
    gen = rng(100 * (1 + ("sym", "asym", "searched").index(mode)) + bits)
    gs = 8
    w = gen.normal(size=(3, 24))
    target = gen.normal(size=(3, 24)) * 0.1
    v, a, b = Q.init_params(3, 24, gs, np.float64)
    v = v + gen.uniform(-0.3, 0.3, size=v.shape)
    a = a * (1.0 + gen.uniform(-0.15, 0.15, size=a.shape))
    b = b * (1.0 + gen.uniform(-0.15, 0.15, size=b.shape))
    init_scale = None
    if mode == "searched":
        init_scale = -np.abs(gen.normal(size=(3, 3))) * 0.3 - 0.05
    fr = _freeze(w, v, a, b, bits, gs, mode, init_scale)
    loss = lambda vv, aa, bb: float(np.sum((_surrogate(w, vv, aa, bb, fr, bits, gs, mode) - target) ** 2))
    qdq = Q.fake_quantize(w, v, a, b, bits=bits, group_size=gs, mode=mode, init_scale=init_scale,
                          dtype=np.float64)[0]
    grads = Q.quantize_grad(w, v, a, b, 2.0 * (qdq - target), bits=bits, group_size=gs, mode=mode,
                            init_scale=init_scale, dtype=np.float64)
    h = 1e-6
    for which, arr in enumerate((v, a, b)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            orig = arr[idx]
            arr[idx] = orig + h
            plus = loss(v, a, b)
            arr[idx] = orig - h
            minus = loss(v, a, b)
            arr[idx] = orig
            num[idx] = (plus - minus) / (2 * h)
        denom = max(1.0, float(np.abs(num).max()))
        assert np.allclose(grads[which] / denom, num / denom, atol=1e-6), (mode, bits, which)


def test_dropping_the_direct_beta_term_fails_finite_differences():
    """A plausible mistake -- omitting the zero-point route to beta -- is caught."""
    gen = rng(7)
    w = gen.normal(size=(2, 16))
    target = gen.normal(size=(2, 16)) * 0.1
    v, a, b = Q.init_params(2, 16, 8, np.float64)
    v = v - 0.45  # push low codes against the clamp so the direct term is active
    a, b = a * 0.6, b * 0.6
    fr = _freeze(w, v, a, b, 2, 8, "asym", None)
    qdq = Q.fake_quantize(w, v, a, b, bits=2, group_size=8, mode="asym", dtype=np.float64)[0]
    g = 2.0 * (qdq - target)
    _, _, gb = Q.quantize_grad(w, v, a, b, g, bits=2, group_size=8, mode="asym", dtype=np.float64)
    _, direct = Q.grad_terms(w, v, a, b, g, bits=2, group_size=8, mode="asym", dtype=np.float64)
    loss = lambda bb: float(np.sum((_surrogate(w, v, a, bb, fr, 2, 8, "asym") - target) ** 2))
    num = np.zeros_like(b)
    for idx in np.ndindex(b.shape):
        bp, bm = b.copy(), b.copy()
        bp[idx] += 1e-6
        bm[idx] -= 1e-6
        num[idx] = (loss(bp) - loss(bm)) / 2e-6
    assert np.allclose(gb, num, atol=1e-6)
    wrong = gb - direct.sum(-1, keepdims=True)
    assert not np.allclose(wrong, num, atol=1e-6)


def test_float32_and_float64_codes_agree():
    """< 0.1 % of codes may differ between the precisions (test_mlx_parity.py:213-234)."""
    w = rng(11).normal(scale=0.02, size=(64, 256))
    v = rng(12).uniform(-0.5, 0.5, size=(64, 4, 64))
    a = np.ones((64, 4, 1)); b = np.ones((64, 4, 1))
    c32 = Q.fake_quantize(w, v, a, b, bits=2, group_size=64, mode="asym", dtype=np.float32)[1]
    c64 = Q.fake_quantize(w, v, a, b, bits=2, group_size=64, mode="asym", dtype=np.float64)[1]
    assert np.mean(c32 != c64) < 1e-3


def test_bf16_rounding_known_values():
    x = np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, -2.5, 3.0e38], dtype=np.float32)
    got = Q.round_to_bf16(x)
    assert got[0] == 1.0
    assert got[1] == 1.0  # tie -> even
    assert got[2] == 1.0 + 4 * 2**-8  # tie -> even (up)
    assert got[3] == -2.5
