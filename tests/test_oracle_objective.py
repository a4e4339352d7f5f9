"""The oracle's objectives (objective/binary.rs:27-50, objective/regression.rs:20-43) against closed forms.

Binary log loss with sigmoid parameter s and p = 1 / (1 + exp(-s * score)): the gradient is s * (p - y) and the
hessian s^2 * p * (1 - p), with y = 1 for a label > 0 and 0 otherwise, both times the row weight. The reference
computes them as -sign * s / (1 + exp(sign * s * score)) and |r| * (s - |r|); the closed form below is written with
scipy's logistic function instead, so a sign, a missing s, or an s that should be s^2 fails it. The sweep covers
three values of s: at s = 1 a hessian written with 1 in place of s would pass.
"""

import numpy as np
import pytest
from scipy.special import expit

import oracle
from silvic_amd import _abi

F32_ULP = np.float64(2.0 ** -23)


def _within(got, want, rel_ulps, abs_tol=0.0):
    got = got.astype(np.float64)
    return np.abs(got - want) <= rel_ulps * F32_ULP * np.abs(want) + abs_tol


@pytest.mark.parametrize("sigma", [0.5, 1.0, 2.0])
@pytest.mark.parametrize("weighted", [False, True])
def test_binary_gradients_match_the_closed_form(sigma, weighted):
    n = 40_000
    rng = np.random.default_rng(int(sigma * 10) + weighted)
    scores = np.concatenate([np.linspace(-30, 30, n // 2), rng.standard_normal(n // 2) * 4]).astype(np.float32)
    label = rng.choice(np.array([0.0, 1.0, 0.5, -1.0], np.float32), n, p=[0.45, 0.45, 0.05, 0.05])
    weight = rng.uniform(0.1, 3.0, n).astype(np.float32) if weighted else None
    g, h, mg, mh = oracle.gradients(_abi.OBJ_BINARY, scores, label, sigma, weight)

    z = sigma * scores.astype(np.float64)
    pos = label > 0
    w = np.ones(n) if weight is None else weight.astype(np.float64)
    want_g = np.where(pos, -sigma * expit(-z), sigma * expit(z)) * w  # s * (p - y), p - 1 = -expit(-z)
    want_h = sigma * sigma * expit(z) * expit(-z) * w
    assert _within(g, want_g, 3).all()
    # |r| * (s - |r|) cancels when |r| is near s: its absolute error is a few f64 ulps of s^2 * w
    assert _within(h, want_h, 3, 4 * sigma * sigma * 2.0 ** -52 * w).all()
    assert (np.sign(g[pos]) <= 0).all() and (np.sign(g[~pos]) >= 0).all()
    assert mg == np.abs(g).astype(np.float64).max() and mh == h.astype(np.float64).max()


def test_regression_gradients_are_f32_residuals():
    # regression.rs:20-43: g = (score - y) * w, h = w, in f32 arithmetic
    rng = np.random.default_rng(1)
    n = 10_000
    scores = (rng.standard_normal(n) * 3).astype(np.float32)
    label = (rng.standard_normal(n) * 3).astype(np.float32)
    weight = rng.uniform(0.1, 3.0, n).astype(np.float32)
    g, h, _, _ = oracle.gradients(_abi.OBJ_REGRESSION, scores, label)
    assert np.array_equal(g, scores - label) and (h == 1.0).all()
    g, h, mg, mh = oracle.gradients(_abi.OBJ_REGRESSION, scores, label, 1.0, weight)
    assert np.array_equal(g, (scores - label) * weight) and np.array_equal(h, weight)
    assert mg == np.abs(g).astype(np.float64).max() and mh == h.astype(np.float64).max()
