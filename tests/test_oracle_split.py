"""The oracle's split.rs restatement against the reference's split tests (split.rs:1150-1506): brute force over
every candidate, the NaN-vs-rest, one-hot, sorted categorical, constraint, zero-hessian and tie cases."""

import numpy as np

import oracle
from silvic_amd import _abi
from tests.helpers import Lcg
from tests.split_cases import (MIN_SCORE, brute_force, categorical, close, config, goes_left, leaf_gain,
                               leaf_output, numerical, numerical_candidates, numerical_cases, quantized_cases,
                               random_hist, side_sums, sums)


def check_children(split, meta, hist, rows, cfg, case):
    """split.rs:1110-1148."""
    left = goes_left(split, meta, len(rows))
    lg, lh, ln = side_sums(hist, rows, left)
    assert close(split.left.grad, lg), case
    assert close(split.left.hess, lh), case
    assert split.left.count == ln, case
    l2 = cfg.lambda_l2
    if split.categorical and (split.num_cat_bins > 1 or len(rows) > cfg.max_cat_to_onehot):
        l2 = cfg.lambda_l2 + cfg.cat_l2
    assert close(split.left_output, leaf_output(lg, lh, cfg.lambda_l1, l2)), case


def test_numerical_matches_brute_force():
    for name, hist, rows, meta, cfg in numerical_cases():
        best, _ = oracle.find_best_split(hist, [meta], [1], sums(hist, rows), 1.0, 1.0, cfg)
        expected = brute_force(hist, rows, cfg, numerical_candidates(len(rows), meta.nan_bin))
        if not best.found:
            assert expected == MIN_SCORE, f"{name}: brute force found a split"
        else:
            assert close(best.gain, expected), (name, best.gain, expected)
            check_children(best, meta, hist, rows, cfg, name)


def test_quantized_scale_matches_real_sums():
    for case, units, rows, meta in quantized_cases():
        real = units.copy()
        real[0::2] *= 0.37
        real[1::2] *= 0.125
        cfg = config()
        total = int(rows.sum())
        q, _ = oracle.find_best_split(units, [meta], [1], (units[0::2].sum(), units[1::2].sum(), total), 0.37, 0.125, cfg)
        f, _ = oracle.find_best_split(real, [meta], [1], (real[0::2].sum(), real[1::2].sum(), total), 1.0, 1.0, cfg)
        assert bool(q.found) == bool(f.found), case
        if q.found:
            assert (q.threshold, q.default_left) == (f.threshold, f.default_left), case
            assert close(q.gain, f.gain), case
            assert close(q.left.grad * 0.37, f.left.grad), case


def test_nan_against_rest_is_a_candidate():
    # split.rs:1234-1250
    hist = np.array([-10.0, 10.0, -10.0, 10.0, -10.0, 10.0, 30.0, 10.0])
    rows = np.array([10, 10, 10, 10])
    best, _ = oracle.find_best_split(hist, [numerical(4, True)], [1], sums(hist, rows), 1.0, 1.0, config())
    assert best.found and not best.categorical
    assert (best.threshold, best.default_left) == (2, 0)
    assert best.left.count == 30


def test_onehot_matches_brute_force():
    # split.rs:1252-1285
    rng = Lcg(3)
    for case in range(200):
        num_bins = 2 + rng.below(3)
        hist, rows = random_hist(rng, num_bins, 1.0)
        meta = categorical(num_bins)
        cfg = config()
        best, _ = oracle.find_best_split(hist, [meta], [1], sums(hist, rows), 1.0, 1.0, cfg)
        cands = [lambda b, t=t: b == t for t in range(1, num_bins)]
        expected = brute_force(hist, rows, cfg, cands)
        if not best.found:
            assert expected == MIN_SCORE, case
        else:
            assert close(best.gain, expected), case
            assert best.categorical and best.num_cat_bins == 1, case
            check_children(best, meta, hist, rows, cfg, case)


def test_sorted_categorical_matches_brute_force():
    # split.rs:1287-1349
    rng = Lcg(5)
    found = 0
    for case in range(200):
        num_bins = 6 + rng.below(12)
        hist, rows = random_hist(rng, num_bins, 1.0)
        cfg = config(min_data_per_group=1, cat_smooth=1.0, max_cat_threshold=4)
        meta = categorical(num_bins)
        best, _ = oracle.find_best_split(hist, [meta], [1], sums(hist, rows), 1.0, 1.0, cfg)

        def ctr(t):
            return hist[2 * t] / (hist[2 * t + 1] + cfg.cat_smooth)

        srt = sorted([t for t in range(1, num_bins) if rows[t] >= cfg.cat_smooth], key=ctr)
        used = len(srt)
        max_cat = min(cfg.max_cat_threshold, (used + 1) // 2)
        cands = []
        for k in range(1, min(max_cat, used) + 1):
            low, high = set(srt[:k]), set(srt[used - k:])
            cands.append(lambda b, s=low: b in s)
            cands.append(lambda b, s=high: b in s)
        bcfg = config(min_data_per_group=1, cat_smooth=1.0, max_cat_threshold=4, lambda_l2=cfg.lambda_l2 + cfg.cat_l2)
        tg, th, _ = sums(hist, rows)
        shift_fix = leaf_gain(tg, th, 0.0, bcfg.lambda_l2) - leaf_gain(tg, th, 0.0, cfg.lambda_l2)
        expected = brute_force(hist, rows, bcfg, cands)
        expected = expected if expected == MIN_SCORE else expected + shift_fix
        if not best.found:
            assert expected <= 0.0, (case, expected)
        else:
            found += 1
            assert close(best.gain, expected), (case, best.gain, expected)
            check_children(best, meta, hist, rows, cfg, case)
            assert all(best.cat_bins[i] >= 1 for i in range(best.num_cat_bins))
    assert found > 50


def test_constraints_reject_splits():
    # split.rs:1351-1412
    hist = np.array([-20.0, 10.0, 20.0, 10.0, -5.0, 5.0])
    rows = np.array([10, 10, 5])
    meta = numerical(3, False)

    def run(cfg, ev=(1,)):
        return oracle.find_best_split(hist, [meta], list(ev), sums(hist, rows), 1.0, 1.0, cfg)

    assert run(config())[0].found
    for kw in (dict(min_data_in_leaf=16), dict(min_sum_hessian_in_leaf=16.0), dict(min_gain_to_split=1e6),
               dict(lambda_l1=100.0)):
        assert not run(config(**kw))[0].found, kw
    best, spl = run(config(), ev=(0,))
    assert not best.found and list(spl) == [False]


def test_zero_hessian_rows_never_make_empty_children():
    # split.rs:1414-1471
    cfg = config(min_data_in_leaf=0, min_sum_hessian_in_leaf=0.0)
    hist = np.array([0.0, 0.0, 0.0, 0.0, -3.0, 2.0, 0.0, 0.0, 4.0, 2.0, 0.0, 0.0])
    best, _ = oracle.find_best_split(hist, [numerical(6, False)], [1], (hist[0::2].sum(), hist[1::2].sum(), 400),
                                     1.0, 1.0, cfg)
    assert best.found
    assert best.left.hess > 0 and best.right.hess > 0 and best.left.count > 0 and best.right.count > 0
    zero = np.zeros(12)
    best, _ = oracle.find_best_split(zero, [numerical(6, False)], [1], (0.0, 0.0, 400), 1.0, 1.0, cfg)
    assert not best.found
    for nb in (3, 8):
        h = np.array([0.0, 0.0, -3.0, 2.0, 0.0, 0.0, 4.0, 2.0, 0.0, 0.0, 1.0, 1.0, 0.0, 0.0, 0.0, 0.0])[: 2 * nb]
        c = config(min_data_in_leaf=0, min_sum_hessian_in_leaf=0.0, min_data_per_group=0, cat_smooth=0.0)
        best, _ = oracle.find_best_split(h, [categorical(nb)], [1], (h[0::2].sum(), h[1::2].sum(), 400), 1.0, 1.0, c)
        if best.found:
            assert best.left.hess > 0 and best.right.hess > 0


def test_ties_go_to_the_lower_feature():
    # split.rs:1473-1489
    hist = np.array([-20.0, 10.0, 20.0, 10.0, -20.0, 10.0, 20.0, 10.0])
    feats = [numerical(2, False), numerical(2, False, hist_offset=2)]
    best, spl = oracle.find_best_split(hist, feats, [1, 1], (hist[0:4:2].sum(), hist[1:4:2].sum(), 20), 1.0, 1.0,
                                       config())
    assert best.feature == 0
    assert list(spl) == [True, True]


def test_feature_mask_samples_the_lightgbm_count():
    # split.rs:1491-1506
    feats = [numerical(4, False) for _ in range(10)]
    feats[3] = type(feats[3])(0, 0, 0, 0, _abi.BINS_TRIVIAL, False)
    for fraction, expected in [(1.0, 9), (0.5, 5), (0.8, 7), (0.01, 1)]:
        m = oracle.feature_mask(feats, fraction, 2, 0)
        assert m.sum() == expected, fraction
        assert not m[3]
    assert (oracle.feature_mask(feats, 0.5, 2, 4) == oracle.feature_mask(feats, 0.5, 2, 4)).all()
    distinct = {tuple(oracle.feature_mask(feats, 0.5, 2, i)) for i in range(20)}
    assert len(distinct) > 5


def test_gain_and_output_closed_forms():
    # split.rs:159-192: ThresholdL1(G)^2 / (H + l2), -ThresholdL1(G) / (H + l2)
    L = oracle.lib()
    assert L.oracle_leaf_gain(-3.0, 2.0, 0.0, 1.0) == 3.0
    assert L.oracle_leaf_gain(-3.0, 2.0, 1.0, 0.0) == 2.0
    assert L.oracle_leaf_gain(0.5, 2.0, 1.0, 0.0) == 0.0
    assert L.oracle_leaf_output(-3.0, 2.0, 1.0, 0.0) == 1.0
    assert L.oracle_leaf_output(3.0, 1.0, 0.0, 2.0) == -1.0
    assert L.oracle_leaf_output(0.0, 1.0, 0.0, 0.0) == 0.0
