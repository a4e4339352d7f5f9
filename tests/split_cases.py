"""Split-search cases of crates/silvic-core/src/split.rs:987-1507 and an independent brute force over every
candidate (split.rs:1070-1100), shared by the oracle tests and the device parity tests."""

import numpy as np

import oracle
from silvic_amd import _abi
from silvic_amd.dataset import FeatureMeta
from tests.helpers import Lcg

MIN_SCORE = -np.inf


def numerical(num_bins, nan_bin, hist_offset=0):
    return FeatureMeta(num_bins, 0, 0, hist_offset, _abi.BINS_NUMERICAL, nan_bin)


def categorical(num_bins):
    return FeatureMeta(num_bins, 0, 0, 0, _abi.BINS_CATEGORICAL, False)


def config(**kw):
    """split.rs:1040-1045: defaults with min_data_in_leaf 5."""
    base = dict(min_data_in_leaf=5)
    base.update(kw)
    return oracle.split_config(**base)


def random_hist(rng, num_bins, hess_per_row):
    """split.rs:1048-1055."""
    rows = [rng.below(40) for _ in range(num_bins)]
    hist = []
    for n in rows:
        hist += [(rng.next() - 0.45) * n, n * hess_per_row]
    return np.array(hist, np.float64), np.array(rows, np.int64)


def leaf_gain(g, h, l1, l2):
    r = max(abs(g) - l1, 0.0)
    return r * r / (h + l2)


def leaf_output(g, h, l1, l2):
    r = max(abs(g) - l1, 0.0)
    return -np.sign(g) * r / (h + l2)


def sums(hist, rows):
    return float(hist[0::2].sum()), float(hist[1::2].sum()), int(rows.sum())


def side_sums(hist, rows, left):
    idx = [b for b in range(len(rows)) if left(b)]
    return (sum(hist[2 * b] for b in idx), sum(hist[2 * b + 1] for b in idx), sum(int(rows[b]) for b in idx))


def brute_force(hist, rows, cfg, candidates):
    """split.rs:1070-1088: the best gain - shift over every allowed candidate, by direct summation."""
    tg, th, tn = sums(hist, rows)
    shift = leaf_gain(tg, th, cfg.lambda_l1, cfg.lambda_l2) + cfg.min_gain_to_split
    best = MIN_SCORE
    for left in candidates:
        lg, lh, ln = side_sums(hist, rows, left)
        rg, rh, rn = tg - lg, th - lh, tn - ln

        def ok(n, h):
            return n >= cfg.min_data_in_leaf and n > 0 and h >= cfg.min_sum_hessian_in_leaf and h > 0.0

        if not ok(ln, lh) or not ok(rn, rh):
            continue
        gain = leaf_gain(lg, lh, cfg.lambda_l1, cfg.lambda_l2) + leaf_gain(rg, rh, cfg.lambda_l1, cfg.lambda_l2)
        if gain > shift:
            best = max(best, gain - shift)
    return best


def numerical_candidates(num_bins, nan_bin):
    """split.rs:1090-1100."""
    numeric = num_bins - int(nan_bin)
    end = numeric if nan_bin else numeric - 1
    out = []
    for t in range(end):
        for nan_left in (False, True):
            out.append(lambda b, t=t, nl=nan_left: nl if b == numeric else b <= t)
    return out


def close(found, expected):
    return abs(found - expected) <= 1e-9 * max(abs(expected), 1.0)


def goes_left(split, meta, num_bins):
    if split.categorical if hasattr(split, "categorical") else False:
        bins = set(split.cat_bins[i] for i in range(split.num_cat_bins))
        return lambda b: b in bins
    nan = meta.nan_bin
    return lambda b: bool(split.default_left) if (nan and b == num_bins - 1) else b <= split.threshold


def numerical_cases():
    """The 400 cases of split.rs:1150-1179: (name, hist, rows, meta, cfg)."""
    rng = Lcg(7)
    out = []
    for case in range(400):
        nan_bin = case % 2 == 1
        num_bins = 2 + rng.below(30)
        hist, rows = random_hist(rng, num_bins, 0.25)
        cfg = config(lambda_l1=0.5 if case % 3 == 0 else 0.0, lambda_l2=2.0 if case % 5 == 0 else 0.0)
        out.append((f"case {case} bins {num_bins} nan {nan_bin}", hist, rows, numerical(num_bins, nan_bin), cfg))
    return out


def quantized_cases():
    """split.rs:1181-1232: integer units with real scales 0.37 / 0.125."""
    rng = Lcg(11)
    out = []
    for case in range(100):
        num_bins = 3 + rng.below(20)
        rows = np.array([rng.below(40) for _ in range(num_bins)], np.int64)
        units = []
        for n in rows:
            units += [rng.below(9) - 4.0, 2.0 * n]
        out.append((case, np.array(units, np.float64), rows, numerical(num_bins, case % 2 == 0)))
    return out


def categorical_cases():
    """split.rs:1252-1349 one-hot and sorted categorical cases, sorted cases under the default categorical
    parameters with larger bins, and split.rs:1414-1471's zero-hessian bins with cat_smooth 0 (a 0/0 ratio):
    (name, hist, rows, meta, cfg)."""
    out = []
    rng = Lcg(3)
    for case in range(200):
        num_bins = 2 + rng.below(3)
        hist, rows = random_hist(rng, num_bins, 1.0)
        out.append((f"one-hot {case}", hist, rows, categorical(num_bins), config()))
    rng = Lcg(5)
    for case in range(200):
        num_bins = 6 + rng.below(12)
        hist, rows = random_hist(rng, num_bins, 1.0)
        cfg = config(min_data_per_group=1, cat_smooth=1.0, max_cat_threshold=4)
        out.append((f"sorted {case}", hist, rows, categorical(num_bins), cfg))
    rng = Lcg(13)
    for case in range(100):
        num_bins = 20 + rng.below(200)
        rows = np.array([rng.below(300) for _ in range(num_bins)], np.int64)
        hist = []
        for n in rows:
            hist += [(rng.next() - 0.45) * n, n * 1.0]
        out.append((f"sorted default {case}", np.array(hist, np.float64), rows, categorical(num_bins), config()))
    zero = np.array([0.0, 0.0, -3.0, 2.0, 0.0, 0.0, 4.0, 2.0, 0.0, 0.0, 1.0, 1.0, 0.0, 0.0, 0.0, 0.0])
    for nb in (3, 8):
        h = zero[: 2 * nb]
        cfg = config(min_data_in_leaf=0, min_sum_hessian_in_leaf=0.0, min_data_per_group=0, cat_smooth=0.0)
        out.append((f"zero hessian {nb}", h, h[1::2].astype(np.int64), categorical(nb), cfg))
    return out


def wide_numerical_cases(count=40):
    """Numerical features of 257..1024 bins (2-byte bins, an extension the reference does not have), generated as
    the cases above: (name, hist, rows, meta, cfg)."""
    rng = Lcg(19)
    out = []
    for case in range(count):
        nan_bin = case % 2 == 1
        num_bins = 257 + rng.below(768)
        hist, rows = random_hist(rng, num_bins, 0.25)
        cfg = config(lambda_l1=0.5 if case % 3 == 0 else 0.0, lambda_l2=2.0 if case % 5 == 0 else 0.0)
        out.append((f"wide case {case} bins {num_bins} nan {nan_bin}", hist, rows, numerical(num_bins, nan_bin), cfg))
    return out


def brute_force_numerical(hist, rows, cfg, nan_bin):
    """brute_force over numerical_candidates with the sides' sums from cumulative sums (the candidates of a
    1000-bin feature are too many for the direct loop)."""
    num_bins = len(rows)
    numeric = num_bins - int(nan_bin)
    g, h, n = hist[0::2], hist[1::2], rows.astype(np.int64)
    tg, th, tn = float(g.sum()), float(h.sum()), int(n.sum())
    shift = leaf_gain(tg, th, cfg.lambda_l1, cfg.lambda_l2) + cfg.min_gain_to_split
    end = numeric if nan_bin else numeric - 1
    cg, ch, cn = np.cumsum(g[:numeric]), np.cumsum(h[:numeric]), np.cumsum(n[:numeric])
    best = MIN_SCORE
    for t in range(end):
        for nan_left in (False, True):
            lg, lh, ln = float(cg[t]), float(ch[t]), int(cn[t])
            if nan_left and nan_bin:
                lg, lh, ln = lg + g[numeric], lh + h[numeric], ln + int(n[numeric])
            rg, rh, rn = tg - lg, th - lh, tn - ln
            if not (ln >= cfg.min_data_in_leaf and ln > 0 and lh >= cfg.min_sum_hessian_in_leaf and lh > 0.0):
                continue
            if not (rn >= cfg.min_data_in_leaf and rn > 0 and rh >= cfg.min_sum_hessian_in_leaf and rh > 0.0):
                continue
            gain = leaf_gain(lg, lh, cfg.lambda_l1, cfg.lambda_l2) + leaf_gain(rg, rh, cfg.lambda_l1, cfg.lambda_l2)
            if gain > shift:
                best = max(best, gain - shift)
    return best
