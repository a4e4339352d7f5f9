"""The oracle's 2-byte bins, an extension silvic does not have (it rejects max_bin > 255, config.rs:407-412), so
these pin the extension by closed forms only: histograms against direct sums, the stable partition by its
numerical rule, the split search over up to 1024 bins against a brute force, and grown trees whose rules send
every row to the leaf holding it."""

import ctypes as C

import numpy as np

import oracle
import silvic_amd
from silvic_amd import _abi
from tests.helpers import naive_histogram
from tests.split_cases import (MIN_SCORE, brute_force_numerical, close, sums, wide_numerical_cases)


def wide_data(rows=30_000, cols=12, seed=5):
    data = silvic_amd.synthetic(5, rows=rows, cols=cols, seed=seed, max_bin=1023)
    assert all(g.bin_bits == 16 for g in data.groups)
    assert max(f.num_bins for f in data.features) > 256
    return data


def test_wide_histogram_matches_direct_sums():
    data = wide_data()
    rng = np.random.default_rng(1)
    g = (rng.standard_normal(data.num_rows)).astype(np.float32)
    h = rng.uniform(0.1, 1.0, data.num_rows).astype(np.float32)
    spec = oracle.quant_spec(float(np.abs(g).max()), float(h.max()), None, 16, True, 3, 0)
    packed = oracle.quantize(spec, g, h)
    gq, hq = oracle.unpack(packed)
    rows = np.sort(rng.choice(data.num_rows, 9_000, replace=False)).astype(np.uint32)
    got = oracle.histogram(data, packed, 16, rows)
    want = naive_histogram(data, rows, gq[rows], hq[rows])
    assert np.array_equal(got, want)


def test_wide_partition_follows_the_numerical_rule():
    data = wide_data(rows=10_000)
    f = 3
    meta = data.features[f]
    bins = data.bin(f)
    rows = np.arange(data.num_rows, dtype=np.uint32)[::3].copy()
    for thr, nan_left in ((600, False), (40, True), (meta.num_bins - 2, True)):
        words = [thr, meta.num_bins if (nan_left and meta.nan_bin) else 0] + [0] * 6
        split = _abi.BinSplit(meta.group, meta.column, (C.c_uint32 * 8)(*words))
        out, left = oracle.partition(data, rows, split)
        b = bins[rows]
        goes = (b <= thr) | (nan_left and meta.nan_bin and (b == meta.num_bins - 1))
        assert left == int(goes.sum())
        assert np.array_equal(out[:left], rows[goes]) and np.array_equal(out[left:], rows[~goes])


def test_wide_split_matches_brute_force():
    for name, hist, rows, meta, cfg in wide_numerical_cases():
        best, _ = oracle.find_best_split(hist, [meta], [1], sums(hist, rows), 1.0, 1.0, cfg)
        expected = brute_force_numerical(hist, rows, cfg, meta.nan_bin)
        if not best.found:
            assert expected == MIN_SCORE, name
        else:
            assert close(best.gain, expected), (name, best.gain, expected)
            assert best.threshold < meta.num_bins


def test_wide_trees_send_every_row_to_its_leaf():
    data = wide_data(rows=40_000, cols=10, seed=7)
    rng = np.random.default_rng(3)
    g = (data.label - data.label.mean() + rng.standard_normal(data.num_rows) * 0.1).astype(np.float32)
    tree, ranges, part = oracle.grow_tree(data, g, np.ones_like(g), oracle.default_params(num_leaves=63))
    assert tree["num_leaves"] == 63 and tree["threshold_bin"].max() > 255
    leaf_of = np.empty(data.num_rows, np.int64)
    for leaf, (b, c) in enumerate(ranges):
        leaf_of[part[b:b + c]] = leaf
        rows = part[b:b + c]
        G, H = g[rows].astype(np.float64).sum(), float(c)
        assert abs(tree["leaf_value"][leaf] - (-G / H)) <= 1e-6 * max(abs(G / H), 1.0)
    bins = np.stack([data.bin(f) for f in range(len(data.features))], 1).astype(np.int64)
    words = tree["left_bins"]
    for n, f in enumerate(tree["split_feature"]):
        meta = data.features[f]
        assert words[n][0] == tree["threshold_bin"][n] and not words[n][2:].any()
        nan_left = bool(tree["decision_type"][n] & 2) and meta.nan_bin
        assert words[n][1] == (meta.num_bins if nan_left else 0)
    node = np.zeros(data.num_rows, np.int64)
    active = np.ones(data.num_rows, bool)
    while active.any():
        idx = np.flatnonzero(active)
        nd = node[idx]
        f = tree["split_feature"][nd]
        b = bins[idx, f]
        w = words[nd]
        left = (b <= w[:, 0]) | ((w[:, 1] != 0) & (b == w[:, 1].astype(np.int64) - 1))
        node[idx] = np.where(left, tree["left_child"][nd], tree["right_child"][nd])
        active[idx] = node[idx] >= 0
    assert np.array_equal(~node, leaf_of)
