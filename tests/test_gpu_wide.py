"""Two-byte bins (max_bin up to 1023) on the device, against the oracle's restatement of them.

silvic rejects max_bin > 255 (config.rs:407-412), so these bins are an extension of the reference: the oracle's
handling of them is pinned by closed forms only (direct sums, the numerical rule, a brute-force split search). Here
the device must match that oracle bit for bit, as for one-byte bins: histograms, the partition row for row, split
search, grown trees and boosted scores.
"""

import numpy as np
import pytest

import oracle
import silvic_amd
from silvic_amd import bin_split, wide_bin_split
from tests.helpers import joined
from tests.split_cases import wide_numerical_cases
from tests.test_gpu_parity import (binary_gradients, boost_both, compare_split, compare_trees, quantized_setup, say)

pytestmark = pytest.mark.gpu


def wide_data(rows, cols, seed):
    data = silvic_amd.synthetic(5, rows=rows, cols=cols, seed=seed, max_bin=1023)
    assert all(g.bin_bits == 16 for g in data.groups)
    assert max(f.num_bins for f in data.features) > 256
    return data


def wide_rule(meta, threshold, nan_left):
    """A numerical rule on a two-byte feature: bins <= threshold, and the NaN bin when `nan_left`."""
    return wide_bin_split(meta.group, meta.column, threshold, meta.num_bins - 1 if nan_left and meta.nan_bin else None)


def regression_gradients(data, seed):
    rng = np.random.default_rng(seed)
    g = (data.label - data.label.mean() + rng.standard_normal(data.num_rows) * 0.1).astype(np.float32)
    return g, np.ones_like(g)


# 32 two-byte features (one slab of 128 columns); 9 (a 64-column slab); 12 byte features beside 20 two-byte ones
@pytest.mark.parametrize("rows,cols,mixed", [(300_000, 32, False), (120_000, 9, False), (200_000, 20, True)])
def test_wide_histograms_and_partition_bit_exact(rocm, rows, cols, mixed):
    say("wide histogram", rows, cols, mixed)
    data = wide_data(rows, cols, 11)
    if mixed:
        data = joined(silvic_amd.synthetic(2, rows=rows, cols=12, seed=4), data)
    g, h = binary_gradients(data)
    spec, packed = quantized_setup(rocm, data, g, h, num_bins=16)
    assert rocm.reset_partition() == rows
    root = rocm.histogram((0, rows))
    assert np.array_equal(root, oracle.histogram(data, packed, 16, np.arange(rows, dtype=np.uint32)))
    f = len(data.features) - 3
    meta = data.features[f]
    assert meta.num_bins > 256
    for thr, nan_left in ((meta.num_bins // 3, True), (700, False)):
        rocm.reset_partition()
        split = wide_rule(meta, thr, nan_left)
        left = rocm.partition((0, rows), split)
        o_rows, o_left = oracle.partition(data, np.arange(rows, dtype=np.uint32), split)
        assert left == o_left
        assert np.array_equal(rocm.partition_rows(rows), o_rows)
        for b, c in [(0, left), (left, rows - left), (left + 7, min(5000, rows - left - 7))]:
            assert np.array_equal(rocm.histogram((b, c)), oracle.histogram(data, packed, 16, o_rows[b:b + c])), (b, c)
    # a byte feature's rule in the mixed dataset still reads the (two-byte) column-major bins
    if mixed:
        m0 = data.features[2]
        rocm.reset_partition()
        split = bin_split(m0.group, m0.column, range(0, m0.num_bins // 2))
        left = rocm.partition((0, rows), split)
        o_rows, o_left = oracle.partition(data, np.arange(rows, dtype=np.uint32), split)
        assert left == o_left and np.array_equal(rocm.partition_rows(rows), o_rows)


def test_wide_split_search_matches_the_oracle(rocm):
    say("wide split search: 40 cases of 257..1024 bins")
    for name, hist, rows, meta, cfg in wide_numerical_cases():
        units = np.round(hist * 64.0)
        s = (units[0::2].sum(), units[1::2].sum(), int(rows.sum()))
        o, ospl = oracle.find_best_split(units, [meta], [1], s, 1.0 / 64, 1.0 / 64, cfg)
        d, dspl = rocm.find_best_split(units, [meta], [1], s, 1.0 / 64, 1.0 / 64, cfg)
        compare_split(d, o, name)
        assert np.array_equal(dspl, ospl), name


@pytest.mark.parametrize("rows,cols,leaves,mixed", [(400_000, 32, 255, False), (2_000_000, 32, 2047, False),
                                                    (300_000, 20, 127, True)])
def test_wide_grown_tree_matches_the_oracle(rocm, rows, cols, leaves, mixed):
    say("wide grow", rows, cols, leaves, mixed)
    data = wide_data(rows, cols, 3)
    if mixed:  # byte features first, the target still the two-byte features'
        wide = data
        data = joined(silvic_amd.synthetic(2, rows=rows, cols=12, seed=6), wide)
        data.label = wide.label
    g, h = regression_gradients(data, 8)
    p = oracle.default_params(num_leaves=leaves, min_data_in_leaf=20)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    assert o_tree["num_leaves"] == leaves and o_tree["threshold_bin"].max() > 255
    spec, _ = quantized_setup(rocm, data, g, h, seed=p.data_random_seed)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d = rocm.grow(p.cfg, p.num_leaves, p.max_depth, spec.grad_scale, spec.hess_scale, mask, (0, n), n)
    compare_trees(d, dict(o_tree), f"wide grow {leaves}")
    assert np.array_equal(d["left_bins"], o_tree["left_bins"])
    assert np.array_equal(d["leaf_range"].astype(np.int64), o_ranges)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])


# the 50M x 32, max_bin 1023, 2047-leaf regression shape at 2M rows; and a validation set scored by the row walk
def test_wide_boosting_matches_the_oracle():
    say("wide boost 2047 leaves")
    data = wide_data(2_000_000, 32, 4)
    o, t = boost_both(data, dict(num_leaves=2047), 3)
    assert len(t.trees) == len(o.trees) == 3
    for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
        assert ot["num_leaves"] == 2047
        compare_trees(d, ot, f"tree {i}", exact_values=False)
    assert np.array_equal(t.backend.scores(0), o.scores)
    t.backend.close()
