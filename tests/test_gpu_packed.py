"""Packed slabs on the device. Byte features are laid out in slabs by bin class, and a slab's LDS columns hold
several features each when its bin counts allow (four of at most 64 bins, two of at most 128), so a slab of 256
features takes one histogram launch and a slab of 128 small features a quarter of the LDS and partials. The layout
is the backend's own; the results must stay the oracle's bit for bit: histograms of the whole range and of leaves,
the partition row for row, grown trees and boosted scores, with numerical and categorical features in packed slabs
and beside byte and two-byte slabs.
"""

import numpy as np
import pytest

import oracle
import silvic_amd
from silvic_amd import _abi, bin_split
from tests.helpers import joined
from tests.test_gpu_parity import binary_gradients, boost_both, compare_trees, quantized_setup, say

pytestmark = pytest.mark.gpu


def mixed_bins(rows, seed, small=150, mid=90, full=40, categorical=False, wide=0):
    """`small` features of at most 64 bins, `mid` of at most 128, `full` of up to 255, then `wide` two-byte ones;
    the label is the first part's."""
    data = silvic_amd.synthetic(2, rows=rows, cols=small, seed=seed, max_bin=63, categorical=categorical)
    for cols, max_bin, cfg in ((mid, 127, 2), (full, None, 2), (wide, 1023, 5)):
        if cols:
            part = silvic_amd.synthetic(cfg, rows=rows, cols=cols, seed=seed + cols, max_bin=max_bin)
            label = data.label
            data = joined(data, part)
            data.label = label
    nb = np.array([f.num_bins for f in data.features])
    assert ((nb > 1) & (nb <= 64)).sum() > 0
    assert mid == 0 or ((nb > 64) & (nb <= 128)).sum() > 0
    return data


@pytest.mark.parametrize("rows,kw", [(200_000, {}), (90_000, dict(small=600, mid=0, full=0)),
                                     (120_000, dict(small=300, mid=260, full=10, categorical=True))])
def test_packed_histograms_and_partition_bit_exact(rocm, rows, kw):
    say("packed histogram", rows, kw)
    data = mixed_bins(rows, 3, **kw)
    g, h = binary_gradients(data)
    spec, packed = quantized_setup(rocm, data, g, h, num_bins=16)
    assert rocm.reset_partition() == rows
    root = rocm.histogram((0, rows))
    assert np.array_equal(root, oracle.histogram(data, packed, 16, np.arange(rows, dtype=np.uint32)))
    f = next(i for i, m in enumerate(data.features) if 16 < m.num_bins <= 64)
    meta = data.features[f]
    split = bin_split(meta.group, meta.column, range(0, meta.num_bins // 2))
    left = rocm.partition((0, rows), split)
    o_rows, o_left = oracle.partition(data, np.arange(rows, dtype=np.uint32), split)
    assert left == o_left
    assert np.array_equal(rocm.partition_rows(rows), o_rows)
    for b, c in [(0, left), (left, rows - left), (left + 5, min(3000, rows - left - 5))]:
        assert np.array_equal(rocm.histogram((b, c)), oracle.histogram(data, packed, 16, o_rows[b:b + c])), (b, c)


# a packed slab beside a byte slab; 600 features of at most 64 bins (three packed slabs, 256-, 256- and 128-byte
# rows); categorical features in packed slabs; two-byte features beside a packed slab; 100 features of at most 128
# bins in one slab of 64 columns, two features each
@pytest.mark.parametrize("rows,leaves,kw", [(300_000, 127, {}), (100_000, 63, dict(small=600, mid=0, full=0)),
                                            (150_000, 63, dict(categorical=True)),
                                            (150_000, 127, dict(small=200, mid=0, full=0, wide=12)),
                                            (200_000, 63, dict(small=40, mid=60, full=0))])
def test_packed_grown_tree_matches_the_oracle(rocm, rows, leaves, kw):
    say("packed grow", rows, leaves, kw)
    data = mixed_bins(rows, 7, **kw)
    g, h = binary_gradients(data, 5)
    p = oracle.default_params(num_leaves=leaves)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    spec, _ = quantized_setup(rocm, data, g, h, seed=p.data_random_seed)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d = rocm.grow(p.cfg, p.num_leaves, p.max_depth, spec.grad_scale, spec.hess_scale, mask, (0, n), n)
    compare_trees(d, dict(o_tree), f"packed grow {kw}")
    assert np.array_equal(d["left_bins"], o_tree["left_bins"])
    assert np.array_equal(d["leaf_range"].astype(np.int64), o_ranges)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])


def test_packed_boosting_matches_the_oracle():
    say("packed boost: binary, 63 leaves, bagging and feature fraction, 4 rounds")
    data = mixed_bins(80_000, 11, small=400, mid=100, full=20, categorical=True)
    params = dict(objective=_abi.OBJ_BINARY, num_leaves=63, bagging_fraction=0.8, bagging_freq=1, feature_fraction=0.8)
    o, t = boost_both(data, params, 4)
    assert len(t.trees) == len(o.trees) == 4
    for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
        compare_trees(d, ot, f"tree {i}", exact_values=False)
    assert np.array_equal(t.backend.scores(0), o.scores)
    t.backend.close()


# Dense slabs: when byte features take more than one slab, the backend may stack them in the 128 LDS columns by
# their bin counts instead (fewer columns, so fewer partial words and launches). Each case checks the layout it
# means to exercise, then the results against the oracle: 280 mixed features in one dense slab (3 a column); the
# sparse shape's 2000 features in one (16 a column, 8 passes a row); 2100 in two dense slabs of one launch;
# 800 with categorical features beside a slab of two-byte features; 600 of 64 bins, which do not fit (packed).
def sparse_mixed(rows, seed, cols, wide=0, categorical=False):
    data = silvic_amd.synthetic(4, rows=rows, cols=cols, seed=seed)
    if categorical:
        cat = silvic_amd.synthetic(2, rows=rows, cols=40, seed=seed + 1, max_bin=63, categorical=True)
        data = joined(data, cat)
    if wide:
        label = data.label
        data = joined(data, silvic_amd.synthetic(5, rows=rows, cols=wide, seed=seed + 2, max_bin=1023))
        data.label = label
    return data


DENSE_CASES = [
    ("mixed280", lambda rows: mixed_bins(rows, 7), dict(dense=1, per=3)),
    ("sparse2000", lambda rows: sparse_mixed(rows, 3, 2000), dict(dense=1, per=16)),
    ("sparse2100", lambda rows: sparse_mixed(rows, 4, 2100), dict(dense=2, per=9)),
    ("sparse800+cat+wide", lambda rows: sparse_mixed(rows, 5, 800, wide=8, categorical=True), dict(dense=1, wide=1)),
    ("bins600", lambda rows: mixed_bins(rows, 3, small=600, mid=0, full=0), dict(dense=0)),
]


def check_layout(rocm, want):
    layout = rocm.slab_layout()
    dense = [s for s in layout if s["dense"]]
    assert len(dense) == want["dense"], layout
    if "per" in want:
        assert all(s["row_bytes"] == 128 * want["per"] for s in dense), layout
    if "wide" in want:
        assert sum(s["wide"] for s in layout) == want["wide"], layout
    return layout


@pytest.mark.parametrize("name", [c[0] for c in DENSE_CASES])
def test_dense_histograms_and_partition_bit_exact(rocm, name):
    _, make, want = next(c for c in DENSE_CASES if c[0] == name)
    rows = 60_000
    say("dense histogram", name, rows)
    data = make(rows)
    g, h = binary_gradients(data, 4)
    spec, packed = quantized_setup(rocm, data, g, h, num_bins=16)
    check_layout(rocm, want)
    assert rocm.reset_partition() == rows
    assert np.array_equal(rocm.histogram((0, rows)), oracle.histogram(data, packed, 16, np.arange(rows, dtype=np.uint32)))
    f = next(i for i, m in enumerate(data.features) if m.num_bins > 2 and data.groups[m.group].bin_bits != 16)
    meta = data.features[f]
    split = bin_split(meta.group, meta.column, range(0, meta.num_bins // 2))
    left = rocm.partition((0, rows), split)
    o_rows, o_left = oracle.partition(data, np.arange(rows, dtype=np.uint32), split)
    assert left == o_left
    for b, c in [(0, left), (left, rows - left), (left + 3, min(2000, rows - left - 3))]:
        assert np.array_equal(rocm.histogram((b, c)), oracle.histogram(data, packed, 16, o_rows[b:b + c])), (b, c)


@pytest.mark.parametrize("name", [c[0] for c in DENSE_CASES])
def test_dense_grown_tree_matches_the_oracle(rocm, name):
    _, make, want = next(c for c in DENSE_CASES if c[0] == name)
    rows = 200_000
    say("dense grow", name, rows)
    data = make(rows)
    g, h = binary_gradients(data, 9)
    p = oracle.default_params(num_leaves=63)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    spec, _ = quantized_setup(rocm, data, g, h, seed=p.data_random_seed)
    check_layout(rocm, want)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d = rocm.grow(p.cfg, p.num_leaves, p.max_depth, spec.grad_scale, spec.hess_scale, mask, (0, n), n)
    compare_trees(d, dict(o_tree), f"dense grow {name}")
    assert np.array_equal(d["left_bins"], o_tree["left_bins"])
    assert np.array_equal(d["leaf_range"].astype(np.int64), o_ranges)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])


def test_dense_boosting_matches_the_oracle():
    say("dense boost: the sparse shape at 100k x 2000, 63 leaves, bagging, 4 rounds")
    data = sparse_mixed(100_000, 6, 2000)
    params = dict(objective=_abi.OBJ_BINARY, num_leaves=63, bagging_fraction=0.8, bagging_freq=1)
    o, t = boost_both(data, params, 4)
    assert [s["dense"] for s in t.backend.slab_layout()] == [True]
    for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
        compare_trees(d, ot, f"tree {i}", exact_values=False)
    assert np.array_equal(t.backend.scores(0), o.scores)
    t.backend.close()
