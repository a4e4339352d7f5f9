"""Quantization wider than the reference's num_grad_quant_bins <= 64 (config.rs:416-421), up to 16-bit units
(32766 bins: g_q within +-16383, h_q at most 32766), on the device against the oracle.

Above 127 gradient or 255 hessian units the packed 16/16 LDS words would be flushed every few rows, so the backend
accumulates separate 32-bit g and h counters instead, in slabs of at most 64 columns that it lays out again on the
device when the mode changes. The reference has no such units, so the oracle's side is pinned by closed forms only
(tests/test_oracle_quantize.py); here the device must equal the oracle bit for bit: histograms, the partition row
for row, grown trees and boosted scores, across mode switches in one context.
"""

import numpy as np
import pytest

import oracle
import silvic_amd
from silvic_amd import _abi, bin_split
from tests.helpers import joined
from tests.test_gpu_parity import binary_gradients, boost_both, compare_trees, quantized_setup, say

pytestmark = pytest.mark.gpu


def check_histograms(rocm, data, g, h, bins, seed):
    """Quantizes at `bins`, then the root and both children of a split, against the oracle."""
    rows = data.num_rows
    spec, packed = quantized_setup(rocm, data, g, h, seed=seed, num_bins=bins)
    mq = max(spec.grad_max_q, spec.hess_max_q)
    assert rocm.reset_partition() == rows
    assert np.array_equal(rocm.histogram((0, rows)), oracle.histogram(data, packed, mq, np.arange(rows, dtype=np.uint32)))
    meta = data.features[3]
    split = bin_split(meta.group, meta.column, range(0, meta.num_bins // 3))
    left = rocm.partition((0, rows), split)
    o_rows, o_left = oracle.partition(data, np.arange(rows, dtype=np.uint32), split)
    assert left == o_left
    assert np.array_equal(rocm.partition_rows(rows), o_rows)
    for b, c in [(0, left), (left, rows - left), (left + 9, min(4000, rows - left - 9))]:
        assert np.array_equal(rocm.histogram((b, c)), oracle.histogram(data, packed, mq, o_rows[b:b + c])), (bins, b, c)


# 100 byte features (two 64-column slabs with separate counters, one 128-column slab packed); 20 two-byte features
# beside 12 byte ones. Each case switches the mode three times in one context.
@pytest.mark.parametrize("kind", ["bytes", "mixed"])
def test_sixteen_bit_unit_histograms_bit_exact(rocm, kind):
    say("16-bit units histogram", kind)
    rows = 200_000
    if kind == "bytes":
        data = silvic_amd.synthetic(2, rows=rows, cols=100, seed=12, categorical=True)
    else:
        wide = silvic_amd.synthetic(5, rows=rows, cols=20, seed=12, max_bin=1023)
        data = joined(silvic_amd.synthetic(2, rows=rows, cols=12, seed=13), wide)
    g, h = binary_gradients(data, 2)
    for bins, seed in ((32766, 1), (4, 2), (1024, 3), (256, 4)):
        check_histograms(rocm, data, g, h, bins, seed)


@pytest.mark.parametrize("rows,cols,leaves,bins", [(300_000, 100, 127, 1024), (200_000, 40, 255, 32766),
                                                   (700_000, 16, 63, 32766)])
def test_sixteen_bit_unit_grown_tree_matches_the_oracle(rocm, rows, cols, leaves, bins):
    say("16-bit units grow", rows, cols, leaves, bins)
    data = silvic_amd.synthetic(2, rows=rows, cols=cols, seed=31)
    g, h = binary_gradients(data, 6)
    p = oracle.default_params(num_leaves=leaves, num_grad_quant_bins=bins)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    spec, _ = quantized_setup(rocm, data, g, h, seed=p.data_random_seed, num_bins=bins)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d = rocm.grow(p.cfg, leaves, -1, spec.grad_scale, spec.hess_scale, mask, (0, n), n)
    compare_trees(d, dict(o_tree), f"grow at {bins} bins")
    assert np.array_equal(d["leaf_range"].astype(np.int64), o_ranges)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])


@pytest.mark.parametrize("config,rows,cols,params,rounds", [
    (2, 150_000, 64, dict(objective=_abi.OBJ_BINARY, num_leaves=63, num_grad_quant_bins=256), 5),
    (2, 150_000, 64, dict(objective=_abi.OBJ_BINARY, num_leaves=63, num_grad_quant_bins=32766), 5),
    (2, 150_000, 64, dict(objective=_abi.OBJ_BINARY, num_leaves=63, num_grad_quant_bins=4096,
                          quant_train_renew_leaf=0, bagging_fraction=0.7, bagging_freq=1), 5),
    (2, 120_000, 28, dict(objective=_abi.OBJ_BINARY, num_leaves=63, num_grad_quant_bins=32766, categorical=True), 4),
    # config 5's shape with 16-bit units: two-byte bins and gradients
    (5, 400_000, 32, dict(num_leaves=255, num_grad_quant_bins=32766), 3),
    (1, 100_000, 28, dict(num_leaves=31, weighted=True, num_grad_quant_bins=2048), 5),
])
def test_sixteen_bit_unit_boosting_matches_the_oracle(config, rows, cols, params, rounds):
    say("16-bit units boost", config, rows, cols, params, rounds)
    params = dict(params)
    categorical = bool(params.pop("categorical", False))
    weighted = bool(params.pop("weighted", False))
    kw = dict(max_bin=1023) if config == 5 else {}
    data = silvic_amd.synthetic(config, rows=rows, cols=cols, seed=17, categorical=categorical, **kw)
    if weighted:
        data.weight = np.random.default_rng(8).uniform(0.2, 3.0, rows).astype(np.float32)
    o, t = boost_both(data, params, rounds)
    assert len(t.trees) == len(o.trees) == rounds
    for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
        compare_trees(d, ot, f"tree {i}", exact_values=False)
    assert np.array_equal(t.backend.scores(0), o.scores)
    t.backend.close()


# 20M rows at 16-bit units: one workgroup per compute unit would add up 78k rows, past (2^31 - 1) / 32766, so the
# histogram and split-step workgroups are spread wider; the tree and the partition must still be the oracle's
def test_sixteen_bit_units_over_many_rows_spread_the_workgroups(rocm):
    say("16-bit units, 20M rows x 8 two-byte features, 63 leaves")
    rows, bins = 20_000_000, 32766
    data = silvic_amd.synthetic(5, rows=rows, cols=8, seed=41, max_bin=1023)
    rng = np.random.default_rng(2)
    g = (data.label - data.label.mean() + rng.standard_normal(rows) * 0.1).astype(np.float32)
    h = np.ones_like(g)
    p = oracle.default_params(num_leaves=63, num_grad_quant_bins=bins)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    spec, _ = quantized_setup(rocm, data, g, h, seed=p.data_random_seed, num_bins=bins)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d = rocm.grow(p.cfg, 63, -1, spec.grad_scale, spec.hess_scale, mask, (0, n), n)
    compare_trees(d, dict(o_tree), "grow over 20M rows at 16-bit units")
    assert np.array_equal(d["leaf_range"].astype(np.int64), o_ranges)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])
