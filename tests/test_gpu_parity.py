"""Parity of the HIP backend with the oracle, through the C ABI, on an MI355X.

Integer work (quantization, histograms, partitions, leaf sums) must match bit for bit; split decisions, tree
arrays and leaf values must be identical; scores must agree within 1e-6 relative (the f32 adds are the same, so
they match exactly in practice). Every test prints the case it runs before touching the GPU.
"""

import ctypes as C

import numpy as np
import pytest

import oracle
import silvic_amd
from silvic_amd import _abi, bin_split, device_node
from tests.helpers import cpu_dataset, cpu_gradients, learner_dataset, learner_gradients, mirrored, row_slice
from tests.split_cases import categorical_cases, config, numerical_cases, quantized_cases, sums

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def quantized_setup(rocm, data, grad, hess, seed=1, iteration=0, num_bins=4):
    """Loads `data`, hands both sides the same gradients and quantizes them; returns (spec, oracle packed)."""
    rocm.load(data)
    mg, mh = rocm.set_gradients(grad, hess)
    assert mg == float(np.abs(grad).max()) and mh == float(np.abs(hess).max())
    spec = oracle.quant_spec(mg, mh, None, num_bins, True, seed, iteration)
    rocm.quantize(spec)
    packed = oracle.quantize(spec, grad, hess, data.row_offset)
    return spec, packed


def binary_gradients(data, seed=0):
    rng = np.random.default_rng(seed)
    scores = (rng.standard_normal(data.num_rows) * 0.5).astype(np.float32)
    g, h, _, _ = oracle.gradients(_abi.OBJ_BINARY, scores, data.label)
    return g, h


@pytest.mark.parametrize("rows,cols", [(5_000, 28), (300_000, 128), (120_000, 136)])
def test_root_and_leaf_histograms_bit_exact(rocm, rows, cols):
    say("histogram", rows, cols)
    data = silvic_amd.synthetic(2, rows=rows, cols=cols, seed=11)
    g, h = binary_gradients(data)
    spec, packed = quantized_setup(rocm, data, g, h)
    n = rocm.reset_partition()
    assert n == rows
    root = rocm.histogram((0, rows))
    expected = oracle.histogram(data, packed, 4, np.arange(rows, dtype=np.uint32))
    assert np.array_equal(root, expected)
    # a leaf: partition the root on a feature, then both children and sub-ranges (which pin the row order)
    f = 5
    meta = data.features[f]
    split = bin_split(meta.group, meta.column, list(range(0, meta.num_bins // 2)) + [meta.num_bins - 1])
    left = rocm.partition((0, rows), split)
    o_rows, o_left = oracle.partition(data, np.arange(rows, dtype=np.uint32), split)
    assert left == o_left
    for b, c in [(0, left), (left, rows - left), (0, min(777, left)), (left + 13, min(1000, rows - left - 13))]:
        got = rocm.histogram((b, c))
        want = oracle.histogram(data, packed, 4, o_rows[b:b + c])
        assert np.array_equal(got, want), (b, c)


def test_partition_and_histogram_fused(rocm):
    say("partition_and_histogram")
    data = silvic_amd.synthetic(2, rows=200_000, cols=64, seed=3)
    g, h = binary_gradients(data, 1)
    spec, packed = quantized_setup(rocm, data, g, h)
    rocm.reset_partition()
    meta = data.features[40]
    split = bin_split(meta.group, meta.column, range(0, 100))
    o_rows, o_left = oracle.partition(data, np.arange(200_000, dtype=np.uint32), split)
    for side in (0, 1):
        rocm.reset_partition()
        left, hist = rocm.partition_and_histogram((0, 200_000), split, side)
        assert left == o_left
        b, c = (0, o_left) if side == 0 else (o_left, 200_000 - o_left)
        assert np.array_equal(hist, oracle.histogram(data, packed, 4, o_rows[b:b + c]))


def test_bagged_partition_is_ascending_and_exact(rocm):
    say("bagging")
    data = silvic_amd.synthetic(2, rows=100_000, cols=32, seed=5)
    g, h = binary_gradients(data, 2)
    spec, packed = quantized_setup(rocm, data, g, h)
    bag = _abi.Bag(_abi.BAG_BERNOULLI, 4, 1, 0, 0.7)
    n = rocm.reset_partition(bag)
    rows = np.array([r for r in range(100_000) if oracle.lib().oracle_in_bag(4, 1, r, 0.7)], np.uint32)
    assert n == len(rows)
    for b, c in [(0, n), (0, 1000), (n - 500, 500)]:
        assert np.array_equal(rocm.histogram((b, c)), oracle.histogram(data, packed, 4, rows[b:b + c]))


def test_reference_backend_cases(rocm):
    # cpu.rs:1014-1179 on the device: histograms over a bag, stable partition, add_tree, leaf sums
    say("cpu.rs cases")
    data = cpu_dataset(50_000)
    grad, hess = cpu_gradients(50_000)
    rocm.load(data)
    rocm.set_gradients(grad, hess)
    spec = oracle.quant_spec(1.5, 0.75, None, 16, True, 9, 3)
    rocm.quantize(spec)
    packed = oracle.quantize(spec, grad, hess, data.row_offset)
    n = rocm.reset_partition(_abi.Bag(_abi.BAG_BERNOULLI, 4, 1, 0, 0.7))
    part = np.array([r for r in range(50_000) if oracle.lib().oracle_in_bag(4, 1, 100 + r, 0.7)], np.uint32)
    assert n == len(part)
    got = rocm.histogram((1000, 30_000))
    assert np.array_equal(got, oracle.histogram(data, packed, 16, part[1000:31_000]))
    rocm.reset_partition()
    split = bin_split(0, 0, [1, 2, 4])
    left = rocm.partition((500, 25_000), split)
    o_rows, o_left = oracle.partition(data, np.arange(500, 25_500, dtype=np.uint32), split)
    assert left == o_left
    sums = rocm.leaf_sums([(500, left), (500 + left, 25_000 - left)], 1024.0, 256.0)
    full = np.arange(50_000, dtype=np.uint32)
    full[500:25_500] = o_rows
    want = oracle.leaf_sums(grad, hess, full, [(500, left), (500 + left, 25_000 - left)], 1024.0, 256.0)
    assert np.array_equal(sums, want)
    tsplit = bin_split(1, 0, [0, 1])
    rocm.init_scores(0, 1.0)
    rocm.add_tree([device_node(tsplit, ~0, ~1)], [0.5, -0.25])
    assert np.array_equal(rocm.scores(0), np.where(data.bin(2) < 2, 1.5, 0.75).astype(np.float32))


def test_binary_gradients_are_the_oracles_bit_for_bit(rocm):
    # objective/binary.rs:27-50 on the device (exp restated bit-exactly) vs the oracle (C library exp)
    say("binary gradients")
    data = silvic_amd.synthetic(2, rows=400_000, cols=16, seed=17)
    rocm.load(data, objective=_abi.OBJ_BINARY, sigmoid=1.0)
    # diverse scores: a 255-leaf tree with leaf values over [-40, 40] on top of a constant
    rocm.init_scores(0, 0.3)
    rng = np.random.default_rng(5)
    nodes = []
    for k in range(127):
        meta = data.features[k % 16]
        left = 2 * k + 1 if 2 * k + 1 < 127 else ~(2 * k + 1 - 127)
        right = 2 * k + 2 if 2 * k + 2 < 127 else ~(2 * k + 2 - 127)
        nodes.append(device_node(bin_split(meta.group, meta.column, range(int(rng.integers(1, meta.num_bins)))),
                                 left, right))
    leaf_values = (rng.uniform(-40, 40, 128)).astype(np.float32)
    rocm.add_tree(nodes, leaf_values)
    scores = rocm.scores(0)
    assert len(np.unique(scores)) > 50
    mg, mh = rocm.compute_gradients()
    g, h = rocm.gradients()
    og, oh, omg, omh = oracle.gradients(_abi.OBJ_BINARY, scores, data.label, sigmoid=1.0)
    assert np.array_equal(g.view(np.uint32), og.view(np.uint32))
    assert np.array_equal(h.view(np.uint32), oh.view(np.uint32))
    assert (mg, mh) == (omg, omh)
    for sig in (0.5, 2.0):
        rocm.load(data, objective=_abi.OBJ_BINARY, sigmoid=sig)
        rocm.init_scores(0, 0.0)
        rocm.add_tree(nodes, leaf_values)
        rocm.compute_gradients()
        g, h = rocm.gradients()
        og, oh, _, _ = oracle.gradients(_abi.OBJ_BINARY, rocm.scores(0), data.label, sigmoid=sig)
        assert np.array_equal(g.view(np.uint32), og.view(np.uint32)), sig
        assert np.array_equal(h.view(np.uint32), oh.view(np.uint32)), sig


def test_regression_gradients_are_exact(rocm):
    say("regression gradients")
    data = silvic_amd.synthetic(1, rows=100_000, seed=3)
    rocm.load(data)
    rocm.init_scores(0, 0.25)
    mg, mh = rocm.compute_gradients()
    g, h = rocm.gradients()
    og, oh, omg, omh = oracle.gradients(_abi.OBJ_REGRESSION, np.full(100_000, 0.25, np.float32), data.label)
    assert np.array_equal(g, og) and np.array_equal(h, oh) and (mg, mh) == (omg, omh)


def test_errors_are_reported_not_crashes(rocm):
    say("errors")
    data = cpu_dataset(1000)
    rocm.load(data)
    g, h = cpu_gradients(1000)
    rocm.set_gradients(g, h)
    rocm.quantize(oracle.quant_spec(1.0, 1.0, None, 4, True, 1, 0))
    rocm.reset_partition()
    with pytest.raises(_abi.DeviceError):
        rocm.histogram((900, 200))
    with pytest.raises(_abi.SilvicError) as e:
        rocm.histogram((0, 10), quantized=False)
    assert e.value.kind == "unsupported"
    with pytest.raises(_abi.DeviceError):
        rocm.add_tree([device_node(bin_split(0, 0, [0]), 0, ~1)], [0.0, 1.0])
    with pytest.raises(_abi.DeviceError):
        rocm.partition((0, 10), bin_split(7, 0, [0]))
    assert rocm.histogram((0, 0)).sum() == 0


def compare_split(d, o, name):
    assert bool(d.found) == bool(o.found), name
    if not o.found:
        return
    assert d.feature == o.feature, name
    assert (d.threshold, d.default_left) == (o.threshold, o.default_left), name
    assert d.gain == o.gain, (name, d.gain, o.gain)
    for side in ("left", "right"):
        ds, os_ = getattr(d, side), getattr(o, side)
        assert (ds.grad, ds.hess, ds.count) == (os_.grad, os_.hess, os_.count), (name, side)
    assert d.left_output == o.left_output and d.right_output == o.right_output, name
    assert bool(d.categorical) == bool(o.categorical), name
    if o.categorical:
        assert d.num_cat_bins == o.num_cat_bins, name
        assert list(d.cat_bins[: d.num_cat_bins]) == list(o.cat_bins[: o.num_cat_bins]), name


def test_categorical_split_search_matches_the_oracle_bit_for_bit(rocm):
    say("split search: one-hot, sorted and zero-hessian categorical cases")
    for name, hist, rows, meta, cfg in categorical_cases():
        units = np.round(hist * 64.0)
        s = (units[0::2].sum(), units[1::2].sum(), int(rows.sum()))
        o, ospl = oracle.find_best_split(units, [meta], [1], s, 1.0 / 64, 1.0 / 64, cfg)
        d, dspl = rocm.find_best_split(units, [meta], [1], s, 1.0 / 64, 1.0 / 64, cfg)
        compare_split(d, o, name)
        assert np.array_equal(dspl, ospl), name


def test_split_search_matches_the_oracle_bit_for_bit(rocm):
    say("split search: 400 numerical cases")
    for name, hist, rows, meta, cfg in numerical_cases():
        s = sums(hist, rows)
        # histograms hold integer units on the device path: scale the reference's real-valued cases
        units = np.round(hist * 64.0)
        s = (units[0::2].sum(), units[1::2].sum(), s[2])
        o, ospl = oracle.find_best_split(units, [meta], [1], s, 1.0 / 64, 1.0 / 64, cfg)
        d, dspl = rocm.find_best_split(units, [meta], [1], s, 1.0 / 64, 1.0 / 64, cfg)
        compare_split(d, o, name)
        assert np.array_equal(dspl, ospl), name
    say("split search: quantized-scale cases")
    for case, units, rows, meta in quantized_cases():
        s = (units[0::2].sum(), units[1::2].sum(), int(rows.sum()))
        o, _ = oracle.find_best_split(units, [meta], [1], s, 0.37, 0.125, config())
        d, _ = rocm.find_best_split(units, [meta], [1], s, 0.37, 0.125, config())
        compare_split(d, o, case)


def test_split_search_over_a_real_histogram(rocm):
    say("split search on a config-2 histogram")
    data = silvic_amd.synthetic(2, rows=200_000, cols=128, seed=9)
    g, h = binary_gradients(data, 4)
    spec, packed = quantized_setup(rocm, data, g, h)
    hist = oracle.histogram(data, packed, 4, np.arange(200_000, dtype=np.uint32))
    f0 = data.features[0]
    s = (hist[2 * f0.hist_offset:2 * (f0.hist_offset + f0.num_bins):2].sum(),
         hist[2 * f0.hist_offset + 1:2 * (f0.hist_offset + f0.num_bins):2].sum(), 200_000)
    for ev_seed in range(4):
        ev = np.random.default_rng(ev_seed).random(len(data.features)) < (1.0 if ev_seed == 0 else 0.5)
        for kw in ({}, dict(lambda_l1=0.5, lambda_l2=2.0), dict(min_data_in_leaf=5000)):
            cfg = oracle.split_config(**kw)
            o, ospl = oracle.find_best_split(hist, data.features, ev, s, spec.grad_scale, spec.hess_scale, cfg)
            d, dspl = rocm.find_best_split(hist, data.features, ev, s, spec.grad_scale, spec.hess_scale, cfg)
            compare_split(d, o, (ev_seed, kw))
            assert np.array_equal(dspl, ospl)


def compare_trees(d, o, name, exact_values=True):
    assert d["num_leaves"] == o["num_leaves"], name
    for k in ("split_feature", "threshold_bin", "left_child", "right_child", "internal_count", "leaf_count",
              "leaf_depth"):
        assert np.array_equal(d[k], o[k]), (name, k)
    dl = (o["decision_type"] & 2) != 0
    assert np.array_equal(d["default_left"].astype(bool), dl), name
    assert np.array_equal(d["split_gain"], o["split_gain"]), name
    for k in ("leaf_value", "leaf_weight", "internal_value", "internal_weight"):
        if exact_values:
            assert np.array_equal(d[k], o[k]), (name, k, np.abs(d[k] - o[k]).max())
        else:
            np.testing.assert_allclose(d[k], o[k], rtol=1e-6, atol=0, err_msg=f"{name} {k}")


# (rows, features, leaves, gradient bins): the 700k-row root partitions in several tiles per workgroup; 300
# features span three slabs; 32 gradient bins keep every workgroup's sums in {g, h} pairs; with 64 gradient bins
# (1023 rows fill a packed word) the 1M-row steps flush their words several times within a workgroup.
@pytest.mark.parametrize("rows,cols,leaves,qbins", [(20_000, 16, 31, 4), (400_000, 128, 255, 4), (700_000, 8, 63, 4),
                                                    (60_000, 300, 63, 4), (150_000, 40, 63, 32),
                                                    (1_000_000, 8, 63, 64)])
def test_grown_tree_matches_the_oracle(rocm, rows, cols, leaves, qbins):
    say("grow", rows, cols, leaves, qbins)
    data = silvic_amd.synthetic(2, rows=rows, cols=cols, seed=21)
    g, h = binary_gradients(data, 7)
    p = oracle.default_params(num_leaves=leaves, num_grad_quant_bins=qbins)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    spec, _ = quantized_setup(rocm, data, g, h, seed=p.data_random_seed, num_bins=qbins)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d = rocm.grow(p.cfg, leaves, -1, spec.grad_scale, spec.hess_scale, mask, (0, n), n)
    o = dict(o_tree)
    o["leaf_value"] = o_tree["leaf_value"]
    compare_trees(d, o, "grow")
    assert np.array_equal(d["leaf_range"].astype(np.int64), o_ranges)
    # the stable partition, row for row (cpu.rs:556-599)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])


# Edge cases of device growth, each against the oracle with the final partition row for row: one split; the
# largest tree of the register replay (512 leaves); a depth limit (jobs whose children are not histogrammed); a
# min_data_in_leaf that stops the tree early; a tiny dataset; zero gradients (no split at all).
@pytest.mark.parametrize("rows,cols,kw", [
    (50_000, 16, dict(num_leaves=2)),
    (200_000, 32, dict(num_leaves=512)),
    (200_000, 32, dict(num_leaves=255, max_depth=4)),
    (100_000, 16, dict(num_leaves=255, min_data_in_leaf=5000)),
    (300, 16, dict(num_leaves=31, min_data_in_leaf=5)),
    (20_000, 16, dict(num_leaves=31, zero=True)),
])
def test_grown_tree_edge_cases(rocm, rows, cols, kw):
    say("grow edge", rows, cols, kw)
    kw = dict(kw)
    zero = kw.pop("zero", False)
    data = silvic_amd.synthetic(2, rows=rows, cols=cols, seed=5)
    g, h = binary_gradients(data, 3)
    if zero:
        g = np.zeros_like(g)
    p = oracle.default_params(**kw)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    spec, _ = quantized_setup(rocm, data, g, h, seed=p.data_random_seed)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d = rocm.grow(p.cfg, p.num_leaves, p.max_depth, spec.grad_scale, spec.hess_scale, mask, (0, n), n)
    compare_trees(d, dict(o_tree), f"edge {kw}")
    assert np.array_equal(d["leaf_range"].astype(np.int64), o_ranges)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])


# Exact ties between leaves: two mirrored halves (negated gradients in exact quantized units, each numerical bin
# order reversed) split apart at the root; every split of one half then has a twin of exactly equal gain in the
# other (the same sums with the sides swapped), so best_leaf (learner.rs:418-429) breaks ties by the lower leaf id.
def test_grown_tree_breaks_exact_gain_ties_by_leaf_id(rocm):
    say("grow mirrored halves")
    half = silvic_amd.synthetic(2, rows=30_000, cols=16, seed=11)
    f0 = next(j for j, f in enumerate(half.features) if f.num_bins >= 3)
    data = mirrored(half, f0)
    rng = np.random.default_rng(4)
    ga = rng.choice(np.array([-1.0, -0.5, 0.5, 1.0], np.float32), size=half.num_rows, p=[0.2, 0.2, 0.3, 0.3])
    g = np.concatenate([ga, -ga]).astype(np.float32)
    h = np.ones(data.num_rows, np.float32)
    p = oracle.default_params(num_leaves=63, stochastic_rounding=0)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    gains = o_tree["split_gain"]
    assert o_tree["split_feature"][0] == f0 and len(set(gains[1:].tolist())) <= (len(gains) - 1) // 2 + 1
    rocm.load(data)
    rocm.set_gradients(g, h)
    spec = oracle.quant_spec(1.0, 1.0, None, 4, False, p.data_random_seed, 0)
    rocm.quantize(spec)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d = rocm.grow(p.cfg, p.num_leaves, p.max_depth, spec.grad_scale, spec.hess_scale, mask, (0, n), n)
    compare_trees(d, dict(o_tree), "mirrored")
    assert np.array_equal(d["leaf_range"].astype(np.int64), o_ranges)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])


def test_grow_rejects_more_leaves_than_the_device_grows(rocm):
    say("grow 2049 leaves")
    data = silvic_amd.synthetic(2, rows=5_000, cols=8, seed=5)
    g, h = binary_gradients(data, 3)
    spec, _ = quantized_setup(rocm, data, g, h)
    n = rocm.reset_partition()
    p = oracle.default_params(num_leaves=2049)
    with pytest.raises(_abi.SilvicError) as e:
        rocm.grow(p.cfg, 2049, -1, spec.grad_scale, spec.hess_scale, np.ones(len(data.features), bool), (0, n), n)
    assert e.value.kind == _abi.KIND_NAMES[_abi.ERR_UNSUPPORTED]


# Trees beyond 512 leaves (the replay keeps its leaves in LDS): config 5's shape (U[0,1) features, a
# piecewise-constant regression target) at 2M rows, max_bin 255, grown to 1000 and 2047 leaves with the final
# partition row for row, and boosted to 2047 leaves per tree.
@pytest.mark.parametrize("leaves", [1000, 2047])
def test_large_trees_match_the_oracle(rocm, leaves):
    say("grow large", leaves)
    data = silvic_amd.synthetic(5, rows=2_000_000, cols=32, seed=3, max_bin=255)
    rng = np.random.default_rng(8)
    g = (data.label - rng.standard_normal(data.num_rows).astype(np.float32) * 0.1).astype(np.float32)
    h = np.ones_like(g)
    p = oracle.default_params(num_leaves=leaves, min_data_in_leaf=20)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    assert o_tree["num_leaves"] == leaves
    spec, _ = quantized_setup(rocm, data, g, h, seed=p.data_random_seed)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d = rocm.grow(p.cfg, p.num_leaves, p.max_depth, spec.grad_scale, spec.hess_scale, mask, (0, n), n)
    compare_trees(d, dict(o_tree), f"grow {leaves}")
    assert np.array_equal(d["leaf_range"].astype(np.int64), o_ranges)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])


def test_boosting_large_trees_matches_the_oracle():
    say("boost 2047 leaves")
    data = silvic_amd.synthetic(5, rows=2_000_000, cols=32, seed=4, max_bin=255)
    o, t = boost_both(data, dict(num_leaves=2047), 3)
    assert len(t.trees) == len(o.trees) == 3
    for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
        assert ot["num_leaves"] == 2047
        compare_trees(d, ot, f"tree {i}", exact_values=False)
    assert np.array_equal(t.backend.scores(0), o.scores)
    t.backend.close()


# categorical columns: the default parameters search sorted categorical rules (21 bins > max_cat_to_onehot 4);
# max_cat_to_onehot 32 searches one-hot rules; cat_smooth 0 with min_data_per_group 1 ranks raw ratios.
@pytest.mark.parametrize("rows,cols,leaves,kw", [(200_000, 28, 63, {}), (300_000, 12, 255, dict(max_cat_to_onehot=32)),
                                                 (60_000, 16, 31, dict(cat_smooth=0.0, min_data_per_group=1,
                                                                       max_cat_threshold=8))])
def test_categorical_tree_matches_the_oracle(rocm, rows, cols, leaves, kw):
    say("categorical grow", rows, cols, leaves, kw)
    data = silvic_amd.synthetic(2, rows=rows, cols=cols, seed=23, categorical=True)
    assert any(f.kind == _abi.BINS_CATEGORICAL for f in data.features)
    g, h = binary_gradients(data, 9)
    p = oracle.default_params(num_leaves=leaves, **kw)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    spec, _ = quantized_setup(rocm, data, g, h, seed=p.data_random_seed)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d = rocm.grow(p.cfg, leaves, -1, spec.grad_scale, spec.hess_scale, mask, (0, n), n)
    compare_trees(d, o_tree, "categorical grow")
    cat_nodes = (o_tree["decision_type"] & 1) != 0
    assert cat_nodes.any(), "the case must split on a categorical feature"
    assert np.array_equal(d["left_bins"], o_tree["left_bins"])
    assert np.array_equal(d["leaf_range"].astype(np.int64), o_ranges)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])


def test_learner_cases_on_the_device(rocm):
    # learner.rs:690-740 on numerical features: max_depth, zero-gradient rows
    say("learner cases")
    data, bins = learner_dataset(0, 6000)
    data.features[2].kind = _abi.BINS_NUMERICAL
    g, h = learner_gradients(0, 6000, bins, zeros=True)
    for kw in (dict(max_depth=2), dict(min_data_in_leaf=0, min_sum_hessian_in_leaf=0.0, num_leaves=31)):
        p = oracle.default_params(num_leaves=kw.get("num_leaves", 8), min_data_in_leaf=kw.get("min_data_in_leaf", 20),
                                  min_sum_hessian_in_leaf=kw.get("min_sum_hessian_in_leaf", 1e-3),
                                  max_depth=kw.get("max_depth", -1))
        o_tree, o_ranges, _ = oracle.grow_tree(data, g, h, p, renew=False)
        spec, _ = quantized_setup(rocm, data, g, h)
        n = rocm.reset_partition()
        d = rocm.grow(p.cfg, p.num_leaves, p.max_depth, spec.grad_scale, spec.hess_scale, np.ones(3, bool),
                      (0, n), n)
        compare_trees(d, o_tree, kw)


def boost_both(data, params, rounds):
    o = oracle.train(data, oracle.default_params(num_iterations=rounds, **params))
    t = silvic_amd.Trainer(dict(params_to_lightgbm(params), num_iterations=rounds, device_type="rocm"), data)
    t.step(rounds)
    return o, t


def params_to_lightgbm(params):
    out = dict(params)
    if "objective" in out:
        out["objective"] = {_abi.OBJ_REGRESSION: "regression", _abi.OBJ_BINARY: "binary",
                            _abi.OBJ_LAMBDARANK: "lambdarank"}[out["objective"]]
    return out


@pytest.mark.parametrize("config,rows,cols,params,rounds", [
    (1, 100_000, 28, dict(num_leaves=31), 20),
    (2, 200_000, 128, dict(objective=_abi.OBJ_BINARY, num_leaves=255), 6),
    (2, 100_000, 64, dict(objective=_abi.OBJ_BINARY, num_leaves=63, bagging_fraction=0.8, bagging_freq=2,
                          feature_fraction=0.7, lambda_l2=1.0), 8),
    (2, 120_000, 28, dict(objective=_abi.OBJ_BINARY, num_leaves=63, categorical=True), 6),
    # the wide sparse shape: 2000 features of at most 63 bins (mostly a handful) in 8 packed slabs
    (4, 30_000, 2000, dict(objective=_abi.OBJ_BINARY, num_leaves=63), 4),
    # leaves not renewed: the tree's own outputs from the device scales (GrowState's scales, no host copy)
    (2, 150_000, 64, dict(objective=_abi.OBJ_BINARY, num_leaves=127, quant_train_renew_leaf=0), 6),
    # the smallest and the largest quantization the reference accepts (config.rs:416-421)
    (2, 150_000, 64, dict(objective=_abi.OBJ_BINARY, num_leaves=63, num_grad_quant_bins=2), 6),
    (2, 150_000, 64, dict(objective=_abi.OBJ_BINARY, num_leaves=63, num_grad_quant_bins=64), 6),
    (2, 150_000, 64, dict(objective=_abi.OBJ_BINARY, num_leaves=63, num_grad_quant_bins=64,
                          quant_train_renew_leaf=0), 4),
    # weighted regression: non-constant hessians (objective/mod.rs:84-89), weighted sums in the leaf renewal
    (1, 100_000, 28, dict(num_leaves=31, weighted=True), 8),
    (1, 100_000, 28, dict(num_leaves=31, weighted=True, num_grad_quant_bins=16, quant_train_renew_leaf=0), 5),
])
def test_boosting_matches_the_oracle(config, rows, cols, params, rounds):
    say("boost", config, rows, cols, params, rounds)
    params = dict(params)
    categorical = bool(params.pop("categorical", False))
    weighted = bool(params.pop("weighted", False))
    data = silvic_amd.synthetic(config, rows=rows, cols=cols, seed=13, categorical=categorical)
    if weighted:
        data.weight = np.random.default_rng(5).uniform(0.2, 3.0, rows).astype(np.float32)
    o, t = boost_both(data, params, rounds)
    assert len(t.trees) == len(o.trees) == rounds
    assert t.init_score == o.init_score
    for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
        compare_trees(d, ot, f"tree {i}", exact_values=False)
    s = t.backend.scores(0)
    np.testing.assert_allclose(s, o.scores, rtol=1e-6, atol=1e-6)
    assert np.array_equal(s, o.scores), "scores are the same f32 adds"
    t.backend.close()


def test_headline_workload_at_full_size(rocm):
    # config 2 as the bench runs it: 10M rows x 128 features, binary, 255 leaves, num_grad_quant_bins 4. The root
    # histogram bit for bit, then three boosted trees and the scores identical to the oracle's
    say("full size 10M x 128")
    data = silvic_amd.synthetic(2)
    assert (data.num_rows, len(data.features)) == (10_000_000, 128)
    g, h = binary_gradients(data)
    spec, packed = quantized_setup(rocm, data, g, h)
    n = rocm.reset_partition()
    root = rocm.histogram((0, n))
    assert np.array_equal(root, oracle.histogram(data, packed, 4, np.arange(n, dtype=np.uint32)))
    say("full size boost 3")
    o, t = boost_both(data, dict(objective=_abi.OBJ_BINARY, num_leaves=255), 3)
    assert len(t.trees) == len(o.trees) == 3
    for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
        assert ot["num_leaves"] == 255
        compare_trees(d, ot, f"tree {i}", exact_values=False)
    assert np.array_equal(t.backend.scores(0), o.scores)
    t.backend.close()


# Config 3 (lambdarank, ndcg): queries of 10..200 documents, 136 features, labels 0..4. The gradients are computed
# on the host in f64 (objective/lambdarank.rs), the trees on the device.
def test_lambdarank_gradients_match_the_oracle():
    say("lambdarank gradients 200k")
    data = silvic_amd.synthetic(3, rows=200_000, seed=5)
    p = oracle.default_params(objective=_abi.OBJ_LAMBDARANK)
    t = silvic_amd.Trainer(dict(objective="lambdarank", num_leaves=31, device_type="rocm"), data)
    try:
        for step in range(3):  # tied scores (all 0: rank order by row), then the scores of 1 and 2 trees
            scores = t.backend.scores(0)
            mg, mh = t.backend.compute_gradients()
            g, h = t.backend.gradients()
            og, oh = oracle.lambdarank_gradients(data, p, scores)
            assert np.array_equal(g, og) and np.array_equal(h, oh), step
            assert mg == float(np.abs(og).max()) and mh == float(oh.max())
            t.step(1)
    finally:
        t.backend.close()


# The device path (k_rank_pairs: every query of at most 512 rows) under other settings: no normalization, a short
# truncation, row weights, sigmoid 2, labels drawn uniformly (most pairs taken, where the synthetic queries take
# few), a query of 500 rows (the 512-row kernel); and queries of more than 512 rows on the host's threads beside the
# device's (one such query, copied by itself; 70, with every row's scores copied), against the oracle bit for bit.
@pytest.mark.parametrize("case", ["no norm, truncation 5", "weights, sigmoid 2", "uniform labels",
                                  "one query of 500 rows, uniform labels", "one query of 700 rows", "NaN labels",
                                  "70 queries of 600 rows", "70 queries of 600 rows, no norm, weights"])
def test_lambdarank_gradient_paths_match_the_oracle(case):
    say("lambdarank gradients", case)
    data = silvic_amd.synthetic(3, rows=60_000, seed=9)
    kw = {}
    if "uniform labels" in case:
        data.label = np.random.default_rng(4).integers(0, 5, data.num_rows).astype(np.float32)
    if case == "NaN labels":  # Rust's `as` casts: a NaN label passes silvic's checks and takes label 0's gain
        data.label = data.label.copy()
        data.label[np.random.default_rng(6).random(data.num_rows) < 0.05] = np.nan
        assert oracle.check_labels(data.label, 31) == 0
    if case.startswith("no norm"):
        kw = dict(lambdarank_norm=False, lambdarank_truncation_level=5)
    elif case.startswith("weights"):
        data.weight = np.random.default_rng(3).uniform(0.5, 2.0, data.num_rows).astype(np.float32)
        kw = dict(sigmoid=2.0)
    elif case.startswith("one query of 500"):
        qb = data.query_boundaries
        k = int(np.searchsorted(qb, 500))
        data.query_boundaries = np.concatenate([[0, 500], qb[k + 1:]]).astype(qb.dtype)
        assert 256 < np.diff(data.query_boundaries).max() <= 512
    elif case.startswith("one query of 700"):
        qb = data.query_boundaries
        k = int(np.searchsorted(qb, 700))
        data.query_boundaries = np.concatenate([[0], qb[k:]]).astype(qb.dtype)  # rows 0..qb[k] become one query
        sizes = np.diff(data.query_boundaries)
        assert sizes.max() > 512 and (sizes > 512).sum() == 1  # that one on the host, every other on the device
    elif case.startswith("70 queries of 600"):  # more host queries than are copied one at a time
        qb = data.query_boundaries
        k = int(np.searchsorted(qb, 42_000))
        data.query_boundaries = np.concatenate([np.arange(0, 42_000, 600), qb[k:]]).astype(qb.dtype)
        sizes = np.diff(data.query_boundaries)
        assert (sizes > 512).sum() >= 70 and (sizes <= 512).sum() > 100
        if "no norm" in case:
            data.weight = np.random.default_rng(3).uniform(0.5, 2.0, data.num_rows).astype(np.float32)
            kw = dict(lambdarank_norm=False)
    p = oracle.default_params(objective=_abi.OBJ_LAMBDARANK, **kw)
    t = silvic_amd.Trainer(dict(objective="lambdarank", num_leaves=31, device_type="rocm", **kw), data)
    try:
        for step in range(3):
            scores = t.backend.scores(0)
            mg, mh = t.backend.compute_gradients()
            g, h = t.backend.gradients()
            og, oh = oracle.lambdarank_gradients(data, p, scores)
            assert np.array_equal(g.view(np.uint32), og.view(np.uint32)), step
            assert np.array_equal(h.view(np.uint32), oh.view(np.uint32)), step
            assert mg == float(np.abs(og).max()) and mh == float(np.abs(oh).max())
            t.step(1)
    finally:
        t.backend.close()


def test_lambdarank_labels_are_checked_as_the_reference_checks_them():
    # lambdarank.rs:172-188 with Rust's saturating casts: 3e9 saturates to i32::MAX and fails the integer check,
    # -1 fails the sign check, 31 the gain check (31 default gains); the oracle's restatement agrees on each
    say("lambdarank label checks")
    for bad, code, text in ((3e9, 1, "int type"), (-1.0, 2, "non-negative"), (31.0, 3, "label mappings")):
        data = silvic_amd.synthetic(3, rows=5_000, seed=9)
        data.label = data.label.copy()
        data.label[17] = bad
        assert oracle.check_labels(data.label, 31) == code
        with pytest.raises(_abi.SilvicError) as e:
            silvic_amd.Trainer(dict(objective="lambdarank", num_leaves=7, device_type="rocm"), data)
        assert e.value.kind == "data" and text in str(e.value), (bad, str(e.value))


@pytest.mark.parametrize("rows,params,rounds", [
    (200_000, dict(num_leaves=127), 6),
    (120_000, dict(num_leaves=63, bagging_fraction=0.7, bagging_freq=1, lambdarank_truncation_level=10), 5),
])
def test_lambdarank_boosting_matches_the_oracle(rows, params, rounds):
    say("boost lambdarank", rows, params, rounds)
    data = silvic_amd.synthetic(3, rows=rows, seed=7)
    params = dict(params, objective=_abi.OBJ_LAMBDARANK)
    o, t = boost_both(data, params, rounds)
    assert len(t.trees) == len(o.trees) == rounds
    assert t.init_score == o.init_score == 0.0
    for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
        compare_trees(d, ot, f"tree {i}", exact_values=False)
    assert np.array_equal(t.backend.scores(0), o.scores)
    t.backend.close()


# The fallback of the device-made lambdarank normalization factors (SROCM_TEST_RANK_FALLBACK=1 at load makes every
# device query raise the flag that some row's f32 gradient could depend on the last bit of the C library's log2): the
# gradients are made again with the host's factors, and each boosting iteration is taken again after its first
# attempt was kept from the scores (by the leaf-renewal gate; without renewal the host never applies it). Gradients,
# trees and scores equal the oracle's, and the profile counts one redo per gradient computation.
@pytest.mark.parametrize("renew", [1, 0])
def test_lambdarank_host_factor_fallback_matches_the_oracle(monkeypatch, renew):
    say("lambdarank host-factor fallback", renew)
    monkeypatch.setenv("SROCM_TEST_RANK_FALLBACK", "1")
    data = silvic_amd.synthetic(3, rows=60_000, seed=13)
    prof = (C.c_double * 26)()
    p = oracle.default_params(objective=_abi.OBJ_LAMBDARANK)
    t = silvic_amd.Trainer(dict(objective="lambdarank", num_leaves=31, device_type="rocm"), data)
    try:
        t.backend._check(t.backend._lib.srocm_profile(t.backend._h, 0))  # the counters from zero
        scores = t.backend.scores(0)
        mg, mh = t.backend.compute_gradients()
        g, h = t.backend.gradients()
        og, oh = oracle.lambdarank_gradients(data, p, scores)
        assert np.array_equal(g, og) and np.array_equal(h, oh)
        assert mg == float(np.abs(og).max()) and mh == float(oh.max())
        t.backend._check(t.backend._lib.srocm_profile_read(t.backend._h, prof, 26))
        assert prof[25] == 1
    finally:
        t.backend.close()
    rounds = 4
    o, t = boost_both(data, dict(objective=_abi.OBJ_LAMBDARANK, num_leaves=31, quant_train_renew_leaf=renew), rounds)
    try:
        assert len(t.trees) == len(o.trees) == rounds
        for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
            compare_trees(d, ot, f"tree {i}", exact_values=False)
        assert np.array_equal(t.backend.scores(0), o.scores)
        t.backend._check(t.backend._lib.srocm_profile_read(t.backend._h, prof, 26))
        assert prof[25] == rounds
    finally:
        t.backend.close()


# Validation sets (Backend::load's `valid`, cpu.rs:707-728; scores(1), cpu.rs:929): two sets binned with the
# training set's layout; after boosting, their scores equal the oracle's trees replayed onto their rows with its
# add_tree (cpu.rs:605-695), the initial score first and the first tree's values without it (replay.rs:38-40).
@pytest.mark.parametrize("objective,renew", [(_abi.OBJ_BINARY, 1), (_abi.OBJ_REGRESSION, 0)])
def test_validation_scores_match_the_oracle(objective, renew):
    say("validation sets", objective, renew)
    full = silvic_amd.synthetic(2 if objective == _abi.OBJ_BINARY else 1, rows=160_000, cols=40, seed=17)
    train, valid1, valid2 = row_slice(full, 0, 100_000), row_slice(full, 100_000, 140_000), row_slice(full, 140_000, 160_000)
    params = dict(objective=objective, num_leaves=63, quant_train_renew_leaf=renew)
    rounds = 6
    o = oracle.train(train, oracle.default_params(num_iterations=rounds, **params))
    t = silvic_amd.Trainer(dict(params_to_lightgbm(params), num_iterations=rounds, device_type="rocm"), train,
                           valid_sets=[valid1, valid2])
    try:
        t.step(rounds)
        assert len(t.trees) == len(o.trees) == rounds
        for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
            compare_trees(d, ot, f"tree {i}", exact_values=False)
        assert np.array_equal(t.backend.scores(0), o.scores)
        for k, valid in ((1, valid1), (2, valid2)):
            vs = np.full(valid.num_rows, np.float32(o.init_score), np.float32)
            for i, tr in enumerate(o.trees):
                assert tr["num_leaves"] > 1
                nodes = [device_node(_abi.BinSplit(full.features[f].group, full.features[f].column,
                                                   (C.c_uint32 * 8)(*[int(w) for w in tr["left_bins"][n]])),
                                     int(tr["left_child"][n]), int(tr["right_child"][n]))
                         for n, f in enumerate(tr["split_feature"])]
                lv = tr["leaf_value"] - (o.init_score if i == 0 else 0.0)
                vs = oracle.add_tree(valid, nodes, lv.astype(np.float32), vs)
            assert np.array_equal(t.backend.scores(k), vs), k
    finally:
        t.backend.close()


def test_the_widest_units_spread_the_workgroups_and_wider_ones_are_rejected(rocm):
    # a workgroup's histogram sums are i32, so for units of up to 65535 the histogram and split-step workgroups are
    # spread until none adds up more than (2^31 - 1) / 65535 rows (at 8M rows, one a compute unit would add 31k);
    # units past the packed word's halves are refused before any kernel runs
    wide = oracle.quant_spec(1.0, 1.0, None, 4, True, 1, 0)
    wide.grad_max_q, wide.hess_max_q = 32767, 65535
    for rows in (400_000, 8_000_000):
        say("widest units", rows)
        data = silvic_amd.synthetic(2, rows=rows, cols=4, seed=3)
        g, h = binary_gradients(data)
        rocm.load(data)
        rocm.set_gradients(g, h)
        rocm.quantize(wide)
        packed = oracle.quantize(wide, g, h)
        assert rocm.reset_partition() == rows
        assert np.array_equal(rocm.histogram((0, rows)), oracle.histogram(data, packed, 65535, np.arange(rows, dtype=np.uint32)))
    for gq, hq in ((32768, 4), (2, 65536), (0, 4)):
        bad = oracle.quant_spec(1.0, 1.0, None, 4, True, 1, 0)
        bad.grad_max_q, bad.hess_max_q = gq, hq
        with pytest.raises(_abi.SilvicError) as e:
            rocm.quantize(bad)
        assert e.value.kind == "unsupported" and "must lie in" in str(e.value)
    rocm.quantize(oracle.quant_spec(1.0, 1.0, None, 64, True, 1, 0))  # the reference's largest setting passes
