"""The oracle's learner.rs / boosting.rs restatement against the reference's learner and training tests
(learner.rs:657-740, crates/silvic-core/tests/train_cpu.rs:175-267)."""

import numpy as np

import oracle
import silvic_amd
from silvic_amd import _abi
from tests.helpers import learner_dataset, learner_gradients


def learner_params(**kw):
    """learner.rs:580-591."""
    base = dict(num_leaves=8, min_data_in_leaf=20, max_cat_to_onehot=4, min_data_per_group=10, cat_smooth=1.0,
                cat_l2=0.0)
    base.update(kw)
    return oracle.default_params(**base)


def test_leaves_match_the_partition_and_their_sums():
    # learner.rs:657-688, quantized with leaf renewal: leaves hold -G/H of their rows
    data, bins = learner_dataset(0, 3000)
    g, h = learner_gradients(0, 3000, bins)
    p = learner_params()
    tree, ranges, part = oracle.grow_tree(data, g, h, p)
    assert tree["num_leaves"] == 8
    assert 2 in tree["split_feature"], "the categorical feature splits"
    assert sorted(np.concatenate([part[b:b + c] for b, c in ranges])) == list(range(3000))
    for leaf, (b, c) in enumerate(ranges):
        rows = part[b:b + c]
        assert c == tree["leaf_count"][leaf]
        assert c >= 20
        G, H = g[rows].astype(np.float64).sum(), h[rows].astype(np.float64).sum()
        assert abs(tree["leaf_value"][leaf] - (-G / H)) <= 1e-6 * max(abs(G / H), 1.0)
        assert abs(tree["leaf_weight"][leaf] - H) <= 1e-6 * H


def test_left_bin_masks_route_every_row_to_its_leaf():
    # learner.rs:459-485 apply_split: a numerical node sends bins 0..=threshold (and the NaN bin iff default_left)
    # left, a categorical node exactly its rule's bins; walking each row down the masks must reach the leaf whose
    # range holds it
    data, bins = learner_dataset(0, 3000)
    g, h = learner_gradients(0, 3000, bins)
    tree, ranges, part = oracle.grow_tree(data, g, h, learner_params())
    masks = tree["left_bins"]
    for node, f in enumerate(tree["split_feature"]):
        meta = data.features[f]
        cat = (tree["decision_type"][node] & 1) != 0
        assert cat == (meta.kind == _abi.BINS_CATEGORICAL)
        left = [b for b in range(256) if (masks[node][b >> 5] >> (b & 31)) & 1]
        if cat:
            assert tree["threshold_bin"][node] == 0 and 0 < len(left) < meta.num_bins
        else:
            want = list(range(tree["threshold_bin"][node] + 1))
            if meta.nan_bin and (tree["decision_type"][node] & 2):
                want.append(meta.num_bins - 1)
            assert left == want
    leaf_of = np.empty(3000, np.int64)
    for leaf, (b, c) in enumerate(ranges):
        leaf_of[part[b:b + c]] = leaf
    for r in range(3000):
        node = 0
        while node >= 0:
            b = int(bins[r, tree["split_feature"][node]])
            go_left = (masks[node][b >> 5] >> (b & 31)) & 1
            node = tree["left_child"][node] if go_left else tree["right_child"][node]
        assert ~node == leaf_of[r]


def test_max_depth_limits_growth():
    # learner.rs:690-699
    data, bins = learner_dataset(0, 3000)
    g, h = learner_gradients(0, 3000, bins)
    tree, _, _ = oracle.grow_tree(data, g, h, learner_params(max_depth=2))
    assert tree["num_leaves"] == 4
    assert tree["leaf_depth"].max() == 2


def test_zero_gradient_rows_never_make_empty_leaves():
    # learner.rs:724-740
    data, bins = learner_dataset(0, 6000)
    g, h = learner_gradients(0, 6000, bins, zeros=True)
    tree, _, _ = oracle.grow_tree(data, g, h, learner_params(min_data_in_leaf=0, min_sum_hessian_in_leaf=0.0,
                                                             num_leaves=31))
    assert tree["num_leaves"] > 8
    assert (tree["leaf_count"] > 0).all()
    assert np.isfinite(tree["leaf_value"]).all()


def test_node_numbering_follows_lightgbm():
    # tree.rs:8-21, 143-177: the split leaf keeps its index (left), the new leaf is num_leaves, children < 0 are ~leaf
    data, bins = learner_dataset(0, 3000)
    g, h = learner_gradients(0, 3000, bins)
    tree, _, _ = oracle.grow_tree(data, g, h, learner_params())
    n = tree["num_leaves"]
    seen_leaves = set()
    for node in range(n - 1):
        for c in (tree["left_child"][node], tree["right_child"][node]):
            if c < 0:
                seen_leaves.add(~c)
            else:
                assert c > node
    assert seen_leaves == set(range(n))
    assert tree["internal_count"][0] == 3000


def small_config1(rows=20_000):
    return silvic_amd.synthetic(1, rows=rows)


def test_identical_runs_are_identical_across_thread_counts():
    # train_cpu.rs:249-267
    data = small_config1()
    p = oracle.default_params(num_iterations=8, num_leaves=31)
    before = oracle.threads()
    try:
        oracle.set_threads(1)
        a = oracle.train(data, p)
        oracle.set_threads(4)
        b = oracle.train(data, p)
    finally:
        oracle.set_threads(before)
    assert len(a.trees) == len(b.trees) == 8
    for ta, tb in zip(a.trees, b.trees):
        for k in ta:
            assert np.array_equal(ta[k], tb[k]), k
    assert np.array_equal(a.scores, b.scores)


def test_every_objective_learns():
    # train_cpu.rs:175-243
    data = small_config1()
    m = oracle.train(data, oracle.default_params(num_iterations=20, num_leaves=31))
    mse0 = ((data.label - data.label.mean()) ** 2).mean()
    mse = ((data.label - m.scores) ** 2).mean()
    assert mse < 0.5 * mse0
    bdata = silvic_amd.synthetic(2, rows=30_000, cols=32)
    mb = oracle.train(bdata, oracle.default_params(objective=_abi.OBJ_BINARY, num_iterations=20, num_leaves=31))
    p = 1 / (1 + np.exp(-mb.scores.astype(np.float64)))
    y = bdata.label
    loss = -(y * np.log(p) + (1 - y) * np.log(1 - p)).mean()
    p0 = y.mean()
    loss0 = -(p0 * np.log(p0) + (1 - p0) * np.log(1 - p0))
    assert loss < loss0
