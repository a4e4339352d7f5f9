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


def _commit_order_violations(tree, num_leaves_cap):
    """best_leaf (learner.rs:418-429) commits the open leaf with the largest gain, the lowest leaf id among equal
    gains, while that gain is positive. Checked from the finished tree alone: node t split leaf `leaf[t]` (the
    leftmost leaf under t, since a split leaf keeps its id on the left); the leaf split at node j > t was open at t
    when j's parent node came before t; a leaf never split was open after its parent node."""
    n = tree["num_leaves"]
    left, right = tree["left_child"], tree["right_child"]
    gain, open_gain = tree["commit_gain"], tree["open_gain"]
    parent = np.full(n - 1, -1)
    leaf_parent = np.full(n, -1)
    for p in range(n - 1):
        for c in (left[p], right[p]):
            if c >= 0:
                parent[c] = p
            else:
                leaf_parent[~c] = p
    leaf = np.empty(n - 1, np.int64)
    for t in range(n - 1):
        c = t
        while c >= 0:
            c = left[c]
        leaf[t] = ~c
    bad = []
    for t in range(n - 1):
        if not gain[t] > 0:
            bad.append(("non-positive commit", t))
        for j in range(t + 1, n - 1):
            if parent[j] < t and not (gain[j] < gain[t] or (gain[j] == gain[t] and leaf[j] > leaf[t])):
                bad.append(("later commit beats", t, j))
        for l in range(n):
            if leaf_parent[l] < t and not (open_gain[l] < gain[t] or (open_gain[l] == gain[t] and l > leaf[t])):
                bad.append(("open leaf beats", t, l))
    if n < num_leaves_cap and (open_gain > 0).any():
        bad.append(("stopped with a positive gain",))
    return bad


def test_grown_trees_commit_leaves_in_best_first_order():
    # learner.rs:167-169, 418-429: every tree of a boosted model and a single large tree
    data = silvic_amd.synthetic(2, rows=40_000, cols=24, seed=9)
    m = oracle.train(data, oracle.default_params(objective=_abi.OBJ_BINARY, num_iterations=4, num_leaves=63))
    for tree in m.trees:
        assert tree["num_leaves"] > 8
        assert _commit_order_violations(tree, 63) == []
    data1 = small_config1(30_000)
    rng = np.random.default_rng(2)
    g = (data1.label - rng.standard_normal(data1.num_rows)).astype(np.float32)
    tree, _, _ = oracle.grow_tree(data1, g, np.ones_like(g), oracle.default_params(num_leaves=255,
                                                                                   min_data_in_leaf=40))
    assert tree["num_leaves"] > 100
    assert _commit_order_violations(tree, 255) == []


def test_exact_gain_ties_commit_the_lower_leaf_first():
    # two mirrored halves: every split of one half has a twin of exactly equal f64 gain in the other
    from tests.helpers import mirrored

    half = silvic_amd.synthetic(2, rows=30_000, cols=16, seed=11)
    f0 = next(j for j, f in enumerate(half.features) if f.num_bins >= 3)
    data = mirrored(half, f0)
    rng = np.random.default_rng(4)
    ga = rng.choice(np.array([-1.0, -0.5, 0.5, 1.0], np.float32), size=half.num_rows, p=[0.2, 0.2, 0.3, 0.3])
    g = np.concatenate([ga, -ga]).astype(np.float32)
    tree, _, _ = oracle.grow_tree(data, g, np.ones_like(g), oracle.default_params(num_leaves=63,
                                                                                   stochastic_rounding=0),
                                  renew=False)
    gains = tree["commit_gain"][1:]
    assert len(np.unique(gains)) < len(gains), "the halves produce exactly tied gains"
    assert _commit_order_violations(tree, 63) == []
