"""A learner over the trait calls alone: Learner::grow / split_leaf / best_leaf / find_split (learner.rs:121-352,
418-452) driving Backend::histogram, partition, partition_and_histogram and the device split search one split at a
time, with the sibling's histogram by subtraction on the host (learner.rs:356-371), or (SlotBackend) with every
histogram, the subtraction and the split search on the device over histogram slots. It is how a binding grows trees
of more leaves than srocm_grow takes (2048; silvic takes up to 131072, config.rs:389-391), so a test grows such a
tree with it and checks it against the oracle's learner. Test infrastructure: it restates the reference's learner
in Python, as the oracle restates it in C++.
"""

import numpy as np

from silvic_amd import _abi, bin_split, wide_bin_split


class TraitTree:
    """Tree::split's arrays (tree.rs:108-178): node k is the k-th split; leaf `leaf` keeps its id as the left child
    and the right child takes the next one."""

    def __init__(self):
        self.num_leaves = 1
        self.split_feature, self.threshold_bin, self.left_child, self.right_child = [], [], [], []
        self.default_left = []
        self.internal_count, self.internal_value, self.internal_weight, self.split_gain = [], [], [], []
        self.leaf_value, self.leaf_weight, self.leaf_count = [0.0], [0.0], [0]
        self.leaf_parent, self.leaf_depth = [-1], [0]
        self.left_bins = []

    def split(self, leaf, feature, threshold, default_left, children, gain, words):
        node = self.num_leaves - 1
        new_leaf = self.num_leaves
        parent = self.leaf_parent[leaf]
        if parent >= 0:
            if self.left_child[parent] == ~leaf:
                self.left_child[parent] = node
            else:
                self.right_child[parent] = node
        lv, rv, lc, rc, lw, rw = children
        self.split_feature.append(feature)
        self.split_gain.append(np.float32(gain))
        self.threshold_bin.append(threshold)
        self.default_left.append(1 if default_left else 0)
        self.left_child.append(~leaf)
        self.right_child.append(~new_leaf)
        self.internal_weight.append(self.leaf_weight[leaf])
        self.internal_value.append(self.leaf_value[leaf])
        self.internal_count.append(lc + rc)
        self.left_bins.append(words)
        nz = lambda v: 0.0 if v != v else v
        self.leaf_value[leaf], self.leaf_weight[leaf], self.leaf_count[leaf] = nz(lv), lw, lc
        self.leaf_value.append(nz(rv))
        self.leaf_weight.append(rw)
        self.leaf_count.append(rc)
        self.leaf_parent[leaf] = node
        self.leaf_parent.append(node)
        depth = self.leaf_depth[leaf] + 1
        self.leaf_depth[leaf] = depth
        self.leaf_depth.append(depth)
        self.num_leaves += 1
        return new_leaf

    def arrays(self):
        i32 = lambda v: np.array(v, np.int32)
        return {
            "num_leaves": self.num_leaves, "split_feature": i32(self.split_feature),
            "threshold_bin": np.array(self.threshold_bin, np.uint32), "left_child": i32(self.left_child),
            "default_left": np.array(self.default_left, np.uint8),
            "right_child": i32(self.right_child), "internal_count": np.array(self.internal_count, np.int64),
            "leaf_count": np.array(self.leaf_count, np.int64), "leaf_depth": i32(self.leaf_depth),
            "leaf_value": np.array(self.leaf_value), "leaf_weight": np.array(self.leaf_weight),
            "internal_value": np.array(self.internal_value), "internal_weight": np.array(self.internal_weight),
            "split_gain": np.array(self.split_gain, np.float32),
            "left_bins": np.array(self.left_bins, np.uint32).reshape(-1, 8),
        }


class Leaf:
    def __init__(self, rng, sums, nf):
        self.range = rng
        self.sums = sums  # (grad, hess, count) in histogram units
        self.splittable = np.ones(nf, bool)
        self.best = None
        self.hist = None


def grow(backend, data, params, feature_mask, grad_scale, hess_scale, root, root_count):
    """learner.rs:121-169 over the trait calls; returns (tree arrays, leaf ranges)."""
    cfg = params.cfg
    L = params.num_leaves
    nf = len(data.features)
    feats = data.features
    sums_feature = next((f for f, m in enumerate(feats) if m.num_bins), None)
    depth_allows = lambda d: params.max_depth <= 0 or d < params.max_depth  # learner.rs:178-180
    may_split = lambda d, l, r: depth_allows(d) and (l >= 2 * cfg.min_data_in_leaf or r >= 2 * cfg.min_data_in_leaf)
    tree = TraitTree()
    leaves = [Leaf(root, (0.0, 0.0, root_count), nf)]

    def find_split(leaf, hist, evaluate):  # learner.rs:236-246
        info, spl = backend.find_best_split(hist, feats, evaluate, leaf.sums, grad_scale, hess_scale, cfg)
        leaf.splittable = spl
        leaf.best = info if info.found else None
        leaf.hist = hist

    def split_words(m, info):  # learner.rs:432-452
        if data.groups[m.group].bin_bits == 16:
            return wide_bin_split(m.group, m.column, info.threshold,
                                  m.num_bins - 1 if info.default_left and m.nan_bin else None)
        if info.categorical:
            return bin_split(m.group, m.column, [info.cat_bins[i] for i in range(info.num_cat_bins)])
        bins = list(range(info.threshold + 1))
        if info.default_left and m.kind == _abi.BINS_NUMERICAL and m.nan_bin:
            bins.append(m.num_bins - 1)
        return bin_split(m.group, m.column, bins)

    if sums_feature is not None and may_split(0, root_count, 0):
        used = np.array(feature_mask, bool)
        used[sums_feature] = True
        backend.set_histogram_features(used)
        hist = backend.histogram(root)
        m = feats[sums_feature]
        sg = sh = 0.0
        for b in range(m.num_bins):  # split.rs:101-108, in bin order
            sg += hist[2 * (m.hist_offset + b)]
            sh += hist[2 * (m.hist_offset + b) + 1]
        leaves[0].sums = (sg, sh, root_count)
        find_split(leaves[0], hist, np.array(feature_mask, bool))

    while tree.num_leaves < L:
        best = None  # learner.rs:418-429: the first highest gain, positive
        for i, l in enumerate(leaves):
            if l.best is not None and (best is None or l.best.gain > leaves[best].best.gain):
                best = i
        if best is None or not leaves[best].best.gain > 0.0:
            break
        leaf = leaves[best]
        info = leaf.best
        leaf.best = None
        m = feats[info.feature]
        split = split_words(m, info)
        (pb, pc), parent_count = leaf.range, leaf.sums[2]
        depth = tree.leaf_depth[best]
        may_search = leaf.hist is not None and tree.num_leaves + 1 < L and depth_allows(depth + 1)
        built_left = info.left.count <= info.right.count  # learner.rs:269-275
        evaluate = np.array(feature_mask, bool) & leaf.splittable
        built = None
        if may_search:
            backend.set_histogram_features(evaluate)
            left, built = backend.partition_and_histogram(leaf.range, split, 0 if built_left else 1)
        else:
            left = backend.partition(leaf.range, split)
        lc, rc = left, parent_count - left
        assert lc > 0 and rc > 0, "a split sent no rows to one side"
        children = (info.left_output, info.right_output, lc, rc, info.left.hess * hess_scale,
                    info.right.hess * hess_scale)
        right = tree.split(best, info.feature, 0 if info.categorical else info.threshold,
                           bool(info.default_left) and not info.categorical, children,
                           info.gain + cfg.min_gain_to_split, list(split.left_bins))
        parent_hist = leaf.hist
        lo = Leaf((pb, left), (info.left.grad, info.left.hess, lc), nf)
        ro = Leaf((pb + left, pc - left), (info.right.grad, info.right.hess, rc), nf)
        leaves[best] = lo
        leaves.append(ro)
        assert right == len(leaves) - 1
        if parent_hist is not None and built is not None and may_split(depth + 1, lc, rc):
            other_hist = parent_hist - built  # learner.rs:356-371: exact, integers in f64
            b_leaf, o_leaf = (lo, ro) if built_left else (ro, lo)
            find_split(b_leaf, built, evaluate)
            find_split(o_leaf, other_hist, evaluate)
    return tree.arrays(), np.array([l.range for l in leaves], np.int64)


class SlotHist:
    """A histogram in a device slot (srocm_hist_slots). `parent - built` subtracts on the device, so the parent's slot
    becomes the other child's histogram (learner.rs:365-367); indexing reads the slot to the host once."""

    def __init__(self, backend, slot):
        self.backend, self.slot, self._host = backend, slot, None

    def __sub__(self, built):
        self.backend.rocm.subtract(self.slot, built.slot)
        return SlotHist(self.backend, self.slot)

    def __getitem__(self, i):
        if self._host is None:
            self._host = self.backend.rocm.read_slot(self.slot)
        return self._host[i]


class SlotBackend:
    """The device backend with every histogram grow() makes kept in a device slot: the slot calls for the histogram,
    the fused partition and histogram, the subtraction and the split search, so no histogram crosses to the host
    (the root's, read once for its sums, aside). A histogram takes the next slot; a sibling reuses its parent's."""

    def __init__(self, rocm, num_slots):
        self.rocm, self.num_slots, self.used = rocm, num_slots, 0
        rocm.hist_slots(num_slots)

    def _slot(self):
        assert self.used < self.num_slots, "out of histogram slots"
        self.used += 1
        return self.used - 1

    def set_histogram_features(self, used):
        self.rocm.set_histogram_features(used)

    def histogram(self, leaf):
        slot = self._slot()
        self.rocm.histogram_slot(leaf, slot)
        return SlotHist(self, slot)

    def partition(self, leaf, split):
        return self.rocm.partition(leaf, split)

    def partition_and_histogram(self, leaf, split, side):
        slot = self._slot()
        left = self.rocm.partition_and_histogram_slot(leaf, split, side, slot)
        return left, SlotHist(self, slot)

    def find_best_split(self, hist, features, evaluate, sums, grad_scale, hess_scale, cfg):
        return self.rocm.find_best_split_slot(hist.slot, features, evaluate, sums, grad_scale, hess_scale, cfg)


class OracleBackend:
    """The trait calls grow() makes, answered by the oracle on the host (its histogram, stable partition and split
    search over a partition it keeps), so that the learner restatement itself is checked against the oracle's own
    learner without a device."""

    def __init__(self, data, packed, max_quant):
        import oracle

        self.oracle, self.data, self.packed, self.max_quant = oracle, data, packed, max_quant
        self.part = np.arange(data.num_rows, dtype=np.uint32)

    def set_histogram_features(self, used):
        pass

    def histogram(self, leaf):
        b, c = leaf
        return self.oracle.histogram(self.data, self.packed, self.max_quant, self.part[b:b + c])

    def partition(self, leaf, split):
        b, c = leaf
        rows, left = self.oracle.partition(self.data, self.part[b:b + c], split)
        self.part[b:b + c] = rows
        return left

    def partition_and_histogram(self, leaf, split, side):
        b, c = leaf
        left = self.partition(leaf, split)
        return left, self.histogram((b, left) if side == 0 else (b + left, c - left))

    def find_best_split(self, hist, features, evaluate, sums, grad_scale, hess_scale, cfg):
        return self.oracle.find_best_split(hist, features, evaluate, sums, grad_scale, hess_scale, cfg)
