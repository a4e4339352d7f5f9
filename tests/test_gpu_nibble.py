"""4-bit bins (two to a byte; an extension silvic does not have) on the device: a dataset whose features of at most
16 bins are stored two to a byte must give, bit for bit, what the oracle gives on the same features stored as
bytes: histograms, the partition row for row, grown trees and boosted scores."""

import numpy as np
import pytest

import oracle
import silvic_amd
from silvic_amd import _abi, bin_split
from silvic_amd.dataset import pack_nibbles
from tests.test_gpu_parity import binary_gradients, boost_both, compare_trees, quantized_setup, say

pytestmark = pytest.mark.gpu


def both(rows, cols, seed):
    data = silvic_amd.synthetic(4, rows=rows, cols=cols, seed=seed)
    packed = pack_nibbles(data)
    assert sum(len(g.features) for g in packed.groups if g.bin_bits == 4) > cols // 2
    return data, packed


def test_nibble_histograms_and_partition_bit_exact(rocm):
    say("nibble histogram")
    data, packed = both(300_000, 300, 4)
    g, h = binary_gradients(data)
    spec, q = quantized_setup(rocm, packed, g, h)
    rows = data.num_rows
    assert rocm.reset_partition() == rows
    assert np.array_equal(rocm.histogram((0, rows)), oracle.histogram(data, q, 4, np.arange(rows, dtype=np.uint32)))
    f = next(k for k, m in enumerate(packed.features) if packed.groups[m.group].bin_bits == 4 and m.num_bins > 3)
    m, pm = data.features[f], packed.features[f]
    left = list(range(0, m.num_bins, 2))
    got = rocm.partition((0, rows), bin_split(pm.group, pm.column, left))
    o_rows, o_left = oracle.partition(data, np.arange(rows, dtype=np.uint32), bin_split(m.group, m.column, left))
    assert got == o_left and np.array_equal(rocm.partition_rows(rows), o_rows)
    for b, c in [(0, o_left), (o_left, rows - o_left)]:
        assert np.array_equal(rocm.histogram((b, c)), oracle.histogram(data, q, 4, o_rows[b:b + c]))


def test_nibble_grown_tree_matches_the_oracle(rocm):
    say("nibble grow")
    data, packed = both(200_000, 400, 6)
    g, h = binary_gradients(data, 3)
    p = oracle.default_params(num_leaves=63)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    spec, _ = quantized_setup(rocm, packed, g, h, seed=p.data_random_seed)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d = rocm.grow(p.cfg, p.num_leaves, p.max_depth, spec.grad_scale, spec.hess_scale, mask, (0, n), n)
    compare_trees(d, o_tree, "nibble grow")
    assert np.array_equal(d["leaf_range"].astype(np.int64), o_ranges)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])


def test_nibble_boosting_matches_the_oracle():
    say("nibble boost")
    data, packed = both(60_000, 1000, 9)
    o = oracle.train(data, oracle.default_params(objective=_abi.OBJ_BINARY, num_leaves=63, num_iterations=4))
    t = silvic_amd.Trainer(dict(objective="binary", num_leaves=63, num_iterations=4, device_type="rocm"), packed)
    t.step(4)
    assert len(t.trees) == len(o.trees) == 4
    for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
        compare_trees(d, ot, f"tree {i}", exact_values=False)
    assert np.array_equal(t.backend.scores(0), o.scores)
    t.backend.close()
