"""Trees of more leaves than srocm_grow takes (2048), grown split by split over the trait calls as a binding's
Learner::grow does (tests/trait_learner.py, learner.rs:121-352 with the subtraction of learner.rs:356-371), with the
histograms on the host or kept in device slots, against the oracle's learner: the tree arrays, every split's bins, the leaf ranges and the final partition row for row.
silvic takes num_leaves up to 131072 (config.rs:389-391)."""

import numpy as np
import pytest

import oracle
import silvic_amd
from tests import trait_learner
from tests.test_gpu_parity import compare_trees, quantized_setup, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("slots", [False, True], ids=["host-histograms", "device-slots"])
@pytest.mark.parametrize("rows,leaves,max_bin", [(1_000_000, 3000, 255), (400_000, 2600, 1023)])
def test_trait_learner_grows_more_than_2048_leaves_as_the_oracle(rocm, rows, leaves, max_bin, slots):
    say("trait learner", rows, leaves, max_bin, "slots" if slots else "host")
    data = silvic_amd.synthetic(5, rows=rows, cols=32, seed=19, max_bin=max_bin)
    rng = np.random.default_rng(4)
    g = (data.label - rng.standard_normal(rows).astype(np.float32) * 0.1).astype(np.float32)
    h = np.ones_like(g)
    p = oracle.default_params(num_leaves=leaves, min_data_in_leaf=20)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    assert o_tree["num_leaves"] == leaves
    spec, _ = quantized_setup(rocm, data, g, h, seed=p.data_random_seed)
    n = rocm.reset_partition()
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    backend = trait_learner.SlotBackend(rocm, leaves) if slots else rocm
    d, ranges = trait_learner.grow(backend, data, p, mask, spec.grad_scale, spec.hess_scale, (0, n), n)
    compare_trees(d, dict(o_tree), f"trait learner {leaves}")
    assert np.array_equal(d["left_bins"], o_tree["left_bins"])
    assert np.array_equal(ranges, o_ranges)
    assert np.array_equal(rocm.partition_rows(n), o_part[:n])
