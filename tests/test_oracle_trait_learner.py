"""The trait-call learner restatement (tests/trait_learner.py, learner.rs:121-352) answered by the oracle's own
histogram, partition and split search: it must grow exactly the oracle learner's tree (arrays, split bins, leaf
ranges, partition), which pins it before the GPU test uses it for trees beyond srocm_grow's 2048 leaves."""

import numpy as np
import pytest

import oracle
import silvic_amd
from tests import trait_learner


@pytest.mark.parametrize("config,rows,cols,leaves,kw", [(2, 20_000, 12, 200, {}), (5, 30_000, 6, 300, dict(max_bin=1023))])
def test_trait_learner_matches_the_oracle_learner(config, rows, cols, leaves, kw):
    data = silvic_amd.synthetic(config, rows=rows, cols=cols, seed=5, **kw)
    rng = np.random.default_rng(3)
    g = (data.label - data.label.mean() + rng.standard_normal(rows) * 0.1).astype(np.float32)
    h = np.ones_like(g)
    p = oracle.default_params(num_leaves=leaves, min_data_in_leaf=20)
    o_tree, o_ranges, o_part = oracle.grow_tree(data, g, h, p, renew=False)
    spec = oracle.quant_spec(float(np.abs(g).max()), float(np.abs(h).max()), None, 4, True, p.data_random_seed, 0)
    packed = oracle.quantize(spec, g, h, data.row_offset)
    be = trait_learner.OracleBackend(data, packed, max(spec.grad_max_q, spec.hess_max_q))
    mask = oracle.feature_mask(data.features, 1.0, 2, 0)
    d, ranges = trait_learner.grow(be, data, p, mask, spec.grad_scale, spec.hess_scale, (0, rows), rows)
    assert d["num_leaves"] == o_tree["num_leaves"] > 100
    for k in ("split_feature", "threshold_bin", "left_child", "right_child", "internal_count", "leaf_count",
              "leaf_depth", "leaf_value", "internal_value", "split_gain"):
        assert np.array_equal(d[k], o_tree[k]), k
    assert np.array_equal(d["default_left"].astype(bool), (o_tree["decision_type"] & 2) != 0)
    assert np.array_equal(d["left_bins"], o_tree["left_bins"])
    assert np.array_equal(ranges, o_ranges)
    assert np.array_equal(be.part, o_part)
