"""The benchmark workloads other than the headline one, boosted at the sizes and settings they are defined with,
against the oracle on the same binned data: identical trees, scores bit for bit, and the last tree's partition row
for row (the boosting loop restores the reference's row order after the last tree of a call).

- 50M x 32 U[0,1) features, max_bin 1023, 2047 leaves, 16-bit gradient units (num_grad_quant_bins 32766), here at
  2M rows: all three settings together (separate-counter two-byte slabs, the 2048-leaf select, spread workgroups).
  silvic takes neither max_bin > 255 nor more than 64 gradient bins (config.rs:407-421), so the oracle's side of
  these two settings is pinned by closed forms only.
- lambdarank over 2M documents x 136 features in about 20,000 queries of 10..200 documents, 127 leaves.
- 1M x 2000 features with 98% zeros at max_bin 63, 63 leaves, binary.

The headline workload (10M x 128 binary, 255 leaves) is boosted at full size in test_gpu_parity.py.
"""

import numpy as np
import pytest

import silvic_amd
from silvic_amd import _abi
from tests.test_gpu_parity import boost_both, compare_trees, say

pytestmark = pytest.mark.gpu


def check_boost(data, params, rounds, leaves=None):
    o, t = boost_both(data, params, rounds)
    try:
        assert len(t.trees) == len(o.trees) == rounds
        assert t.init_score == o.init_score
        for i, (d, ot) in enumerate(zip(t.trees, o.trees)):
            if leaves is not None:
                assert ot["num_leaves"] == leaves, (i, ot["num_leaves"])
            compare_trees(d, ot, f"tree {i}", exact_values=False)
            assert np.array_equal(d["left_bins"], ot["left_bins"]), i
        assert np.array_equal(t.backend.scores(0), o.scores)
        n = data.num_rows
        assert np.array_equal(t.backend.partition_rows(n), o.partition[:n])
    finally:
        t.backend.close()
    return o, t


def test_two_byte_bins_2047_leaves_16_bit_units_match_the_oracle():
    say("U[0,1) 2M x 32, max_bin 1023, 2047 leaves, num_grad_quant_bins 32766, 2 trees")
    data = silvic_amd.synthetic(5, rows=2_000_000, cols=32, seed=23, max_bin=1023)
    assert all(g.bin_bits == 16 for g in data.groups)
    assert max(f.num_bins for f in data.features) > 1000
    o, _ = check_boost(data, dict(num_leaves=2047, num_grad_quant_bins=32766), 2, leaves=2047)
    assert max(int(t["threshold_bin"].max()) for t in o.trees) > 255


def test_lambdarank_2m_documents_127_leaves_match_the_oracle():
    say("lambdarank 2M documents (about 20000 queries) x 136, 127 leaves, 3 trees")
    data = silvic_amd.synthetic(3, seed=29)
    assert 19_000 <= len(data.query_boundaries) - 1 <= 21_000 and data.num_rows == 2_000_000
    assert len(data.features) == 136
    check_boost(data, dict(objective=_abi.OBJ_LAMBDARANK, num_leaves=127), 3, leaves=127)


def test_wide_sparse_1m_x_2000_63_leaves_match_the_oracle():
    say("binary 1M x 2000 (98% zeros), max_bin 63, 63 leaves, 3 trees")
    data = silvic_amd.synthetic(4, seed=31)
    assert (data.num_rows, len(data.features)) == (1_000_000, 2000)
    assert max(f.num_bins for f in data.features) <= 64
    check_boost(data, dict(objective=_abi.OBJ_BINARY, num_leaves=63), 3, leaves=63)
