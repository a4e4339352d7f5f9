"""The oracle on 4-bit bins (two to a byte), an extension silvic does not have (its bins are always bytes,
data/mod.rs:57-58). Parity against silvic is unpinned; these pin the format by equivalence: the same features
stored two to a byte read back the same bins, and give the same histograms, partitions and trees as the byte
layout, which the reference's own tests pin."""

import ctypes as C

import numpy as np

import oracle
import silvic_amd
from silvic_amd import _abi, bin_split
from silvic_amd.dataset import pack_nibbles
from tests.helpers import naive_histogram


def both(rows=20_000, cols=200, seed=3):
    data = silvic_amd.synthetic(4, rows=rows, cols=cols, seed=seed)
    packed = pack_nibbles(data)
    assert any(g.bin_bits == 4 for g in packed.groups) and any(g.bin_bits == 8 for g in packed.groups)
    return data, packed


def test_nibbles_read_back_the_same_bins():
    data, packed = both()
    for f, meta in enumerate(data.features):
        if meta.num_bins:
            assert np.array_equal(packed.bin(f), data.bin(f)), f
    # a 4-bit slot holds the low half of its byte when even, the high half when odd
    g = next(g for g in packed.groups if g.bin_bits == 4 and len(g.features) >= 2)
    rows = g.data.reshape(packed.num_rows, g.row_stride)
    f0, f1 = g.features[0], g.features[1]
    assert np.array_equal(rows[:, 0] & 15, data.bin(f0)) and np.array_equal(rows[:, 0] >> 4, data.bin(f1))


def test_nibble_histograms_equal_the_byte_layout_and_direct_sums():
    data, packed = both()
    rng = np.random.default_rng(2)
    g = rng.standard_normal(data.num_rows).astype(np.float32)
    h = rng.uniform(0.1, 1.0, data.num_rows).astype(np.float32)
    spec = oracle.quant_spec(float(np.abs(g).max()), float(h.max()), None, 16, True, 5, 0)
    q = oracle.quantize(spec, g, h)
    gq, hq = oracle.unpack(q)
    rows = np.sort(rng.choice(data.num_rows, 7_000, replace=False)).astype(np.uint32)
    got = oracle.histogram(packed, q, 16, rows)
    assert np.array_equal(got, oracle.histogram(data, q, 16, rows))
    assert np.array_equal(got, naive_histogram(data, rows, gq[rows], hq[rows]))


def test_nibble_partition_equals_the_byte_layout():
    data, packed = both(rows=8_000)
    rows = np.arange(data.num_rows, dtype=np.uint32)[::2].copy()
    for f in (0, 7, 31):
        m, pm = data.features[f], packed.features[f]
        assert packed.groups[pm.group].bin_bits == 4
        left = list(range(0, m.num_bins, 3))
        a = oracle.partition(data, rows, bin_split(m.group, m.column, left))
        b = oracle.partition(packed, rows, bin_split(pm.group, pm.column, left))
        assert a[1] == b[1] and np.array_equal(a[0], b[0]), f


def test_nibble_boosting_equals_the_byte_layout():
    data, packed = both(rows=30_000, cols=120, seed=8)
    p = oracle.default_params(objective=_abi.OBJ_BINARY, num_leaves=31, num_iterations=4)
    a, b = oracle.train(data, p), oracle.train(packed, p)
    assert len(a.trees) == len(b.trees) == 4
    for ta, tb in zip(a.trees, b.trees):
        for k in ("split_feature", "threshold_bin", "left_child", "right_child", "leaf_count", "leaf_value"):
            assert np.array_equal(ta[k], tb[k]), k
    assert np.array_equal(a.scores, b.scores)
