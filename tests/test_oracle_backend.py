"""The oracle's CpuBackend restatement (cpu.rs), pinned by the reference's own tests (cpu.rs:1014-1179) and by
brute-force direct sums."""

import numpy as np
import pytest

import oracle
from silvic_amd import bin_split, device_node
from tests.helpers import cpu_dataset, cpu_gradients, naive_histogram


def bagged_rows(data, seed, round_, fraction):
    return np.array([r for r in range(data.num_rows)
                     if oracle.lib().oracle_in_bag(seed, round_, data.row_offset + r, fraction)], np.uint32)


def test_histograms_match_direct_sums():
    # cpu.rs:1014-1056
    data = cpu_dataset(50_000)
    grad, hess = cpu_gradients(50_000)
    spec = oracle.quant_spec(1.5, 0.75, None, 16, True, 9, 3)
    packed = oracle.quantize(spec, grad, hess, data.row_offset)
    part = bagged_rows(data, 4, 1, 0.7)
    rows = part[1000:31_000]
    out = oracle.histogram(data, packed, 16, rows)
    g, h = oracle.unpack(packed[rows])
    expected = naive_histogram(data, rows, g, h)
    assert (out == expected).all()
    for used in ([1, 0, 1], [0, 1, 0], [0, 0, 1]):
        masked = oracle.histogram(data, packed, 16, rows, used)
        for f, meta in enumerate(data.features):
            if used[f]:
                sl = slice(2 * meta.hist_offset, 2 * (meta.hist_offset + meta.num_bins))
                assert (masked[sl] == expected[sl]).all(), (used, f)


def test_packed_accumulators_flush_before_overflow():
    # cpu.rs:1058-1090: g_q = -32000, h_q = 3 on every row; a bound of 1000 rows per accumulator forces flushes
    n = 400_000
    data = cpu_dataset(n)
    rows = np.arange(n, dtype=np.uint32)
    packed = np.full(n, 3 * 65536 - 32000, np.int32)
    out = oracle.histogram(data, packed, 2147483647 // 1000, rows)
    g, h = oracle.unpack(packed)
    expected = naive_histogram(data, rows, g, h)
    assert (out == expected).all()
    assert (out[::2] < -2.0 ** 31).any(), "sums leave i32"


def test_partition_is_stable():
    # cpu.rs:1092-1121
    data = cpu_dataset(30_000)
    rows = np.arange(30_000, dtype=np.uint32)
    split = bin_split(0, 0, [1, 2, 4])  # 0b10110
    seg, left = oracle.partition(data, rows[500:25_500], split)
    b = data.bin(0)
    goes = np.isin(b, [1, 2, 4])
    expected_left = np.arange(500, 25_500)[goes[500:25_500]]
    expected_right = np.arange(500, 25_500)[~goes[500:25_500]]
    assert left == len(expected_left)
    assert (seg[:left] == expected_left).all()
    assert (seg[left:] == expected_right).all()


def test_add_tree_and_leaf_sums():
    # cpu.rs:1123-1179
    data = cpu_dataset(10_000)
    grad, hess = cpu_gradients(10_000)
    split = bin_split(1, 0, [0, 1])
    rows, left = oracle.partition(data, np.arange(10_000, dtype=np.uint32), split)
    node = device_node(split, ~0, ~1)
    scores = oracle.add_tree(data, [node], [0.5, -0.25], np.full(10_000, 1.0, np.float32))
    expected = np.where(data.bin(2) < 2, 1.5, 0.75).astype(np.float32)
    assert (scores == expected).all()
    leaves = [(0, left), (left, 10_000 - left)]
    sums = oracle.leaf_sums(grad, hess, rows, leaves, 1024.0, 256.0)
    for i, (b, c) in enumerate(leaves):
        r = rows[b:b + c]
        assert sums[i, 0] == int(np.rint(grad[r].astype(np.float64) * 1024.0).sum())
        assert sums[i, 1] == int(np.rint(hess[r].astype(np.float64) * 256.0).sum())


def test_malformed_tree_is_a_device_error():
    data = cpu_dataset(100)
    split = bin_split(0, 0, [0])
    bad = device_node(split, 0, ~1)  # a child pointing at itself
    with pytest.raises(Exception):
        oracle.add_tree(data, [bad], [0.0, 1.0], np.zeros(100, np.float32))


def test_histogram_thread_count_does_not_change_results():
    data = cpu_dataset(60_000)
    grad, hess = cpu_gradients(60_000)
    spec = oracle.quant_spec(2.0, 1.0, None, 4, True, 1, 0)
    packed = oracle.quantize(spec, grad, hess, data.row_offset)
    rows = np.arange(60_000, dtype=np.uint32)
    before = oracle.threads()
    try:
        oracle.set_threads(1)
        a = oracle.histogram(data, packed, 4, rows)
        oracle.set_threads(4)
        b = oracle.histogram(data, packed, 4, rows)
    finally:
        oracle.set_threads(before)
    assert (a == b).all()
