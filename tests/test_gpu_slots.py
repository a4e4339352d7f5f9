"""The histogram-slot calls (srocm_hist_slots and the calls on slots), which keep a binding's learner histograms on
the device: a slot's histogram equals srocm_histogram's and the oracle's, the fused partition into a slot equals the
oracle's partition and child histogram, the device subtraction leaves parent - built (learner.rs:365-367), and the
split search over a slot equals the search over the same histogram from the host and the oracle's (split.rs:919-961).
Slots past the set-up count, and a slot subtracted from itself, are refused."""

import numpy as np
import pytest

import oracle
import silvic_amd
from silvic_amd import _abi, bin_split
from tests.split_cases import config
from tests.test_gpu_parity import binary_gradients, compare_split, quantized_setup, say

pytestmark = pytest.mark.gpu


def test_histogram_slots_match_the_host_calls_and_the_oracle(rocm):
    say("histogram slots")
    data = silvic_amd.synthetic(2, rows=200_000, cols=64, seed=3)
    g, h = binary_gradients(data, 1)
    spec, packed = quantized_setup(rocm, data, g, h)
    n = rocm.reset_partition()
    rows = np.arange(n, dtype=np.uint32)
    rocm.hist_slots(3)
    rocm.histogram_slot((0, n), 0)
    root = rocm.read_slot(0)
    assert np.array_equal(root, rocm.histogram((0, n)))
    assert np.array_equal(root, oracle.histogram(data, packed, 4, rows))

    meta = data.features[40]
    split = bin_split(meta.group, meta.column, range(0, 100))
    o_rows, o_left = oracle.partition(data, rows, split)
    left = rocm.partition_and_histogram_slot((0, n), split, 1, 1)  # the right child's histogram into slot 1
    assert left == o_left
    right = rocm.read_slot(1)
    assert np.array_equal(right, oracle.histogram(data, packed, 4, o_rows[o_left:]))
    rocm.subtract(0, 1)  # slot 0 becomes the left child's
    left_hist = rocm.read_slot(0)
    assert np.array_equal(left_hist, root - right)
    assert np.array_equal(left_hist, oracle.histogram(data, packed, 4, o_rows[:o_left]))
    assert np.array_equal(rocm.read_slot(1), right)

    m = next(f for f in data.features if f.num_bins)  # the leaf's sums, as learner.rs:143-153 takes them
    sums = (float(sum(left_hist[2 * (m.hist_offset + b)] for b in range(m.num_bins))),
            float(sum(left_hist[2 * (m.hist_offset + b) + 1] for b in range(m.num_bins))), o_left)
    ev = np.ones(len(data.features), bool)
    ev[5] = False
    cfg = config(min_data_in_leaf=20)
    d, dspl = rocm.find_best_split_slot(0, data.features, ev, sums, spec.grad_scale, spec.hess_scale, cfg)
    hd, hspl = rocm.find_best_split(left_hist, data.features, ev, sums, spec.grad_scale, spec.hess_scale, cfg)
    o, ospl = oracle.find_best_split(left_hist, data.features, ev, sums, spec.grad_scale, spec.hess_scale, cfg)
    assert d.found
    compare_split(d, hd, "slot against host histogram")
    compare_split(d, o, "slot against oracle")
    assert np.array_equal(dspl, hspl) and np.array_equal(dspl, np.asarray(ospl, bool))

    # an empty leaf's slot holds zeros
    rocm.histogram_slot((0, 0), 2)
    assert not rocm.read_slot(2).any()
    for bad in (lambda: rocm.histogram_slot((0, n), 3), lambda: rocm.subtract(1, 1), lambda: rocm.read_slot(7),
                lambda: rocm.subtract(0, 3)):
        with pytest.raises(_abi.SilvicError):
            bad()
