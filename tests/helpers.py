"""Datasets and generators shared by the tests (ports of the reference's test fixtures)."""

import numpy as np

import oracle
from silvic_amd import _abi
from silvic_amd.dataset import BinnedDataset, FeatureGroup, FeatureMeta, from_bins


def mix32(x):
    return oracle.lib().oracle_mix32(int(x) & 0xFFFFFFFF)


def mix32_np(x):
    """lowbias32 vectorized (quantize.rs:16-23), used only to generate test data."""
    x = np.asarray(x, dtype=np.uint64) & 0xFFFFFFFF
    x ^= x >> 16
    x = (x * 0x7FEB352D) & 0xFFFFFFFF
    x ^= x >> 15
    x = (x * 0x846CA68B) & 0xFFFFFFFF
    x ^= x >> 16
    return x.astype(np.uint32)


def cpu_dataset(rows):
    """crates/silvic-core/src/backend/cpu.rs:950-989: two groups, features 0-1 (7, 3 bins) and feature 2 (5 bins),
    bins from a hash, row_offset 100."""
    bins = [7, 3, 5]
    r = np.arange(rows, dtype=np.uint64)
    b = [(mix32_np(r * 3 + f) % bins[f]).astype(np.uint8) for f in range(3)]
    feats = [FeatureMeta(7, 0, 0, 0, _abi.BINS_CATEGORICAL), FeatureMeta(3, 0, 1, 7, _abi.BINS_CATEGORICAL),
             FeatureMeta(5, 1, 0, 10, _abi.BINS_CATEGORICAL)]
    g0 = np.zeros((rows, 4), np.uint8)
    g0[:, 0], g0[:, 1] = b[0], b[1]
    g1 = np.zeros((rows, 4), np.uint8)
    g1[:, 0] = b[2]
    groups = [FeatureGroup([0, 1], 4, 0, 10, g0.reshape(-1)), FeatureGroup([2], 4, 10, 5, g1.reshape(-1))]
    return BinnedDataset(rows, feats, groups, 15, np.zeros(rows, np.float32), row_offset=100)


def cpu_gradients(rows):
    """cpu.rs:991-998 `loaded`: g = (r % 13)/4 - 1.5, h = 0.25 + (r % 5)/8."""
    r = np.arange(rows)
    return ((r % 13) / 4.0 - 1.5).astype(np.float32), (0.25 + (r % 5) / 8.0).astype(np.float32)


def naive_histogram(data, rows, g, h):
    """cpu.rs:1000-1012: direct per-bin sums over every feature."""
    out = np.zeros(2 * data.total_bins, np.float64)
    for f, meta in enumerate(data.features):
        if meta.num_bins == 0:
            continue
        idx = meta.hist_offset + data.bin(f, rows).astype(np.int64)
        np.add.at(out, 2 * idx, g.astype(np.float64))
        np.add.at(out, 2 * idx + 1, h.astype(np.float64))
    return out


class Lcg:
    """crates/silvic-core/src/split.rs:992-1006."""

    def __init__(self, seed):
        self.s = seed

    def next(self):
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        return (self.s >> 11) / float(1 << 53)

    def below(self, n):
        return int(self.next() * n)


def learner_dataset(first, last):
    """crates/silvic-core/src/learner.rs:497-578: features of 8 (numerical), 5 (numerical + NaN bin) and 6
    (categorical) bins from a hash of the global row."""
    rows = np.arange(first, last, dtype=np.uint64)

    def h(stream):
        return mix32_np((rows & 0xFFFFFFFF) ^ mix32(stream))

    bins = [8, 5, 6]
    b = np.stack([(h(f) % bins[f]).astype(np.uint8) for f in range(3)], axis=1)
    data = from_bins(b, bins, np.zeros(len(rows), np.float32),
                     kinds=[_abi.BINS_NUMERICAL, _abi.BINS_NUMERICAL, _abi.BINS_CATEGORICAL],
                     nan_bins=[False, True, False], row_offset=first)
    return data, b


def learner_gradients(first, last, bins, zeros=False):
    """learner.rs:545-553 row_gradient."""
    rows = np.arange(first, last, dtype=np.uint64)
    noise = (mix32_np((rows & 0xFFFFFFFF) ^ 0x5BD1E995) % 1000).astype(np.float32) / np.float32(1000.0) - np.float32(0.5)
    signal = np.where(bins[:, 0] > 3, 1.0, -1.0) + np.where(bins[:, 1] == 4, 2.0, 0.0)
    cat = np.where((bins[:, 2] == 2) | (bins[:, 2] == 4), -1.5, 0.0)
    g = (signal.astype(np.float32) + cat.astype(np.float32) + noise).astype(np.float32)
    hh = (np.float32(0.5) + (rows % 7).astype(np.float32) / np.float32(7.0)).astype(np.float32)
    if zeros:
        z = (rows % 3) != 0
        g = np.where(z, 0, g).astype(np.float32)
        hh = np.where(z, 0, hh).astype(np.float32)
    return g, hh


def mirrored(half, feature):
    """`half`, then `half` again with every other numerical feature's bin order reversed (missing values stay in the
    NaN bin); `feature` is bin 0 in the first copy and bin 1 in the second."""
    n = half.num_rows
    groups = []
    for gi, g in enumerate(half.groups):
        d = np.concatenate([g.data, g.data]).reshape(2 * n, g.row_stride)
        for j in g.features:
            f = half.features[j]
            if j == feature or f.num_bins == 0:
                continue
            assert f.kind == _abi.BINS_NUMERICAL
            top = f.num_bins - 1 - int(bool(f.nan_bin))  # the last numerical bin
            col = d[n:, f.column].astype(np.int64)
            d[n:, f.column] = np.where(col <= top, top - col, col).astype(np.uint8)
        if gi == half.features[feature].group:
            c = half.features[feature].column
            d[:n, c] = 0
            d[n:, c] = 1
        groups.append(FeatureGroup(g.features, g.row_stride, g.hist_offset, g.total_bins, d.reshape(-1).copy()))
    return BinnedDataset(2 * n, half.features, groups, half.total_bins, np.concatenate([half.label, half.label]))


def row_slice(data, start, stop):
    """Rows [start, stop) of ``data`` as a dataset with the same features, groups and bins (a validation set binned
    with the training set's mappers, as silvic requires, cpu.rs:707-728)."""
    groups = []
    for g in data.groups:
        d = g.data.reshape(data.num_rows, g.row_stride)[start:stop]
        groups.append(FeatureGroup(g.features, g.row_stride, g.hist_offset, g.total_bins, d.reshape(-1).copy(),
                                   g.bin_bits))
    weight = None if data.weight is None else data.weight[start:stop].copy()
    return BinnedDataset(stop - start, data.features, groups, data.total_bins, data.label[start:stop].copy(), weight)


def joined(a, b):
    """The features of ``a`` and then ``b`` (same rows) as one dataset, ``b``'s groups and bins after ``a``'s, with
    ``a``'s labels: a dataset of both one-byte and two-byte groups."""
    assert a.num_rows == b.num_rows
    ng = len(a.groups)
    feats = list(a.features)
    for f in b.features:
        feats.append(FeatureMeta(f.num_bins, f.group + ng, f.column, f.hist_offset + a.total_bins, f.kind, f.nan_bin,
                                 f.bounds))
    groups = list(a.groups)
    nf = len(a.features)
    for g in b.groups:
        groups.append(FeatureGroup([j + nf for j in g.features], g.row_stride, g.hist_offset + a.total_bins,
                                   g.total_bins, g.data, g.bin_bits))
    return BinnedDataset(a.num_rows, feats, groups, a.total_bins + b.total_bins, a.label, a.weight)
