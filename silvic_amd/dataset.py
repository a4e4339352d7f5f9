"""Binned training data as silvic lays it out (crates/silvic-core/src/data/mod.rs:24-88).

``BinnedDataset`` holds every feature's metadata and the row-major bins of each feature group, and turns itself
into the ``srocm_dataset`` struct of ``include/silvic_rocm.h`` for both the HIP backend and the oracle.
``synthetic`` builds the benchmark configurations through the native generator.
"""

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _abi

GROUP_BIN_BUDGET = 8192  # data/mod.rs:22


@dataclass
class FeatureMeta:
    """FeatureMeta (data/mod.rs:24-36); ``bounds`` are a numerical feature's upper bounds."""

    num_bins: int
    group: int
    column: int
    hist_offset: int
    kind: int = _abi.BINS_NUMERICAL
    nan_bin: bool = False
    bounds: np.ndarray = None

    @property
    def is_trivial(self):
        return self.num_bins == 0


@dataclass
class FeatureGroup:
    """FeatureGroup (data/mod.rs:48-59): ``data[row * row_stride + column]``. ``bin_bits`` (extensions silvic does
    not have): 8, silvic's byte bins; 16, each bin a little-endian u16 at byte offset ``column`` (max_bin > 255);
    4, two bins a byte, ``column`` counting 4-bit slots (the low half of byte column // 2 first)."""

    features: list
    row_stride: int
    hist_offset: int
    total_bins: int
    data: np.ndarray
    bin_bits: int = 8


@dataclass
class BinnedDataset:
    """BinnedDataset (data/mod.rs:61-74)."""

    num_rows: int
    features: list
    groups: list
    total_bins: int
    label: np.ndarray
    weight: np.ndarray = None
    row_offset: int = 0
    query_boundaries: np.ndarray = None  # ranking: num_queries + 1 row offsets
    _keep: list = field(default_factory=list, repr=False)

    def bin(self, feature, rows=None):
        """Bins of ``feature`` at ``rows`` (all rows by default), as ``BinnedDataset::bin`` (data/mod.rs:81-87)."""
        meta = self.features[feature]
        g = self.groups[meta.group]
        m = g.data.reshape(self.num_rows, g.row_stride)
        if g.bin_bits == 16:
            col = m[:, meta.column].astype(np.uint16) | (m[:, meta.column + 1].astype(np.uint16) << 8)
        elif g.bin_bits == 4:
            col = (m[:, meta.column // 2] >> (4 * (meta.column % 2))) & 15
        else:
            col = m[:, meta.column]
        return col if rows is None else col[rows]

    def as_c(self):
        """The ``srocm_dataset`` view of this dataset; valid while the dataset lives."""
        feats = (_abi.Feature * max(1, len(self.features)))()
        for i, f in enumerate(self.features):
            feats[i] = _abi.Feature(f.num_bins, f.group, f.column, f.hist_offset, f.kind, int(bool(f.nan_bin)))
        groups = (_abi.Group * max(1, len(self.groups)))()
        keep = [feats, groups]
        for i, g in enumerate(self.groups):
            fidx = np.ascontiguousarray(np.asarray(g.features, dtype=np.uint32))
            data = np.ascontiguousarray(g.data, dtype=np.uint8)
            keep += [fidx, data]
            groups[i] = _abi.Group(g.row_stride, g.hist_offset, g.total_bins, len(g.features),
                                   fidx.ctypes.data_as(C.POINTER(C.c_uint32)),
                                   data.ctypes.data_as(C.POINTER(C.c_uint8)), g.bin_bits)
        label = np.ascontiguousarray(self.label, dtype=np.float32)
        keep.append(label)
        weight = None
        if self.weight is not None:
            weight = np.ascontiguousarray(self.weight, dtype=np.float32)
            keep.append(weight)
        qb, nq = None, 0
        if self.query_boundaries is not None:
            qarr = np.ascontiguousarray(self.query_boundaries, dtype=np.uint32)
            keep.append(qarr)
            qb, nq = qarr.ctypes.data_as(C.POINTER(C.c_uint32)), len(qarr) - 1
        ds = _abi.Dataset(
            self.num_rows, self.row_offset, len(self.features), len(self.groups), feats, groups, self.total_bins,
            label.ctypes.data_as(C.POINTER(C.c_float)),
            weight.ctypes.data_as(C.POINTER(C.c_float)) if weight is not None else None, qb, nq)
        self._keep = keep
        return ds


def layout(num_bins, kinds=None, nan_bins=None):
    """Feature metadata and groups for per-feature bin counts, as ``layout`` (data/build.rs:336-383): non-trivial
    features in order, a new group whenever the next feature would take the current one over 8192 bins, each
    group's row stride its feature count rounded up to 4. Returns ``(features, group_members, total_bins)``."""
    features, groups = [], []
    offset = 0
    totals = []
    for j, nb in enumerate(num_bins):
        kind = _abi.BINS_NUMERICAL if kinds is None else kinds[j]
        nan = False if nan_bins is None else bool(nan_bins[j])
        if nb == 0:
            features.append(FeatureMeta(0, 0, 0, offset, _abi.BINS_TRIVIAL, False))
            continue
        if not groups or totals[-1] + nb > GROUP_BIN_BUDGET:
            groups.append([])
            totals.append(0)
        features.append(FeatureMeta(nb, len(groups) - 1, len(groups[-1]), offset, kind, nan))
        groups[-1].append(j)
        totals[-1] += nb
        offset += nb
    return features, groups, offset


def from_bins(bins, num_bins, label, kinds=None, nan_bins=None, weight=None, row_offset=0):
    """A dataset from a dense ``rows x features`` uint8 bin matrix (bins below each feature's ``num_bins``)."""
    bins = np.asarray(bins, dtype=np.uint8)
    rows = bins.shape[0]
    features, members, total = layout(num_bins, kinds, nan_bins)
    groups = []
    for gi, mem in enumerate(members):
        stride = (len(mem) + 3) // 4 * 4
        data = np.zeros((rows, stride), dtype=np.uint8)
        for c, j in enumerate(mem):
            data[:, c] = bins[:, j]
        first = features[mem[0]].hist_offset
        groups.append(FeatureGroup(list(mem), stride, first, sum(features[j].num_bins for j in mem),
                                   data.reshape(-1)))
    return BinnedDataset(rows, features, groups, total, np.asarray(label, dtype=np.float32),
                         None if weight is None else np.asarray(weight, dtype=np.float32), row_offset)


# The benchmark configurations: (config id, rows, features, max_bin, objective)
CONFIGS = {
    1: (100_000, 28, 255, _abi.OBJ_REGRESSION),
    2: (10_000_000, 128, 255, _abi.OBJ_BINARY),
    3: (2_000_000, 136, 255, _abi.OBJ_LAMBDARANK),
    4: (1_000_000, 2000, 63, _abi.OBJ_BINARY),
    5: (50_000_000, 32, 1023, _abi.OBJ_REGRESSION),
}


def as_categorical(data, features):
    """``data`` with the numerical ``features`` turned categorical: the NaN bin (or none) becomes bin 0, the bin of
    silvic's categorical mappers for negative / missing / unseen values (data/bin_mapper.rs), and value bin b becomes
    category bin b + 1. The bin count is unchanged when the feature has a NaN bin. Modifies ``data`` in place."""
    for j in features:
        m = data.features[j]
        if m.kind != _abi.BINS_NUMERICAL or not m.num_bins:
            raise ValueError(f"feature {j} is not a numerical feature with bins")
        if not m.nan_bin:
            raise ValueError(f"feature {j} has no NaN bin to become the categorical bin 0")
        g = data.groups[m.group]
        col = g.data.reshape(data.num_rows, g.row_stride)[:, m.column]
        nan = m.num_bins - 1
        col[:] = np.where(col == nan, 0, col.astype(np.int32) + 1).astype(np.uint8)
        m.kind = _abi.BINS_CATEGORICAL
        m.nan_bin = False
        m.bounds = None
    return data


def pack_nibbles(data, min_run=2):
    """``data`` with its features of at most 16 bins stored two to a byte (``bin_bits`` 4), the others as they were:
    each run of at least ``min_run`` consecutive such features of one byte group becomes a group of its own. Bins,
    histogram offsets, feature order and every bin value are unchanged, so a learner sees the same dataset."""
    new_groups, metas = [], [FeatureMeta(**vars(f)) for f in data.features]
    for g in data.groups:
        if g.bin_bits not in (0, 8):
            new_groups.append(g)
            continue
        rows = g.data.reshape(data.num_rows, g.row_stride)
        runs, cur = [], []  # consecutive features, split where a feature has more than 16 bins
        for f in g.features:
            small = 0 < data.features[f].num_bins <= 16
            if cur and small != cur[0][1]:
                runs.append(cur)
                cur = []
            cur.append((f, small))
        if cur:
            runs.append(cur)
        for run in runs:
            fs = [f for f, _ in run]
            nib = run[0][1] and len(fs) >= min_run
            slots = len(fs)
            stride = ((slots + 1) // 2 + 3) // 4 * 4 if nib else (slots + 3) // 4 * 4
            packed = np.zeros((data.num_rows, stride), np.uint8)
            for k, f in enumerate(fs):
                b = rows[:, data.features[f].column]
                if nib:
                    packed[:, k // 2] |= (b & 15) << (4 * (k % 2))
                else:
                    packed[:, k] = b
                metas[f].group = len(new_groups)
                metas[f].column = k
            lo = min(data.features[f].hist_offset for f in fs)
            hi = max(data.features[f].hist_offset + data.features[f].num_bins for f in fs)
            new_groups.append(FeatureGroup(fs, stride, lo, hi - lo, packed.reshape(-1), 4 if nib else 8))
    return BinnedDataset(data.num_rows, metas, new_groups, data.total_bins, data.label, data.weight,
                         data.row_offset, data.query_boundaries)


def synthetic(config, rows=None, cols=None, seed=7, max_bin=None, categorical=False):
    """Configuration ``config`` (1-5) as a binned dataset, generated natively; ``rows``/``cols`` shrink it.
    Configuration 3 carries query boundaries (Zipf-like sizes in 10..200).
    ``categorical``: config 2's integer features (the last quarter) as categorical features (see as_categorical)."""
    lib = _abi.load_synth()
    drows, dcols, dbin, _ = CONFIGS[config]
    rows = drows if rows is None else rows
    cols = dcols if cols is None else cols
    max_bin = dbin if max_bin is None else max_bin
    h = lib.synth_create(config, rows, cols, seed, max_bin)
    if not h:
        raise ValueError(f"cannot generate config {config} with {rows} rows x {cols} features")
    try:
        meta = np.zeros(6 * cols, dtype=np.uint32)
        lib.synth_features(h, meta.ctypes.data_as(C.POINTER(C.c_uint32)))
        meta = meta.reshape(cols, 6)
        features = []
        for j in range(cols):
            nb, g, c, off, kind, nan = (int(v) for v in meta[j])
            bounds = None
            if nb:
                nbounds = nb - nan
                bounds = np.ctypeslib.as_array(lib.synth_bounds(h, j), shape=(nbounds,)).copy()
            features.append(FeatureMeta(nb, g, c, off, kind, bool(nan), bounds))
        groups = []
        info = (C.c_uint32 * 5)()
        for g in range(lib.synth_num_groups(h)):
            lib.synth_group(h, g, info)
            stride, off, total, nf, bits = (int(v) for v in info)
            fidx = np.ctypeslib.as_array(lib.synth_group_features(h, g), shape=(nf,)).copy()
            data = np.ctypeslib.as_array(lib.synth_group_data(h, g), shape=(rows * stride,)).copy()
            groups.append(FeatureGroup([int(f) for f in fidx], stride, off, total, data, bits))
        label = np.ctypeslib.as_array(lib.synth_label(h), shape=(rows,)).copy()
        total = int(lib.synth_total_bins(h))
        nq = int(lib.synth_num_queries(h))
        queries = np.ctypeslib.as_array(lib.synth_query_boundaries(h), shape=(nq + 1,)).copy() if nq else None
    finally:
        lib.synth_free(h)
    data = BinnedDataset(rows, features, groups, total, label, query_boundaries=queries)
    if categorical:
        if config != 2:
            raise ValueError("categorical features are defined for configuration 2")
        ints = [j for j in range(3 * cols // 4, cols) if features[j].num_bins and features[j].nan_bin]
        as_categorical(data, ints)
    return data
