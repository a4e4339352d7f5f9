"""``RocmBackend``: silvic-core's ``trait Backend`` (crates/silvic-core/src/backend/mod.rs:115-179) over the C ABI
of ``include/silvic_rocm.h``, plus the device-side extension (split search, whole-tree growth, boosting).

Method names, argument meaning and errors follow the trait: a failure raises ``SilvicError`` whose ``kind`` is
``SilvicError::kind()`` (``DeviceError`` for ``device``), never a crash; histograms come back as ``2 *
total_bins`` float64 integers in quantized mode.
"""

import ctypes as C

import numpy as np

from . import _abi
from ._abi import BinSplit, DeviceNode, LeafRange


# LightGBM's default label_gain: 2^i - 1 for i < 31 (config.rs:118-121)
DEFAULT_LABEL_GAIN = [float((1 << i) - 1) for i in range(31)]

def _p(a, t):
    return a.ctypes.data_as(C.POINTER(t))


class RocmBackend:
    """One MI355X (gfx950) device. ``available()`` never raises."""

    @staticmethod
    def available():
        try:
            return bool(_abi.load_rocm().srocm_is_available())
        except (ImportError, OSError):
            return False

    def __init__(self, ordinal=-1):
        self._lib = _abi.load_rocm()
        h = C.c_void_p()
        rc = self._lib.srocm_create(ordinal, C.byref(h))
        if rc != _abi.OK:
            self._raise(rc, self._lib.srocm_last_error(None))
        self._h = h
        self.total_bins = 0
        self.num_features = 0
        self._datasets = []

    def close(self):
        if getattr(self, "_h", None):
            self._lib.srocm_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _raise(rc, msg):
        kind = _abi.KIND_NAMES.get(rc, "internal")
        msg = (msg or b"").decode("utf-8", "replace")
        if rc == _abi.ERR_DEVICE:
            raise _abi.DeviceError(kind, msg)
        raise _abi.SilvicError(kind, msg)

    def _check(self, rc):
        if rc != _abi.OK:
            self._raise(rc, self._lib.srocm_last_error(self._h))

    # -- trait Backend ------------------------------------------------------------------------------

    def name(self):
        buf = C.create_string_buffer(256)
        self._check(self._lib.srocm_name(self._h, buf, 256))
        return buf.value.decode()

    def slab_layout(self):
        """The loaded training set's slabs (``srocm_slab_layout``): per slab its LDS columns, row bytes, features a
        column (0: stacked by bin count) and whether it holds two-byte bins, separate 32-bit g/h counters or stacked
        features."""
        n = C.c_uint32()
        self._check(self._lib.srocm_slab_layout(self._h, None, 0, C.byref(n)))
        out = (C.c_uint32 * (4 * max(n.value, 1)))()
        self._check(self._lib.srocm_slab_layout(self._h, out, n.value, C.byref(n)))
        return [dict(width=out[4 * i], row_bytes=out[4 * i + 1], pack=out[4 * i + 2], wide=bool(out[4 * i + 3] & 1),
                     q32=bool(out[4 * i + 3] & 2), dense=bool(out[4 * i + 3] & 4)) for i in range(n.value)]

    def load(self, train, valid=(), objective=_abi.OBJ_REGRESSION, sigmoid=1.0, norm=True, truncation_level=30,
             label_gain=None, inverse_max_dcg=None):
        """``Backend::load`` (mod.rs:125-126). Lambdarank takes ``ObjectiveSetup::LambdaRank``'s fields
        (mod.rs:62-71): ``label_gain`` defaults to LightGBM's 2^i - 1 (i < 31), and ``inverse_max_dcg`` (one per
        training query) is derived from the labels by the backend when not given."""
        t = train.as_c()
        vs = [v.as_c() for v in valid]
        arr = (C.POINTER(_abi.Dataset) * max(1, len(vs)))(*[C.pointer(v) for v in vs])
        gain = np.ascontiguousarray(DEFAULT_LABEL_GAIN if label_gain is None else label_gain, dtype=np.float64)
        inv = None if inverse_max_dcg is None else np.ascontiguousarray(inverse_max_dcg, dtype=np.float64)
        obj = _abi.Objective(objective, sigmoid, int(bool(norm)), int(truncation_level), _p(gain, C.c_double),
                             len(gain), None if inv is None else _p(inv, C.c_double))
        self._check(self._lib.srocm_load(self._h, C.byref(t), arr, len(vs), C.byref(obj)))
        self._datasets = [train, *valid]
        self.total_bins = train.total_bins
        self.num_features = len(train.features)

    def init_scores(self, dataset, value):
        self._check(self._lib.srocm_init_scores(self._h, dataset, value))

    def compute_gradients(self):
        """``Backend::compute_gradients``: (max |g|, max |h|)."""
        g, h = C.c_double(), C.c_double()
        self._check(self._lib.srocm_compute_gradients(self._h, C.byref(g), C.byref(h)))
        return g.value, h.value

    def set_gradients(self, grad, hess):
        grad = np.ascontiguousarray(grad, dtype=np.float32)
        hess = np.ascontiguousarray(hess, dtype=np.float32)
        g, h = C.c_double(), C.c_double()
        self._check(self._lib.srocm_set_gradients(self._h, _p(grad, C.c_float), _p(hess, C.c_float), len(grad),
                                                  C.byref(g), C.byref(h)))
        return g.value, h.value

    def gradients(self):
        """The training gradients and hessians on the device (float32 arrays)."""
        n = self._datasets[0].num_rows
        g = np.zeros(n, np.float32)
        h = np.zeros(n, np.float32)
        self._check(self._lib.srocm_gradients(self._h, _p(g, C.c_float), _p(h, C.c_float), n))
        return g, h

    def partition_rows(self, count=None):
        """The backend's partition (row ids in leaf-range order), its first `count` entries (default: all rows)."""
        n = self._datasets[0].num_rows if count is None else int(count)
        out = np.zeros(n, np.uint32)
        self._check(self._lib.srocm_partition_rows(self._h, _p(out, C.c_uint32), n))
        return out

    def quantize(self, spec):
        self._check(self._lib.srocm_quantize(self._h, C.byref(spec)))

    def reset_partition(self, bag=None):
        n = C.c_uint32()
        b = bag if bag is not None else _abi.Bag(_abi.BAG_ALL, 0, 0, 0, 0.0)
        self._check(self._lib.srocm_reset_partition(self._h, C.byref(b), C.byref(n)))
        return n.value

    def set_histogram_features(self, used):
        u = np.ascontiguousarray(used, dtype=np.uint8)
        self._check(self._lib.srocm_set_histogram_features(self._h, _p(u, C.c_uint8), len(u)))

    def histogram(self, leaf, quantized=True, out=None):
        """``Backend::histogram``: ``leaf`` is (begin, count); returns (or fills) 2 * total_bins float64."""
        out = np.zeros(2 * self.total_bins, np.float64) if out is None else out
        self._check(self._lib.srocm_histogram(self._h, LeafRange(*leaf), int(quantized), _p(out, C.c_double), len(out)))
        return out

    def partition(self, leaf, split):
        left = C.c_uint32()
        self._check(self._lib.srocm_partition(self._h, LeafRange(*leaf), C.byref(split), C.byref(left)))
        return left.value

    def partition_and_histogram(self, leaf, split, side, quantized=True, out=None):
        out = np.zeros(2 * self.total_bins, np.float64) if out is None else out
        left = C.c_uint32()
        self._check(self._lib.srocm_partition_and_histogram(self._h, LeafRange(*leaf), C.byref(split), side,
                                                            int(quantized), _p(out, C.c_double), len(out),
                                                            C.byref(left)))
        return left.value, out

    def leaf_sums(self, leaves, grad_scale, hess_scale):
        arr = (LeafRange * max(1, len(leaves)))(*[LeafRange(b, c) for b, c in leaves])
        out = np.zeros(2 * len(leaves), np.int64)
        self._check(self._lib.srocm_leaf_sums(self._h, arr, len(leaves), grad_scale, hess_scale, _p(out, C.c_int64)))
        return out.reshape(-1, 2)

    def add_tree(self, nodes, leaf_values):
        arr = (DeviceNode * max(1, len(nodes)))(*nodes)
        lv = np.ascontiguousarray(leaf_values, dtype=np.float32)
        self._check(self._lib.srocm_add_tree(self._h, arr, len(nodes), _p(lv, C.c_float), len(lv)))

    def scores(self, dataset=0):
        n = self._datasets[dataset].num_rows
        out = np.zeros(n, np.float32)
        self._check(self._lib.srocm_scores(self._h, dataset, _p(out, C.c_float), n))
        return out

    # -- device-side extension ----------------------------------------------------------------------

    # Histogram slots: the learner's histograms kept on the device (srocm_hist_slots and the calls after it).
    def hist_slots(self, n):
        self._check(self._lib.srocm_hist_slots(self._h, n))

    def histogram_slot(self, leaf, slot):
        self._check(self._lib.srocm_histogram_slot(self._h, LeafRange(*leaf), slot))

    def partition_and_histogram_slot(self, leaf, split, side, slot):
        left = C.c_uint32()
        self._check(self._lib.srocm_partition_and_histogram_slot(self._h, LeafRange(*leaf), C.byref(split), side, slot,
                                                                 C.byref(left)))
        return left.value

    def subtract(self, parent_slot, child_slot):
        """learner.rs:365-367 on the device: the parent's slot becomes parent - child."""
        self._check(self._lib.srocm_subtract(self._h, parent_slot, child_slot))

    def read_slot(self, slot):
        out = np.zeros(2 * self.total_bins, np.float64)
        self._check(self._lib.srocm_read_slot(self._h, slot, _p(out, C.c_double), len(out)))
        return out

    def find_best_split_slot(self, slot, features, evaluate, sums, grad_scale, hess_scale, cfg):
        ev = np.ascontiguousarray(evaluate, dtype=np.uint8)
        feats = (_abi.Feature * max(1, len(features)))()
        for i, f in enumerate(features):
            feats[i] = _abi.Feature(f.num_bins, f.group, f.column, f.hist_offset, f.kind, int(bool(f.nan_bin)))
        out = _abi.SplitInfo()
        spl = np.zeros(len(features), np.uint8)
        s = _abi.Sums(*sums)
        self._check(self._lib.srocm_find_best_split_slot(self._h, slot, feats, len(features), _p(ev, C.c_uint8),
                                                         C.byref(s), grad_scale, hess_scale, C.byref(cfg),
                                                         C.byref(out), _p(spl, C.c_uint8)))
        return out, spl.astype(bool)

    def find_best_split(self, hist, features, evaluate, sums, grad_scale, hess_scale, cfg):
        """``split::find_best_split`` (split.rs:919-961) on the device: returns (SplitInfo, splittable bools)."""
        hist = np.ascontiguousarray(hist, dtype=np.float64)
        ev = np.ascontiguousarray(evaluate, dtype=np.uint8)
        feats = (_abi.Feature * max(1, len(features)))()
        for i, f in enumerate(features):
            feats[i] = _abi.Feature(f.num_bins, f.group, f.column, f.hist_offset, f.kind, int(bool(f.nan_bin)))
        out = _abi.SplitInfo()
        spl = np.zeros(len(features), np.uint8)
        s = _abi.Sums(*sums)
        self._check(self._lib.srocm_find_best_split(self._h, _p(hist, C.c_double), len(hist), feats, len(features),
                                                    _p(ev, C.c_uint8), C.byref(s), grad_scale, hess_scale,
                                                    C.byref(cfg), C.byref(out), _p(spl, C.c_uint8)))
        return out, spl.astype(bool)

    def grow(self, cfg, num_leaves, max_depth, grad_scale, hess_scale, feature_mask, root, root_count):
        """``Learner::grow`` on the device; returns the tree as a dict of numpy arrays."""
        mask = np.ascontiguousarray(feature_mask, dtype=np.uint8)
        spec = _abi.GrowSpec(cfg, num_leaves, max_depth, grad_scale, hess_scale, _p(mask, C.c_uint8),
                             LeafRange(*root), root_count)
        t, keep = new_tree(num_leaves)
        self._check(self._lib.srocm_grow(self._h, C.byref(spec), C.byref(t)))
        return tree_dict(t, keep)


def new_tree(capacity):
    """An ``srocm_grown_tree`` with numpy storage for ``capacity`` leaves."""
    ni = max(capacity - 1, 1)
    keep = {
        "split_feature": np.zeros(ni, np.int32), "threshold_bin": np.zeros(ni, np.uint32),
        "default_left": np.zeros(ni, np.uint8), "left_child": np.zeros(ni, np.int32),
        "right_child": np.zeros(ni, np.int32), "split_gain": np.zeros(ni, np.float32),
        "internal_value": np.zeros(ni, np.float64), "internal_weight": np.zeros(ni, np.float64),
        "internal_count": np.zeros(ni, np.int64), "leaf_value": np.zeros(capacity, np.float64),
        "leaf_weight": np.zeros(capacity, np.float64), "leaf_count": np.zeros(capacity, np.int64),
        "leaf_parent": np.zeros(capacity, np.int32), "leaf_depth": np.zeros(capacity, np.int32),
        "leaf_range": np.zeros(2 * capacity, np.uint32), "left_bins": np.zeros(8 * ni, np.uint32),
    }
    types = {np.int32: C.c_int32, np.uint32: C.c_uint32, np.uint8: C.c_uint8, np.float32: C.c_float,
             np.float64: C.c_double, np.int64: C.c_int64}
    args = {k: _p(v, types[v.dtype.type]) for k, v in keep.items() if k != "leaf_range"}
    t = _abi.GrownTree(capacity, 0, leaf_range=keep["leaf_range"].ctypes.data_as(C.POINTER(LeafRange)), **args)
    return t, keep


def tree_dict(t, keep):
    n = t.num_leaves
    ni = max(n - 1, 0)
    out = {"num_leaves": n}
    for k, v in keep.items():
        if k == "leaf_range":
            out[k] = v[: 2 * n].reshape(-1, 2).copy()
        elif k == "left_bins":
            out[k] = v[: 8 * ni].reshape(-1, 8).copy()
        elif k.startswith("leaf_"):
            out[k] = v[:n].copy()
        else:
            out[k] = v[:ni].copy()
    return out


def bin_split(group, column, left_bins):
    """A ``BinSplit`` from the set of bins going left."""
    words = [0] * 8
    for b in left_bins:
        words[b // 32] |= 1 << (b % 32)
    return BinSplit(group, column, (C.c_uint32 * 8)(*words))


def wide_bin_split(group, column, threshold, nan_bin=None):
    """A ``BinSplit`` on a feature of two-byte bins: bins up to ``threshold`` go left, and the NaN bin ``nan_bin``
    too when given (words 0 and 1 hold the rule; a bit set cannot hold 1024 bins)."""
    words = [threshold, 0 if nan_bin is None else nan_bin + 1] + [0] * 6
    return BinSplit(group, column, (C.c_uint32 * 8)(*words))


def device_node(split, left, right):
    return DeviceNode(split, left, right)
