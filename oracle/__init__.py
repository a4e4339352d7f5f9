"""The oracle: ctypes bindings of the CPU restatement of silvic's quantized path (``silvic_oracle.cpp``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg, as the checker and the CPU baseline; the product package ``silvic_amd`` never imports it.
Build with ``make -C oracle`` (``__graft_entry__.build()`` does).
"""

import ctypes as C
import os

import numpy as np

from silvic_amd import _abi

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libsilvic_oracle.so")


class SplitInfo(C.Structure):
    """``oracle_split_info`` (silvic_oracle.h)."""

    _fields_ = [("found", C.c_int32), ("feature", C.c_int32), ("gain", C.c_double), ("categorical", C.c_int32),
                ("threshold", C.c_uint32), ("default_left", C.c_uint32), ("num_cat_bins", C.c_uint32),
                ("cat_bins", C.c_uint32 * 256), ("left", _abi.Sums), ("right", _abi.Sums),
                ("left_output", C.c_double), ("right_output", C.c_double)]


class Params(C.Structure):
    """``oracle_params`` (silvic_oracle.h); defaults from config.rs:123-167."""

    _fields_ = [("objective", C.c_uint32), ("sigmoid", C.c_double), ("num_iterations", C.c_uint32),
                ("learning_rate", C.c_double), ("num_leaves", C.c_uint32), ("max_depth", C.c_int32),
                ("cfg", _abi.SplitConfig), ("bagging_fraction", C.c_double), ("bagging_freq", C.c_uint32),
                ("bagging_seed", C.c_uint32), ("feature_fraction", C.c_double),
                ("feature_fraction_seed", C.c_uint32), ("data_random_seed", C.c_uint32),
                ("num_grad_quant_bins", C.c_uint32), ("use_quantized_grad", C.c_uint8),
                ("quant_train_renew_leaf", C.c_uint8), ("stochastic_rounding", C.c_uint8),
                ("boost_from_average", C.c_uint8), ("lambdarank_norm", C.c_uint32),
                ("lambdarank_truncation_level", C.c_uint32), ("label_gain", C.POINTER(C.c_double)),
                ("num_label_gain", C.c_uint32)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise ImportError(f"{LIB} is missing: run `make -C oracle`")
        L = C.CDLL(LIB)
        P = C.POINTER
        sig = {
            "oracle_mix32": (C.c_uint32, [C.c_uint32]),
            "oracle_mix32_n": (None, [P(C.c_uint32), C.c_uint64, P(C.c_uint32)]),
            "oracle_uniform": (C.c_float, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64]),
            "oracle_quant_spec": (None, [C.c_double, C.c_double, C.c_int, C.c_double, C.c_uint32, C.c_int,
                                         C.c_uint32, C.c_uint32, P(_abi.QuantSpec)]),
            "oracle_quantize": (None, [P(_abi.QuantSpec), P(C.c_float), P(C.c_float), C.c_uint64, C.c_uint64,
                                       P(C.c_int32)]),
            "oracle_unpack": (None, [C.c_int32, P(C.c_int32), P(C.c_int32)]),
            "oracle_in_bag": (C.c_int, [C.c_uint32, C.c_uint32, C.c_uint64, C.c_double]),
            "oracle_fixed_point_scale": (C.c_float, [C.c_double]),
            "oracle_to_fixed": (C.c_int64, [C.c_float, C.c_float]),
            "oracle_gradients": (None, [C.c_uint32, C.c_double, P(C.c_float), P(C.c_float), P(C.c_float),
                                        C.c_uint64, P(C.c_float), P(C.c_float), P(C.c_double), P(C.c_double)]),
            "oracle_init_score": (C.c_double, [C.c_uint32, C.c_double, P(C.c_float), P(C.c_float), C.c_uint64]),
            "oracle_set_threads": (None, [C.c_int]),
            "oracle_threads": (C.c_int, []),
            "oracle_histogram": (None, [P(_abi.Dataset), P(C.c_int32), C.c_int64, P(C.c_uint32), C.c_uint64,
                                        P(C.c_uint8), P(C.c_double)]),
            "oracle_partition": (C.c_uint32, [P(_abi.Dataset), P(C.c_uint32), C.c_uint64, P(_abi.BinSplit)]),
            "oracle_leaf_sums": (None, [P(C.c_float), P(C.c_float), P(C.c_uint32), P(_abi.LeafRange), C.c_uint32,
                                        C.c_float, C.c_float, P(C.c_int64)]),
            "oracle_add_tree": (C.c_int, [P(_abi.Dataset), P(_abi.DeviceNode), C.c_uint32, P(C.c_float),
                                          C.c_uint32, P(C.c_float)]),
            "oracle_find_best_split": (None, [P(C.c_double), P(_abi.Feature), C.c_uint32, P(C.c_uint8),
                                              P(_abi.Sums), C.c_double, C.c_double, P(_abi.SplitConfig),
                                              P(SplitInfo), P(C.c_uint8)]),
            "oracle_leaf_gain": (C.c_double, [C.c_double] * 4),
            "oracle_leaf_output": (C.c_double, [C.c_double] * 4),
            "oracle_feature_mask": (None, [P(_abi.Feature), C.c_uint32, C.c_double, C.c_uint32, C.c_uint32,
                                           P(C.c_uint8)]),
            "oracle_default_params": (None, [P(Params)]),
            "oracle_lambdarank_query": (None, [P(C.c_float), P(C.c_float), P(C.c_float), C.c_uint32, P(C.c_double),
                                               C.c_uint32, C.c_double, C.c_double, C.c_int, C.c_uint32,
                                               P(C.c_float), P(C.c_float)]),
            "oracle_max_dcg_at_k": (C.c_double, [C.c_uint32, P(C.c_float), C.c_uint32, P(C.c_double), C.c_uint32]),
            "oracle_sigmoid_table_get": (C.c_double, [C.c_double, C.c_double]),
            "oracle_check_labels": (C.c_int, [P(C.c_float), C.c_uint64, C.c_uint32]),
            "oracle_lambdarank_gradients": (None, [P(_abi.Dataset), P(Params), P(C.c_float), P(C.c_float),
                                                   P(C.c_float)]),
            "oracle_train": (C.c_void_p, [P(_abi.Dataset), P(Params)]),
            "oracle_model_free": (None, [C.c_void_p]),
            "oracle_model_num_trees": (C.c_uint32, [C.c_void_p]),
            "oracle_model_init_score": (C.c_double, [C.c_void_p]),
            "oracle_model_tree_leaves": (C.c_uint32, [C.c_void_p, C.c_uint32]),
            "oracle_model_tree": (None, [C.c_void_p, C.c_uint32, P(C.c_int32), P(C.c_uint32), P(C.c_int8),
                                         P(C.c_int32), P(C.c_int32), P(C.c_float), P(C.c_double), P(C.c_double),
                                         P(C.c_int64), P(C.c_double), P(C.c_double), P(C.c_int64),
                                         P(C.c_int32)]),
            "oracle_model_scores": (None, [C.c_void_p, P(C.c_float), C.c_uint64]),
            "oracle_model_times": (None, [C.c_void_p, P(C.c_double)]),
            "oracle_model_hist_bins": (C.c_double, [C.c_void_p]),
            "oracle_model_tree_left_bins": (None, [C.c_void_p, C.c_uint32, C.POINTER(C.c_uint32)]),
            "oracle_model_tree_gains": (None, [C.c_void_p, C.c_uint32, P(C.c_double), P(C.c_double)]),
            "oracle_grow_tree": (C.c_void_p, [P(_abi.Dataset), P(C.c_float), P(C.c_float), P(Params), C.c_int]),
            "oracle_model_leaf_ranges": (None, [C.c_void_p, P(_abi.LeafRange)]),
            "oracle_model_partition": (None, [C.c_void_p, P(C.c_uint32)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ptr(a, ctype):
    return a.ctypes.data_as(C.POINTER(ctype))


def set_threads(n):
    lib().oracle_set_threads(int(n))


def threads():
    return lib().oracle_threads()


def uniform(seed, stream, iteration, row):
    return lib().oracle_uniform(seed, stream, iteration, row)


def mix32(x):
    """mix32 of every element of a uint32 array."""
    x = np.ascontiguousarray(x, dtype=np.uint32)
    out = np.empty_like(x)
    lib().oracle_mix32_n(ptr(x, C.c_uint32), x.size, ptr(out, C.c_uint32))
    return out


def quant_spec(max_abs_grad, max_hess, constant_hessian=None, num_bins=4, stochastic=True, seed=1, iteration=0):
    s = _abi.QuantSpec()
    lib().oracle_quant_spec(max_abs_grad, max_hess, int(constant_hessian is not None),
                            0.0 if constant_hessian is None else constant_hessian, num_bins, int(stochastic), seed,
                            iteration, C.byref(s))
    return s


def quantize(spec, grad, hess, row_offset=0):
    grad = np.ascontiguousarray(grad, dtype=np.float32)
    hess = np.ascontiguousarray(hess, dtype=np.float32)
    out = np.empty(len(grad), dtype=np.int32)
    lib().oracle_quantize(C.byref(spec), ptr(grad, C.c_float), ptr(hess, C.c_float), len(grad), row_offset,
                          ptr(out, C.c_int32))
    return out


def unpack(packed):
    """quantize.rs:140-143, vectorized: (g, h)."""
    packed = np.asarray(packed, dtype=np.int32)
    g = (packed.astype(np.uint32) & 0xFFFF).astype(np.uint16).view(np.int16).astype(np.int32)
    h = (packed - g) >> 16
    return g, h


def gradients(objective, scores, label, sigmoid=1.0, weight=None):
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    label = np.ascontiguousarray(label, dtype=np.float32)
    n = len(scores)
    g = np.empty(n, dtype=np.float32)
    h = np.empty(n, dtype=np.float32)
    mg, mh = C.c_double(), C.c_double()
    w = None if weight is None else np.ascontiguousarray(weight, dtype=np.float32)
    lib().oracle_gradients(objective, sigmoid, ptr(scores, C.c_float), ptr(label, C.c_float),
                           None if w is None else ptr(w, C.c_float), n, ptr(g, C.c_float), ptr(h, C.c_float),
                           C.byref(mg), C.byref(mh))
    return g, h, mg.value, mh.value


def lambdarank_query(scores, label, label_gain, inverse_max_dcg, sigmoid=1.0, norm=True, truncation_level=30,
                     weight=None):
    """One query's lambdarank gradients (objective/lambdarank.rs:254-301)."""
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    label = np.ascontiguousarray(label, dtype=np.float32)
    gain = np.ascontiguousarray(label_gain, dtype=np.float64)
    n = len(scores)
    g = np.full(n, np.nan, np.float32)
    h = np.full(n, np.nan, np.float32)
    w = None if weight is None else np.ascontiguousarray(weight, dtype=np.float32)
    lib().oracle_lambdarank_query(ptr(scores, C.c_float), ptr(label, C.c_float),
                                  None if w is None else ptr(w, C.c_float), n, ptr(gain, C.c_double), len(gain),
                                  inverse_max_dcg, sigmoid, int(norm), truncation_level, ptr(g, C.c_float),
                                  ptr(h, C.c_float))
    return g, h


def max_dcg_at_k(k, labels, label_gain):
    labels = np.ascontiguousarray(labels, dtype=np.float32)
    gain = np.ascontiguousarray(label_gain, dtype=np.float64)
    return lib().oracle_max_dcg_at_k(k, ptr(labels, C.c_float), len(labels), ptr(gain, C.c_double), len(gain))


def check_labels(label, num_gains):
    """lambdarank.rs:172-188: 0 when every label passes, else 1 (not an integer), 2 (negative) or 3 (too large)."""
    label = np.ascontiguousarray(label, dtype=np.float32)
    return lib().oracle_check_labels(ptr(label, C.c_float), len(label), num_gains)


def lambdarank_gradients(data, params, scores):
    """Every query's gradients of a dataset with query boundaries, under ``params``' lambdarank settings."""
    ds = data.as_c()
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    g = np.empty(data.num_rows, np.float32)
    h = np.empty(data.num_rows, np.float32)
    lib().oracle_lambdarank_gradients(C.byref(ds), C.byref(params), ptr(scores, C.c_float), ptr(g, C.c_float),
                                      ptr(h, C.c_float))
    return g, h


def histogram(data, packed, max_quant, rows, used=None):
    ds = data.as_c()
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    rows = np.ascontiguousarray(rows, dtype=np.uint32)
    out = np.zeros(2 * data.total_bins, dtype=np.float64)
    u = None if used is None else np.ascontiguousarray(used, dtype=np.uint8)
    lib().oracle_histogram(C.byref(ds), ptr(packed, C.c_int32), max_quant, ptr(rows, C.c_uint32), len(rows),
                           None if u is None else ptr(u, C.c_uint8), ptr(out, C.c_double))
    return out


def partition(data, rows, split):
    """Stable partition of a copy of ``rows``; returns (rows, left)."""
    ds = data.as_c()
    rows = np.array(rows, dtype=np.uint32)
    left = lib().oracle_partition(C.byref(ds), ptr(rows, C.c_uint32), len(rows), C.byref(split))
    return rows, left


def leaf_sums(grad, hess, partition_rows, leaves, grad_scale, hess_scale):
    grad = np.ascontiguousarray(grad, dtype=np.float32)
    hess = np.ascontiguousarray(hess, dtype=np.float32)
    part = np.ascontiguousarray(partition_rows, dtype=np.uint32)
    arr = (_abi.LeafRange * len(leaves))(*[_abi.LeafRange(b, c) for b, c in leaves])
    out = np.zeros(2 * len(leaves), dtype=np.int64)
    lib().oracle_leaf_sums(ptr(grad, C.c_float), ptr(hess, C.c_float), ptr(part, C.c_uint32), arr, len(leaves),
                           grad_scale, hess_scale, ptr(out, C.c_int64))
    return out.reshape(-1, 2)


def add_tree(data, nodes, leaf_values, scores):
    ds = data.as_c()
    arr = (_abi.DeviceNode * max(1, len(nodes)))(*nodes)
    lv = np.ascontiguousarray(leaf_values, dtype=np.float32)
    scores = np.array(scores, dtype=np.float32)
    rc = lib().oracle_add_tree(C.byref(ds), arr, len(nodes), ptr(lv, C.c_float), len(lv), ptr(scores, C.c_float))
    if rc != 0:
        raise _abi.SilvicError("device", "malformed device tree")
    return scores


def split_config(**kw):
    """SplitConfig from config.rs defaults (min_data_in_leaf 20, ...), overridden by ``kw``."""
    c = _abi.SplitConfig(20, 1e-3, 0.0, 0.0, 0.0, 4, 32, 10.0, 10.0, 100)
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def features_c(features):
    arr = (_abi.Feature * max(1, len(features)))()
    for i, f in enumerate(features):
        arr[i] = _abi.Feature(f.num_bins, f.group, f.column, f.hist_offset, f.kind, int(bool(f.nan_bin)))
    return arr


def find_best_split(hist, features, evaluate, sums, grad_scale=1.0, hess_scale=1.0, cfg=None):
    """split.rs:919-961; ``sums`` is (grad, hess, count). Returns (SplitInfo, splittable)."""
    hist = np.ascontiguousarray(hist, dtype=np.float64)
    ev = np.ascontiguousarray(evaluate, dtype=np.uint8)
    cfg = split_config() if cfg is None else cfg
    out = SplitInfo()
    spl = np.zeros(len(features), dtype=np.uint8)
    s = _abi.Sums(*sums)
    lib().oracle_find_best_split(ptr(hist, C.c_double), features_c(features), len(features), ptr(ev, C.c_uint8),
                                 C.byref(s), grad_scale, hess_scale, C.byref(cfg), C.byref(out), ptr(spl, C.c_uint8))
    return out, spl.astype(bool)


def feature_mask(features, fraction, seed, iteration):
    m = np.zeros(len(features), dtype=np.uint8)
    lib().oracle_feature_mask(features_c(features), len(features), fraction, seed, iteration, ptr(m, C.c_uint8))
    return m.astype(bool)


def default_params(**kw):
    p = Params()
    lib().oracle_default_params(C.byref(p))
    for k, v in kw.items():
        if k in {f[0] for f in _abi.SplitConfig._fields_}:
            setattr(p.cfg, k, v)
        else:
            setattr(p, k, v)
    return p


class Model:
    """A trained oracle model: trees as numpy arrays, final scores, per-op times."""

    def __init__(self, handle, num_rows):
        L = lib()
        self.init_score = L.oracle_model_init_score(handle)
        self.trees = []
        for t in range(L.oracle_model_num_trees(handle)):
            nl = L.oracle_model_tree_leaves(handle, t)
            ni = max(nl - 1, 0)
            a = {
                "split_feature": np.zeros(ni, np.int32), "threshold_bin": np.zeros(ni, np.uint32),
                "decision_type": np.zeros(ni, np.int8), "left_child": np.zeros(ni, np.int32),
                "right_child": np.zeros(ni, np.int32), "split_gain": np.zeros(ni, np.float32),
                "internal_value": np.zeros(ni, np.float64), "internal_weight": np.zeros(ni, np.float64),
                "internal_count": np.zeros(ni, np.int64), "leaf_value": np.zeros(nl, np.float64),
                "leaf_weight": np.zeros(nl, np.float64), "leaf_count": np.zeros(nl, np.int64),
                "leaf_depth": np.zeros(nl, np.int32),
            }
            types = [C.c_int32, C.c_uint32, C.c_int8, C.c_int32, C.c_int32, C.c_float, C.c_double, C.c_double,
                     C.c_int64, C.c_double, C.c_double, C.c_int64, C.c_int32]
            L.oracle_model_tree(handle, t, *[ptr(v, ty) for v, ty in zip(a.values(), types)])
            a["num_leaves"] = nl
            lb = np.zeros(8 * max(ni, 1), np.uint32)
            L.oracle_model_tree_left_bins(handle, t, ptr(lb, C.c_uint32))
            a["left_bins"] = lb[: 8 * ni].reshape(-1, 8)
            a["commit_gain"], a["open_gain"] = np.zeros(ni, np.float64), np.zeros(nl, np.float64)
            L.oracle_model_tree_gains(handle, t, ptr(a["commit_gain"], C.c_double), ptr(a["open_gain"], C.c_double))
            self.trees.append(a)
        self.scores = np.zeros(num_rows, np.float32)
        L.oracle_model_scores(handle, ptr(self.scores, C.c_float), num_rows)
        t = np.zeros(9, np.float64)
        L.oracle_model_times(handle, ptr(t, C.c_double))
        self.times = dict(zip(["gradients", "quantize", "reset_partition", "histogram", "partition",
                               "split_search", "leaf_sums", "add_tree", "total"], t.tolist()))
        self.hist_bins = L.oracle_model_hist_bins(handle)
        # the last tree's partition (empty for a model that grew no tree)
        self.partition = np.zeros(num_rows, np.uint32)
        if self.trees:
            L.oracle_model_partition(handle, ptr(self.partition, C.c_uint32))


def train(data, params):
    ds = data.as_c()
    h = lib().oracle_train(C.byref(ds), C.byref(params))
    if not h:
        raise _abi.SilvicError("internal", "oracle training failed")
    try:
        return Model(h, data.num_rows)
    finally:
        lib().oracle_model_free(h)


def grow_tree(data, grad, hess, params, renew=True):
    """One tree from given gradients; returns (tree dict, leaf ranges (n x 2), partition)."""
    ds = data.as_c()
    grad = np.ascontiguousarray(grad, dtype=np.float32)
    hess = np.ascontiguousarray(hess, dtype=np.float32)
    h = lib().oracle_grow_tree(C.byref(ds), ptr(grad, C.c_float), ptr(hess, C.c_float), C.byref(params), int(renew))
    if not h:
        raise _abi.SilvicError("internal", "oracle grow failed")
    try:
        m = Model(h, data.num_rows)
        tree = m.trees[0]
        ranges = (_abi.LeafRange * tree["num_leaves"])()
        lib().oracle_model_leaf_ranges(h, ranges)
        part = np.zeros(data.num_rows, np.uint32)
        lib().oracle_model_partition(h, ptr(part, C.c_uint32))
        return tree, np.array([[r.begin, r.count] for r in ranges], np.int64), part
    finally:
        lib().oracle_model_free(h)
