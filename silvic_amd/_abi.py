"""ctypes mirror of ``include/silvic_rocm.h`` and the loader of the built native libraries.

The structs below are field-for-field the header's; ``tests/test_abi.py`` checks their sizes against the
header with the C compiler. The loader fails loudly: a missing HIP library is an ``ImportError`` naming the
file and the build command, never a silent fallback.
"""

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "_lib")
ROCM_LIB = os.path.join(LIB_DIR, "libsilvic_rocm.so")
SYNTH_LIB = os.path.join(LIB_DIR, "libsilvic_synth.so")

# status codes: SilvicError::kind() (crates/silvic-core/src/error.rs:33-45)
OK = 0
ERR_CONFIG = 1
ERR_DATA = 2
ERR_DEVICE = 3
ERR_COLLECTIVE = 4
ERR_MODEL = 5
ERR_UNSUPPORTED = 6
ERR_INTERRUPTED = 7
ERR_INTERNAL = 8
KIND_NAMES = {
    ERR_CONFIG: "config",
    ERR_DATA: "data",
    ERR_DEVICE: "device",
    ERR_COLLECTIVE: "collective",
    ERR_MODEL: "model",
    ERR_UNSUPPORTED: "unsupported",
    ERR_INTERRUPTED: "interrupted",
    ERR_INTERNAL: "internal",
}

BINS_TRIVIAL, BINS_NUMERICAL, BINS_CATEGORICAL = 0, 1, 2
OBJ_REGRESSION, OBJ_BINARY, OBJ_LAMBDARANK = 0, 1, 2
BAG_ALL, BAG_BERNOULLI = 0, 1
SIDE_LEFT, SIDE_RIGHT = 0, 1


class Feature(C.Structure):
    _fields_ = [("num_bins", C.c_uint32), ("group", C.c_uint32), ("column", C.c_uint32),
                ("hist_offset", C.c_uint32), ("kind", C.c_uint32), ("nan_bin", C.c_uint32)]


class Group(C.Structure):
    _fields_ = [("row_stride", C.c_uint32), ("hist_offset", C.c_uint32), ("total_bins", C.c_uint32),
                ("num_features", C.c_uint32), ("features", C.POINTER(C.c_uint32)),
                ("data", C.POINTER(C.c_uint8)), ("bin_bits", C.c_uint32)]


class Dataset(C.Structure):
    _fields_ = [("num_rows", C.c_uint64), ("row_offset", C.c_uint64), ("num_features", C.c_uint32),
                ("num_groups", C.c_uint32), ("features", C.POINTER(Feature)), ("groups", C.POINTER(Group)),
                ("total_bins", C.c_uint64), ("label", C.POINTER(C.c_float)), ("weight", C.POINTER(C.c_float)),
                ("query_boundaries", C.POINTER(C.c_uint32)), ("num_queries", C.c_uint32)]


class Objective(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("sigmoid", C.c_double), ("norm", C.c_uint32), ("truncation_level", C.c_uint32),
                ("label_gain", C.POINTER(C.c_double)), ("num_label_gain", C.c_uint32),
                ("inverse_max_dcg", C.POINTER(C.c_double))]


class QuantSpec(C.Structure):
    _fields_ = [("inv_grad_scale", C.c_float), ("inv_hess_scale", C.c_float), ("grad_scale", C.c_double),
                ("hess_scale", C.c_double), ("grad_max_q", C.c_int32), ("hess_max_q", C.c_int32),
                ("constant_hessian", C.c_uint8), ("stochastic", C.c_uint8), ("pad_", C.c_uint8 * 2),
                ("seed", C.c_uint32), ("iteration", C.c_uint32)]


class Bag(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("seed", C.c_uint32), ("round", C.c_uint32), ("pad_", C.c_uint32),
                ("fraction", C.c_double)]


class LeafRange(C.Structure):
    _fields_ = [("begin", C.c_uint32), ("count", C.c_uint32)]


class BinSplit(C.Structure):
    _fields_ = [("group", C.c_uint32), ("column", C.c_uint32), ("left_bins", C.c_uint32 * 8)]


class DeviceNode(C.Structure):
    _fields_ = [("split", BinSplit), ("left", C.c_int32), ("right", C.c_int32)]


class SplitConfig(C.Structure):
    _fields_ = [("min_data_in_leaf", C.c_int64), ("min_sum_hessian_in_leaf", C.c_double),
                ("lambda_l1", C.c_double), ("lambda_l2", C.c_double), ("min_gain_to_split", C.c_double),
                ("max_cat_to_onehot", C.c_uint64), ("max_cat_threshold", C.c_uint64), ("cat_l2", C.c_double),
                ("cat_smooth", C.c_double), ("min_data_per_group", C.c_int64)]


class Sums(C.Structure):
    _fields_ = [("grad", C.c_double), ("hess", C.c_double), ("count", C.c_int64)]


class SplitInfo(C.Structure):
    _fields_ = [("found", C.c_int32), ("feature", C.c_int32), ("gain", C.c_double), ("threshold", C.c_uint32),
                ("default_left", C.c_uint32), ("left", Sums), ("right", Sums), ("left_output", C.c_double),
                ("right_output", C.c_double), ("categorical", C.c_uint32), ("num_cat_bins", C.c_uint32),
                ("cat_bins", C.c_uint32 * 256)]


class GrownTree(C.Structure):
    _fields_ = [("capacity_leaves", C.c_uint32), ("num_leaves", C.c_uint32),
                ("split_feature", C.POINTER(C.c_int32)), ("threshold_bin", C.POINTER(C.c_uint32)),
                ("default_left", C.POINTER(C.c_uint8)), ("left_child", C.POINTER(C.c_int32)),
                ("right_child", C.POINTER(C.c_int32)), ("split_gain", C.POINTER(C.c_float)),
                ("internal_value", C.POINTER(C.c_double)), ("internal_weight", C.POINTER(C.c_double)),
                ("internal_count", C.POINTER(C.c_int64)), ("leaf_value", C.POINTER(C.c_double)),
                ("leaf_weight", C.POINTER(C.c_double)), ("leaf_count", C.POINTER(C.c_int64)),
                ("leaf_parent", C.POINTER(C.c_int32)), ("leaf_depth", C.POINTER(C.c_int32)),
                ("leaf_range", C.POINTER(LeafRange)), ("left_bins", C.POINTER(C.c_uint32))]


class GrowSpec(C.Structure):
    _fields_ = [("cfg", SplitConfig), ("num_leaves", C.c_uint32), ("max_depth", C.c_int32),
                ("grad_scale", C.c_double), ("hess_scale", C.c_double), ("feature_mask", C.POINTER(C.c_uint8)),
                ("root", LeafRange), ("root_count", C.c_int64)]


class TrainParams(C.Structure):
    _fields_ = [("objective", C.c_uint32), ("num_leaves", C.c_uint32), ("sigmoid", C.c_double),
                ("learning_rate", C.c_double), ("max_depth", C.c_int32), ("num_grad_quant_bins", C.c_uint32),
                ("cfg", SplitConfig), ("bagging_fraction", C.c_double), ("bagging_freq", C.c_uint32),
                ("bagging_seed", C.c_uint32), ("feature_fraction", C.c_double),
                ("feature_fraction_seed", C.c_uint32), ("data_random_seed", C.c_uint32),
                ("stochastic_rounding", C.c_uint8), ("quant_train_renew_leaf", C.c_uint8),
                ("boost_from_average", C.c_uint8), ("pad_", C.c_uint8)]


# Every entry point include/silvic_rocm.h declares, with its ctypes signature.
_P = C.c_void_p
_SIGNATURES = {
    "srocm_is_available": (C.c_int, []),
    "srocm_create": (C.c_int, [C.c_int, C.POINTER(C.c_void_p)]),
    "srocm_destroy": (None, [_P]),
    "srocm_last_error": (C.c_char_p, [_P]),
    "srocm_name": (C.c_int, [_P, C.c_char_p, C.c_size_t]),
    "srocm_load": (C.c_int, [_P, C.POINTER(Dataset), C.POINTER(C.POINTER(Dataset)), C.c_uint32,
                             C.POINTER(Objective)]),
    "srocm_init_scores": (C.c_int, [_P, C.c_uint32, C.c_double]),
    "srocm_compute_gradients": (C.c_int, [_P, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "srocm_set_gradients": (C.c_int, [_P, C.POINTER(C.c_float), C.POINTER(C.c_float), C.c_uint64,
                                      C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "srocm_gradients": (C.c_int, [_P, C.POINTER(C.c_float), C.POINTER(C.c_float), C.c_size_t]),
    "srocm_partition_rows": (C.c_int, [_P, C.POINTER(C.c_uint32), C.c_size_t]),
    "srocm_quantize": (C.c_int, [_P, C.POINTER(QuantSpec)]),
    "srocm_reset_partition": (C.c_int, [_P, C.POINTER(Bag), C.POINTER(C.c_uint32)]),
    "srocm_set_histogram_features": (C.c_int, [_P, C.POINTER(C.c_uint8), C.c_uint32]),
    "srocm_histogram": (C.c_int, [_P, LeafRange, C.c_int, C.POINTER(C.c_double), C.c_size_t]),
    "srocm_histogram_noalloc": (C.c_int, [_P, LeafRange, C.c_void_p, C.c_size_t, C.c_int]),
    "srocm_partition": (C.c_int, [_P, LeafRange, C.POINTER(BinSplit), C.POINTER(C.c_uint32)]),
    "srocm_partition_and_histogram": (C.c_int, [_P, LeafRange, C.POINTER(BinSplit), C.c_uint32, C.c_int,
                                                C.POINTER(C.c_double), C.c_size_t, C.POINTER(C.c_uint32)]),
    "srocm_leaf_sums": (C.c_int, [_P, C.POINTER(LeafRange), C.c_uint32, C.c_float, C.c_float,
                                  C.POINTER(C.c_int64)]),
    "srocm_add_tree": (C.c_int, [_P, C.POINTER(DeviceNode), C.c_uint32, C.POINTER(C.c_float), C.c_uint32]),
    "srocm_scores": (C.c_int, [_P, C.c_uint32, C.POINTER(C.c_float), C.c_size_t]),
    "srocm_find_best_split": (C.c_int, [_P, C.POINTER(C.c_double), C.c_size_t, C.POINTER(Feature), C.c_uint32,
                                        C.POINTER(C.c_uint8),
                                        C.POINTER(Sums), C.c_double, C.c_double, C.POINTER(SplitConfig),
                                        C.POINTER(SplitInfo), C.POINTER(C.c_uint8)]),
    "srocm_hist_slots": (C.c_int, [_P, C.c_uint32]),
    "srocm_histogram_slot": (C.c_int, [_P, LeafRange, C.c_uint32]),
    "srocm_partition_and_histogram_slot": (C.c_int, [_P, LeafRange, C.POINTER(BinSplit), C.c_uint32, C.c_uint32,
                                                     C.POINTER(C.c_uint32)]),
    "srocm_subtract": (C.c_int, [_P, C.c_uint32, C.c_uint32]),
    "srocm_find_best_split_slot": (C.c_int, [_P, C.c_uint32, C.POINTER(Feature), C.c_uint32, C.POINTER(C.c_uint8),
                                             C.POINTER(Sums), C.c_double, C.c_double, C.POINTER(SplitConfig),
                                             C.POINTER(SplitInfo), C.POINTER(C.c_uint8)]),
    "srocm_read_slot": (C.c_int, [_P, C.c_uint32, C.POINTER(C.c_double), C.c_size_t]),
    "srocm_grow": (C.c_int, [_P, C.POINTER(GrowSpec), C.POINTER(GrownTree)]),
    "srocm_boost_init": (C.c_int, [_P, C.POINTER(TrainParams), C.POINTER(C.c_double)]),
    "srocm_boost": (C.c_int, [_P, C.POINTER(TrainParams), C.c_uint32, C.c_uint32, C.POINTER(GrownTree),
                              C.POINTER(C.c_uint32)]),
    "srocm_profile": (C.c_int, [_P, C.c_int]),
    "srocm_profile_read": (C.c_int, [_P, C.POINTER(C.c_double), C.c_uint32]),
    "srocm_slab_layout": (C.c_int, [_P, C.POINTER(C.c_uint32), C.c_uint32, C.POINTER(C.c_uint32)]),
}

EXPORTS = tuple(_SIGNATURES)

_rocm = None
_synth = None


def load_rocm():
    """The HIP backend library; raises ImportError when it has not been built."""
    global _rocm
    if _rocm is None:
        if not os.path.exists(ROCM_LIB):
            raise ImportError(f"{ROCM_LIB} is missing: build it with `python -m silvic_amd.build`")
        lib = C.CDLL(ROCM_LIB)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _rocm = lib
    return _rocm


def load_synth():
    """The synthetic-workload generator (host code only)."""
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_LIB):
            raise ImportError(f"{SYNTH_LIB} is missing: build it with `python -m silvic_amd.build`")
        lib = C.CDLL(SYNTH_LIB)
        lib.synth_create.restype = C.c_void_p
        lib.synth_create.argtypes = [C.c_uint32, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32]
        lib.synth_free.argtypes = [C.c_void_p]
        lib.synth_features.argtypes = [C.c_void_p, C.POINTER(C.c_uint32)]
        lib.synth_num_groups.restype = C.c_uint32
        lib.synth_num_groups.argtypes = [C.c_void_p]
        lib.synth_total_bins.restype = C.c_uint64
        lib.synth_total_bins.argtypes = [C.c_void_p]
        lib.synth_group.argtypes = [C.c_void_p, C.c_uint32, C.POINTER(C.c_uint32)]
        lib.synth_group_features.restype = C.POINTER(C.c_uint32)
        lib.synth_group_features.argtypes = [C.c_void_p, C.c_uint32]
        lib.synth_group_data.restype = C.POINTER(C.c_uint8)
        lib.synth_group_data.argtypes = [C.c_void_p, C.c_uint32]
        lib.synth_label.restype = C.POINTER(C.c_float)
        lib.synth_label.argtypes = [C.c_void_p]
        lib.synth_bounds.restype = C.POINTER(C.c_double)
        lib.synth_bounds.argtypes = [C.c_void_p, C.c_uint32]
        lib.synth_num_queries.restype = C.c_uint32
        lib.synth_num_queries.argtypes = [C.c_void_p]
        lib.synth_query_boundaries.restype = C.POINTER(C.c_uint32)
        lib.synth_query_boundaries.argtypes = [C.c_void_p]
        _synth = lib
    return _synth


class SilvicError(RuntimeError):
    """A failure reported by the backend; ``kind`` is ``SilvicError::kind()`` (error.rs:33-45)."""

    def __init__(self, kind, message):
        super().__init__(f"{kind}: {message}")
        self.kind = kind


class DeviceError(SilvicError):
    """``SilvicError::Device``, which the Python package raises as ``silvic.DeviceError``."""
