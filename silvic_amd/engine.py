"""``train``: silvic's ``train`` (python/silvic/engine.py:152-200) for ``device_type`` ``rocm``/``hip`` (and ``gpu``
or ``auto`` when an MI355X is present), on a binned dataset.

Parameter names and defaults are LightGBM's as silvic reads them (crates/silvic-core/src/config.rs:123-167).
The boosting loop runs natively (``srocm_boost``); every tree comes back as LightGBM tree arrays with
thresholds as bins.
"""

import ctypes as C

from . import _abi
from .backend import RocmBackend, new_tree, tree_dict

DEFAULTS = {
    "objective": "regression",
    "num_iterations": 100,
    "learning_rate": 0.1,
    "num_leaves": 31,
    "max_depth": -1,
    "min_data_in_leaf": 20,
    "min_sum_hessian_in_leaf": 1e-3,
    "lambda_l1": 0.0,
    "lambda_l2": 0.0,
    "min_gain_to_split": 0.0,
    "bagging_fraction": 1.0,
    "bagging_freq": 0,
    "bagging_seed": 3,
    "feature_fraction": 1.0,
    "feature_fraction_seed": 2,
    "data_random_seed": 1,
    "max_cat_to_onehot": 4,
    "max_cat_threshold": 32,
    "cat_l2": 10.0,
    "cat_smooth": 10.0,
    "min_data_per_group": 100,
    "boost_from_average": True,
    "sigmoid": 1.0,
    "label_gain": None,
    "lambdarank_truncation_level": 30,
    "lambdarank_norm": True,
    "use_quantized_grad": True,
    "num_grad_quant_bins": 4,
    "quant_train_renew_leaf": True,
    "stochastic_rounding": True,
    "device_type": "auto",
    "gpu_device_id": -1,
}

# LightGBM aliases silvic accepts for the keys this path reads (config.rs:169-311)
ALIASES = {
    "num_boost_round": "num_iterations", "n_estimators": "num_iterations", "num_round": "num_iterations",
    "num_trees": "num_iterations", "eta": "learning_rate", "shrinkage_rate": "learning_rate",
    "num_leaf": "num_leaves", "max_leaves": "num_leaves", "min_data": "min_data_in_leaf",
    "min_child_samples": "min_data_in_leaf", "min_child_weight": "min_sum_hessian_in_leaf",
    "reg_alpha": "lambda_l1", "reg_lambda": "lambda_l2", "min_split_gain": "min_gain_to_split",
    "subsample": "bagging_fraction", "subsample_freq": "bagging_freq", "colsample_bytree": "feature_fraction",
    "sub_feature": "feature_fraction", "device": "device_type", "application": "objective", "app": "objective",
}

OBJECTIVES = {"regression": _abi.OBJ_REGRESSION, "l2": _abi.OBJ_REGRESSION, "regression_l2": _abi.OBJ_REGRESSION,
              "mse": _abi.OBJ_REGRESSION, "binary": _abi.OBJ_BINARY, "lambdarank": _abi.OBJ_LAMBDARANK}


def resolve_params(params):
    out = dict(DEFAULTS)
    for k, v in (params or {}).items():
        out[ALIASES.get(k, k)] = v
    if out["objective"] not in OBJECTIVES:
        raise _abi.SilvicError("unsupported", f"objective {out['objective']!r} does not run on the rocm device")
    if not out["use_quantized_grad"]:  # float training stays on the CPU backend (a config error, not a device one)
        raise _abi.SilvicError("config", "device_type=rocm trains with quantized gradients only "
                                         "(use_quantized_grad=true), or use device_type=cpu")
    # the reference takes 2..=64 (config.rs:416-421); up to 32766 (16-bit units) is this backend's extension
    if not 2 <= int(out["num_grad_quant_bins"]) <= 32766 or int(out["num_grad_quant_bins"]) % 2:
        raise _abi.SilvicError("config", "num_grad_quant_bins must be even and in 2..=32766")
    return out


def choose_device(params):
    """``choose_device`` (crates/silvic-python/src/training.rs:79-105) with the rocm device added."""
    dev = str(params["device_type"]).lower()
    if dev in ("rocm", "hip", "gpu", "auto"):
        if RocmBackend.available():
            return "rocm"
        raise _abi.DeviceError("device", f"device_type={dev} but no MI355X (gfx950) device is available")
    raise _abi.SilvicError("unsupported", f"device_type={dev} is not served by silvic_amd")


def train_params(p):
    cfg = _abi.SplitConfig(int(p["min_data_in_leaf"]), float(p["min_sum_hessian_in_leaf"]), float(p["lambda_l1"]),
                           float(p["lambda_l2"]), float(p["min_gain_to_split"]), int(p["max_cat_to_onehot"]),
                           int(p["max_cat_threshold"]), float(p["cat_l2"]), float(p["cat_smooth"]),
                           int(p["min_data_per_group"]))
    return _abi.TrainParams(OBJECTIVES[p["objective"]], int(p["num_leaves"]), float(p["sigmoid"]),
                            float(p["learning_rate"]), int(p["max_depth"]), int(p["num_grad_quant_bins"]), cfg,
                            float(p["bagging_fraction"]), int(p["bagging_freq"]), int(p["bagging_seed"]),
                            float(p["feature_fraction"]), int(p["feature_fraction_seed"]),
                            int(p["data_random_seed"]), int(bool(p["stochastic_rounding"])),
                            int(bool(p["quant_train_renew_leaf"])), int(bool(p["boost_from_average"])), 0)


class Booster:
    """The trained trees (LightGBM arrays, thresholds as bins) and the initial score."""

    def __init__(self, trees, init_score, params):
        self.trees = trees
        self.init_score = init_score
        self.params = params

    def num_trees(self):
        return len(self.trees)


class Trainer:
    """A loaded device with the boosting state, so iterations can be run in steps (``step``)."""

    def __init__(self, params, train_set, backend=None, valid_sets=()):
        self.params = resolve_params(params)
        choose_device(self.params) if backend is None else None
        self.backend = backend or RocmBackend(int(self.params["gpu_device_id"]))
        p = self.params
        self.backend.load(train_set, valid=tuple(valid_sets), objective=OBJECTIVES[p["objective"]],
                          sigmoid=float(p["sigmoid"]),
                          norm=bool(p["lambdarank_norm"]), truncation_level=int(p["lambdarank_truncation_level"]),
                          label_gain=p["label_gain"])
        self.tp = train_params(self.params)
        init = C.c_double()
        self.backend._check(self.backend._lib.srocm_boost_init(self.backend._h, C.byref(self.tp), C.byref(init)))
        self.init_score = init.value
        self.iteration = 0
        self.trees = []
        self.finished = False

    def step(self, count=1):
        """Runs up to ``count`` boosting iterations; returns the trees added."""
        if self.finished or count <= 0:
            return []
        cap = int(self.params["num_leaves"])
        store = [new_tree(cap) for _ in range(count)]
        arr = (_abi.GrownTree * count)(*[t for t, _ in store])
        trained = C.c_uint32()
        self.backend._check(self.backend._lib.srocm_boost(self.backend._h, C.byref(self.tp), self.iteration, count,
                                                          arr, C.byref(trained)))
        n = trained.value
        added = [tree_dict(arr[i], store[i][1]) for i in range(n)]
        self.trees.extend(added)
        self.iteration += count
        if n < count:
            self.finished = True
        return added


def train(params, train_set, num_boost_round=100, valid_sets=()):
    """Trains ``num_boost_round`` trees (``num_iterations`` in ``params`` wins, as LightGBM's alias rules);
    ``valid_sets`` (binned with the training set's layout) have their scores updated with every tree."""
    p = resolve_params(params)
    rounds = int(p.get("num_iterations", num_boost_round)) if "num_iterations" in (params or {}) else num_boost_round
    t = Trainer(params, train_set, valid_sets=valid_sets)
    t.step(rounds)
    return Booster(t.trees, t.init_score, p)
