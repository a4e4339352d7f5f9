"""silvic_amd: an MI355X-native (gfx950) backend for silvic's quantized-gradient histogram / split path.

- ``RocmBackend``: silvic-core's ``trait Backend`` over the C ABI of ``include/silvic_rocm.h``;
- ``train``/``Trainer``: the boosting loop with whole-tree growth on the device;
- ``BinnedDataset``/``synthetic``: silvic's binned data layout and the benchmark workloads.

The native library is required: importing the backend without it raises ``ImportError`` naming the build
command (``python -m silvic_amd.build``); nothing falls back to a CPU path.
"""

from ._abi import DeviceError, SilvicError
from .backend import RocmBackend, bin_split, device_node, wide_bin_split
from .dataset import BinnedDataset, FeatureGroup, FeatureMeta, from_bins, synthetic
from .engine import Booster, Trainer, train

__all__ = ["BinnedDataset", "Booster", "DeviceError", "FeatureGroup", "FeatureMeta", "RocmBackend", "SilvicError",
           "Trainer", "bin_split", "device_node", "from_bins", "synthetic", "train", "wide_bin_split"]
