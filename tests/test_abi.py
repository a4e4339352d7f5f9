"""The C ABI: the libraries load on a host without a GPU, export every entry point include/silvic_rocm.h declares,
and the ctypes structs match the header's layout. No compute call is made here."""

import ctypes as C
import os
import re
import subprocess

import pytest

from silvic_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "silvic_rocm.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(srocm_\w+)\s*\(", text, re.M)))


def test_header_declarations_are_mirrored():
    assert set(declared()) == set(_abi.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _abi.load_rocm()
    for name in declared():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.ROCM_LIB], capture_output=True, text=True).stdout
    for name in declared():
        assert re.search(rf"\bT {name}$", out, re.M), name


STRUCTS = {
    "srocm_feature": _abi.Feature, "srocm_group": _abi.Group, "srocm_dataset": _abi.Dataset,
    "srocm_objective": _abi.Objective, "srocm_quant_spec": _abi.QuantSpec, "srocm_bag": _abi.Bag,
    "srocm_leaf_range": _abi.LeafRange, "srocm_bin_split": _abi.BinSplit, "srocm_device_node": _abi.DeviceNode,
    "srocm_split_config": _abi.SplitConfig, "srocm_sums": _abi.Sums, "srocm_split_info": _abi.SplitInfo,
    "srocm_grown_tree": _abi.GrownTree, "srocm_grow_spec": _abi.GrowSpec, "srocm_train_params": _abi.TrainParams,
}


def test_struct_layouts_match_the_header(tmp_path):
    src = tmp_path / "sizes.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for name in STRUCTS:
        lines.append(f'  printf("{name} %zu\\n", sizeof({name}));')
    lines.append("  return 0; }")
    src.write_text("\n".join(lines))
    exe = tmp_path / "sizes"
    subprocess.run(["gcc", "-o", str(exe), str(src)], check=True)
    sizes = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True).stdout.splitlines())
    for name, cls in STRUCTS.items():
        assert int(sizes[name]) == C.sizeof(cls), name


def test_probe_and_create_never_abort():
    lib = _abi.load_rocm()
    avail = lib.srocm_is_available()
    assert avail in (0, 1)
    if not avail:
        h = C.c_void_p()
        rc = lib.srocm_create(0, C.byref(h))
        assert rc == _abi.ERR_DEVICE
        assert lib.srocm_last_error(None)
        from silvic_amd import RocmBackend

        with pytest.raises(_abi.DeviceError):
            RocmBackend()


def test_null_context_is_an_error():
    lib = _abi.load_rocm()
    assert lib.srocm_init_scores(None, 0, 0.0) == _abi.ERR_DEVICE


def test_oracle_is_not_linked_by_the_product():
    out = subprocess.run(["nm", "-D", _abi.ROCM_LIB], capture_output=True, text=True).stdout
    assert "oracle_" not in out
    deps = subprocess.run(["ldd", _abi.ROCM_LIB], capture_output=True, text=True).stdout
    assert "oracle" not in deps


def test_float_training_is_refused_at_device_selection():
    # the backend serves quantized histograms only; float training (use_quantized_grad=false) is refused when the
    # parameters are resolved, before any device is touched, as the binding's choose_device refuses it
    import pytest

    from silvic_amd import _abi
    from silvic_amd.engine import resolve_params

    with pytest.raises(_abi.SilvicError) as e:
        resolve_params({"objective": "binary", "use_quantized_grad": False, "device_type": "rocm"})
    assert e.value.kind == "config" and "quantized gradients only" in str(e.value)
    assert resolve_params({"objective": "binary"})["use_quantized_grad"]
