"""srocm_histogram_noalloc (the entry point that allocates nothing) against srocm_histogram, through the C ABI: calls
in a row, each on a smaller leaf, each bit for bit equal to the allocating entry point's histogram, with and without
waiting; and the device's free memory unchanged over many calls. The device output buffer comes from the HIP runtime
the library itself links (ctypes), not from torch."""

import ctypes as C

import numpy as np
import pytest

import oracle
import silvic_amd
from silvic_amd import _abi, bin_split

pytestmark = pytest.mark.gpu


def _hip():
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    hip.hipFree.argtypes = [C.c_void_p]
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    return hip


def _free_bytes(hip):
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipDeviceSynchronize() == 0
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def _noalloc(rocm, hip, dbuf, leaf, n, wait=1):
    rc = rocm._lib.srocm_histogram_noalloc(rocm._h, _abi.LeafRange(*leaf), dbuf, n, wait)
    rocm._check(rc)
    if not wait:
        assert hip.hipDeviceSynchronize() == 0
    out = np.empty(n, np.int64)
    assert hip.hipMemcpy(out.ctypes.data, dbuf, n * 8, 2) == 0  # hipMemcpyDeviceToHost
    return out


def test_noalloc_histogram_matches_the_allocating_one():
    print("[case] noalloc histogram 400000 x 128", flush=True)
    data = silvic_amd.synthetic(2, rows=400_000, cols=128, seed=21)
    rng = np.random.default_rng(0)
    scores = (rng.standard_normal(data.num_rows) * 0.5).astype(np.float32)
    g, h, _, _ = oracle.gradients(_abi.OBJ_BINARY, scores, data.label)
    rocm = silvic_amd.RocmBackend(0)
    hip = _hip()
    dbuf = C.c_void_p()
    n = 2 * data.total_bins
    assert hip.hipMalloc(C.byref(dbuf), n * 8) == 0
    try:
        rocm.load(data)
        mg, mh = rocm.set_gradients(g, h)
        rocm.quantize(oracle.quant_spec(mg, mh, None, 4, True, 1, 0))
        rows = rocm.reset_partition()
        meta = data.features[3]
        left = rocm.partition((0, rows), bin_split(meta.group, meta.column, list(range(meta.num_bins // 3))))
        for leaf in ((0, rows), (left, rows - left), (17, min(5000, left - 17))):
            print("[case] leaf", leaf, flush=True)
            want = rocm.histogram(leaf)
            got = _noalloc(rocm, hip, dbuf, leaf, n)
            assert np.array_equal(got.astype(np.float64), want), leaf
        # an empty leaf is zeros, as the allocating entry point's
        assert not _noalloc(rocm, hip, dbuf, (5, 0), n).any()
        # without waiting: the result is there once the device has finished
        want = rocm.histogram((left, rows - left))
        assert np.array_equal(_noalloc(rocm, hip, dbuf, (left, rows - left), n, wait=0).astype(np.float64), want)
        # no device memory is taken by the calls: the free bytes do not move over many of them, waiting or not
        before = _free_bytes(hip)
        for k in range(24):
            leaf = (0, rows) if k % 3 == 0 else (left, rows - left) if k % 3 == 1 else (17, 4000 + k)
            rc = rocm._lib.srocm_histogram_noalloc(rocm._h, _abi.LeafRange(*leaf), dbuf, n, k % 2)
            rocm._check(rc)
        assert _free_bytes(hip) == before
    finally:
        rocm.close()
        hip.hipFree(dbuf)


def test_noalloc_refuses_units_its_scratch_cannot_spread():
    # with the widest units a workgroup may add at most (2^31 - 1) / 65535 rows; the allocating entry point spreads a
    # 10M-row leaf over enough workgroups, the scratch holds too few of them, so the no-allocation one refuses it
    print("[case] noalloc widest units 10000000 x 4", flush=True)
    data = silvic_amd.synthetic(2, rows=10_000_000, cols=4, seed=5)
    rng = np.random.default_rng(1)
    scores = (rng.standard_normal(data.num_rows) * 0.5).astype(np.float32)
    g, h, _, _ = oracle.gradients(_abi.OBJ_BINARY, scores, data.label)
    rocm = silvic_amd.RocmBackend(0)
    hip = _hip()
    dbuf = C.c_void_p()
    n = 2 * data.total_bins
    assert hip.hipMalloc(C.byref(dbuf), n * 8) == 0
    try:
        rocm.load(data)
        rocm.set_gradients(g, h)
        wide = oracle.quant_spec(1.0, 1.0, None, 4, True, 1, 0)
        wide.grad_max_q, wide.hess_max_q = 32767, 65535
        rocm.quantize(wide)
        rows = rocm.reset_partition()
        want = rocm.histogram((0, rows))
        assert np.array_equal(want, oracle.histogram(data, oracle.quantize(wide, g, h), 65535,
                                                     np.arange(rows, dtype=np.uint32)))
        with pytest.raises(_abi.SilvicError) as e:
            _noalloc(rocm, hip, dbuf, (0, rows), n)
        assert e.value.kind == "unsupported" and "scratch's limit" in str(e.value)
        # a leaf the scratch's workgroups can take still matches
        print("[case] noalloc widest units, 2M-row leaf", flush=True)
        assert np.array_equal(_noalloc(rocm, hip, dbuf, (0, 2_000_000), n).astype(np.float64),
                              rocm.histogram((0, 2_000_000)))
    finally:
        rocm.close()
        hip.hipFree(dbuf)
