"""Benchmark: boosting iterations/s and histogram bins/s on the 10M x 128 binary workload (int8-quantized
gradients, 255 leaves), on one MI355X, with the oracle (a C++ restatement of silvic's CPU trainer) timed on the
host's cores beside it.

One step is one boosting iteration (gradients, quantization, partition reset, whole-tree growth with every
histogram/subtraction/split scan/partition on the device, leaf renewal, score update) over the resident dataset.
Prints one JSON line.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "histogram bins/s + boosting iters/s at 10M×128 int8-quantized; % HBM peak"
HBM_PEAK_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "split_step_traffic_10Mx128.md")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes (scaled by a
    copy kernel of known size), for the default workload; None when the summary is absent."""
    import re

    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch " + re.escape(kernel) + r": (\d+)$", text, re.M)
    return float(m.group(1)) if m else None


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def copy_calibration(nbytes):
    """Four device-to-device copies of `nbytes` through the HIP runtime (its copy kernel reads and writes each byte
    once): the reference point for FETCH_SIZE / WRITE_SIZE counters."""
    import ctypes as C

    hip = C.CDLL("libamdhip64.so")
    src, dst = C.c_void_p(), C.c_void_p()
    for buf in (src, dst):
        if hip.hipMalloc(C.byref(buf), C.c_size_t(nbytes)) != 0:
            raise RuntimeError("hipMalloc failed")
    if hip.hipMemset(src, 1, C.c_size_t(nbytes)) != 0:
        raise RuntimeError("hipMemset failed")
    for _ in range(4):
        if hip.hipMemcpy(dst, src, C.c_size_t(nbytes), 3) != 0:  # hipMemcpyDeviceToDevice
            raise RuntimeError("hipMemcpy failed")
    hip.hipDeviceSynchronize()
    hip.hipFree(src)
    hip.hipFree(dst)
    log(f"copy calibration: 4 x {nbytes} B device-to-device")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--rows", type=int, default=10_000_000)
    ap.add_argument("--cols", type=int, default=128)
    ap.add_argument("--leaves", type=int, default=255)
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of oracle work for the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                    help="first run 4 device-to-device copies of MB MiB (the runtime's copy kernel): known bytes for "
                         "scaling hardware memory counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: --gpus {args.gpus} is not supported (the path is single-GPU; "
              "multi-GPU sharding is a design note, not a measured configuration)", file=sys.stderr)
        sys.exit(2)

    import ctypes as C

    import numpy as np

    import silvic_amd
    from silvic_amd import _abi

    if args.calibrate_copy:
        copy_calibration(args.calibrate_copy << 20)

    t0 = time.perf_counter()
    data = silvic_amd.synthetic(2, rows=args.rows, cols=args.cols, seed=7)
    log(f"generated {args.rows} x {args.cols} in {time.perf_counter() - t0:.1f}s; total_bins {data.total_bins}")
    params = {"objective": "binary", "num_leaves": args.leaves, "max_bin": 255, "num_grad_quant_bins": 4,
              "device_type": "rocm"}
    params.pop("max_bin")
    t0 = time.perf_counter()
    trainer = silvic_amd.Trainer(params, data)
    log(f"loaded on {trainer.backend.name()} in {time.perf_counter() - t0:.1f}s")
    lib, h = trainer.backend._lib, trainer.backend._h

    warm = trainer.step(args.warmup)
    log(f"warmup {len(warm)} iterations done")
    trainer.backend._check(lib.srocm_profile(h, 1))
    t0 = time.perf_counter()
    timed = trainer.step(args.steps)
    elapsed = time.perf_counter() - t0
    prof = (C.c_double * 15)()
    trainer.backend._check(lib.srocm_profile_read(h, prof, 15))
    trainer.backend._check(lib.srocm_profile(h, 0))
    if len(timed) != args.steps:
        log(f"training ended after {len(timed)} of {args.steps} timed iterations")
    (hist_launches, hist_ms, hist_bytes, step_launches, step_ms, step_bytes, builds, hist_rows, hist_bins,
     part_rows, _, _, grow_steps, expansions, kept) = list(prof)
    steps = max(len(timed), 1)
    iters_per_s = steps / elapsed
    # every histogram is built by k_hist (roots) or k_step_rows (split steps, which also partition)
    bins_per_s = hist_bins / ((hist_ms + step_ms) / 1e3) if hist_ms + step_ms else 0.0
    step_gbps = step_bytes / (step_ms / 1e3) / 1e9 if step_ms else 0.0
    default_workload = (args.rows, args.cols, args.leaves) == (10_000_000, 128, 255)
    traffic = measured_traffic("k_step_rows<128>") if default_workload else None
    root_gbps = hist_bytes / (hist_ms / 1e3) / 1e9 if hist_ms else 0.0
    log(f"{steps} iterations in {elapsed:.3f}s; k_step_rows: {step_launches:.0f} launches, {step_ms:.1f} ms, "
        f"{step_gbps:.0f} GB/s algorithmic; k_hist (roots): {hist_launches:.0f} launches, {hist_ms:.1f} ms, "
        f"{root_gbps:.0f} GB/s; {builds:.0f} histograms, {part_rows:.3g} rows partitioned; {grow_steps:.0f} split "
        f"steps expanded {expansions:.0f} leaves for {kept:.0f} kept splits")

    cpu = None
    if not args.no_cpu:
        import oracle

        oracle.set_threads(0)
        threads = oracle.threads()
        p = oracle.default_params(objective=_abi.OBJ_BINARY, num_leaves=args.leaves, num_iterations=1)
        t0 = time.perf_counter()
        m1 = oracle.train(data, p)
        one = time.perf_counter() - t0
        n_cpu = max(1, min(args.warmup + steps, int(args.cpu_budget / max(one, 1e-3))))
        if n_cpu > 1:
            p = oracle.default_params(objective=_abi.OBJ_BINARY, num_leaves=args.leaves, num_iterations=n_cpu)
            t0 = time.perf_counter()
            m = oracle.train(data, p)
            cpu_elapsed = time.perf_counter() - t0
        else:
            m, cpu_elapsed = m1, one
        cpu_iters = len(m.trees) / cpu_elapsed
        # the trees the oracle grew must be the device's (split features, threshold bins, counts; values 1e-6)
        gpu_trees = trainer.trees
        same = 0
        for d, o in zip(gpu_trees, m.trees):
            ok = (d["num_leaves"] == o["num_leaves"] and np.array_equal(d["split_feature"], o["split_feature"])
                  and np.array_equal(d["threshold_bin"], o["threshold_bin"])
                  and np.array_equal(d["leaf_count"], o["leaf_count"])
                  and np.allclose(d["leaf_value"], o["leaf_value"], rtol=1e-6, atol=0))
            same += int(ok)
        compared = min(len(gpu_trees), len(m.trees))
        log(f"oracle: {len(m.trees)} iterations in {cpu_elapsed:.1f}s on {threads} threads; "
            f"trees identical to the device's: {same}/{compared}")
        cpu = {"value": cpu_iters, "unit": "iters/s", "cores": threads, "kind": "port",
               "sample": f"{len(m.trees)} boosting iterations of the same {args.rows}x{args.cols} binary workload "
                         f"({args.leaves} leaves), oracle (C++ restatement of silvic's CPU trainer) on {threads} "
                         f"threads",
               "hist_bins_per_s": m.hist_bins / m.times["histogram"] if m.times["histogram"] else None,
               "trees_identical": f"{same}/{compared}", "seconds": cpu_elapsed}

    out = {
        "metric": METRIC,
        "value": iters_per_s,
        "unit": "iters/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed / steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8-quantized gradients (integer histograms), f64 split search",
        "data": "synthetic",
        "config": {"workload": f"binary, {args.rows} rows x {args.cols} f32 features binned to <=255 bins "
                               f"(half N(0,1), quarter lognormal, quarter integers, 10% NaN), {args.leaves} leaves, "
                               "num_grad_quant_bins=4", "rows": args.rows, "features": args.cols,
                   "num_leaves": args.leaves, "total_bins": data.total_bins, "parallelism": "single GPU"},
        "hist_bins_per_s": bins_per_s,
        "step_kernel_ms_per_iter": step_ms / steps,
        "root_hist_ms_per_iter": hist_ms / steps,
        "roofline": {"bound": "hbm", "achieved": step_gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": step_gbps / HBM_PEAK_GBPS, "traffic": traffic,
                     "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT) if traffic else None,
                     "kernel": "k_step_rows<128> (split step: stable partition + built-child histogram)",
                     "launches": step_launches, "avg_launch_us": step_ms / step_launches * 1e3 if step_launches else None,
                     "bytes_per_launch": step_bytes / step_launches if step_launches else None,
                     "root_k_hist": {"launches": hist_launches, "achieved": root_gbps,
                                     "avg_launch_us": hist_ms / hist_launches * 1e3 if hist_launches else None}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    trainer.backend.close()


if __name__ == "__main__":
    main()
