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
# The workloads: the headline (binary, the default) and two more shapes of the same path, each with its synthetic
# configuration, objective, leaves and bins. Only the headline carries the metric above; the others name theirs.
WORKLOADS = {
    "binary": dict(config=2, rows=10_000_000, cols=128, leaves=255, max_bin=255, objective="binary",
                   describe="binary, {rows} rows x {cols} f32 features binned to <=255 bins (half N(0,1), quarter "
                            "lognormal, quarter integers, 10% NaN), {leaves} leaves, num_grad_quant_bins={bins}"),
    "lambdarank": dict(config=3, rows=2_000_000, cols=136, leaves=127, max_bin=255, objective="lambdarank",
                       describe="lambdarank NDCG, {rows} documents in queries of 10-200 (Zipf-like), {cols} f32 "
                                "features, labels 0-4, <=255 bins, {leaves} leaves, truncation 30, "
                                "num_grad_quant_bins={bins}"),
    "sparse": dict(config=4, rows=1_000_000, cols=2000, leaves=63, max_bin=63, objective="binary",
                   describe="binary, {rows} rows x {cols} f32 features, 98% exact zeros (nonzeros exp(1) or integers "
                            "of cardinality 2-16), binned to <=63 bins, {leaves} leaves, num_grad_quant_bins={bins}"),
    "wide": dict(config=5, rows=50_000_000, cols=32, leaves=2047, max_bin=1023, objective="regression",
                 describe="L2 regression, {rows} rows x {cols} U[0,1) f32 features binned to <=1023 bins (two-byte "
                          "bins), piecewise-constant target, {leaves} leaves, num_grad_quant_bins={bins}"),
}
HBM_PEAK_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "split_step_traffic_10Mx128.md")


def measured_traffic(kernel, per):
    """HBM bytes per `per` ("launch" or "tree") of the kernel whose name starts with `kernel`, from the committed
    summary of rocprofv3 FETCH_SIZE / WRITE_SIZE passes over this script's timed iterations (scaled by a copy of
    known size), for the default workload; None when the summary is absent."""
    import re

    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_" + per + " " + re.escape(kernel) + r"[^:]*: (\d+)$", text, re.M)
    return float(m.group(1)) if m else None


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def kernel_key(name):
    """A short, stable name for a dispatch's kernel: the template instance of the step and histogram kernels, the
    plain name otherwise."""
    n = name.replace("void ", "").replace("srocm::", "").replace("(anonymous namespace)::", "")
    return n.split("(")[0].strip()


def timed_window(rows, warmup, steps):
    """The dispatch records of the timed iterations (after `warmup` iterations, `steps` of them) of a run of this
    script. An iteration starts after the previous tree's score update (k_add_leaf_values) that precedes its tree's
    k_grow_init, so a window begins with an iteration's gradients. `rows` are rocprofv3 CSV records in dispatch
    order."""
    starts = [i for i, r in enumerate(rows) if kernel_key(r["Kernel_Name"]).startswith("k_grow_init")]
    if warmup < 1 or len(starts) < warmup + steps:
        raise SystemExit(f"the profile holds {len(starts)} trees; a window of {steps} after {warmup} warm-up "
                         "iterations (at least one) needs more")

    def begin(t):
        if t >= len(starts):
            return len(rows)
        ends = [i for i in range(starts[t]) if kernel_key(rows[i]["Kernel_Name"]).startswith("k_add_leaf_values")]
        return ends[-1] + 1 if ends else starts[t]

    return rows[begin(warmup):begin(warmup + steps)]


def step_kernels(layout, quant_bins):
    """The k_step_rows instances the backend launches for a slab layout (RocmBackend.slab_layout()), with their
    slab counts: the last parameter says the built rows' gradients travel as one-byte codes beside the row ids
    (units of at most 7 and 15, i.e. num_grad_quant_bins up to 14, and no separate counters)."""
    out = {}
    for sl in layout:
        dp = (4 if sl["row_bytes"] <= 1024 else 8) if sl["dense"] else 0
        codes = not sl["q32"] and quant_bins <= 14
        k = (f"k_step_rows<{sl['width']}, {'true' if sl['wide'] else 'false'}, {max(sl['pack'], 1)}, "
             f"{'true' if sl['q32'] else 'false'}, {dp}, {'true' if codes else 'false'}>")
        out[k] = out.get(k, 0) + 1
    return ", ".join(f"{k} x{n}" for k, n in out.items())


def read_counters(folder):
    """rocprofv3 --pmc CSV of `folder` as (dispatch records in order, {dispatch: {counter: value}})."""
    import csv
    import glob

    files = glob.glob(os.path.join(folder, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {folder}")
    recs, vals = {}, {}
    for f in files:
        for r in csv.DictReader(open(f)):
            d = int(r["Dispatch_Id"])
            recs[d] = r
            vals.setdefault(d, {})
            vals[d][r["Counter_Name"]] = vals[d].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    order = [recs[d] for d in sorted(recs)]
    return order, vals


def pmc_summary(args):
    """Per-tree and per-launch counters of the timed window (--steps iterations after --warmup) from rocprofv3 runs
    of this script; prints a markdown summary. FETCH_SIZE / WRITE_SIZE (KiB per dispatch) are scaled by what each reads
    for the runtime's copy kernel moving a known size (--calibrate-copy): the copies are the
    `__amd_rocclr_copyBuffer` dispatches before the dataset upload (`k_repack`)."""
    fetch_dir, write_dir = args.pmc_summary[:2]
    lds_dir = args.pmc_summary[2] if len(args.pmc_summary) > 2 else None
    out = []
    extra = []
    per_tree = {}
    launches = {}
    scale = {}
    for counter, folder in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        order, vals = read_counters(folder)
        first_load = next((i for i, r in enumerate(order) if "k_repack" in r["Kernel_Name"]), len(order))
        copies = [vals[int(r["Dispatch_Id"])].get(counter, 0.0) for r in order[:first_load]
                  if "copyBuffer" in r["Kernel_Name"]][:4]
        known_kib = args.calibrate_copy * 1024.0
        if not copies or not known_kib:
            raise SystemExit(f"{counter}: no calibration copies (run the profile with --calibrate-copy MB and pass "
                             "the same --calibrate-copy here)")
        measured = sum(copies) / len(copies)
        scale[counter] = known_kib / measured
        win = timed_window(order, args.warmup, args.steps)
        for r in win:
            k = kernel_key(r["Kernel_Name"])
            v = vals[int(r["Dispatch_Id"])].get(counter, 0.0) * 1024.0 * scale[counter]
            per_tree.setdefault(k, {}).setdefault(counter, 0.0)
            per_tree[k][counter] += v / args.steps
            if counter == "FETCH_SIZE":
                launches[k] = launches.get(k, 0) + 1
        out.append(f"- {counter}: the {len(copies)} calibration copies of {args.calibrate_copy} MiB read "
                   f"{measured:.0f} KiB each; scale {scale[counter]:.3f}")
    out.append("")
    out.append("| kernel | launches per tree | FETCH MB per tree | WRITE MB per tree | HBM MB per tree | "
               "HBM MB per launch |")
    out.append("|---|---:|---:|---:|---:|---:|")
    rank = sorted(per_tree, key=lambda k: -(per_tree[k].get("FETCH_SIZE", 0) + per_tree[k].get("WRITE_SIZE", 0)))
    for k in rank[:12]:
        f, w = per_tree[k].get("FETCH_SIZE", 0.0), per_tree[k].get("WRITE_SIZE", 0.0)
        lpt = launches.get(k, 0) / args.steps
        out.append(f"| `{k}` | {lpt:.2f} | {f / 1e6:.1f} | {w / 1e6:.1f} | {(f + w) / 1e6:.1f} | "
                   f"{(f + w) / lpt / 1e6 if lpt else 0:.1f} |")
    out.append("")
    for k in rank:
        if k.startswith("k_step_rows") or k.startswith("k_hist<"):
            t = per_tree[k].get("FETCH_SIZE", 0.0) + per_tree[k].get("WRITE_SIZE", 0.0)
            lpt = launches.get(k, 0) / args.steps
            out.append(f"traffic_bytes_per_tree {k}: {t:.0f}")
            out.append(f"traffic_bytes_per_launch {k}: {t / lpt if lpt else 0:.0f}")
    if args.pmc_sizes:
        # the read requests by size: true bytes 32 / 64 / 128 a request, beside FETCH_SIZE scaled by the copy (which
        # reads 128-byte requests, so its scale fits 128-byte traffic only)
        order, vals = read_counters(args.pmc_sizes)
        first_load = next((i for i, r in enumerate(order) if "k_repack" in r["Kernel_Name"]), len(order))
        names = ("TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum", "TCC_EA0_RDREQ_sum")
        copies = [vals[int(r["Dispatch_Id"])] for r in order[:first_load] if "copyBuffer" in r["Kernel_Name"]][:4]
        sizes = {}
        for r in timed_window(order, args.warmup, args.steps):
            k = kernel_key(r["Kernel_Name"])
            a = sizes.setdefault(k, dict.fromkeys(names, 0.0))
            for c in names:
                a[c] += vals[int(r["Dispatch_Id"])].get(c, 0.0) / args.steps
        out.append("")
        out.append("Read requests by size (`TCC_EA0_RDREQ_32B/64B/128B`, all of `TCC_EA0_RDREQ`), per tree; bytes = 32, "
                   "64 and 128 a request:")
        out.append("")
        if copies:
            c = copies[0]
            n32, n64, n128 = (c.get(x, 0.0) for x in names[:3])
            out.append(f"- calibration copy of {args.calibrate_copy} MiB: {n32:.0f} x 32 B + {n64:.0f} x 64 B + {n128:.0f} "
                       f"x 128 B = {(32 * n32 + 64 * n64 + 128 * n128) / 2**20:.1f} MiB read")
        out.append("")
        out.append("| kernel | 32 B requests | 64 B requests | 128 B requests | all requests | read MB by request size | "
                   "FETCH_SIZE x copy scale, MB |")
        out.append("|---|---:|---:|---:|---:|---:|---:|")
        for k in rank[:8]:
            a = sizes.get(k)
            if not a:
                continue
            b = 32 * a[names[0]] + 64 * a[names[1]] + 128 * a[names[2]]
            out.append(f"| `{k}` | {a[names[0]]:.3g} | {a[names[1]]:.3g} | {a[names[2]]:.3g} | {a[names[3]]:.3g} | "
                       f"{b / 1e6:.1f} | {per_tree[k].get('FETCH_SIZE', 0.0) / 1e6:.1f} |")
            if k.startswith("k_step_rows") or k.startswith("k_hist<"):
                extra.append(f"read_bytes_by_request_size_per_tree {k}: {b:.0f}")
        out.append("")
        out.extend(extra)
    if lds_dir:
        order, vals = read_counters(lds_dir)
        win = timed_window(order, args.warmup, args.steps)
        agg = {}
        for r in win:
            k = kernel_key(r["Kernel_Name"])
            a = agg.setdefault(k, {"n": 0, "ns": 0.0})
            a["n"] += 1
            a["ns"] += float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
            for c, v in vals[int(r["Dispatch_Id"])].items():
                a[c] = a.get(c, 0.0) + v
        out.append("")
        out.append("| kernel | launches per tree | LDS atomic lane-ops per launch | LDS atomics/s | LDS instructions per "
                   "launch | bank-conflict share of LDS cycles |")
        out.append("|---|---:|---:|---:|---:|---:|")
        for k in sorted(agg, key=lambda k: -agg[k].get("SQ_INSTS_LDS_ATOMIC", 0.0)):
            a = agg[k]
            atom = a.get("SQ_INSTS_LDS_ATOMIC", 0.0) * 64  # wave instructions x 64 lanes
            if not a.get("SQ_INSTS_LDS", 0.0):
                continue
            rate = atom / (a["ns"] * 1e-9) if a["ns"] else 0.0
            act = a.get("SQ_LDS_IDX_ACTIVE", 0.0)
            share = a.get("SQ_LDS_BANK_CONFLICT", 0.0) / act if act else 0.0
            out.append(f"| `{k}` | {a['n'] / args.steps:.2f} | {atom / a['n']:.3g} | {rate:.3g} | "
                       f"{a.get('SQ_INSTS_LDS', 0.0) / a['n']:.3g} | {share:.1%} |")
    print("\n".join(out))


def trace_summary(args):
    """Per-iteration kernel time of the timed window (--steps iterations after --warmup) from a rocprofv3
    --kernel-trace run of this script, with the idle time between consecutive dispatches; prints a markdown table."""
    import csv
    import glob

    files = glob.glob(os.path.join(args.trace_summary, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no kernel_trace.csv under {args.trace_summary}")
    rows = []
    for f in files:
        rows += list(csv.DictReader(open(f)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    win = timed_window(rows, args.warmup, args.steps)
    agg, gaps, where = {}, 0.0, {}
    prev, prev_k = None, None
    for r in win:
        s, e = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        k = kernel_key(r["Kernel_Name"])
        a = agg.setdefault(k, [0, 0.0])
        a[0] += 1
        a[1] += (e - s) / 1e3
        if prev is not None and s > prev:
            gaps += (s - prev) / 1e3
            w = where.setdefault((prev_k, k), [0, 0.0])
            w[0] += 1
            w[1] += (s - prev) / 1e3
        if prev is None or e >= prev:
            prev, prev_k = e, k
    span = (int(win[-1]["End_Timestamp"]) - int(win[0]["Start_Timestamp"])) / 1e3
    print(f"{args.steps} iterations, {span / args.steps:.1f} us per iteration from the first dispatch of the window "
          f"to the last; busy {sum(v[1] for v in agg.values()) / args.steps:.1f} us, idle between dispatches "
          f"{gaps / args.steps:.1f} us per iteration")
    print()
    print("| kernel | launches per iteration | us per iteration | avg us per launch | share of busy time |")
    print("|---|---:|---:|---:|---:|")
    busy = sum(v[1] for v in agg.values())
    for k, (n, us) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        print(f"| `{k}` | {n / args.steps:.2f} | {us / args.steps:.1f} | {us / n:.1f} | {us / busy:.1%} |")
    print()
    print("Where the idle time falls (the dispatch that ended last, then the next one to start):")
    print()
    print("| after | before | gaps per iteration | idle us per iteration |")
    print("|---|---|---:|---:|")
    for (k0, k1), (n, us) in sorted(where.items(), key=lambda kv: -kv[1][1])[:6]:
        print(f"| `{k0}` | `{k1}` | {n / args.steps:.2f} | {us / args.steps:.1f} |")


def line_floor(v, layout, args, trees):
    """The HBM bytes per tree k_step_rows cannot avoid with this layout, from the device's line counts (srocm_profile
    mode 2) over the repeated iterations: every L2 miss fetches a 128-byte line (the request-size counters show no
    other size), so 128 bytes per distinct line its gathers touch (the split bins of the parent rows; the packed
    gradients of the built rows, unless they travel as one-byte codes beside the row ids), every built row's slab
    row whole, the row ids read once (whole lines) and written once, and the partials as written. Also the split-bin bytes if jobs that split on the same feature in a
    step shared their lines, and the sparse jobs' share (fewer than two parent rows a split-bin line)."""
    prow, plines, brow, blines, shared, partials, packed, sp_rows, sp_lines, sp_built = v
    trees = max(trees, 1)
    first = layout[0] if layout else {"width": 128, "row_bytes": 128, "q32": False}
    slab_lines = -(-first["row_bytes"] // 128)
    pbytes = 256 * first["width"] * 4
    # small units travel as one-byte codes beside the row ids (read and written with every partitioned row);
    # otherwise every built row gathers its packed word
    codes = not first.get("q32", False) and args.quant_bins <= 14
    parts = {
        "split_bins": 128.0 * plines, "gradients": 2.0 * prow if codes else 128.0 * blines,
        "slab_rows": 128.0 * slab_lines * brow,
        "row_ids_read": 4.0 * prow, "row_ids_written": 4.0 * prow,
        "partials": pbytes * packed + 2 * pbytes * (partials - packed),
    }
    floor = sum(parts.values())
    reads = (parts["split_bins"] + parts["gradients"] / (2.0 if codes else 1.0) + parts["slab_rows"] +
             parts["row_ids_read"])
    algorithmic = 9.0 * prow + brow * (first["width"] + 4.0)
    out = {k + "_per_tree": b / trees for k, b in parts.items()}
    out.update({
        "floor_bytes_per_tree": floor / trees, "floor_read_bytes_per_tree": reads / trees,
        "floor_over_algorithmic": floor / algorithmic if algorithmic else None,
        "parent_rows_per_tree": prow / trees, "built_rows_per_tree": brow / trees,
        "split_bin_lines_per_parent_row": plines / prow if prow else None,
        "gradient_lines_per_built_row": blines / brow if brow else None, "gradients_carried_as_codes": codes,
        "split_bins_shared_per_step_per_tree": 128.0 * shared / trees,
        "sparse_jobs": {"parent_rows_per_tree": sp_rows / trees, "split_bin_lines_per_tree": sp_lines / trees,
                        "built_rows_per_tree": sp_built / trees},
        "note": "one slab; 128-byte lines; the first slab's partials (packed: 256 x width x 4 B, pairs twice that)",
    })
    log(f"line model per tree: {prow / trees:.3g} parent rows ({plines / max(prow, 1):.3f} split-bin lines a row), "
        f"{brow / trees:.3g} built rows ({blines / max(brow, 1):.3f} gradient lines a row); floor "
        f"{floor / trees / 1e9:.2f} GB ({reads / trees / 1e9:.2f} GB read) = {out['floor_over_algorithmic']:.2f} x "
        f"algorithmic; split bins {parts['split_bins'] / trees / 1e9:.2f} GB per job, {128.0 * shared / trees / 1e9:.2f} "
        f"GB if a step's jobs shared lines; sparse jobs: {sp_rows / trees:.3g} parent rows, {sp_lines / trees:.3g} "
        f"lines, {sp_built / trees:.3g} built rows")
    return out


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
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="binary",
                    help="binary: the headline 10M x 128 workload; lambdarank: 2M documents x 136; sparse: 1M x 2000 "
                         "mostly-zero features of <=63 bins; wide: 50M x 32 at 1023 bins and 2047 leaves")
    ap.add_argument("--rows", type=int, default=None)
    ap.add_argument("--cols", type=int, default=None)
    ap.add_argument("--leaves", type=int, default=None)
    ap.add_argument("--quant-bins", type=int, default=4, metavar="B",
                    help="num_grad_quant_bins (the reference takes 2..64; up to 32766, 16-bit units, is an extension)")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of oracle work for the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                    help="first run 4 device-to-device copies of MB MiB (the runtime's copy kernel): known bytes for "
                         "scaling hardware memory counters")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="no GPU: summarize rocprofv3 --pmc runs of this script (FETCH_SIZE dir, WRITE_SIZE dir, and "
                         "optionally an LDS-counter dir) over its timed iterations (--warmup, --steps as in the run)")
    ap.add_argument("--line-model", action="store_true",
                    help="in the repeat with kernel events, also count the distinct 128-byte lines each split step's "
                         "gathers touch (kernels between the steps; the timed iterations are unaffected) and report "
                         "the traffic floor they set for k_step_rows")
    ap.add_argument("--pmc-sizes", metavar="DIR",
                    help="with --pmc-summary: a rocprofv3 --pmc run of TCC_EA0_RDREQ_32B_sum TCC_EA0_RDREQ_64B_sum "
                         "TCC_EA0_RDREQ_128B_sum TCC_EA0_RDREQ_sum, for the read bytes by request size")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="no GPU: per-iteration kernel times of a rocprofv3 --kernel-trace run of this script over "
                         "its timed iterations (--warmup, --steps as in the run)")
    args = ap.parse_args()
    wl = WORKLOADS[args.workload]
    args.rows = wl["rows"] if args.rows is None else args.rows
    args.cols = wl["cols"] if args.cols is None else args.cols
    args.leaves = wl["leaves"] if args.leaves is None else args.leaves
    if args.pmc_summary:
        pmc_summary(args)
        return
    if args.trace_summary:
        trace_summary(args)
        return
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
    data = silvic_amd.synthetic(wl["config"], rows=args.rows, cols=args.cols, seed=7, max_bin=wl["max_bin"])
    log(f"generated {args.workload}: {args.rows} x {args.cols} in {time.perf_counter() - t0:.1f}s; total_bins "
        f"{data.total_bins}")
    params = {"objective": wl["objective"], "num_leaves": args.leaves, "num_grad_quant_bins": args.quant_bins,
              "device_type": "rocm"}
    t0 = time.perf_counter()
    trainer = silvic_amd.Trainer(params, data)
    log(f"loaded on {trainer.backend.name()} in {time.perf_counter() - t0:.1f}s")

    lib, h = trainer.backend._lib, trainer.backend._h

    warm = trainer.step(args.warmup)
    log(f"warmup {len(warm)} iterations done")
    layout = trainer.backend.slab_layout()  # as the boosting loop left it (the quantization picks the counters)
    log(f"slabs: {step_kernels(layout, args.quant_bins)}")
    # The timed iterations run without the per-kernel events (each event is a marker in the stream that idles the
    # GPU for a few microseconds). Training is deterministic, so a second trainer repeats the same warm-up and the
    # same iterations with the events on: the kernel times and work counts are those of the timed trees.
    t0 = time.perf_counter()
    timed = trainer.step(args.steps)
    elapsed = time.perf_counter() - t0
    if len(timed) != args.steps:
        log(f"training ended after {len(timed)} of {args.steps} timed iterations")
    gpu_trees = trainer.trees
    trainer.backend.close()
    trainer = silvic_amd.Trainer(params, data)
    lib, h = trainer.backend._lib, trainer.backend._h
    trainer.step(args.warmup)
    trainer.backend._check(lib.srocm_profile(h, 2 if args.line_model else 1))
    t1 = time.perf_counter()
    profiled = trainer.step(args.steps)
    elapsed_profiled = time.perf_counter() - t1
    prof = (C.c_double * 26)()
    trainer.backend._check(lib.srocm_profile_read(h, prof, 26))
    trainer.backend._check(lib.srocm_profile(h, 0))
    same_trees = all(np.array_equal(a["split_feature"], b["split_feature"]) and
                     np.array_equal(a["threshold_bin"], b["threshold_bin"]) for a, b in zip(gpu_trees, trainer.trees))
    if not same_trees:
        log("the repeated iterations grew different trees")
    (hist_launches, hist_ms, hist_bytes, step_launches, step_ms, step_bytes, builds, hist_rows, hist_bins,
     part_rows, _, _, grow_steps, expansions, kept) = list(prof)[:15]
    line_model = line_floor(list(prof)[15:25], layout, args, len(profiled)) if args.line_model else None
    steps = max(len(timed), 1)
    iters_per_s = steps / elapsed
    psteps = max(len(profiled), 1)
    # every histogram is built by k_hist (roots) or k_step_rows (split steps, which also partition)
    bins_per_s = hist_bins / ((hist_ms + step_ms) / 1e3) if hist_ms + step_ms else 0.0
    step_gbps = step_bytes / (step_ms / 1e3) / 1e9 if step_ms else 0.0
    # the committed counter summary covers iterations 6-25 of the default workload: a window late in the run (deeper
    # trees, sparser leaves) moves other bytes, so it gets no traffic figure
    default_workload = (args.workload == "binary" and (args.rows, args.cols, args.leaves) == (10_000_000, 128, 255)
                        and args.quant_bins == 4 and args.warmup + args.steps <= 50)
    traffic = measured_traffic("k_step_rows<128", "launch") if default_workload else None
    traffic_tree = measured_traffic("k_step_rows<128", "tree") if default_workload else None
    root_gbps = hist_bytes / (hist_ms / 1e3) / 1e9 if hist_ms else 0.0
    log(f"{steps} iterations in {elapsed:.3f}s; the same {psteps} again with kernel events in {elapsed_profiled:.3f}s: "
        f"k_step_rows: {step_launches:.0f} launches, {step_ms:.1f} ms, "
        f"{step_gbps:.0f} GB/s algorithmic; k_hist (roots): {hist_launches:.0f} launches, {hist_ms:.1f} ms, "
        f"{root_gbps:.0f} GB/s; {builds:.0f} histograms, {part_rows:.3g} rows partitioned; {grow_steps:.0f} split "
        f"steps expanded {expansions:.0f} leaves for {kept:.0f} kept splits")

    cpu = None
    if not args.no_cpu:
        import oracle

        oracle.set_threads(0)
        threads = oracle.threads()
        objective = {"binary": _abi.OBJ_BINARY, "lambdarank": _abi.OBJ_LAMBDARANK,
                     "regression": _abi.OBJ_REGRESSION}[wl["objective"]]
        p = oracle.default_params(objective=objective, num_leaves=args.leaves, num_iterations=1,
                                  num_grad_quant_bins=args.quant_bins)
        t0 = time.perf_counter()
        m1 = oracle.train(data, p)
        one = time.perf_counter() - t0
        n_cpu = max(1, min(args.warmup + steps, int(args.cpu_budget / max(one, 1e-3))))
        if n_cpu > 1:
            p = oracle.default_params(objective=objective, num_leaves=args.leaves, num_iterations=n_cpu,
                                      num_grad_quant_bins=args.quant_bins)
            t0 = time.perf_counter()
            m = oracle.train(data, p)
            cpu_elapsed = time.perf_counter() - t0
        else:
            m, cpu_elapsed = m1, one
        cpu_iters = len(m.trees) / cpu_elapsed
        # the trees the oracle grew must be the device's (split features, threshold bins, counts; values 1e-6)
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
               "sample": f"{len(m.trees)} boosting iterations of the same {args.rows}x{args.cols} {args.workload} workload "
                         f"({args.leaves} leaves), oracle (C++ restatement of silvic's CPU trainer) on {threads} "
                         f"threads",
               "hist_bins_per_s": m.hist_bins / m.times["histogram"] if m.times["histogram"] else None,
               "trees_identical": f"{same}/{compared}", "seconds": cpu_elapsed}

    describe = wl["describe"].format(rows=args.rows, cols=args.cols, leaves=args.leaves, bins=args.quant_bins)
    slab = step_kernels(layout, args.quant_bins)
    out = {
        "metric": METRIC if args.workload == "binary" and args.quant_bins == 4 else
                  f"boosting iters/s, {args.workload} workload at num_grad_quant_bins={args.quant_bins}; % HBM peak",
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
        "config": {"workload": describe, "rows": args.rows, "features": args.cols,
                   "num_leaves": args.leaves, "total_bins": data.total_bins, "parallelism": "single GPU"},
        "hist_bins_per_s": bins_per_s,
        "step_kernel_ms_per_iter": step_ms / psteps,
        "root_hist_ms_per_iter": hist_ms / psteps,
        "roofline": {"bound": "hbm", "achieved": step_gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": step_gbps / HBM_PEAK_GBPS, "traffic": traffic,
                     "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT) if traffic else None,
                     "kernel": f"{slab} (split step: stable partition + built-child histogram)",
                     "launches": step_launches, "avg_launch_us": step_ms / step_launches * 1e3 if step_launches else None,
                     "bytes_per_launch": step_bytes / step_launches if step_launches else None,
                     "per_tree": {"launches": step_launches / psteps, "kernel_ms": step_ms / psteps,
                                  "algorithmic_bytes": step_bytes / psteps, "traffic_bytes": traffic_tree,
                                  "traffic_over_algorithmic": traffic_tree / (step_bytes / psteps)
                                  if traffic_tree and step_bytes else None},
                     "timing": f"HIP events around every k_step_rows / k_hist launch on the backend's stream, over "
                               f"a repeat of the {psteps} timed iterations (same trees: "
                               f"{'yes' if same_trees else 'NO'})",
                     "root_k_hist": {"launches": hist_launches, "achieved": root_gbps,
                                     "avg_launch_us": hist_ms / hist_launches * 1e3 if hist_launches else None}},
        "cpu_baseline": cpu,
    }
    if line_model:
        out["roofline"]["line_model"] = line_model
    if args.workload == "lambdarank":  # iterations of the repeat taken again with the host's normalization factors
        out["lambdarank_host_factor_redos"] = list(prof)[25]
    print(json.dumps(out), flush=True)
    trainer.backend.close()


if __name__ == "__main__":
    main()
