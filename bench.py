#!/usr/bin/env python3
"""Benchmark of the gfx950 quantized linear path; prints ONE JSON line.

A step is one call of the device entry point (``i4_matmul_dev``: activation
quantization, MFMA block dots and the FP32 epilogue chain) over one batch of
synthetic input already resident in HBM.  The timed workload is the W4 GEMV
M=1 K=4096 N=12288 with group-128 scales; ``value`` is its algorithmic HBM
throughput (packed weights + one fp32 per distinct scale + fp32 activations
in + fp32 outputs out, divided by the time per call).  Packed weights rotate
over >= 512 MB of copies so no call is served from the 256 MB last-level
cache.  The other workloads are timed the same way and reported under
``workloads``.

Each workload: prepack, one untimed call per weight copy, the warmup
calls, synchronize, then the timed calls between two HIP events on the
library's stream (a short spin kernel ahead of the first event keeps the
host's first enqueue out of the region), synchronize.  The other workloads
run first and the headline last, on a GPU that has been busy.

``cpu_baseline`` times the reference CPU kernel (kernel/quantized_matmul.cpp
of breeze-engine, compiled from its own source into oracle/_ref) on this
host's cores for every workload (oracle/cpu_bench.py, a child process with
the reference benchmark's OpenMP placement, one thread per physical core of
the GPU's NUMA node); without that build, the oracle's scalar C port.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--headline-only]
                       [--no-cpu-baseline] [--workload NAME[:ROWS]]

--workload times one workload alone and prints its own JSON line (for
profiling one kernel); the default run prints the contract line above.
``--workload rmsnorm[:ROWS]`` times the decoder's exact RMSNorm at width 5120,
``--workload rmsnorm_worst[:ROWS]`` its one-wave fallback (rows that
defeat the parallel in-order rebuild, with that rebuild forced), and
``--workload multi[:ROWS]`` the decoder's projections of one activation (one
launch, one launch per projection, and with the RMSNorm in front).
"""
import argparse
import csv
import glob
import hashlib
import json
import os
import statistics
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "breeze-engine_amd")
for _p in (ROOT, PKG_DIR):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HEADLINE = "w4_gemv"
METRIC = "W4/W8 GEMV us + achieved HBM GB/s at M=1; prefill INT8 TOPS at M=512"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
ROTATE_BYTES = 512 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_w4_gemv.json")
HEADLINE_KERNEL = "dec_kernel"


def kernel_source_files():
    """The files whose change can change a kernel's code: every file under
    the package's csrc/ and the build script (its compiler flags)."""
    files = sorted(glob.glob(os.path.join(PKG_DIR, "csrc", "*")))
    return files + [os.path.join(PKG_DIR, "breeze_amd", "_build.py")]


def kernel_sources_digest(files=None):
    """First 16 hex digits of a sha256 over the kernel sources (path relative
    to the repository, then content, in name order).  Profiles record it, and
    a profile whose digest differs from the tree's was taken on other
    kernels."""
    h = hashlib.sha256()
    for f in files or kernel_source_files():
        h.update(os.path.relpath(f, ROOT).encode() + b"\0")
        with open(f, "rb") as fh:
            h.update(fh.read())
        h.update(b"\0")
    return h.hexdigest()[:16]


def traffic_record(path=TRAFFIC_FILE):
    """The headline's profile record and whether it is stale (its kernel
    sources digest differs from this tree's, or it has none)."""
    if not os.path.exists(path):
        return None, True
    with open(path) as f:
        tr = json.load(f)
    return tr, tr.get("sources_digest") != kernel_sources_digest()


def _handles(hb, d, min_bytes):
    """Enough packed copies of one workload's weights to cover min_bytes."""
    n = max(1, -(-min_bytes // d["qweight"].nbytes))
    return [hb.prepack(d["qweight"], d["scales"], d["qzeros"], d["K"], d["N"], bits=d["bits"])
            for _ in range(n)]


def gate(torch, stream):
    """Holds the stream for ~0.1-1 ms with a spin kernel ahead of the timed
    region, so the host has enqueued the first timed calls before the GPU
    reaches them.  Without it, the region would start on an idle GPU and
    count the host's first ctypes enqueue (a few us) once per region, which
    at 20 steps adds ~5% to a 7.5 us call: the timed calls then measure
    the back-to-back rate of a loop whose host stays ahead of the GPU, as
    in serving.  The spin kernel ends before e0 is recorded."""
    with torch.cuda.stream(stream):
        torch.cuda._sleep(1_000_000)


def time_workload(hb, torch, name, rows, steps, warmup, argmax=False, graph=False):
    """Per-call time (s) of one workload: `warmup` untimed calls, then
    `steps` calls bracketed by synchronisation and HIP events on the stream
    the library launches on.  graph: the `steps` calls are captured in one
    HIP graph on a stream of their own and the timed region is one replay of
    it (dispatches then follow each other at the GPU's own pace, also under a
    profiler whose interception slows the host's enqueue)."""
    from breeze_amd import workloads

    d = workloads.make_config(name, rows)
    hs = _handles(hb, d, ROTATE_BYTES)
    N = d["N"]
    A = torch.from_numpy(d["A"]).cuda()
    M = A.shape[0]
    out = torch.empty((M, N), dtype=torch.float32, device="cuda")
    idx = torch.empty((M,), dtype=torch.int64, device="cuda")
    if graph:
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
    else:
        stream = torch.cuda.current_stream()
    sp = hb._vp(stream.cuda_stream)
    ap, op, ip = hb._vp(A.data_ptr()), hb._vp(out.data_ptr()), hb._vp(idx.data_ptr())
    lib = hb._lib
    if argmax:
        def call(h):
            return lib.i4_matmul_argmax_dev(hb._vp(h), ap, M, op, ip, sp)
    else:
        def call(h):
            return lib.i4_matmul_dev(hb._vp(h), ap, M, op, sp)
    try:
        # One untimed call per weight copy first: the first touch of each
        # copy's pages (and TLB entries) is set-up, not a step.  Then the
        # `warmup` steps.
        for h in hs:
            if call(h) != 0:
                raise RuntimeError(f"{name}: {hb.last_error()}")
        for i in range(warmup):
            if call(hs[i % len(hs)]) != 0:
                raise RuntimeError(f"{name}: {hb.last_error()}")
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        if graph:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for i in range(steps):
                    call(hs[i % len(hs)])
            with torch.cuda.stream(stream):
                g.replay()  # untimed: the graph's first launch uploads it
                torch.cuda.synchronize()
                gate(torch, stream)
                e0.record(stream)
                g.replay()
                e1.record(stream)
        else:
            gate(torch, stream)
            e0.record(stream)
            for i in range(steps):
                call(hs[i % len(hs)])
            e1.record(stream)
        torch.cuda.synchronize()
        err = hb.last_error()
        if err:
            raise RuntimeError(f"{name}: {err}")
        return e0.elapsed_time(e1) * 1e-3 / steps, M
    finally:
        for h in hs:
            hb.free(h)


def gpu_local_cpus(torch):
    """Logical CPUs of the GPU's NUMA node that this process may use, and
    how they were found.  Falls back to the whole affinity mask."""
    allowed = sorted(os.sched_getaffinity(0))
    note = "affinity mask (GPU NUMA node unknown)"
    try:
        p = torch.cuda.get_device_properties(0)
        bdf = f"{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}.0"
        with open(f"/sys/bus/pci/devices/{bdf}/numa_node") as f:
            node = int(f.read())
        if node >= 0:
            with open(f"/sys/devices/system/node/node{node}/cpulist") as f:
                from oracle.cpu_bench import parse_cpulist
                local = sorted(parse_cpulist(f.read()) & set(allowed))
            if local:
                return local, f"NUMA node {node} of GPU {bdf}, within this process's affinity mask"
            note = f"affinity mask (none of NUMA node {node}'s CPUs is allowed)"
        else:
            note = f"affinity mask (GPU {bdf} reports no NUMA node)"
    except (OSError, ValueError, AttributeError, RuntimeError) as e:
        note = f"affinity mask (GPU NUMA node unknown: {type(e).__name__}: {e})"
    return allowed, note


def cpu_baseline(torch):
    """The reference CPU kernel on this host's cores for every workload, in
    a child process (oracle/cpu_bench.py) with the reference benchmark's
    OpenMP placement: one thread per physical core of the GPU's NUMA node,
    OMP_PROC_BIND=spread, OMP_PLACES=cores, OMP_WAIT_POLICY=active."""
    import subprocess

    from oracle.cpu_bench import physical_cores

    cpus, where = gpu_local_cpus(torch)
    T = len(physical_cores(cpus))
    env = dict(os.environ, OMP_NUM_THREADS=str(T), OMP_PROC_BIND="spread", OMP_PLACES="cores",
               OMP_WAIT_POLICY="active")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "oracle", "cpu_bench.py"),
                        "--cpus", ",".join(map(str, cpus))],
                       env=env, stdout=subprocess.PIPE, text=True, timeout=900)
    if r.returncode != 0:
        raise RuntimeError(f"cpu baseline failed ({r.returncode})")
    res = json.loads(r.stdout.strip().splitlines()[-1])
    head = next(w for w in res["workloads"] if w["workload"] == workloads_label(HEADLINE))
    return {
        "value": head["gbs"],
        "unit": "GB/s",
        "cores": res["threads"],
        "kind": res["kind"],
        "sample": f"{head['workload']}, hi-prec mode set once, the native i4_matmul on preallocated input "
                  f"and output, {head['calls']} timed calls after 3 warmup (mean {head['us']} us/call, median "
                  f"{head['us_median']}, min {head['us_min']}; value from the mean, as the reference's benchmark "
                  f"reports); every workload below the same way (at most 20 calls or about 4 s each); threads "
                  f"one per physical core on {where}",
        "cpu_model": res["cpu_model"],
        "cpus": res["cpus"],
        "omp": res["omp"],
        "build": res["build"],
        "workloads": res["workloads"],
    }


def workloads_label(name, M=None):
    from breeze_amd import workloads

    return workloads.LABELS[name].format(M=M)


# Projections of one activation in the Qwen3.5-27B decoder
# (kernel/qwen35_decoder.cpp:285-288 and 334-336), W4 group-128 weights.
MULTI_SHAPES = {
    "linear-attention in_qkv/in_z/in_b/in_a": (5120, (10240, 6144, 48, 48)),
    "full-attention q/k/v": (5120, (12288, 1024, 1024)),
}


def time_multi(hb, torch, label, rows, steps, warmup):
    """Per-call time (s) of the projections of one activation as one
    i4_matmul_multi_dev launch and as one i4_matmul_dev launch each, timed
    like the matmul workloads (weights rotated over >= 512 MB)."""
    import ctypes

    import numpy as np

    from breeze_amd import workloads

    K, Ns = MULTI_SHAPES[label]
    rng = np.random.default_rng(11)
    sets = []
    per_set = sum(N * K // 2 for N in Ns)
    for _ in range(max(1, -(-ROTATE_BYTES // per_set))):
        hs = []
        for N in Ns:
            qw, sc = workloads.make_weights(rng, 4, N, K, 4)
            hs.append(hb.prepack(qw, sc, None, K, N, bits=4))
        sets.append(hs)
    A = torch.from_numpy(rng.standard_normal((rows, K)).astype(np.float32)).cuda()
    outs = [torch.empty((rows, N), dtype=torch.float32, device="cuda") for N in Ns]
    stream = torch.cuda.current_stream()
    sp, ap = hb._vp(stream.cuda_stream), hb._vp(A.data_ptr())
    cv = (ctypes.c_void_p * len(Ns))(*[o.data_ptr() for o in outs])
    hvs = [(ctypes.c_void_p * len(Ns))(*[int(h) for h in hs]) for hs in sets]
    lib = hb._lib

    def one(i):
        return lib.i4_matmul_multi_dev(hvs[i % len(sets)], len(Ns), ap, rows, cv, sp)

    def each(i):
        rc = 0
        for h, o in zip(sets[i % len(sets)], outs):
            rc |= lib.i4_matmul_dev(hb._vp(h), ap, rows, hb._vp(o.data_ptr()), sp)
        return rc

    # The decoder's RMSNorm ahead of the projections: in the projection
    # launch's prologue, or as its own launch first.
    ln = torch.from_numpy((1 + 0.1 * rng.standard_normal(K)).astype(np.float32)).cuda()
    hn = torch.empty_like(A)
    lp, hp = hb._vp(ln.data_ptr()), hb._vp(hn.data_ptr())

    def norm_one(i):
        return lib.i4_rmsnorm_matmul_multi_dev(ap, lp, 1e-6, hvs[i % len(sets)], len(Ns), rows, cv, None, sp)

    def norm_then_one(i):
        rc = lib.i4_rmsnorm_dev(ap, lp, rows, K, 1e-6, hp, sp)
        return rc | lib.i4_matmul_multi_dev(hvs[i % len(sets)], len(Ns), hp, rows, cv, sp)

    res = {}
    try:
        for key, call in (("one_launch", one), ("per_projection", each), ("norm_in_launch", norm_one),
                          ("norm_then_launch", norm_then_one)):
            for i in range(len(sets) + warmup):
                if call(i) != 0:
                    raise RuntimeError(f"{label}: {hb.last_error()}")
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            gate(torch, stream)
            e0.record(stream)
            for i in range(steps):
                call(i)
            e1.record(stream)
            torch.cuda.synchronize()
            res[key] = e0.elapsed_time(e1) * 1e-3 / steps
    finally:
        for hs in sets:
            for h in hs:
                hb.free(h)
    return res


# ---------------------------------------------------------------- profile summaries
#
# A profile of one workload is four runs of `bench.py --workload NAME` on one
# box, each its own process, with their output under one directory D:
#   D/trace   rocprofv3 --kernel-trace --stats --output-format csv -d D/trace -o t
#             (200 timed calls);
#   D/fetch, D/write   rocprofv3 --pmc FETCH_SIZE (or WRITE_SIZE) --output-format csv
#             -d D/fetch -o p (50 timed calls);
#   D/plain.json   the same workload without the profiler (its JSON line).
# and the calibration of the two counters, `bench.py --copy-calibration` under
# each --pmc run (C/fetch, C/write).  --profile-summary D turns them into the
# text summary kept under profiles/, stamped with the kernel sources digest.


def _trace_rows(path, kernel, last):
    rows = [r for r in csv.DictReader(open(path)) if kernel in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    return rows[-last:]


def _counter_median(path, kernel, last=50):
    per = {}
    for r in csv.DictReader(open(path)):
        if kernel in r["Kernel_Name"]:
            per[int(r["Dispatch_Id"])] = per.get(int(r["Dispatch_Id"]), 0.0) + float(r["Counter_Value"])
    vals = [per[k] for k in sorted(per)][-last:]
    if not vals:
        raise SystemExit(f"no {kernel} dispatch in {path}")
    return statistics.median(vals)


def _short_name(name):
    """A kernel's name without its return type and parameter list."""
    if name.startswith("void "):
        name = name[5:]
    if name.endswith(")"):
        depth = 0
        for i in range(len(name) - 1, -1, -1):
            depth += {")": 1, "(": -1}.get(name[i], 0)
            if depth == 0:
                return name[:i]
    return name


def _pct(vals, q):
    v = sorted(vals)
    return v[min(len(v) - 1, int(q * (len(v) - 1) + 0.5))]


def profile_summary(d, cal, workload, kernel, steps, commit, out, traffic_out=None, graph=False):
    """Writes the summary of the profile in directory d (see above) of one
    workload's dominant kernel (`kernel`: a substring of its name)."""
    from breeze_amd import workloads

    name, _, r = workload.partition(":")
    rows = int(r) if r else None
    prefill = name.endswith("prefill")
    if name in workloads.LABELS:
        M = workloads.CONFIGS[name][1] if rows is None else rows
        label = workloads.LABELS[name].format(M=M)
        alg = workloads.algorithmic_ops(name, M) if prefill else workloads.algorithmic_bytes(name, M)
    else:
        # The decoder workloads (multi, rmsnorm): kernel times only.
        label, alg = f"{name} workload, {rows or 1} row(s) (bench.py --workload {workload})", None
    tr = _trace_rows(os.path.join(d, "trace", "t_kernel_trace.csv"), kernel, steps)
    if len(tr) < steps:
        raise SystemExit(f"{len(tr)} {kernel} dispatches in the trace, expected {steps}")
    us = [(int(x["End_Timestamp"]) - int(x["Start_Timestamp"])) / 1e3 for x in tr]
    starts = [int(x["Start_Timestamp"]) for x in tr]
    spacing = statistics.median([(b - a) / 1e3 for a, b in zip(starts, starts[1:])])
    mean, med = statistics.mean(us), statistics.median(us)
    # Other kernels of the same calls (the stand-alone quantizer ahead of a
    # staged decode or prefill call), over the same span of the trace.
    t0, t1 = starts[0], int(tr[-1]["End_Timestamp"])
    others = {}
    for x in csv.DictReader(open(os.path.join(d, "trace", "t_kernel_trace.csv"))):
        if kernel not in x["Kernel_Name"] and t0 <= int(x["Start_Timestamp"]) <= t1:
            others.setdefault(x["Kernel_Name"], []).append(
                (int(x["End_Timestamp"]) - int(x["Start_Timestamp"])) / 1e3)
    plain = None
    pj = os.path.join(d, "plain.json")
    if os.path.exists(pj) and alg is not None:
        plain = json.loads(open(pj).read().strip().splitlines()[-1])

    def rate(t_us):
        if alg is None:
            return f"{t_us:.3f} us"
        if prefill:
            v = alg / (t_us * 1e-6) / 1e12
            return f"{v:.1f} TOPS = {v / INT8_PEAK_TOPS:.4f} of {INT8_PEAK_TOPS / 1000:.1f} POPS"
        v = alg / (t_us * 1e-6) / 1e9
        return f"{v:.1f} GB/s = {v / HBM_PEAK_GBS:.4f} of {HBM_PEAK_GBS / 1000:.0f} TB/s"

    full = tr[0]["Kernel_Name"]
    digest = kernel_sources_digest()
    wl = f"--workload {workload}"
    lines = [
        f"{_short_name(full)} on the {label}, MI355X (gfx950)",
        "",
        f"Kernel sources digest {digest} (sha256 of breeze-engine_amd/csrc/* and breeze_amd/_build.py,",
        f"bench.kernel_sources_digest); taken at commit {commit}.  bench.py marks the roofline stale",
        "when the tree's digest differs.",
        "",
        "Commands (from the repository root, each its own process, all on one box; D and C are",
        "output directories):",
        f"  rocprofv3 --kernel-trace --stats --output-format csv -d D/trace -o t -- "
        f"python3 -u bench.py {wl} --steps {steps} --warmup 5{' --graph' if graph else ''}",
        f"  rocprofv3 --pmc FETCH_SIZE --output-format csv -d D/fetch -o p -- python3 -u bench.py {wl} "
        "--steps 50 --warmup 2",
        f"  rocprofv3 --pmc WRITE_SIZE --output-format csv -d D/write -o p -- python3 -u bench.py {wl} "
        "--steps 50 --warmup 2",
        "  rocprofv3 --pmc FETCH_SIZE (and WRITE_SIZE) --output-format csv -d C/fetch (C/write) -o p -- "
        "python3 -u bench.py --copy-calibration",
        f"  python3 -u bench.py {wl} --steps {steps} --warmup 20 > D/plain.json   (no profiler)",
        f"  python3 bench.py --profile-summary D --calibration C --workload {workload} --kernel '{kernel}' "
        f"--commit {commit}{' --graph' if graph else ''} --out <this file>",
        "",
        f"Kernel trace, the last {steps} timed dispatches of {kernel}"
        + (" (one replay of a HIP graph of the timed calls, so the dispatches follow each other as in "
           "bench.py's timed loop, whose host enqueue the profiler would otherwise slow down):" if graph else ":"),
        f"  mean {mean:.3f} us, median {med:.3f}, p10 {_pct(us, 0.1):.3f}, p90 {_pct(us, 0.9):.3f}, "
        f"min {min(us):.3f}, max {max(us):.3f}",
        f"  consecutive dispatches start {spacing:.3f} us apart (median) under the profiler",
    ]
    if alg is not None:
        lines += [f"  algorithmic {'ops' if prefill else 'bytes'} {alg:,} per call -> over the mean {rate(mean)};",
                  f"  over the median {rate(med)}"]
    # Every other kernel the trace's last calls ran, by name.
    for k, v in sorted(others.items()):
        lines.append(f"  same span, {_short_name(k)}: {len(v)} dispatches, mean {statistics.mean(v):.3f} us, "
                     f"median {statistics.median(v):.3f}")
    if plain:
        pu = plain["us"]
        lines += [
            "",
            f"Without the profiler, same box: {pu:.3f} us per call over {plain['steps']} back-to-back calls "
            f"(HIP events around the timed calls) -> {rate(pu)}.",
            "  bench.py reports this figure; it counts every kernel of a call and the boundary between",
            f"  calls.  Profiled kernel time against it: mean {mean / pu:.3f}x, median {med / pu:.3f}x"
            + ("." if graph else "; under the profiler the host enqueues more slowly (the dispatch "
                                 "spacing above), so each dispatch starts on an idle GPU."),
        ]
    lines += ["", "rocprofv3 kernel_stats.csv (every dispatch of the run, set-up included):"]
    lines += ["  " + x.rstrip() for x in open(os.path.join(d, "trace", "t_kernel_stats.csv"))][:12]
    traffic = None
    if cal and os.path.exists(os.path.join(d, "fetch")):
        f_kib = _counter_median(os.path.join(d, "fetch", "p_counter_collection.csv"), kernel)
        w_kib = _counter_median(os.path.join(d, "write", "p_counter_collection.csv"), kernel)
        cf = _counter_median(os.path.join(cal, "fetch", "p_counter_collection.csv"), "MulFunctor", last=3)
        cw = _counter_median(os.path.join(cal, "write", "p_counter_collection.csv"), "MulFunctor", last=3)
        sf, sw = cf * 1024 / (256 << 20), cw * 1024 / (256 << 20)
        traffic = int(round(f_kib * 1024 / sf + w_kib * 1024 / sw))
        lines += [
            "",
            "HBM traffic per dispatch (medians of the last 50 dispatches, KiB as the counters report them):",
            f"  FETCH_SIZE {f_kib:.1f}   WRITE_SIZE {w_kib:.1f}",
            f"  copy calibration (256 MiB read and written per launch): FETCH_SIZE {cf:.1f} KiB, "
            f"WRITE_SIZE {cw:.1f} KiB",
            f"  -> scale factors (counter / true bytes) FETCH {sf:.5f}, WRITE {sw:.5f}",
        ]
        if not prefill:
            lines.append(f"  HBM bytes per dispatch = {traffic:,} B against {alg:,} algorithmic ({traffic / alg:.4f}x)")
        else:
            lines.append(f"  HBM bytes per dispatch = {traffic:,} B")
    extra = sorted(glob.glob(os.path.join(d, "pmc_*", "p_counter_collection.csv")))
    if extra:
        lines += ["", "Other counters per dispatch of the kernel (medians of the last 50 dispatches; each pass"
                      " its own run,", "  rocprofv3 --pmc <counters> --output-format csv -d D/pmc_<n> -o p -- "
                      f"python3 -u bench.py {wl} --steps 50 --warmup 2):"]
        for path in extra:
            names = sorted({x["Counter_Name"] for x in csv.DictReader(open(path))})
            for cn in names:
                per = {}
                for x in csv.DictReader(open(path)):
                    if kernel in x["Kernel_Name"] and x["Counter_Name"] == cn:
                        per[int(x["Dispatch_Id"])] = per.get(int(x["Dispatch_Id"]), 0.0) + float(x["Counter_Value"])
                vals = [per[k] for k in sorted(per)][-50:]
                if vals:
                    lines.append(f"  {cn:28s} {statistics.median(vals):,.0f}")
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    if traffic_out:
        rec = {
            "bytes_per_launch": traffic,
            "algorithmic_bytes": alg,
            "kernel": _short_name(full),
            "kernel_mean_us": round(mean, 3),
            "kernel_median_us": round(med, 3),
            "bench_us_same_box": plain["us"] if plain else None,
            "sources_digest": digest,
            "commit": commit,
            "source": os.path.relpath(out, ROOT) + " (rocprofv3 kernel trace and FETCH_SIZE/WRITE_SIZE, "
                                                  "copy-calibrated)",
        }
        with open(traffic_out, "w") as f:
            json.dump(rec, f, indent=1)
            f.write("\n")


RMSNORM_H = 5120


def time_rmsnorm(hb, torch, rows, steps, warmup, worst=False):
    """Per-call time (s) of the decoder's exact RMSNorm (i4_rmsnorm_dev) on
    `rows` rows of width 5120 (the hidden size of the prefill and LM-head
    shapes), called through the C ABI with preallocated buffers and timed
    like the matmul workloads.  worst: rows whose partial sums all stay next
    to a power of two (1.0, then 5119 terms of 2^-30), with the in-order sum
    forced (BREEZE_HIP_NORM_EXACT=1), so every row takes the kernel's
    fallback: one wave summing in element order."""
    import numpy as np

    rng = np.random.default_rng(7)
    if worst:
        xa = np.full((rows, RMSNORM_H), 2.0 ** -30, np.float32)
        xa[:, 0] = 1.0
        os.environ["BREEZE_HIP_NORM_EXACT"] = "1"
    else:
        xa = rng.standard_normal((rows, RMSNORM_H)).astype(np.float32)
    x = torch.from_numpy(xa).cuda()
    w = torch.from_numpy((1 + 0.1 * rng.standard_normal(RMSNORM_H)).astype(np.float32)).cuda()
    out = torch.empty_like(x)
    stream = torch.cuda.current_stream()
    sp, xp, wp, op = (hb._vp(v) for v in (stream.cuda_stream, x.data_ptr(), w.data_ptr(), out.data_ptr()))
    lib = hb._lib

    def call():
        return lib.i4_rmsnorm_dev(xp, wp, rows, RMSNORM_H, 1e-6, op, sp)

    for _ in range(warmup):
        if call() != 0:
            raise RuntimeError(f"rmsnorm: {hb.last_error()}")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    gate(torch, stream)
    e0.record(stream)
    for _ in range(steps):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / steps


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--headline-only", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", default=None,
                    help="time only this workload (w8_gemv, w4_gemv, w4_decode:ROWS, w8_lmhead, w8_prefill, "
                         "w4_prefill)")
    ap.add_argument("--graph", action="store_true",
                    help="with --workload: time one replay of a HIP graph of the timed calls")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 256 MiB fp32 elementwise copy 5 times (counter calibration)")
    ap.add_argument("--profile-summary", metavar="DIR", default=None,
                    help="write the summary of the profile runs in DIR (with --workload, --kernel, --out)")
    ap.add_argument("--calibration", metavar="DIR", default=None, help="counter calibration runs (fetch/, write/)")
    ap.add_argument("--kernel", default=HEADLINE_KERNEL, help="dominant kernel of the profiled workload")
    ap.add_argument("--commit", default="unknown", help="commit the profiled tree was at")
    ap.add_argument("--out", default=None, help="summary file to write")
    ap.add_argument("--traffic-out", default=None, help="also write the headline's traffic record here")
    args = ap.parse_args()
    if args.profile_summary:
        if not (args.workload and args.out):
            raise SystemExit("bench.py: --profile-summary needs --workload and --out")
        profile_summary(args.profile_summary, args.calibration, args.workload, args.kernel, args.steps,
                        args.commit, args.out, args.traffic_out, graph=args.graph)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported. "
              "The path would shard by output columns (N) across GPUs with no reduction, "
              "but no multi-GPU run is part of it.", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        # Known traffic for scaling the FETCH_SIZE / WRITE_SIZE counters:
        # each launch reads and writes exactly 256 MiB.
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": 256 << 20, "copy_calibration_bytes_written": 256 << 20}))
        return

    from breeze_amd import hip_backend as hb
    from breeze_amd import workloads

    if not hb.device_available():
        raise SystemExit(f"bench.py: gfx950 path unavailable: {hb.last_error()}")
    hb.set_hi_prec(True)

    if args.workload:
        name, _, r = args.workload.partition(":")
        if name == "multi":
            m = int(r) if r else 1
            for label in MULTI_SHAPES:
                res = time_multi(hb, torch, label, m, args.steps, args.warmup)
                print(json.dumps({"workload": f"{label} M={m}", "us": {k: round(v * 1e6, 3) for k, v in res.items()}}),
                      flush=True)
            return
        if name in ("rmsnorm", "rmsnorm_worst"):
            m = int(r) if r else 1
            worst = name == "rmsnorm_worst"
            t = time_rmsnorm(hb, torch, m, args.steps, args.warmup, worst=worst)
            what = ("in-order fallback of one wave, in-order sum forced" if worst
                    else "bit-identical to the in-order double sum")
            print(json.dumps({"workload": f"RMSNorm M={m} H={RMSNORM_H} ({what})",
                              "steps": args.steps, "us": round(t * 1e6, 3)}), flush=True)
            return
        if name not in workloads.LABELS:
            raise SystemExit(f"bench.py: unknown workload {name!r}; one of {sorted(workloads.LABELS)}")
        rows = int(r) if r else None
        t, m = time_workload(hb, torch, name, rows, args.steps, args.warmup, argmax=name == "w8_lmhead",
                             graph=args.graph)
        entry = {"workload": workloads.LABELS[name].format(M=m), "steps": args.steps, "us": round(t * 1e6, 3)}
        if args.graph:
            entry["graph"] = True
        if name.endswith("prefill"):
            tops = workloads.algorithmic_ops(name, m) / t / 1e12
            entry.update(tops=round(tops, 2), frac_int8_peak=round(tops / INT8_PEAK_TOPS, 4))
        else:
            g = workloads.algorithmic_bytes(name, m) / t / 1e9
            entry.update(gbs=round(g, 1), frac_hbm_peak=round(g / HBM_PEAK_GBS, 4))
        print(json.dumps(entry), flush=True)
        return

    rows = None
    if not args.headline_only:
        # The other workloads first: the headline is timed last, on a GPU
        # that has been busy for a while (clocks settled).
        rows = []
        # The decode workloads take about 10 us a call: same steps and warmup
        # as the headline.  The LM head and the prefill GEMMs take 140-300 us:
        # fewer steps keep the run short.
        # The prefill shape also at 16 and 128 rows (32- and 128-row
        # workgroups of other widths).
        for name, r in (("w8_gemv", None), ("w4_gemv", None), ("w4_decode", 1), ("w4_decode", 2),
                        ("w4_decode", 4), ("w4_decode", 8), ("w8_skinny_k32768", None), ("w8_lmhead", None),
                        ("w8_prefill", None), ("w4_prefill", None), ("w8_prefill", 16), ("w4_prefill", 16),
                        ("w8_prefill", 128)):
            long_call = name in ("w8_lmhead", "w8_prefill", "w4_prefill")
            t, m = time_workload(hb, torch, name, r, max(10, args.steps // 4) if long_call else args.steps,
                                 max(3, args.warmup // 4) if long_call else args.warmup,
                                 argmax=name == "w8_lmhead")
            entry = {"workload": workloads.LABELS[name].format(M=m), "us": round(t * 1e6, 2)}
            if name.endswith("prefill"):
                tops = workloads.algorithmic_ops(name, m) / t / 1e12
                entry.update(tops=round(tops, 2), frac_int8_peak=round(tops / INT8_PEAK_TOPS, 4))
            else:
                g = workloads.algorithmic_bytes(name, m) / t / 1e9
                entry.update(gbs=round(g, 1), frac_hbm_peak=round(g / HBM_PEAK_GBS, 4))
            rows.append(entry)
            print(f"bench: {entry}", file=sys.stderr, flush=True)
        t = time_rmsnorm(hb, torch, 1, args.steps, args.warmup)
        rows.append({"workload": f"RMSNorm M=1 H={RMSNORM_H} (bit-identical to the in-order double sum)", "us": round(t * 1e6, 2)})
        for label in MULTI_SHAPES:
            for m in (1, 4):
                r = time_multi(hb, torch, label, m, args.steps, args.warmup)
                K, Ns = MULTI_SHAPES[label]
                rows.append({"workload": f"Qwen3.5-27B {label} W4 group-128, K={K} N={'/'.join(map(str, Ns))}, "
                                         f"M={m}",
                             "us_one_launch": round(r["one_launch"] * 1e6, 2),
                             "us_per_projection": round(r["per_projection"] * 1e6, 2),
                             "us_rmsnorm_in_launch": round(r["norm_in_launch"] * 1e6, 2),
                             "us_rmsnorm_then_launch": round(r["norm_then_launch"] * 1e6, 2)})
                print(f"bench: {rows[-1]}", file=sys.stderr, flush=True)

    t_step, M = time_workload(hb, torch, HEADLINE, None, args.steps, args.warmup)
    nbytes = workloads.algorithmic_bytes(HEADLINE)
    gbs = nbytes / t_step / 1e9

    tr, stale = traffic_record()
    tr = tr or {}

    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded MatMulNBits weights and N(0,1) activations, breeze_amd.workloads)",
        "config": {
            "workload": workloads.LABELS[HEADLINE],
            "M": 1, "K": 4096, "N": 12288, "bits": 4, "scale_group": 128,
            "activations": "two-pass INT16 (hi-prec)",
            "algorithmic_bytes": nbytes,
            "us_per_call": round(t_step * 1e6, 3),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": tr.get("bytes_per_launch"),
            "kernel": "dec_kernel (one launch per call)",
            "traffic_source": tr.get("source"),
            # The profile's kernel time and the same box's per-call time;
            # stale: the profile was taken on other kernel sources.
            "profiled_kernel_mean_us": tr.get("kernel_mean_us"),
            "profiled_kernel_median_us": tr.get("kernel_median_us"),
            "profiled_bench_us": tr.get("bench_us_same_box"),
            "profile_sources_digest": tr.get("sources_digest"),
            "sources_digest": kernel_sources_digest(),
            "stale": stale,
        },
    }
    if rows is not None:
        result["workloads"] = rows

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch)
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
