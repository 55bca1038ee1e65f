"""CPU baseline leg of bench.py -- TEST INFRASTRUCTURE ONLY.

Times the reference CPU kernel (kernel/quantized_matmul.cpp of breeze-engine,
compiled from its own source into oracle/_ref by oracle/Makefile) on this
host's cores, for the benchmark workloads, as the reference's benchmark
times it (benchmark_cpu_matmul.py:43-54, 64-66; benchmark_qwen35_cpu.py:
132-135): two-pass INT16 activations set once, NUMA replica off, T OpenMP
threads bound one per physical core, prepack untimed, the native i4_matmul
on preallocated input and output, 3 warmup calls, then up to 20 timed calls
(fewer when a call is long, so one workload's sample stays within a few
seconds), reported as the mean (the reference benchmark's figure), median
and minimum per call.  Without the reference build
it times the oracle's scalar C restatement on one core instead.

bench.py runs this file as a child process, so the OpenMP environment
(OMP_NUM_THREADS, OMP_PROC_BIND=spread, OMP_PLACES=cores,
OMP_WAIT_POLICY=active) is in place before the OpenMP runtime starts and no
GPU runtime is loaded beside it.  Prints one JSON object.

Usage: python oracle/cpu_bench.py --cpus 0-15 [--workloads w8_gemv,...]
"""
import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
# Run as a script, this directory leads sys.path and `oracle` would name the
# module oracle.py rather than the package.
sys.path[:] = [p for p in sys.path if os.path.abspath(p or ".") != HERE]
for _p in (ROOT, os.path.join(ROOT, "breeze-engine_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

# (workload, rows): the five benchmark configurations, the W4 decode at each
# of its row counts.
DEFAULT = [("w8_gemv", None), ("w4_gemv", None), ("w4_decode", 1), ("w4_decode", 2), ("w4_decode", 4),
           ("w4_decode", 8), ("w8_prefill", None), ("w8_lmhead", None)]
MAX_CALLS, WARMUP, SAMPLE_S = 20, 3, 4.0


def parse_cpulist(text):
    cpus = set()
    for part in text.strip().split(","):
        if not part:
            continue
        a, _, b = part.partition("-")
        cpus.update(range(int(a), int(b or a) + 1))
    return cpus


def physical_cores(cpus):
    """One logical CPU per physical core (lowest-numbered SMT sibling)."""
    seen, keep = set(), []
    for c in sorted(cpus):
        base = f"/sys/devices/system/cpu/cpu{c}/topology"
        try:
            with open(f"{base}/core_id") as f:
                core = int(f.read())
            with open(f"{base}/physical_package_id") as f:
                pkg = int(f.read())
        except OSError:
            core, pkg = c, 0
        if (pkg, core) not in seen:
            seen.add((pkg, core))
            keep.append(c)
    return keep


def cpu_model():
    """The CPU's brand string (cpuid, as /proc/cpuinfo reports it) with its
    family, model and stepping, which name the part where a virtual machine
    shortens the brand string, and the AVX-512 features the reference kernel
    needs."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first logical CPU is enough
                k, _, v = line.partition(":")
                fields[k.strip()] = v.strip()
    except OSError:
        return "unknown"
    flags = set(fields.get("flags", "").split())
    isa = [x for x in ("avx512f", "avx512_vnni", "avx512vbmi", "avx512_bf16", "avx512_fp16") if x in flags]
    return (f"{fields.get('model name', 'unknown')} (vendor {fields.get('vendor_id', '?')}, family "
            f"{fields.get('cpu family', '?')}, model {fields.get('model', '?')}, stepping "
            f"{fields.get('stepping', '?')}; {' '.join(isa) or 'no AVX-512'})")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--cpus", required=True, help="logical CPUs to run on (one thread per physical core)")
    ap.add_argument("--workloads", default=None, help="comma list of NAME or NAME:ROWS")
    args = ap.parse_args()

    import numpy as np

    from breeze_amd import workloads
    from oracle import oracle

    cpus = physical_cores(parse_cpulist(args.cpus))
    os.sched_setaffinity(0, cpus)
    todo = DEFAULT
    if args.workloads:
        todo = []
        for w in args.workloads.split(","):
            n, _, r = w.partition(":")
            todo.append((n, int(r) if r else None))

    ref = oracle.Ref(threads=len(cpus)) if oracle.ref_available() else None
    orc = None if ref else oracle.c_oracle()
    flags = None
    if ref is not None:
        try:
            with open(os.path.join(HERE, "_ref", "build_flags.txt")) as f:
                flags = f.read().strip()
        except OSError:
            pass
    import ctypes

    if ref is not None:
        ref.lib.i4_set_hi_prec(1)  # two-pass INT16, once, outside the timed calls
    results = []
    for name, rows in todo:
        d = workloads.make_config(name, rows)
        A = np.ascontiguousarray(d["A"], np.float32)
        M = A.shape[0]
        C = np.empty((M, d["N"]), np.float32)
        h = None
        if ref is not None:
            h = ref.prepack(d["qweight"], d["scales"], None, d["N"], d["K"], d["bits"])
            # The native entry point on preallocated input and output, as the
            # reference's benchmark calls it (benchmark_cpu_matmul.py:43-54).
            native = ref.lib.i4_matmul
            args = (ctypes.c_void_p(h), A.ctypes.data_as(ctypes.c_void_p), M, C.ctypes.data_as(ctypes.c_void_p))

            def run():
                native(*args)
        else:
            def run():
                orc.matmul(d["qweight"], d["scales"], None, d["N"], d["K"], d["bits"], A, True)
        try:
            for _ in range(WARMUP):
                run()
            times = []
            t_all = time.perf_counter()
            while len(times) < MAX_CALLS and (len(times) < 3 or time.perf_counter() - t_all < SAMPLE_S):
                t0 = time.perf_counter()
                run()
                times.append(time.perf_counter() - t0)
        finally:
            if h is not None:
                ref.free(h)
        dt = float(np.mean(times))
        entry = {"workload": workloads.LABELS[name].format(M=M), "us": round(dt * 1e6, 1),
                 "us_median": round(float(np.median(times)) * 1e6, 1), "us_min": round(min(times) * 1e6, 1),
                 "calls": len(times)}
        if name.endswith("prefill"):
            entry["tops"] = round(workloads.algorithmic_ops(name, M) / dt / 1e12, 3)
        else:
            entry["gbs"] = round(workloads.algorithmic_bytes(name, M) / dt / 1e9, 2)
        results.append(entry)
        print(f"cpu baseline: {entry}", file=sys.stderr, flush=True)
        del d
    print(json.dumps({
        "kind": "reference" if ref is not None else "port",
        "threads": len(cpus) if ref is not None else 1,
        "cpus": ",".join(map(str, cpus)),
        "cpu_model": cpu_model(),
        "build": flags,
        "omp": {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OMP_PROC_BIND", "OMP_PLACES", "OMP_WAIT_POLICY")},
        "workloads": results,
    }), flush=True)


if __name__ == "__main__":
    main()
