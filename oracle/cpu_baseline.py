"""Timed CPU baseline of the decode workload -- TEST INFRASTRUCTURE ONLY.

Run by bench.py's CPU-baseline leg as a child process, so that the OpenMP
binding it asks for (OMP_PLACES=cores, OMP_PROC_BIND=spread: the reference's
own pinning contract, gnf4_native/cpu_kernels.c:47-51) is in the environment
before any OpenMP runtime loads. It times the reference's CPU kernels
(``oracle/_ref``, compiled from gnf4_native/cpu_kernels.c) -- or, where that
build is absent, this directory's C restatement -- on the headline decode
workload (Qwen3-30B-A3B experts, batch 1, top-8: per layer a gate_up GEMV
over 8 experts of [1536, 2048] and a down GEMV over 8 of [2048, 768]) for
every layer of the model, each layer with its own weight bytes (18.9 MB of
packed bytes per layer, 906 MB per pass over 48 layers, above any host
last-level cache). Only the 8 routed experts of a layer are materialised:
the kernel reads exactly those bytes either way. The weight bytes are
random (timing does not depend on their values); activations are fp32,
converted outside the timed region as the reference's CPU tier does
(kernel/cpu_grouped.py:210-211).

Prints one JSON object: the median over >= 10 timed passes at all physical
cores of the process's CPU set and at one thread, the host CPU model and
core counts from lscpu / sysfs.

    python -m oracle.cpu_baseline [--layers 48] [--min-runs 10] [--seconds 8]
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import time
from pathlib import Path

import numpy as np

from oracle import native

GU = (1536, 2048)
DN = (2048, 768)
TOP_K = 8


def physical_cores(cpus) -> int:
    """Distinct (package, core) pairs among the CPUs this process may run on."""
    seen = set()
    for c in cpus:
        base = Path(f"/sys/devices/system/cpu/cpu{c}/topology")
        try:
            seen.add((base.joinpath("physical_package_id").read_text().strip(),
                      base.joinpath("core_id").read_text().strip()))
        except OSError:
            seen.add(("?", str(c)))
    return len(seen)


def lscpu() -> dict:
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return info
    for line in out.splitlines():
        if ":" in line:
            k, v = line.split(":", 1)
            info[k.strip()] = v.strip()
    keep = ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "CPU(s)",
            "L3 cache")
    return {k: info[k] for k in keep if k in info}


def make_layers(layers: int, seed: int = 0):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(layers):
        lay = []
        for N, K in (GU, DN):
            B = rng.integers(0, 256, size=(TOP_K, N, K // 2), dtype=np.uint8)
            A = (rng.random((TOP_K, N, K // 64), dtype=np.float32) * 0.05 + 0.01)
            x = rng.standard_normal((TOP_K, K), dtype=np.float32)
            lay.append((x, B, A))
        out.append(lay)
    return out


def time_passes(fwd, layers, threads: int, min_runs: int, seconds: float):
    sizes, ids = [1] * TOP_K, list(range(TOP_K))

    def one_pass():
        for lay in layers:
            for x, B, A in lay:
                fwd(x, B, A, sizes, ids, fmt="nf4", threads=threads)

    one_pass()                       # fault the pages in, start the thread team
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - t0)
        if len(times) >= 10 * min_runs:
            break
    return times


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--min-runs", type=int, default=10)
    ap.add_argument("--seconds", type=float, default=8.0)
    args = ap.parse_args()
    inherited = len(os.sched_getaffinity(0))
    try:
        # a parent that ran GPU work may have left this thread pinned to
        # fewer CPUs than the process may use: widen to every online CPU the
        # kernel lets us have, before the OpenMP runtime (loaded with the
        # kernels below) builds its places from the mask
        os.sched_setaffinity(0, range(os.cpu_count() or 1))
    except OSError:
        pass
    cpus = sorted(os.sched_getaffinity(0))
    cores = physical_cores(cpus)
    # (with OMP_PROC_BIND set, the runtime binds this thread to one place
    # when it loads: the CPU set is read above, before that)
    ref = native.ref_lib()
    fwd = native.ref_gemv_grouped if ref is not None else native.gemv_grouped
    layers = make_layers(args.layers)
    nbytes = args.layers * TOP_K * (GU[0] * GU[1] // 2 + DN[0] * DN[1] // 2)
    res = {"kind": "reference" if ref is not None else "port",
           "library": ref.__dict__.get("_name", "") if ref is not None else "oracle/liboracle.so",
           "packed_bytes_per_pass": nbytes, "layers": args.layers,
           "affinity_cpus": len(cpus), "inherited_affinity_cpus": inherited,
           "physical_cores": cores, "lscpu": lscpu(),
           "omp_places": os.environ.get("OMP_PLACES"),
           "omp_proc_bind": os.environ.get("OMP_PROC_BIND")}
    for label, threads, secs in (("all_cores", cores, args.seconds),
                                 ("one_thread", 1, args.seconds / 2)):
        t = time_passes(fwd, layers, threads, args.min_runs, secs)
        med = float(np.median(t))
        res[label] = {"threads": threads, "runs": len(t), "median_ms": round(med * 1e3, 3),
                      "min_ms": round(min(t) * 1e3, 3), "gbs": round(nbytes / med / 1e9, 3)}
    print(json.dumps(res))


if __name__ == "__main__":
    main()
