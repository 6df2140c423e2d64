"""Benchmark: grouped 4-bit MoE expert GEMM on one MI355X.

Headline workload: Qwen3-30B-A3B expert shapes,
NF4 decode. One step = the expert GEMMs of one decode token through all 48
MoE layers: per layer gate_up [128 experts, 1536, 2048] and down [128, 2048,
768], top-8 uniformly routed experts, M = 1 row per active expert. Each layer
has its own packed weights (48 x 302 MB = 14.5 GB resident in HBM), so the
step's 906 MB of packed bytes come from HBM, not the 256 MB Infinity Cache.
The step is captured once as a HIP graph and replayed.

metric value = packed weight bytes of the active experts / step time (GB/s).

Also reported:
  roofline     the dominant kernel (NF4 decode, gate_up) timed per launch
               with HIP events on its stream, against the 8 TB/s HBM peak.
  cpu_baseline the reference's own CPU kernels (gnf4_native/cpu_kernels.c
               compiled by oracle/Makefile) on the host cores, same shapes.
  extra        batch 4 / 16 decode, the fused expert FFN (gate_up -> silu *
               up -> down in one launch) against its two- and three-launch
               forms, a whole device-routed decode MoE layer (top-k ->
               grouping -> gather -> FFN -> combine, one graph), GPT-OSS-20B MXFP4 decode, Qwen3 NF4 Zipf prefill and
               down-projection dgrad TFLOP/s.
  floor        per launch, an empty launch and a plain read of the same
               bytes (csrc/gnf4_floor.hip), next to the roofline.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "grouped-nf4-gemm_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA

QWEN = dict(E=128, gu=(1536, 2048), dn=(2048, 768), top_k=8, layers=48)
GPTOSS = dict(E=32, gu=(5760, 2880), dn=(2880, 2880), top_k=4, layers=24)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def route(rng, tokens, top_k, E, zipf_s=None):
    import numpy as np
    counts = np.zeros(E, dtype=np.int64)
    if zipf_s is None:
        for _ in range(tokens):
            counts[rng.choice(E, size=top_k, replace=False)] += 1
    else:
        p = 1.0 / np.arange(1, E + 1) ** zipf_s
        p = p[rng.permutation(E)]
        p /= p.sum()
        for _ in range(tokens):
            counts[rng.choice(E, size=top_k, replace=False, p=p)] += 1
    ids = [int(e) for e in np.nonzero(counts)[0]]
    return [int(counts[e]) for e in ids], ids


def make_nf4_layers(E, N, K, layers, dev, seed):
    """One genuinely quantized N(0, 0.02) NF4 layer, cloned per layer."""
    import torch
    from nf4_pack_ref import quantize_pack_nf4
    g = torch.Generator(device=dev).manual_seed(seed)
    W = torch.empty(E, N, K // 2, dtype=torch.uint8, device=dev)
    A = torch.empty(E, N, K // 64, dtype=torch.float32, device=dev)
    for e in range(E):
        w = torch.randn(N, K, generator=g, device=dev) * 0.02
        W[e], A[e] = quantize_pack_nf4(w)
    out = [(W, A)]
    for _ in range(layers - 1):
        out.append((W.clone(), A.clone()))
    return out


def make_mx_layers(E, N, K, layers, dev, seed):
    import torch
    from mxfp4_pack_ref import quantize_pack_mxfp4
    g = torch.Generator(device=dev).manual_seed(seed)
    W = torch.empty(E, N, K // 2, dtype=torch.uint8, device=dev)
    S = torch.empty(E, N, K // 32, dtype=torch.uint8, device=dev)
    for e in range(E):
        w = torch.randn(N, K, generator=g, device=dev) * 0.02
        b, s = quantize_pack_mxfp4(w)
        W[e], S[e] = b.reshape(N, K // 2), s
    out = [(W, S)]
    for _ in range(layers - 1):
        out.append((W.clone(), S.clone()))
    return out


class DecodeModel:
    """Expert GEMMs of a decode step through every MoE layer."""

    def __init__(self, fmt, cfg, batch, dev, seed=0, layers=None, weights=None):
        import numpy as np
        import torch
        self.fmt, self.cfg, self.batch, self.dev = fmt, cfg, batch, dev
        L = layers or cfg["layers"]
        E = cfg["E"]
        if weights is None:
            mk = make_nf4_layers if fmt == "nf4" else make_mx_layers
            weights = (mk(E, *cfg["gu"], L, dev, seed), mk(E, *cfg["dn"], L, dev, seed + 1))
        self.gu, self.dn = weights[0][:L], weights[1][:L]
        rng = np.random.default_rng(seed + 7)
        self.routes = []
        self.host_ids = []   # the same expert ids as host lists
        g = torch.Generator(device=dev).manual_seed(seed + 3)
        for _ in range(L):
            sizes, ids = route(rng, batch, cfg["top_k"], E)
            T = sum(sizes)
            x = torch.randn(T, cfg["gu"][1], generator=g, device=dev).to(torch.bfloat16)
            h = torch.randn(T, cfg["dn"][1], generator=g, device=dev).to(torch.bfloat16)
            eids = torch.tensor(ids, dtype=torch.int32, device=dev)
            self.routes.append((sizes, eids, x, h))
            self.host_ids.append(ids)
        N1, K1 = cfg["gu"]
        N2, K2 = cfg["dn"]
        self.bytes_gu = [len(r[0]) * N1 * K1 // 2 for r in self.routes]
        self.bytes_dn = [len(r[0]) * N2 * K2 // 2 for r in self.routes]
        self.packed_bytes = sum(self.bytes_gu) + sum(self.bytes_dn)
        self.L = L

    def op(self):
        if self.fmt == "nf4":
            from nf4_grouped import gemm_4bit_grouped
            return gemm_4bit_grouped
        from mxfp4_grouped import gemm_mxfp4_grouped
        return gemm_mxfp4_grouped

    def step(self, device_ids=False):
        """Every layer's gate_up and down op calls. The expert ids go in as
        host lists (the group sizes are host lists in this API, so a
        caller's ids are on the host with them), or as the device tensor
        (device_ids: the kernels then read them from memory)."""
        op = self.op()
        outs = []
        for l in range(self.L):
            sizes, eids, x, h = self.routes[l]
            ids = eids if device_ids else self.host_ids[l]
            outs.append(op(x, *self.gu[l], sizes, ids))
            outs.append(op(h, *self.dn[l], sizes, ids))
        return outs

    def plans(self):
        if not hasattr(self, "_plans"):
            from nf4_grouped import GroupPlan
            self._plans = [GroupPlan(r[0], r[1], self.dev) for r in self.routes]
        return self._plans

    def eager_us(self, reps=50):
        """Wall time (us) of one op call as a Python caller sees it (host
        planning, the group-table upload and the launch; the reference's
        timing includes the same, bench/phase1/harness.py:915-931): the
        gate_up op of layer 0 called back to back, averaged."""
        import torch
        op = self.op()
        sizes, eids, x, h = self.routes[0]
        ids = eids.cpu().tolist()
        for _ in range(5):
            op(x, *self.gu[0], sizes, ids)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            op(x, *self.gu[0], sizes, ids)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e6 / reps

    def kernel_ms(self, which="gu", replays=20):
        """Average duration (ms) of one projection's kernel: every layer's
        launch (planned, so nothing but the kernel) captured back to back in
        one graph, timed over `replays` replays with HIP events on the launch
        stream."""
        import torch
        from nf4_grouped import launch_planned
        fmt = 0 if self.fmt == "nf4" else 1
        plans = self.plans()
        outs = []
        for l in range(self.L):
            sizes, eids, x, h = self.routes[l]
            a, (W, S) = (x, self.gu[l]) if which == "gu" else (h, self.dn[l])
            outs.append(torch.empty(a.shape[0], W.shape[1], dtype=torch.bfloat16, device=self.dev))

        def run():
            for l in range(self.L):
                sizes, eids, x, h = self.routes[l]
                a, (W, S) = (x, self.gu[l]) if which == "gu" else (h, self.dn[l])
                launch_planned(fmt, a, W, S, plans[l], out=outs[l])

        _, graph = time_graph(run, 1, 2, self.dev)
        stream = torch.cuda.current_stream(self.dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(replays):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (replays * self.L)


    def ffn_ms(self, kind, replays=20):
        """Average time (ms) of one layer's expert FFN, every layer captured
        back to back in one graph and timed with HIP events on the launch
        stream. kind: "pair" = gate_up and down launches only (no
        activation), "composed" = gate_up -> silu-multiply -> down (three
        launches), "fused" = the single fused launch."""
        import torch
        import nf4_ffn
        from nf4_grouped import launch_planned
        plans = self.plans()
        outs = []
        for l in range(self.L):
            x = self.routes[l][2]
            outs.append((torch.empty(x.shape[0], self.cfg["gu"][0], dtype=torch.bfloat16,
                                     device=self.dev),
                         torch.empty(x.shape[0], self.cfg["gu"][0] // 2, dtype=torch.bfloat16,
                                     device=self.dev),
                         torch.empty(x.shape[0], self.cfg["dn"][0], dtype=torch.bfloat16,
                                     device=self.dev)))

        def run():
            for l in range(self.L):
                sizes, eids, x, hin = self.routes[l]
                gu, h, out = outs[l]
                if kind == "fused":
                    nf4_ffn.launch_ffn_planned(x, *self.gu[l], *self.dn[l], plans[l], h=h, out=out)
                    continue
                launch_planned(0, x, *self.gu[l], plans[l], out=gu)
                if kind == "composed":
                    h = nf4_ffn.silu_mul_locked(gu)
                launch_planned(0, h if kind == "composed" else hin, *self.dn[l], plans[l], out=out)

        _, graph = time_graph(run, 1, 2, self.dev)
        stream = torch.cuda.current_stream(self.dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(replays):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (replays * self.L)


def moe_layer_ms(model, replays=20):
    """Average time (ms) of one whole decode MoE expert layer with device
    routing: router logits -> top-k (renormalised softmax) + grouping +
    gather (one launch) -> expert FFN -> weighted combine, every layer
    captured back to back in one graph (nothing is read on the host)."""
    import torch
    import nf4_route
    g = torch.Generator(device=model.dev).manual_seed(99)
    logits = [torch.randn(model.batch, model.cfg["E"], generator=g, device=model.dev)
              for _ in range(model.L)]
    xs = [torch.randn(model.batch, model.cfg["gu"][1], generator=g, device=model.dev)
          .to(torch.bfloat16) for _ in range(model.L)]

    def run():
        for l in range(model.L):
            nf4_route.moe_layer(xs[l], logits[l], model.cfg["top_k"], *model.gu[l],
                                *model.dn[l], mode=0, norm=True)

    _, graph = time_graph(run, 1, 2, model.dev)
    stream = torch.cuda.current_stream(model.dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(replays):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (replays * model.L)


def ffn_report(model):
    """Per-layer expert FFN at decode: the fused launch against the two- and
    three-launch forms, and the fused form's packed-weight rate."""
    per_layer = model.packed_bytes / model.L
    r = {}
    for kind in ("pair", "composed", "fused"):
        ms = model.ffn_ms(kind)
        r[f"{kind}_us_per_layer"] = round(ms * 1e3, 3)
        r[f"{kind}_gbs"] = round(per_layer / (ms * 1e-3) / 1e9, 1)
    if model.batch <= 16:
        r["device_routed_layer_us"] = round(moe_layer_ms(model) * 1e3, 3)
    return r


def _floor_lib():
    """The measurement kernels of grouped-nf4-gemm_amd/csrc/gnf4_floor.hip."""
    import ctypes
    lib = ctypes.CDLL(str(ROOT / "grouped-nf4-gemm_amd" / "libgnf4_floor.so"))
    lib.gnf4_floor_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.gnf4_floor_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                    ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def _graph_us(run, launches, dev, replays=20):
    """Average time (us) per launch of run() (which makes `launches`
    launches), captured once as a graph and replayed, HIP events on the
    launch stream."""
    import torch
    _, graph = time_graph(run, 1, 2, dev, settle=True)
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(replays):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (replays * launches)


def floor_report(m, which="gu"):
    """What a decode launch of this shape can reach, measured like the
    decode kernels (a graph of every layer's launches): an empty launch of
    256 workgroups, and a plain 16-byte-per-lane read of exactly the active
    experts' packed bytes (each layer's own buffer, expert ids from a device
    table) that computes nothing. Returns per-launch times and rates."""
    import torch
    lib = _floor_lib()
    W = [w[0] for w in (m.gu if which == "gu" else m.dn)]
    sink = torch.zeros(1, dtype=torch.int32, device=m.dev)
    region = W[0].shape[1] * W[0].stride(1)

    def run_empty():
        stream = torch.cuda.current_stream(m.dev).cuda_stream   # the capturing stream
        for _ in range(m.L):
            assert lib.gnf4_floor_empty(256, 1, stream) == 0

    def run_read():
        stream = torch.cuda.current_stream(m.dev).cuda_stream
        for l in range(m.L):
            eids = m.routes[l][1]
            assert lib.gnf4_floor_read(W[l].data_ptr(), W[l].stride(0), region, eids.data_ptr(),
                                       eids.numel(), sink.data_ptr(), stream) == 0

    empty = _graph_us(run_empty, m.L, m.dev)
    read = _graph_us(run_read, m.L, m.dev)
    nbytes = sum(m.bytes_gu if which == "gu" else m.bytes_dn) / m.L
    return {"empty_launch_us": round(empty, 3), "plain_read_us": round(read, 3),
            "plain_read_gbs": round(nbytes / (read * 1e-6) / 1e9, 1),
            "plain_read_frac": round(nbytes / (read * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def floor_workload(dev):
    """bench.py --floor: per-launch floors next to the decode kernels at batch
    1, Qwen3 NF4 gate_up / down and GPT-OSS-20B MXFP4 gate_up / down, every
    model layer its own weights (48 x 12.6 MB and 24 x 33 MB per gate_up
    graph: far more than the 256 MB Infinity Cache)."""
    out = {}
    for name, fmt, cfg in (("qwen3_nf4", "nf4", QWEN), ("gptoss_mxfp4", "mxfp4", GPTOSS)):
        L = cfg["layers"]
        m = DecodeModel(fmt, cfg, 1, dev, layers=L)
        for which in ("gu", "dn"):
            f = floor_report(m, which)
            k_us = m.kernel_ms(which) * 1e3
            nbytes = sum(m.bytes_gu if which == "gu" else m.bytes_dn) / m.L
            f["kernel_us"] = round(k_us, 3)
            f["kernel_gbs"] = round(nbytes / (k_us * 1e-6) / 1e9, 1)
            f["kernel_frac"] = round(f["kernel_gbs"] / HBM_PEAK_GBS, 4)
            f["packed_bytes_per_launch"] = int(nbytes)
            out[f"{name}_{'gate_up' if which == 'gu' else 'down'}_b1"] = f
            log(f"[bench] floor {name} {which}: {json.dumps(f)}")
        del m
        import torch
        torch.cuda.empty_cache()
    return out


def decode_report(m):
    """Per-launch rates of one decode configuration: gate_up and down packed
    GB/s (graph of every layer's launches, HIP events), active experts per
    layer, and the eager per-call wall time of the op."""
    gu = m.kernel_ms("gu")
    dn = m.kernel_ms("dn")
    return {"gate_up_us": round(gu * 1e3, 3),
            "gate_up_gbs": round(sum(m.bytes_gu) / m.L / (gu * 1e-3) / 1e9, 1),
            "down_us": round(dn * 1e3, 3),
            "down_gbs": round(sum(m.bytes_dn) / m.L / (dn * 1e-3) / 1e9, 1),
            "experts_per_layer": round(sum(len(r[0]) for r in m.routes) / m.L, 1),
            "eager_op_us": round(m.eager_us(), 2)}


def time_graph(fn, steps, warmup, dev, settle=False):
    """Capture fn() as a graph, then time `steps` replays after `warmup`
    (and, with `settle`, after further replays filling 30 ms)."""
    import torch
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    # settle: replay until 30 ms of GPU work has run since the last idle
    # stretch, so the shader clock has left its idle level (a heavy kernel
    # right after idle runs ~10 % slower for a few milliseconds)
    t_w = time.perf_counter()
    while settle and time.perf_counter() - t_w < 0.03:
        graph.replay()
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps, graph


def cpu_baseline(layers, seconds=8.0):
    """The reference's CPU kernels (oracle/_ref, compiled from
    gnf4_native/cpu_kernels.c; the C restatement where that build is absent)
    on the same decode workload, run by ``python -m oracle.cpu_baseline`` as
    a child process under the reference's pinning contract
    (OMP_PLACES=cores OMP_PROC_BIND=spread, gnf4_native/cpu_kernels.c:47-51),
    at all physical cores of this process's CPU set and at one thread; the
    median of >= 10 timed passes over every layer's own weight bytes."""
    import subprocess
    env = dict(os.environ, OMP_PLACES="cores", OMP_PROC_BIND="spread")
    cmd = [sys.executable, "-m", "oracle.cpu_baseline", "--layers", str(layers),
           "--seconds", str(seconds)]
    r = subprocess.run(cmd, cwd=str(ROOT), env=env, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        log(f"[bench] cpu baseline failed: {r.stderr[-2000:]}")
        return None
    res = json.loads(r.stdout.strip().splitlines()[-1])
    allc, one = res["all_cores"], res["one_thread"]
    model = res["lscpu"].get("Model name", "?")
    return {"value": allc["gbs"], "unit": "GB/s", "cores": allc["threads"], "kind": res["kind"],
            "sample": f"median of {allc['runs']} passes over {res['layers']} layers' own weights "
                      f"(gate_up 8x1536x2048 + down 8x2048x768 NF4 GEMV per layer, batch 1, "
                      f"{res['packed_bytes_per_pass'] / 1e6:.0f} MB packed per pass), "
                      f"{allc['threads']} threads = every physical core of the process's CPU set "
                      f"({res['affinity_cpus']} CPUs), OMP_PLACES=cores OMP_PROC_BIND=spread; "
                      f"{model}",
            "median_ms_per_pass": allc["median_ms"],
            "one_thread": {"value": one["gbs"], "median_ms_per_pass": one["median_ms"],
                           "runs": one["runs"]},
            "lscpu": res["lscpu"], "library": res["library"]}


def _timed(fn, dev, reps=10):
    """(graph-replay ms, eager ms) per call of fn: the graph replays the
    captured launches and group-table copies without the host-side planning,
    the eager figure is what a Python caller sees per op call."""
    import torch
    ms_graph, _ = time_graph(fn, reps, 3, dev, settle=True)
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    evs[0].record()
    for _ in range(reps):
        fn()
    evs[1].record()
    torch.cuda.synchronize()
    return ms_graph, evs[0].elapsed_time(evs[1]) / reps


def prefill_tflops(dev, seed=0):
    """Config 4: Qwen3 NF4 prefill, 4096 tokens x top-8 Zipf(1.1) routing."""
    import numpy as np
    import torch
    from nf4_grouped import gemm_4bit_grouped
    (W, A), = make_nf4_layers(128, 1536, 2048, 1, dev, seed)
    (W2, A2), = make_nf4_layers(128, 2048, 768, 1, dev, seed + 1)
    sizes, ids = route(np.random.default_rng(seed), 4096, 8, 128, zipf_s=1.1)
    T = sum(sizes)
    x = torch.randn(T, 2048, device=dev).to(torch.bfloat16)
    h = torch.randn(T, 768, device=dev).to(torch.bfloat16)
    eids = torch.tensor(ids, dtype=torch.int32, device=dev)
    res = {}
    for name, a, Wt, At, N, K in (("gate_up", x, W, A, 1536, 2048), ("down", h, W2, A2, 2048, 768)):
        ms, eager = _timed(lambda: gemm_4bit_grouped(a, Wt, At, sizes, eids), dev)
        tf = 2.0 * T * N * K / (ms * 1e-3) / 1e12
        res[name] = {"ms": round(ms, 4), "tflops": round(tf, 1),
                     "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4), "eager_op_ms": round(eager, 4)}
    res["rows"] = T
    res["m_min_max"] = [min(sizes), max(sizes)]
    return res


def prefill_uniform_tflops(dev, fmt="nf4", m=256, seed=0):
    """The metric's prefill cell: every expert with m rows (M = 256 per
    expert), Qwen3 NF4 (128 experts) or GPT-OSS MXFP4 (32 experts), gate_up
    and down, timed as graph replays of the op."""
    import torch
    cfg = QWEN if fmt == "nf4" else GPTOSS
    E = cfg["E"]
    make = make_nf4_layers if fmt == "nf4" else make_mx_layers
    if fmt == "nf4":
        from nf4_grouped import gemm_4bit_grouped as op
    else:
        from mxfp4_grouped import gemm_mxfp4_grouped as op
    sizes, ids = [m] * E, list(range(E))
    T = m * E
    eids = torch.tensor(ids, dtype=torch.int32, device=dev)
    res = {"rows_per_expert": m, "experts": E}
    for name, (N, K), s in (("gate_up", cfg["gu"], seed), ("down", cfg["dn"], seed + 1)):
        (W, S), = make(E, N, K, 1, dev, s)
        a = torch.randn(T, K, device=dev).to(torch.bfloat16)
        ms, eager = _timed(lambda: op(a, W, S, sizes, eids), dev)
        tf = 2.0 * T * N * K / (ms * 1e-3) / 1e12
        res[name] = {"ms": round(ms, 4), "tflops": round(tf, 1),
                     "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4), "eager_op_ms": round(eager, 4)}
        del W, S, a
    return res


def dgrad_tflops(dev, seed=0):
    """Config 5: NF4 dgrad on the Qwen3 down projection, 2048 tokens x top-8."""
    import numpy as np
    import torch
    from nf4_grouped import dgrad_4bit_grouped
    (W, A), = make_nf4_layers(128, 2048, 768, 1, dev, seed)
    sizes, ids = route(np.random.default_rng(seed + 1), 2048, 8, 128)
    T = sum(sizes)
    go = (torch.randn(T, 2048, device=dev) * 1e-2).to(torch.bfloat16)
    eids = torch.tensor(ids, dtype=torch.int32, device=dev)
    ms, eager = _timed(lambda: dgrad_4bit_grouped(go, W, A, sizes, eids), dev)
    tf = 2.0 * T * 2048 * 768 / (ms * 1e-3) / 1e12
    return {"ms": round(ms, 4), "tflops": round(tf, 1), "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4),
            "rows": T, "eager_op_ms": round(eager, 4)}


def pmc_workload(model):
    """Kernels for the HBM-traffic counter passes: a plain device copy of
    exactly 256 MiB (reads 256 MiB, writes 256 MiB) whose FETCH_SIZE /
    WRITE_SIZE readings give the scale factor, then every layer's gate_up
    decode launch (cold weights: each layer is its own buffer), twice, then
    every layer's down launch, twice."""
    import torch
    from nf4_grouped import launch_planned
    src = torch.empty(256 << 20, dtype=torch.uint8, device=model.dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    plans = model.plans()
    fmt = 0 if model.fmt == "nf4" else 1
    for which in ("gu", "dn"):
        for _ in range(2):
            for l in range(model.L):
                sizes, eids, x, h = model.routes[l]
                a, (W, S) = (x, model.gu[l]) if which == "gu" else (h, model.dn[l])
                launch_planned(fmt, a, W, S, plans[l])
            torch.cuda.synchronize()
    log(f"[bench] pmc workload ({model.fmt}, batch {model.batch}): 1 copy of {src.numel()} B, "
        f"{2 * model.L} gate_up launches (mean {sum(model.bytes_gu) / model.L:.0f} packed B), "
        f"then {2 * model.L} down launches (mean {sum(model.bytes_dn) / model.L:.0f} packed B)")


def pmc_prefill_workload(dev, seed=0):
    """Kernels for the prefill HBM-traffic counter passes: the 256 MiB copy
    (calibration), then config 4's gate_up and down calls (Zipf routing,
    32768 rows), each three times, then config 5's dgrad (16384 rows), three
    times, eagerly."""
    import numpy as np
    import torch
    from nf4_grouped import gemm_4bit_grouped
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    (W, A), = make_nf4_layers(128, 1536, 2048, 1, dev, seed)
    (W2, A2), = make_nf4_layers(128, 2048, 768, 1, dev, seed + 1)
    sizes, ids = route(np.random.default_rng(seed), 4096, 8, 128, zipf_s=1.1)
    T = sum(sizes)
    x = torch.randn(T, 2048, device=dev).to(torch.bfloat16)
    h = torch.randn(T, 768, device=dev).to(torch.bfloat16)
    eids = torch.tensor(ids, dtype=torch.int32, device=dev)
    for a, Wt, At in ((x, W, A), (h, W2, A2)):
        for _ in range(3):
            gemm_4bit_grouped(a, Wt, At, sizes, eids)
        torch.cuda.synchronize()
    from nf4_grouped import dgrad_4bit_grouped
    d_sizes, d_ids = route(np.random.default_rng(seed + 1), 2048, 8, 128)
    go = (torch.randn(sum(d_sizes), 2048, device=dev) * 1e-2).to(torch.bfloat16)
    d_eids = torch.tensor(d_ids, dtype=torch.int32, device=dev)
    for _ in range(3):
        dgrad_4bit_grouped(go, W2, A2, d_sizes, d_eids)
    torch.cuda.synchronize()
    log(f"[bench] pmc prefill workload: 1 copy of {src.numel()} B, 3 gate_up + 3 down calls, {T} rows")


def traffic_from_profiles():
    """HBM bytes per launch of the dominant kernel from the committed PMC
    summary, if present (line `traffic_bytes_per_launch: <int>`)."""
    p = ROOT / "profiles" / "decode_nf4_qwen3_gate_up_b1_pmc.md"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.strip().startswith("traffic_bytes_per_launch:"):
            try:
                return int(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--layers", type=int, default=QWEN["layers"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--mma-workload", action="store_true",
                    help="for rocprofv3: the prefill (config 4) and dgrad (config 5) "
                         "measurements only")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="for rocprofv3 --pmc: one 256 MiB device copy (the counter "
                         "calibration), then the gate_up decode kernel of every layer, "
                         "launched eagerly twice; prints nothing else")
    ap.add_argument("--fmt", choices=("nf4", "mxfp4"), default="nf4",
                    help="with --pmc-workload: Qwen3 NF4 (default) or GPT-OSS-20B MXFP4 experts")
    ap.add_argument("--floor", action="store_true",
                    help="batch-1 decode launches next to their floors (an empty launch and a "
                         "plain read of the same bytes), Qwen3 NF4 and GPT-OSS MXFP4; one JSON line")
    ap.add_argument("--pmc-prefill-workload", action="store_true",
                    help="for rocprofv3 --pmc: the 256 MiB copy, then config 4's prefill "
                         "gate_up and down calls, three each")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(expert parallelism is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.pmc_prefill_workload:
        pmc_prefill_workload(dev)
        return
    if args.floor:
        print(json.dumps({"floor": floor_workload(dev)}), flush=True)
        return
    if args.mma_workload:
        log(f"[bench] prefill {json.dumps(prefill_tflops(dev))}")
        log(f"[bench] prefill m256 {json.dumps(prefill_uniform_tflops(dev, 'nf4'))}")
        log(f"[bench] dgrad {json.dumps(dgrad_tflops(dev))}")
        return
    log(f"[bench] building Qwen3-30B-A3B NF4 decode model: {args.layers} layers, batch {args.batch}")
    if args.pmc_workload and args.fmt == "mxfp4":
        pmc_workload(DecodeModel("mxfp4", GPTOSS, args.batch, dev, layers=min(args.layers, 8)))
        return
    model = DecodeModel("nf4", QWEN, args.batch, dev, layers=args.layers)
    if args.pmc_workload:
        pmc_workload(model)
        return
    ms, graph = time_graph(model.step, args.steps, args.warmup, dev)
    value = model.packed_bytes / (ms * 1e-3) / 1e9
    log(f"[bench] step {ms:.4f} ms, {model.packed_bytes / 1e6:.1f} MB packed -> {value:.1f} GB/s")
    del graph
    ms_dev, graph_dev = time_graph(lambda: model.step(device_ids=True), args.steps, args.warmup, dev)
    del graph_dev
    step_dev = {"ms_per_step": round(ms_dev, 5),
                "gbs": round(model.packed_bytes / (ms_dev * 1e-3) / 1e9, 2)}
    log(f"[bench] step with device expert ids {ms_dev:.4f} ms -> {step_dev['gbs']} GB/s")

    avg_ms = model.kernel_ms("gu")
    per_launch = sum(model.bytes_gu) / len(model.bytes_gu)
    achieved = per_launch / (avg_ms * 1e-3) / 1e9
    dn_ms = model.kernel_ms("dn")
    dn_gbs = (sum(model.bytes_dn) / len(model.bytes_dn)) / (dn_ms * 1e-3) / 1e9
    log(f"[bench] gate_up decode kernel {avg_ms * 1e3:.2f} us -> {achieved:.1f} GB/s; "
        f"down {dn_ms * 1e3:.2f} us -> {dn_gbs:.1f} GB/s")

    floor_gu, floor_dn = floor_report(model, "gu"), floor_report(model, "dn")
    log(f"[bench] floors: gate_up {json.dumps(floor_gu)}, down {json.dumps(floor_dn)}")
    extra = {"down_kernel": {"us": round(dn_ms * 1e3, 3), "gbs": round(dn_gbs, 1),
                             "floor": floor_dn},
             "step_with_device_expert_ids": step_dev}
    extra[f"qwen3_nf4_ffn_b{args.batch}"] = ffn_report(model)
    log(f"[bench] ffn: {json.dumps(extra[f'qwen3_nf4_ffn_b{args.batch}'])}")
    extra["qwen3_nf4_decode_b1_eager_op_us"] = round(model.eager_us(), 2)
    if not args.no_extra:
        # config 2's batch sweep over the model's layers (their own bytes: at
        # batch 1 a graph of fewer layers could sit in the 256 MB Infinity Cache)
        sweep = {}
        for b in (1, 2, 4, 8, 16):
            m = DecodeModel("nf4", QWEN, b, dev, seed=b, layers=model.L, weights=(model.gu, model.dn))
            sweep[f"b{b}"] = decode_report(m)
            if b in (4, 16):
                extra[f"qwen3_nf4_ffn_b{b}"] = ffn_report(m)
            del m
        extra["qwen3_nf4_decode_sweep"] = sweep
        # config 3's batch sweep, GPT-OSS-20B MXFP4 experts (all 24 layers'
        # own bytes, 33 MB per gate_up launch at batch 1)
        L_mx = GPTOSS["layers"]
        mx = (make_mx_layers(GPTOSS["E"], *GPTOSS["gu"], L_mx, dev, 100),
              make_mx_layers(GPTOSS["E"], *GPTOSS["dn"], L_mx, dev, 101))
        sweep = {}
        for b in (1, 2, 4, 8, 16, 32, 64):
            m = DecodeModel("mxfp4", GPTOSS, b, dev, seed=100 + b, layers=L_mx, weights=mx)
            sweep[f"b{b}"] = decode_report(m)
            del m
        extra["gptoss20b_mxfp4_decode_sweep"] = sweep
        del mx
        torch.cuda.empty_cache()
        extra["qwen3_nf4_prefill_zipf"] = prefill_tflops(dev)
        extra["qwen3_nf4_prefill_m256"] = prefill_uniform_tflops(dev, "nf4")
        extra["gptoss_mxfp4_prefill_m256"] = prefill_uniform_tflops(dev, "mxfp4")
        extra["qwen3_nf4_dgrad_down"] = dgrad_tflops(dev)
        log(f"[bench] extra: {json.dumps(extra)}")

    cpu = None
    if not args.no_cpu:
        log("[bench] timing the CPU baseline")
        cpu = cpu_baseline(model.L, seconds=args.cpu_seconds)
        log(f"[bench] cpu: {cpu}")

    line = {
        "metric": "packed-weight GB/s at M=1 decode (Qwen3-30B-A3B NF4 experts, all 48 MoE layers)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,0.02) weights NF4-quantized (one layer, cloned per layer), "
                "N(0,1) bf16 activations, seeded uniform top-8 routing; expert ids passed as host "
                "lists with the host group sizes (the device-tensor form: "
                "extra.step_with_device_expert_ids)",
        "config": {"workload": "qwen3-30b-a3b nf4 decode: 48 layers x (gate_up 1536x2048 + down 2048x768), "
                               f"E=128, top-8, batch {args.batch}, HIP graph replay",
                   "batch": args.batch, "layers": model.L,
                   "packed_bytes_per_step": model.packed_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(),
                     "kernel": ("k_gemv_nf4<64, 1, 6, false, false> (gate_up, 8 experts x 1536 x "
                                "1024 B per launch)" if args.batch == 1 else
                                "NF4 decode launch of gate_up (kernel class by the largest group)"),
                     "avg_launch_us": round(avg_ms * 1e3, 3),
                     "timing": "HIP events around 20 replays of a graph of 48 back-to-back launches",
                     "floor": dict(floor_gu, note="same launch shape and bytes, nothing computed: "
                                   "an empty launch and a plain 16-byte-per-lane read of the "
                                   "active experts' packed bytes (grouped-nf4-gemm_amd/csrc/"
                                   "gnf4_floor.hip), timed like the kernel")},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
