#!/usr/bin/env python3
"""Benchmark of libortho_amd's fused dual GEMM on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one forward of the dual GEMM (one kernel launch) over one batch:
the headline workload is BASELINE.json's configs[1] at M=1 (OrthoLinear
4096 -> 11008, INT4 group-128, ortho 1 % uniform, alpha = 1), the decode
regime the GB/s metric is quoted on.  Inputs are resident in HBM before the
timed region; the weights rotate over enough copies (>= 16, > 512 MB) that
no step finds its weights in the 256 MB Infinity Cache.  Each copy carries
its ortho plan, built once before timing, as OrthoLinear builds and caches
it on its first call with alpha > 0.  The K timed steps are one replay of a
HIP graph holding exactly K launches (launch cost on the host is not what is
measured) behind untimed launches of the same workload, bracketed by two
device clock stamps (tiny kernels reading the GPU's 100 MHz clock,
orth_hip_clock_stamp) inside that graph.

Printed: one JSON line with the contract fields plus
  roofline      the decode kernel: algorithmic bytes per launch / its average
                launch duration (the device-clock interval around the K
                timed launches, divided by K) against 8 TB/s
  cpu_baseline  the reference CPU forward restated (oracle/cpu_baseline.c,
                reference flags, 1 pinned core) on a bounded sample
                (c2 M=1), plus c1 (whole layer) and c3 (token subset,
                extrapolated) in cpu_baseline.secondary
  secondary     the rest of the metric: M in {2,4,8,16} GB/s, and the
                prefill TFLOP/s at M=2048 (4096->11008 and 4096->4096);
                c1 M=1 (alpha 1 and 0), c4 M=8, the c5 block (seven
                projections back to back, M 1 and 32); the reference's
                8-argument _C_ops.forward called eagerly without a plan (c2
                M=1, c3); then the packing kernels (load time) on the c2
                layer from dense FP32 weights: GB/s of algorithmic bytes (W
                read once, q / scales / CSR written once)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "dual-GEMM GB/s (M=1) & TFLOP/s (M=2048) at 4096x11008, % of MI355X roofline"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 FLOP/clk, dense
ROTATE_MIN_BYTES = 512 << 20
ROTATE_MIN_COPIES = 16
PRE_STEPS = 1500     # untimed launches in the timing graph before its first clock stamp: the
                     # GPU's clocks are still ramping ~1 ms into a burst (20 decode launches
                     # timed after 200 untimed ones: 6.90 us each; after 1,000 or 3,000: 6.63)
STEADY_STEPS = 2000  # launches of the long graph behind ms_per_step_steady


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)  # ~14 ms per replay: start-up < 0.3 %
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="budget for the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--profile", action="store_true",
                    help="eager launches for rocprofv3 --pmc: decode c2 M=1 (alpha 1 and 0), the mid-batch "
                         "kernels at c2 M=8 and M=32, prefill c3 M=2048, then a plain device copy of known size")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="six eager planned prefill forwards at c3 (M=2048, alpha=1), for counter passes "
                         "of rocprofv3 --pmc over the prefill kernel alone")
    ap.add_argument("--profile-workload", metavar="NAME",
                    help="eager launches of one workload for rocprofv3 (kernel trace or counters): "
                         + ", ".join(PROFILE_WORKLOADS))
    ap.add_argument("--profile-steps", type=int, default=50,
                    help="forwards (blocks for c5) per --profile-workload run")
    ap.add_argument("--profile-replays", type=int, default=0,
                    help="--profile-workload: capture the steps in one HIP graph and replay it this many "
                         "times (as the timed bench lines run them); 0: eager launches (counter passes)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="turn two --profile counter runs into profiles/traffic.json")
    return ap.parse_args()


# ---------------------------------------------------------------- CPU leg

def cpu_baseline(layer, x, alpha, budget_s):
    """Single-core timing of the restated reference CPU forward on the same
    layer and input (FP16 -> FP32 conversion outside the timed region)."""
    from oracle import oracle
    if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        oracle.build()
    cpu = sorted(os.sched_getaffinity(0))[0]
    old = os.sched_getaffinity(0)
    os.sched_setaffinity(0, {cpu})
    try:
        xs = x.astype(np.float32)
        t1, _ = oracle.baseline_time(layer.q, layer.scales, layer.row_ptr, layer.col, layer.vals,
                                     xs, alpha, 0, 1)
        iters = max(3, min(200, int(budget_s / max(t1, 1e-6))))
        t, _ = oracle.baseline_time(layer.q, layer.scales, layer.row_ptr, layer.col, layer.vals,
                                    xs, alpha, 2, iters)
    finally:
        os.sched_setaffinity(0, old)
    return t, iters


def cpu_secondary(budget_s):
    """The same single-core restatement on c1 (4096 -> 4096, per-row
    scales, M=1, alpha 1: the whole layer), c3 (4096 -> 4096, M=2048,
    alpha 1) timed on 8 of its 2048 tokens and scaled by 2048 / 8 (each
    token is an independent pass of the reference's loop over the weights,
    /root/reference/src/ortho.c:352-398, so the time is linear in M), c2 at
    4 and 16 tokens, c4 at 8, and the c5 block at 1 and 32 tokens."""
    from libortho_amd import workloads as W
    out = []
    c1 = W.config_layer("c1")
    t, n = cpu_baseline(c1, W.make_x(1, c1.K, 7001), 1.0, budget_s / 3)
    b = W.algorithmic_bytes(c1, 1, 1.0)
    out.append({"workload": "c1 M=1 alpha=1", "ms_per_call": round(t * 1e3, 3), "GB/s": round(b / t / 1e9, 4),
                "cores": 1, "sample": f"whole layer, {n} timed calls"})
    log(f"  cpu {out[-1]}")
    c3 = W.config_layer("c3")
    sub = 8
    t, n = cpu_baseline(c3, W.make_x(sub, c3.K, 9048), 1.0, budget_s / 2)
    t_full = t * 2048 / sub
    f = W.algorithmic_flops(c3, 2048, 1.0)
    out.append({"workload": "c3 M=2048 alpha=1", "ms_per_call": round(t_full * 1e3, 1),
                "GFLOP/s": round(f / t_full / 1e9, 3), "cores": 1,
                "sample": f"{sub} of 2048 tokens, {n} timed calls of {t * 1e3:.1f} ms, scaled by 2048/{sub} "
                          "(linear extrapolation: the loop is per token)"})
    log(f"  cpu {out[-1]}")
    # the other decode-sized configs (4, 5): c2 at 4 and
    # 16 tokens, c4 at 8, and the Llama-2-7B block at 1 token (its seven
    # projections back to back) and at 32 tokens (2 of the 32 tokens timed,
    # scaled by 16: the loop is per token)
    c2 = W.config_layer("c2")
    for M in (4, 16):
        t, n = cpu_baseline(c2, W.make_x(M, c2.K, 7100 + M), 1.0, budget_s / 12)
        b = W.algorithmic_bytes(c2, M, 1.0)
        out.append({"workload": f"c2 M={M} alpha=1", "ms_per_call": round(t * 1e3, 2), "GB/s": round(b / t / 1e9, 4),
                    "cores": 1, "sample": f"whole layer, {n} timed calls"})
        log(f"  cpu {out[-1]}")
    c4 = W.config_layer("c4")
    t, n = cpu_baseline(c4, W.make_x(8, c4.K, 7208), 1.0, budget_s / 12)
    b = W.algorithmic_bytes(c4, 8, 1.0)
    out.append({"workload": "c4 M=8 alpha=1", "ms_per_call": round(t * 1e3, 2), "GB/s": round(b / t / 1e9, 4),
                "cores": 1, "sample": f"whole layer, {n} timed calls"})
    log(f"  cpu {out[-1]}")
    block = W.llama_block()
    for M, sub in ((1, 1), (32, 2)):
        tot, bytes_, flops = 0.0, 0, 0
        ns = []
        for lay in block:
            t, n = cpu_baseline(lay, W.make_x(sub, lay.K, 7300 + lay.K), 1.0, budget_s / 40)
            tot += t * M / sub
            bytes_ += W.algorithmic_bytes(lay, M, 1.0)
            flops += W.algorithmic_flops(lay, M, 1.0)
            ns.append(n)
        sample = ("seven projections, each timed whole" if sub == M else
                  f"{sub} of {M} tokens per projection, scaled by {M}/{sub} (linear extrapolation: the loop is per token)")
        out.append({"workload": f"c5 Llama-2-7B block M={M} alpha=1", "ms_per_call": round(tot * 1e3, 2),
                    "GB/s": round(bytes_ / tot / 1e9, 4), "GFLOP/s": round(flops / tot / 1e9, 3), "cores": 1,
                    "sample": f"{sample}; {min(ns)}-{max(ns)} timed calls per projection"})
        log(f"  cpu {out[-1]}")
    return out


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------- GPU leg

class Rotation:
    """R device copies of one layer (distinct addresses, identical data)."""

    def __init__(self, layer, torch, min_copies=ROTATE_MIN_COPIES, min_bytes=ROTATE_MIN_BYTES,
                 plan=False):
        from libortho_amd import _C_ops, workloads as W
        d = W.to_device(layer)
        self.K, self.N = layer.K, layer.N
        per = sum(t.numel() * t.element_size() for t in d.values())
        self.n = max(min_copies, -(-min_bytes // per))
        self.copies = [d] + [{k: v.clone() for k, v in d.items()} for _ in range(self.n - 1)]
        self.plans = [None] * self.n
        if plan:
            self.plans = [_C_ops.build_plan(c["q"], c["scales"], c["vals"], c["col"], c["row_ptr"],
                                            layer.K) for c in self.copies]

    def desc(self, i, alpha):
        """The C descriptor of copy i % n (built once per copy and alpha)."""
        from libortho_amd import _C_ops
        k = (i % self.n, float(alpha))
        if not hasattr(self, "_descs"):
            self._descs = {}
        if k not in self._descs:
            c = self.copies[k[0]]
            self._descs[k] = _C_ops.make_layer(c["q"], c["scales"], c["vals"], c["col"], c["row_ptr"],
                                               self.K, self.N, alpha, c["q"].device)
        return self._descs[k]

    def call(self, i, x, y, alpha):
        from libortho_amd import _C_ops
        c = self.copies[i % self.n]
        _C_ops.forward_planned(c["q"], c["scales"], c["vals"], c["col"], c["row_ptr"], x, y, alpha,
                               self.plans[i % self.n])


def time_workload(torch, layer, M, alpha, steps, warmup, plan=False, steady=False, dtype=None):
    """Returns dict(ms_per_step, kernel, copies) for `steps` forwards timed
    by graph_steps_time, so ms_per_step is the average launch duration, the
    gaps between launches included; with ``steady``, also
    ms_per_step_steady from a graph of STEADY_STEPS launches.  ``dtype``:
    the activations' and output's dtype (FP16 unless given)."""
    from libortho_amd import _C_ops, workloads as W
    dtype = dtype or torch.float16
    log(f"  [start {layer.name or f'{layer.K}->{layer.N}'} M={M} alpha={alpha} {str(dtype)[6:]} plan={plan}]")
    rot = Rotation(layer, torch, plan=plan)
    x = torch.from_numpy(W.make_x(M, layer.K, 7000 + M)).cuda().to(dtype)
    y = torch.empty(M, layer.N, dtype=dtype, device="cuda")
    for i in range(warmup):
        rot.call(i, x, y, alpha)
    torch.cuda.synchronize()
    kernel = _C_ops.last_kernel()
    assert torch.isfinite(y).all().item(), "non-finite output"

    ms = graph_steps_time(torch, lambda i: rot.call(i, x, y, alpha), steps, max(warmup, PRE_STEPS))
    out = dict(ms_per_step=ms, kernel=kernel, copies=rot.n)
    if steady:
        # the same launches in one long graph (torch.cuda.CUDAGraph), events
        # around its replay: the steady per-launch time a rocprofv3 kernel
        # trace reports, with no fixed timing cost spread over few steps
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            rot.call(0, x, y, alpha)
        torch.cuda.current_stream().wait_stream(s)
        # captured on the warmed-up stream, as torch's graph capture asks
        with torch.cuda.graph(g, stream=s):
            for i in range(STEADY_STEPS):
                rot.call(i, x, y, alpha)
        out["ms_per_step_steady"] = replay_timed(torch, g) / STEADY_STEPS
        del g
    return out


class _Hip:
    """The few HIP runtime calls the timer needs, through ctypes on the HIP
    runtime torch already loaded (torch.cuda.Event cannot be recorded inside
    a captured graph on ROCm)."""

    def __init__(self):
        import ctypes
        self.c = ctypes
        h = ctypes.CDLL("libamdhip64.so")
        V, P = ctypes.c_void_p, ctypes.POINTER
        for name, args in (("hipEventCreateWithFlags", [P(V), ctypes.c_uint]), ("hipEventDestroy", [V]),
                           ("hipStreamCreate", [P(V)]),
                           ("hipStreamDestroy", [V]), ("hipStreamBeginCapture", [V, ctypes.c_int]),
                           ("hipStreamEndCapture", [V, P(V)]), ("hipGraphCreate", [P(V), ctypes.c_uint]),
                           ("hipGraphAddChildGraphNode", [P(V), V, P(V), ctypes.c_size_t, V]),
                           ("hipGraphAddEventRecordNode", [P(V), V, P(V), ctypes.c_size_t, V]),
                           ("hipGraphInstantiate", [P(V), V, V, ctypes.c_char_p, ctypes.c_size_t]),
                           ("hipGraphLaunch", [V, V]), ("hipGraphExecDestroy", [V]), ("hipGraphDestroy", [V]),
                           ("hipStreamSynchronize", [V]),
                           ("hipGraphGetNodes", [V, P(V), P(ctypes.c_size_t)]),
                           ("hipGraphNodeGetDependentNodes", [V, P(V), P(ctypes.c_size_t)]),
                           ("hipGraphNodeGetDependencies", [V, P(V), P(ctypes.c_size_t)]),
                           ("hipGraphAddDependencies", [V, P(V), P(V), ctypes.c_size_t]),
                           ("hipEventElapsedTime", [P(ctypes.c_float), V, V])):
            fn = getattr(h, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        self.h = h

    def __call__(self, name, *args):
        rc = getattr(self.h, name)(*args)
        if rc != 0:
            raise RuntimeError(f"{name} failed: hipError {rc}")

    def new(self, name, *args):
        v = self.c.c_void_p()
        self(name, self.c.byref(v), *args)
        return v


_HIP = None
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hip_runtime_api.h


def _clock_stamp(torch, buf, stream_ptr):
    """Launch the library's device clock stamp into buf (int64 [16]) on the
    stream: 8 workgroups each write (100 MHz device clock, XCD id)."""
    from libortho_amd import _lib
    import ctypes
    _lib.check(_lib.lib().orth_hip_clock_stamp(ctypes.c_void_p(buf.data_ptr()), ctypes.c_void_p(stream_ptr)))


def _stamp_interval_ms(t0, t1) -> float:
    """Milliseconds between two clock stamps (int64 [16] host tensors of
    (clock, XCD) pairs): the median over the XCDs both stamps ran on."""
    a = {int(t0[2 * i + 1]): int(t0[2 * i]) for i in range(8)}
    b = {int(t1[2 * i + 1]): int(t1[2 * i]) for i in range(8)}
    d = sorted(b[k] - a[k] for k in a if k in b)
    if not d:
        raise RuntimeError("clock stamps share no XCD")
    return d[len(d) // 2] * 1e-5  # 100 MHz ticks -> ms


def graph_steps_time(torch, fn, steps, pre):
    """Milliseconds per call of fn(pre + i), i < steps, on the GPU's own
    clock: one captured HIP graph holds [pre untimed calls, clock stamp,
    the `steps` calls, clock stamp].  Each stamp is a tiny kernel whose
    workgroups read the 100 MHz device clock as they start
    (orth_hip_clock_stamp), so the interval between the two covers exactly
    the `steps` calls and one launch gap, with no event record (whose
    cache flush and completion signal cost several microseconds a segment,
    spread over few steps) and no host round trip inside it.  The untimed
    calls put graph start-up and the clock ramp before the first stamp.
    The graph is built on a stream of its own (default priority), replayed
    once untimed, then once timed; the stream is synchronized on both
    sides of each replay."""
    global _HIP
    if _HIP is None:
        _HIP = _Hip()
    H, c = _HIP, _HIP.c
    s = H.new("hipStreamCreate")
    ts = torch.cuda.ExternalStream(s.value)
    graphs, execs = [], []
    stamps = torch.zeros(2, 16, dtype=torch.int64, device="cuda")
    try:
        with torch.cuda.stream(ts):
            fn(0)  # any per-stream set-up outside capture
        torch.cuda.synchronize()
        with torch.cuda.stream(ts):
            H("hipStreamBeginCapture", s, 2)  # relaxed: other threads may allocate
            for i in range(pre):
                fn(i)
            _clock_stamp(torch, stamps[0], s.value)
            for i in range(pre, pre + steps):
                fn(i)
            _clock_stamp(torch, stamps[1], s.value)
            g = c.c_void_p()
            H("hipStreamEndCapture", s, c.byref(g))
        graphs.append(g)
        ex = H.new("hipGraphInstantiate", g, None, None, 0)
        execs.append(ex)
        H("hipGraphLaunch", ex, s)
        H("hipStreamSynchronize", s)
        H("hipGraphLaunch", ex, s)
        H("hipStreamSynchronize", s)
        host = stamps.cpu()
        return _stamp_interval_ms(host[0], host[1]) / steps
    finally:
        torch.cuda.synchronize()
        for ex in execs:
            H("hipGraphExecDestroy", ex)
        for g in graphs:
            H("hipGraphDestroy", g)
        H("hipStreamDestroy", s)


def replay_timed(torch, g):
    """Milliseconds of one replay of graph g, HIP events on the launch stream
    around it.  The graph is replayed once untimed first (clocks up, graph
    resident), then again untimed immediately before the timed replay with
    no host synchronisation in between, so the timed replay starts while the
    GPU is busy: its own launches are all that the events bracket."""
    g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    g.replay()
    t0.record()
    g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1)


def graph_time(torch, fn, steps):
    """Average duration of fn(i) for i < steps, by graph_steps_time with
    min(steps, 50) untimed calls first."""
    return graph_steps_time(torch, lambda i: fn(i), steps, min(steps, 50))


def time_block(torch, M, steps, grouped=False):
    """Config c5: the seven projections of one Llama-2-7B block (q, k, v, o,
    gate, up, down; group-128, ortho 2 %, alpha = 1) back to back per step,
    each with its cached plan, weights rotated over enough block copies to
    exceed the Infinity Cache; with ``grouped``, q/k/v and gate/up each as
    one orth_layers_forward_hip call (one launch at decode sizes).  Returns
    ms per block, algorithmic bytes and flops, and the kernels of the last
    step."""
    log(f"  [start c5 block M={M} grouped={grouped}]")
    from libortho_amd import _C_ops, workloads as W
    layers = W.llama_block()
    per = sum(W.algorithmic_bytes(l, 0, 1.0) for l in layers)
    copies = max(4, -(-ROTATE_MIN_BYTES // per))
    rots = [Rotation(l, torch, min_copies=copies, min_bytes=0, plan=True) for l in layers]
    xs = {K: torch.from_numpy(W.make_x(M, K, 7100 + K)).cuda() for K in {l.K for l in layers}}
    ys = [torch.empty(M, l.N, dtype=torch.float16, device="cuda") for l in layers]
    groups = [[0, 1, 2], [3], [4, 5], [6]] if grouped else [[j] for j in range(len(layers))]
    kernels = []

    def fn(i):
        kernels.clear()
        for g in groups:
            if len(g) == 1:
                rots[g[0]].call(i, xs[layers[g[0]].K], ys[g[0]], 1.0)
            else:
                _C_ops.forward_group([rots[j].desc(i, 1.0) for j in g], xs[layers[g[0]].K], [ys[j] for j in g],
                                     [rots[j].plans[i % rots[j].n] for j in g])
            kernels.append(_C_ops.last_kernel())
    fn(0)
    torch.cuda.synchronize()
    assert all(torch.isfinite(y).all().item() for y in ys), "non-finite output"
    return graph_time(torch, fn, steps), sum(W.algorithmic_bytes(l, M, 1.0) for l in layers), \
        sum(W.algorithmic_flops(l, M, 1.0) for l in layers), list(kernels)


def time_dropin(torch, layer, M, alpha, calls, graph_steps=0):
    """The reference's 8-argument entry, libortho._C_ops.forward(q_weight,
    q_scales, ortho_values, ortho_col_indices, ortho_row_ptr, input, output,
    alpha) (/root/reference/torch_bind/bindings.cpp:9-48), called eagerly
    from Python: wall and GPU time per call (the entry keeps each weight
    set's ortho plan from its first call, so the timed calls are planned);
    with graph_steps, also the per-launch time of that many calls captured in
    a graph (weights rotated as in time_workload; captured calls take no
    plan, so this is the CSR-reading path)."""
    log(f"  [start 8-argument forward {layer.name} M={M} graph_steps={graph_steps}]")
    import time as _t
    import libortho._C_ops as C
    from libortho_amd import workloads as W
    d = W.to_device(layer)
    x = torch.from_numpy(W.make_x(M, layer.K, 7200 + M)).cuda()
    y = torch.empty(M, layer.N, dtype=torch.float16, device="cuda")
    args = (d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y, alpha)
    for _ in range(5):
        C.forward(*args)
    torch.cuda.synchronize()
    import gc
    gc.collect()  # (see time_module)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    w0 = _t.perf_counter()
    t0.record()
    for _ in range(calls):
        C.forward(*args)
    t1.record()
    torch.cuda.synchronize()
    out = {"us_per_call_wall": round((_t.perf_counter() - w0) / calls * 1e6, 2),
           "us_per_call_gpu": round(t0.elapsed_time(t1) * 1e3 / calls, 2)}
    if graph_steps:
        rot = Rotation(layer, torch, plan=False)
        ms = graph_time(torch, lambda i: C.forward(*(lambda c: (c["q"], c["scales"], c["vals"], c["col"],
                                                                   c["row_ptr"]))(rot.copies[i % rot.n]),
                                                   x, y, alpha), graph_steps)
        out["us_per_launch_graph"] = round(ms * 1e3, 3)
    return out


def time_pack(torch, steps=30):
    """The packing kernels on the c2 layer (4096 -> 11008) from dense FP32
    weights rotated over 3 copies (3 x 180 MB, past the Infinity Cache):
    INT4 base packing with group-128 and per-row scales, and the CSR of a
    1 % matrix (row counts + scan, then the fill).  Returns secondary
    entries; algorithmic bytes read W once and write each output once."""
    log("  [start packing kernels]")
    import ctypes
    from libortho_amd import _lib
    L = _lib.lib()
    N, K, nnz, copies = 11008, 4096, 450888, 3
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    S = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    out = []

    wb = [torch.randn(N, K, device="cuda", generator=gen) * 0.05 for _ in range(copies)]
    q = torch.empty(N, K // 2, dtype=torch.uint8, device="cuda")
    for G, label in ((128, "group-128"), (K, "per-row")):
        s16 = torch.empty(N * (K // G), dtype=torch.float16, device="cuda")
        ms = graph_time(torch, lambda i: _lib.check(L.orth_pack_base_hip(
            P(wb[i % copies]), _lib.DT_F32, N, K, G, None, 0, P(q), P(s16), S())), steps)
        b = N * K * 4 + N * K // 2 + 2 * N * (K // G)
        out.append({"workload": f"pack base c2 fp32 {label}", "kernel": "pack_group" if G == 128 else "pack_row",
                    "us_per_step": round(ms * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                    "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
        log(f"  {out[-1]}")
    del wb

    wo = []
    for _ in range(copies):
        w = torch.zeros(N * K, device="cuda")
        idx = torch.randperm(N * K, device="cuda", generator=gen)[:nnz]
        w[idx] = torch.randn(nnz, device="cuda", generator=gen) + 3.0
        wo.append(w.view(N, K))
    rps = [torch.empty(N + 1, dtype=torch.int32, device="cuda") for _ in range(copies)]
    mb = int(L.orth_pack_csr_mask_bytes(P(wo[0]), _lib.DT_F32, N, K))  # the nonzero mask (5.6 MB)
    masks = [torch.empty(mb, dtype=torch.uint8, device="cuda") for _ in range(copies)]
    for i in range(copies):
        _lib.check(L.orth_pack_csr_rows_hip(P(wo[i]), _lib.DT_F32, N, K, P(rps[i]), P(masks[i]), mb, S()))
    torch.cuda.synchronize()
    assert all(int(r[N]) == nnz for r in rps)
    col = torch.empty(nnz, dtype=torch.int32, device="cuda")
    vals = torch.empty(nnz, dtype=torch.float32, device="cuda")
    ms_rows = graph_time(torch, lambda i: _lib.check(L.orth_pack_csr_rows_hip(
        P(wo[i % copies]), _lib.DT_F32, N, K, P(rps[i % copies]), P(masks[i % copies]), mb, S())), steps)
    ms_fill = graph_time(torch, lambda i: _lib.check(L.orth_pack_csr_fill_hip(
        P(wo[i % copies]), _lib.DT_F32, N, K, P(rps[i % copies]), P(masks[i % copies]), mb, P(col), P(vals),
        _lib.DT_F32, S())), steps)
    b = N * K * 4 + 4 * (N + 1) + 8 * nnz
    ms = ms_rows + ms_fill
    out.append({"workload": "pack csr c2 fp32 1 %", "kernel": "csr_count+csr_scan, csr_fill",
                "us_per_step": round(ms * 1e3, 2), "us_rows": round(ms_rows * 1e3, 2),
                "us_fill": round(ms_fill * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    log(f"  {out[-1]}")
    return out


def time_module(torch, calls=300):
    """Python-level OrthoLinear.forward at c2 M=1 (alpha = 1, cached plan),
    called eagerly: wall time per call on the host (ctypes binding, tensor
    checks, plan-cache lookup, launch) and the GPU time per call (HIP
    events around the same loop).  The layer is loaded from a
    reference-layout state_dict of the c2 buffers."""
    log("  [start OrthoLinear.forward eager]")
    import gc
    import time as _t
    from libortho_amd import OrthoLinear, workloads as W
    lay = W.config_layer("c2")
    m = OrthoLinear(lay.K, lay.N)
    m.load_state_dict({"base_weight": torch.from_numpy(lay.q), "base_scales": torch.from_numpy(lay.scales),
                       "ortho_values": torch.from_numpy(lay.vals),
                       "ortho_col_indices": torch.from_numpy(lay.col),
                       "ortho_row_ptr": torch.from_numpy(lay.row_ptr)})
    m = m.cuda()
    x = torch.from_numpy(W.make_x(1, lay.K, 77)).cuda()
    # the earlier sections leave a large heap: collect it now, so that the
    # loop measures the call path and not a full collection every few calls
    gc.collect()
    with torch.no_grad():
        for _ in range(20):
            m(x)
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        w0 = _t.perf_counter()
        t0.record()
        for _ in range(calls):
            m(x)
        t1.record()
        torch.cuda.synchronize()
        wall = (_t.perf_counter() - w0) / calls
    return {"workload": "OrthoLinear.forward c2 M=1 alpha=1 (eager Python calls)",
            "us_per_call_wall": round(wall * 1e6, 2),
            "us_per_call_gpu": round(t0.elapsed_time(t1) * 1e3 / calls, 2)}


COPY_BYTES = 512 << 20  # calibration copy: reads and writes exactly this many bytes
# graph launches timed per secondary line, whatever --steps is: the two
# in-graph timing events cost a fixed ~8 us per measurement (~0.4 us a
# step at K = 20, < 0.03 us at 300); the headline keeps the caller's K
SECONDARY_STEPS = 300
PROFILE_DECODE_STEPS = 100
PROFILE_PREFILL_STEPS = 5
PROFILE_MID_STEPS = 100
PROFILE_MID_M = 8       # the one-launch mid-batch kernel
PROFILE_QUARTER_M = 32  # the quarter-split kernel and its reduction
PROFILE_COPIES = 5


def profile_run(torch):
    """Eager launches (no graph) so that rocprofv3 --pmc sees one dispatch
    per forward: decode c2 M=1 alpha=1, decode c2 M=1 alpha=0, the
    one-launch mid-batch kernel at c2 M=8 alpha=1 and the quarter-split
    kernel (and its reduction) at c2 M=32 alpha=1 (planned), prefill c3
    M=2048 alpha=1 (planned), then PROFILE_COPIES device-to-device copies of
    COPY_BYTES (the calibration for FETCH_SIZE / WRITE_SIZE)."""
    from libortho_amd import workloads as W
    c2 = W.config_layer("c2")
    for alpha in (1.0, 0.0):
        rot = Rotation(c2, torch, plan=alpha > 0)
        x = torch.from_numpy(W.make_x(1, c2.K, 7001)).cuda()
        y = torch.empty(1, c2.N, dtype=torch.float16, device="cuda")
        for i in range(PROFILE_DECODE_STEPS):
            rot.call(i, x, y, alpha)
        torch.cuda.synchronize()
        del rot
    rot = Rotation(c2, torch, plan=True)
    for m in (PROFILE_MID_M, PROFILE_QUARTER_M):
        x = torch.from_numpy(W.make_x(m, c2.K, 7000 + m)).cuda()
        y = torch.empty(m, c2.N, dtype=torch.float16, device="cuda")
        for i in range(PROFILE_MID_STEPS):
            rot.call(i, x, y, 1.0)
        torch.cuda.synchronize()
    del rot
    c3 = W.config_layer("c3")
    rot = Rotation(c3, torch, min_copies=2, min_bytes=0, plan=True)
    x = torch.from_numpy(W.make_x(2048, c3.K, 9048)).cuda()
    y = torch.empty(2048, c3.N, dtype=torch.float16, device="cuda")
    for i in range(PROFILE_PREFILL_STEPS):
        rot.call(i, x, y, 1.0)
    torch.cuda.synchronize()
    del rot
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(PROFILE_COPIES):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"profile": "done", "decode_steps": PROFILE_DECODE_STEPS,
                      "mid_steps": PROFILE_MID_STEPS, "prefill_steps": PROFILE_PREFILL_STEPS,
                      "copies": PROFILE_COPIES,
                      "copy_bytes": COPY_BYTES}), flush=True)


# --profile-workload names: layer, tokens, alpha (c5: the block, grouped or not)
PROFILE_WORKLOADS = {
    "c2_m1_a1": ("c2", 1, 1.0), "c2_m1_a0": ("c2", 1, 0.0), "c2_m2_a1": ("c2", 2, 1.0),
    "c2_m4_a1": ("c2", 4, 1.0), "c2_m8_a1": ("c2", 8, 1.0), "c2_m16_a1": ("c2", 16, 1.0),
    "c2_m32_a1": ("c2", 32, 1.0), "c2_m32_a0": ("c2", 32, 0.0), "c2_m2048_a1": ("c2", 2048, 1.0),
    "c2_m2048_a0": ("c2", 2048, 0.0),
    "c1_m1_a1": ("c1", 1, 1.0),
    "c1_m1_a0": ("c1", 1, 0.0), "c3_m2048_a1": ("c3", 2048, 1.0), "c3_m2048_a0": ("c3", 2048, 0.0),
    "c4_m8_a1": ("c4", 8, 1.0), "c5_m1": ("c5", 1, 1.0), "c5_m1_grouped": ("c5", 1, 1.0),
    # prefill below one round of the tile grid (the K split)
    "c3_m65_a1": ("c3", 65, 1.0), "c3_m512_a1": ("c3", 512, 1.0), "c3_m1024_a1": ("c3", 1024, 1.0),
    "c2_m65_a1": ("c2", 65, 1.0),
    "c5_m32": ("c5", 32, 1.0), "c5_m32_grouped": ("c5", 32, 1.0), "copy": (None, 0, 0.0),
    # the bench's BF16 / FP32-activation lines and its per-row 4000->11008 layer
    "c2_m1_bf16": ("c2", 1, 1.0, "bf16"), "c2_m8_bf16": ("c2", 8, 1.0, "bf16"),
    "c2_m32_bf16": ("c2", 32, 1.0, "bf16"), "c5down_m8_bf16": ("c5down", 8, 1.0, "bf16"),
    "c2_m2048_bf16": ("c2", 2048, 1.0, "bf16"), "c2_m1_fp32": ("c2", 1, 1.0, "fp32"),
    "c2_m8_fp32": ("c2", 8, 1.0, "fp32"), "odd_m1": ("odd", 1, 1.0),
}


def graph_replays(torch, fn, steps, replays):
    """fn(i), i < steps, captured in one HIP graph on a stream of its own
    (after one eager call there, which sizes any per-stream buffer), then
    the graph replayed `replays` times back to back."""
    global _HIP
    if _HIP is None:
        _HIP = _Hip()
    H, c = _HIP, _HIP.c
    s = H.new("hipStreamCreate")
    ts = torch.cuda.ExternalStream(s.value)
    g, ex = None, None
    try:
        with torch.cuda.stream(ts):
            fn(0)
        torch.cuda.synchronize()
        with torch.cuda.stream(ts):
            H("hipStreamBeginCapture", s, 2)
            for i in range(steps):
                fn(i)
            g = c.c_void_p()
            H("hipStreamEndCapture", s, c.byref(g))
        ex = H.new("hipGraphInstantiate", g, None, None, 0)
        for _ in range(replays):
            H("hipGraphLaunch", ex, s)
        H("hipStreamSynchronize", s)
    finally:
        torch.cuda.synchronize()
        if ex is not None:
            H("hipGraphExecDestroy", ex)
        if g is not None:
            H("hipGraphDestroy", g)
        H("hipStreamDestroy", s)


def profile_workload(torch, name, steps, replays=0):
    """Forwards of one workload, each with its cached plan, weights rotated
    past the Infinity Cache as in the timed runs: eager (a counter pass sees
    one dispatch per launch), or with ``replays`` captured in one HIP graph
    and replayed that many times (the launches the timed lines measure);
    ``copy``: device copies of COPY_BYTES (the FETCH_SIZE / WRITE_SIZE
    calibration)."""
    from libortho_amd import _C_ops, workloads as W
    cfg, M, alpha = PROFILE_WORKLOADS[name][:3]
    dtype = {"bf16": torch.bfloat16, "fp32": torch.float32}.get((PROFILE_WORKLOADS[name] + ("",))[3], torch.float16)
    kernels = set()
    if cfg is None:
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(steps):
            dst.copy_(src)
    elif cfg == "c5":
        layers = W.llama_block()
        per = sum(W.algorithmic_bytes(l, 0, 1.0) for l in layers)
        copies = max(4, -(-ROTATE_MIN_BYTES // per))
        rots = [Rotation(l, torch, min_copies=copies, min_bytes=0, plan=True) for l in layers]
        xs = {K: torch.from_numpy(W.make_x(M, K, 7100 + K)).cuda() for K in {l.K for l in layers}}
        ys = [torch.empty(M, l.N, dtype=torch.float16, device="cuda") for l in layers]
        groups = [[0, 1, 2], [3], [4, 5], [6]] if name.endswith("grouped") else [[j] for j in range(len(layers))]

        def fn(i):
            for g in groups:
                if len(g) == 1:
                    rots[g[0]].call(i, xs[layers[g[0]].K], ys[g[0]], 1.0)
                else:
                    _C_ops.forward_group([rots[j].desc(i, 1.0) for j in g], xs[layers[g[0]].K], [ys[j] for j in g],
                                         [rots[j].plans[i % rots[j].n] for j in g])
                kernels.add(_C_ops.last_kernel())
        if replays:
            graph_replays(torch, fn, steps, replays)
        else:
            for i in range(steps):
                fn(i)
    else:
        if cfg == "c5down":
            layer = {l.name: l for l in W.llama_block()}["down_proj"]
        elif cfg == "odd":
            layer = W.make_layer(4000, 11008, None, 0.01, 4000)
        else:
            layer = W.config_layer(cfg)
        rot = Rotation(layer, torch, plan=alpha > 0) if M < 2048 or replays else \
            Rotation(layer, torch, min_copies=2, min_bytes=0, plan=alpha > 0)
        x = torch.from_numpy(W.make_x(M, layer.K, 7000 + M)).cuda().to(dtype)
        y = torch.empty(M, layer.N, dtype=dtype, device="cuda")

        def fn(i):
            rot.call(i, x, y, alpha)
            kernels.add(_C_ops.last_kernel())
        if replays:
            graph_replays(torch, fn, steps, replays)
        else:
            for i in range(steps):
                fn(i)
    torch.cuda.synchronize()
    print(json.dumps({"profile_workload": name, "steps": steps, "kernels": sorted(kernels)}), flush=True)


def _pmc_rows(path, counter):
    import csv
    rows = []
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] == counter:
            rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return rows


def summarize_pmc(fetch_csv, write_csv):
    """Per-launch HBM bytes of each orth kernel from two --profile runs under
    rocprofv3 --pmc (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each
    scaled by the bytes the same counter reports for the calibration copy
    (the last PROFILE_COPIES copy dispatches, COPY_BYTES read and written)."""
    from libortho_amd import workloads as W
    out = {}
    per = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = _pmc_rows(path, counter)
        copies = [v for _, name, v in rows if "copyBuffer" in name][-PROFILE_COPIES:]
        assert len(copies) == PROFILE_COPIES, f"{path}: calibration copies not found"
        factor = (sum(copies) / len(copies)) * 1024.0 / COPY_BYTES
        kern = {}
        for _, name, v in rows:
            if "quarter_reduce_kernel" in name:  # the trace keeps this name mangled
                name = "orth::quarter_reduce_kernel"
            if "orth::" in name:
                kern.setdefault(name, []).append(v)
        per[counter] = (factor, kern)
    c2, c3 = W.config_layer("c2"), W.config_layer("c3")
    f_fac, f_k = per["FETCH_SIZE"]
    w_fac, w_k = per["WRITE_SIZE"]
    for name in f_k:
        if name.startswith("void orth::decode_kernel"):
            # template args <MT, GMODE, XLDS, CPW, SPARSE, PD>: SPARSE is 0
            # for the alpha = 0 launches
            targs = name[name.index("<") + 1:name.index(">")].split(",")
            alpha = 0.0 if targs[4].strip() == "0" else 1.0
            key, algo = f"c2_m1_alpha{int(alpha)}", W.algorithmic_bytes(c2, 1, alpha)
        elif "orth::prefill_kernel" in name:
            key, algo = "c3_m2048_alpha1", W.algorithmic_bytes(c3, 2048, 1.0)
        elif name.startswith("void orth::mid_kernel"):
            m = PROFILE_MID_M
            key, algo = f"c2_m{m}_alpha1", W.algorithmic_bytes(c2, m, 1.0)
        elif name.startswith("void orth::quarter_kernel"):
            m = PROFILE_QUARTER_M
            key, algo = f"c2_m{m}_alpha1", W.algorithmic_bytes(c2, m, 1.0)
        elif "orth::quarter_reduce_kernel" in name:
            # the reduction of the same forwards: its bytes count against the
            # forward's algorithmic bytes in the combined entry
            key, algo = f"c2_m{PROFILE_QUARTER_M}_alpha1_reduce", None
        else:
            continue
        fk = sum(f_k[name]) / len(f_k[name])
        wk = sum(w_k.get(name, [0.0])) / max(1, len(w_k.get(name, [])))
        fb, wb = fk * 1024.0 / f_fac, wk * 1024.0 / w_fac
        out[key] = {"kernel": name, "dispatches": len(f_k[name]),
                    "fetch_kib_raw": round(fk, 2), "write_kib_raw": round(wk, 2),
                    "fetch_factor": round(f_fac, 4), "write_factor": round(w_fac, 4),
                    "fetch_bytes": int(fb), "write_bytes": int(wb), "bytes": int(fb + wb),
                    "algorithmic_bytes": algo,
                    "ratio_to_algorithmic": round((fb + wb) / algo, 4) if algo else None}
    mk, rk = f"c2_m{PROFILE_QUARTER_M}_alpha1", f"c2_m{PROFILE_QUARTER_M}_alpha1_reduce"
    if mk in out and rk in out:
        tot = out[mk]["bytes"] + out[rk]["bytes"]
        out[mk + "_forward"] = {"kernels": [out[mk]["kernel"], out[rk]["kernel"]], "bytes": tot,
                                "algorithmic_bytes": out[mk]["algorithmic_bytes"],
                                "ratio_to_algorithmic": round(tot / out[mk]["algorithmic_bytes"], 4)}
    p = os.path.join(ROOT, "profiles", "traffic.json")
    json.dump(out, open(p, "w"), indent=1)
    print(json.dumps(out, indent=1))


def load_traffic(workload: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE,
    WRITE_SIZE, copy-kernel calibrated), committed in profiles/traffic.json."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        return json.load(open(p)).get(workload)
    except (OSError, ValueError):
        return None


def main():
    args = parse()
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; the dual GEMM shards by output rows "
              "with no collective (each GPU takes a contiguous block of rows and its CSR rows), "
              "and multi-GPU runs are not part of it",
              file=sys.stderr)
        sys.exit(2)

    if args.profile:
        import torch
        profile_run(torch)
        return
    if args.profile_workload:
        import torch
        if args.profile_workload not in PROFILE_WORKLOADS:
            print(f"bench.py: unknown workload {args.profile_workload!r}; one of {', '.join(PROFILE_WORKLOADS)}",
                  file=sys.stderr)
            sys.exit(2)
        profile_workload(torch, args.profile_workload, args.profile_steps, args.profile_replays)
        return
    if args.profile_prefill:
        import torch
        from libortho_amd import _C_ops, workloads as W
        c3 = W.config_layer("c3")
        d = W.to_device(c3)
        plan = _C_ops.build_plan(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], c3.K)
        x = torch.from_numpy(W.make_x(2048, c3.K, 9048)).cuda()
        y = torch.empty(2048, c3.N, dtype=torch.float16, device="cuda")
        for _ in range(6):
            _C_ops.forward_planned(d["q"], d["scales"], d["vals"], d["col"], d["row_ptr"], x, y, 1.0, plan)
        torch.cuda.synchronize()
        print(json.dumps({"profile_prefill": "done", "kernel": _C_ops.last_kernel(), "launches": 6}), flush=True)
        return

    from libortho_amd import workloads as W
    layer = W.config_layer("c2")
    M, alpha = 1, 1.0
    x0 = W.make_x(M, layer.K, 7000 + M)
    bytes_step = W.algorithmic_bytes(layer, M, alpha)
    flops_step = W.algorithmic_flops(layer, M, alpha)

    cpu = None
    if not args.no_cpu:
        log("cpu baseline: c2 M=1 alpha=1, restated orth_layer_forward, 1 core ...")
        t_cpu, iters = cpu_baseline(layer, x0, alpha, args.cpu_seconds)
        cpu = {"value": round(bytes_step / t_cpu / 1e9, 4), "unit": "GB/s", "cores": 1,
               "kind": "port",
               "sample": f"c2 M=1 alpha=1 (the headline workload, whole layer), {iters} timed "
                         f"calls after 2 warmups, {t_cpu * 1e3:.2f} ms/call, same algorithmic "
                         f"bytes; oracle/cpu_baseline.c with the reference's -O3 -ffast-math "
                         f"-funroll-loops; host: {cpu_model()}, nproc={os.cpu_count()}",
               "ms_per_call": round(t_cpu * 1e3, 3)}
        log(f"  {t_cpu * 1e3:.2f} ms/call over {iters} calls")
        cpu["secondary"] = cpu_secondary(args.cpu_seconds)

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    from libortho_amd import _lib
    info = _lib.device_info(0)
    log(f"device: {info['arch']}, {info['compute_units']} CUs, clock {info['clock_khz'] / 1e3:.0f} MHz")

    log(f"decode c2 M=1: warmup {args.warmup}, steps {args.steps} ...")
    r = time_workload(torch, layer, M, alpha, args.steps, args.warmup, plan=True, steady=True)
    gbs = bytes_step / (r["ms_per_step"] * 1e-3) / 1e9
    achieved = gbs  # one kernel per step: the step time is the launch duration
    log(f"  {r['ms_per_step'] * 1e3:.2f} us/step -> {gbs:.0f} GB/s; kernel {r['kernel']}; "
        f"steady {r['ms_per_step_steady'] * 1e3:.3f} us/launch")

    secondary = []
    if not args.no_secondary:
        for m in (2, 4, 8, 16):
            # with the cached ortho plan, as OrthoLinear passes it
            rr = time_workload(torch, layer, m, alpha, SECONDARY_STEPS, 10, plan=True)
            b = W.algorithmic_bytes(layer, m, alpha)
            secondary.append({"workload": f"c2 M={m}", "kernel": rr["kernel"],
                              "us_per_step": round(rr["ms_per_step"] * 1e3, 3),
                              "GB/s": round(b / (rr["ms_per_step"] * 1e-3) / 1e9, 1),
                              "frac_hbm": round(b / (rr["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
            log(f"  {secondary[-1]}")
        # 10-20 ms of launches per graph replay: with 20 launches the replay's
        # start-up (clock ramp, first dispatch) added 10-15 % to the step
        for name, lay, k in (("4096->11008", layer, 80), ("4096->4096 (c3)", W.config_layer("c3"), 100)):
            for a in (1.0, 0.0):
                rr = time_workload(torch, lay, 2048, a, k, 3, plan=True)
                f = W.algorithmic_flops(lay, 2048, a)
                tf = f / (rr["ms_per_step"] * 1e-3) / 1e12
                secondary.append({"workload": f"prefill {name} M=2048 alpha={a}",
                                  "kernel": rr["kernel"],
                                  "us_per_step": round(rr["ms_per_step"] * 1e3, 2),
                                  "TFLOP/s": round(tf, 1),
                                  "frac_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4)})
                log(f"  {secondary[-1]}")
        # c3 at 512 tokens: 64 tiles for 256 CUs, so K is split over the grid
        c3 = W.config_layer("c3")
        rr = time_workload(torch, c3, 512, 1.0, 200, 3, plan=True)
        tf = W.algorithmic_flops(c3, 512, 1.0) / (rr["ms_per_step"] * 1e-3) / 1e12
        secondary.append({"workload": "prefill 4096->4096 (c3) M=512 alpha=1.0", "kernel": rr["kernel"],
                          "us_per_step": round(rr["ms_per_step"] * 1e3, 2), "TFLOP/s": round(tf, 1),
                          "frac_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4)})
        log(f"  {secondary[-1]}")
        for cfg, m, a in (("c1", 1, 1.0), ("c1", 1, 0.0), ("c4", 8, 1.0)):
            lay = W.config_layer(cfg)
            rr = time_workload(torch, lay, m, a, SECONDARY_STEPS, 10, plan=True)
            b = W.algorithmic_bytes(lay, m, a)
            secondary.append({"workload": f"{cfg} M={m} alpha={a}", "kernel": rr["kernel"],
                              "us_per_step": round(rr["ms_per_step"] * 1e3, 3),
                              "GB/s": round(b / (rr["ms_per_step"] * 1e-3) / 1e9, 1),
                              "frac_hbm": round(b / (rr["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
            log(f"  {secondary[-1]}")
        # BF16 activations and output: the same weights and the same
        # algorithmic bytes (2 per activation and output element either way)
        down = {l.name: l for l in W.llama_block()}["down_proj"]
        for lay, m, label in ((layer, 1, "c2"), (layer, 8, "c2"), (layer, 32, "c2"), (down, 8, "c5 down_proj")):
            rr = time_workload(torch, lay, m, alpha, SECONDARY_STEPS, 10, plan=True, dtype=torch.bfloat16)
            b = W.algorithmic_bytes(lay, m, alpha)
            secondary.append({"workload": f"{label} M={m} alpha={alpha}, BF16 activations", "kernel": rr["kernel"],
                              "us_per_step": round(rr["ms_per_step"] * 1e3, 3),
                              "GB/s": round(b / (rr["ms_per_step"] * 1e-3) / 1e9, 1),
                              "frac_hbm": round(b / (rr["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
            log(f"  {secondary[-1]}")
        rr = time_workload(torch, layer, 2048, 1.0, 80, 3, plan=True, dtype=torch.bfloat16)
        tf = W.algorithmic_flops(layer, 2048, 1.0) / (rr["ms_per_step"] * 1e-3) / 1e12
        secondary.append({"workload": "prefill 4096->11008 M=2048 alpha=1.0, BF16 activations", "kernel": rr["kernel"],
                          "us_per_step": round(rr["ms_per_step"] * 1e3, 2), "TFLOP/s": round(tf, 1),
                          "frac_bf16_peak": round(tf / FP16_PEAK_TFLOPS, 4)})
        log(f"  {secondary[-1]}")
        # the general kernel (one wave per output): FP32 activations and
        # output (4 bytes each in the traffic), and an FP16 layer whose K is
        # not a multiple of 128 (per-row scales), which no fast kernel takes
        odd = W.make_layer(4000, 11008, None, 0.01, 4000)
        for lay, m, dt, label in ((layer, 1, torch.float32, "c2 M=1 alpha=1.0, FP32 activations"),
                                  (layer, 8, torch.float32, "c2 M=8 alpha=1.0, FP32 activations"),
                                  (odd, 1, None, "4000->11008 per-row scales M=1 alpha=1.0 (K % 128 != 0)")):
            rr = time_workload(torch, lay, m, 1.0, SECONDARY_STEPS, 10, plan=True, dtype=dt)
            b = W.algorithmic_bytes(lay, m, 1.0) + (2 * m * (lay.K + lay.N) if dt == torch.float32 else 0)
            secondary.append({"workload": label, "kernel": rr["kernel"],
                              "us_per_step": round(rr["ms_per_step"] * 1e3, 3),
                              "GB/s": round(b / (rr["ms_per_step"] * 1e-3) / 1e9, 1),
                              "frac_hbm": round(b / (rr["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
            log(f"  {secondary[-1]}")
        for m in (1, 32):
            for grouped in (False, True):
                # 7 launches per step: a shorter graph (the capture holds them all)
                ms, b, f, ks = time_block(torch, m, SECONDARY_STEPS, grouped)
                secondary.append({"workload": f"c5 Llama-2-7B block (7 projections) M={m}"
                                  + (", q/k/v and gate/up grouped" if grouped else ""),
                                  "kernel": "+".join(ks), "us_per_step": round(ms * 1e3, 3),
                                  "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                                  "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                  "TFLOP/s": round(f / (ms * 1e-3) / 1e12, 2)})
                log(f"  {secondary[-1]}")
        r1 = time_dropin(torch, layer, 1, 1.0, 300, graph_steps=SECONDARY_STEPS)
        b = W.algorithmic_bytes(layer, 1, 1.0)
        r1.update({"workload": "reference 8-argument _C_ops.forward, c2 M=1 alpha=1 (eager: the entry's cached "
                               "plan; graph: CSR read)",
                   "GB/s_graph": round(b / (r1["us_per_launch_graph"] * 1e-6) / 1e9, 1)})
        secondary.append(r1)
        log(f"  {secondary[-1]}")
        c3 = W.config_layer("c3")
        r3 = time_dropin(torch, c3, 2048, 1.0, 20)
        f = W.algorithmic_flops(c3, 2048, 1.0)
        r3.update({"workload": "reference 8-argument _C_ops.forward, c3 M=2048 alpha=1 (the entry's cached plan)",
                   "TFLOP/s_gpu": round(f / (r3["us_per_call_gpu"] * 1e-6) / 1e12, 1)})
        secondary.append(r3)
        log(f"  {secondary[-1]}")
        secondary.extend(time_pack(torch))
        secondary.append(time_module(torch))
        log(f"  {secondary[-1]}")

    workload = "c2_m1_alpha1"
    out = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded PCG64; INT4 weights, FP16 scales/values/activations)",
        "config": {"workload": "OrthoLinear 4096->11008 (BASELINE configs[1]), M=1 decode, "
                               "INT4 group-128 FP16 scales, ortho 1% uniform FP16, alpha=1",
                   "in_features": layer.K, "out_features": layer.N, "tokens": M,
                   "group_size": 128, "ortho_nnz": layer.nnz, "alpha": alpha,
                   "bytes_per_step": bytes_step, "flops_per_step": flops_step,
                   "weight_copies_rotated": r["copies"], "kernel": r["kernel"],
                   "ortho_plan": "built once per copy before timing (as OrthoLinear caches it)",
                   "timing": f"device clock stamps (100 MHz s_memrealtime, per XCD, median) launched "
                             f"inside one HIP graph around the K launches, after {PRE_STEPS} untimed "
                             f"launches in the same graph"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": (load_traffic(workload) or {}).get("bytes"),
                     "launch_us": round(r["ms_per_step"] * 1e3, 3),
                     "launch_us_steady": round(r["ms_per_step_steady"] * 1e3, 3),
                     "steady_note": f"launch_us_steady: {STEADY_STEPS} launches in one graph, events around "
                                    "its replay (the per-launch time a kernel trace reports); launch_us: "
                                    "the timed K steps between two device clock stamps (one launch gap "
                                    "of fixed cost, spread over K)",
                     "bytes_per_launch": bytes_step},
        "cpu_baseline": cpu,
        "secondary": secondary,
        "device": {k: info[k] for k in ("arch", "compute_units", "clock_khz")},
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
