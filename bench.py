"""Benchmark: Gated DeltaNet recurrence forward + backward, tokens/s per layer at the Qwen3.5-4B layer shape.

One step = one forward (qb_gdn_fwd, writing the 64-token checkpoints) and one backward (qb_gdn_bwd) over the
workload's tokens, inputs resident in HBM before the timed region. value = tokens / (wall time per step), the best
design's, timed with nothing between the kernels, after PREWARM_MS of the same step untimed (the device's clocks
settle over about 100 ms of load after idling) and the --warmup steps. Each kernel's duration comes from a second run of as many steps
with HIP events the library records on its launch stream around each kernel (the descriptor's trace_events);
the roofline object is for the kernel with the most time per step, its algorithmic work per launch
divided by its mean duration. A kernel's algorithmic bytes are the compulsory tensors it reads or writes in the
caller's buffers plus the 64-token checkpoints it writes or reads (KERNEL_IO); the design's own intermediates it
moves (chunk tiles, chunk-end cotangents) are reported apart as design_bytes_per_launch. step_roofline is the whole
step against the compulsory I/O plus the checkpoints written once and read once. cpu_baseline times the oracle (the
CPU restatement, float32, OpenMP) on the host on the same inputs.

The line also carries the 9B and packed 4B layer shapes and the 4B shape with float32 activations, the dtype of the
reference op (workloads, each with its own rooflines; float32 runs on the recurrent design), the reference
bench's T sweep at the 4B head shape (t_sweep), the one-token inference step (decode), the layer's pointwise
neighbours and the LoRA training step; --path-only leaves those out.

python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--prewarm-ms 150] [--design auto|1|2] [--workload qwen35_4b]
                [--no-cpu] [--copy-probe-mib N] [--path-only] [--prologue-fusion] [--decode-only]

roofline.traffic is the dominant kernel's HBM bytes per launch as rocprofv3 counted them (FETCH_SIZE + WRITE_SIZE,
each scaled by what the counter reads for a plain device copy of known size), read from profiles/traffic.json
when that file holds a measurement for this workload; --copy-probe-mib runs such a copy first, for those runs.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Gated DeltaNet fwd+bwd tokens/s per layer @4B shape; % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, published
FP32_PEAK_TFLOPS = 157.3   # MI355X FP32 vector, published
# The device's clocks take about 100 ms of sustained load to settle after it has idled: after one second idle, 20
# steps at the 4B shape behind 5 warm-up steps averaged 447 us, behind 150 further ms of the same step 388 us. Each
# design's timing therefore starts with this much wall time of its own step, untimed, before the warm-up steps
# (--prewarm-ms; 0 turns it off).
PREWARM_MS = 150.0
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense BF16 MFMA, published


class Hip:
    """The few HIP event calls the timer needs, from the runtime torch already loaded."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def event(self):
        e = ctypes.c_void_p()
        if self.lib.hipEventCreate(ctypes.byref(e)) != 0:
            raise RuntimeError("hipEventCreate failed")
        return e.value

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        if self.lib.hipEventElapsedTime(ctypes.byref(ms), ctypes.c_void_p(a), ctypes.c_void_p(b)) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value


def _sizes(w, nc):
    """Byte sizes of the path's tensors at their storage types (bf16 or float32 I/O, float32 g and states)."""
    BT, Hk, Hv, Dk, Dv = w.B * w.T, w.Hk, w.Hv, w.Dk, w.Dv
    io = 2 if w.dtype == "bf16" else 4
    state = Hv * Dv * Dk * 4
    return {
        "q": BT * Hk * Dk * io, "k": BT * Hk * Dk * io, "v": BT * Hv * Dv * io, "y": BT * Hv * Dv * io,
        "dy": BT * Hv * Dv * io, "dq": BT * Hk * Dk * io, "dk": BT * Hk * Dk * io, "dv": BT * Hv * Dv * io,
        "g": BT * Hv * 4, "dg": BT * Hv * 4, "beta": BT * Hv * io, "dbeta": BT * Hv * io,
        "s0": w.n_states * state if w.s0_std > 0 else 0, "s_out": w.n_states * state,
        "ds_out": w.n_states * state if w.ds_out else 0, "ds0": w.n_states * state,
        # the checkpoints: every chunk-start state read once by the backward, written by the forward except each
        # sequence's first (its initial state)
        "ckpt_read": nc * state, "ckpt_write": (nc - w.n_states) * state,
    }


# Each kernel's share of the step's algorithmic bytes: the compulsory tensors it reads or writes in the caller's
# buffers, plus the checkpoints it writes or reads, each counted once. Tensors a kernel only sees through the
# design's own intermediates (the chunk tiles, the chunk-end cotangents) are not counted here but in DESIGN_IO.
KERNEL_IO = {
    "chunk_prep": ("q", "k", "g", "beta"),
    "chunk_fwd": ("q", "k", "v", "s0", "y", "s_out", "ckpt_write"),
    "chunk_bwd_state": ("q", "k", "dy", "ds_out", "dv", "ds0"),
    "chunk_bwd_grads": ("q", "k", "v", "dy", "g", "beta", "ckpt_read", "dq", "dk", "dg", "dbeta"),
}
# The design's own intermediates each kernel writes or reads: "tiles" (the per-chunk records prep writes after the
# states in ckpt) and "dsend" (the chunk-end state cotangents the backward state pass hands to the gradient kernel).
DESIGN_IO = {
    "chunk_prep": ("tiles",),
    "chunk_fwd": ("tiles",),
    "chunk_bwd_state": ("tiles", "dsend"),
    "chunk_bwd_grads": ("tiles", "dsend"),
}


def algorithmic_work(w, kernel, nc, tiles_bytes=0):
    """(kind, amount per launch, design bytes per launch) for a kernel. kind "bytes": its share of the step's
    algorithmic HBM bytes (KERNEL_IO), with the design's intermediates it moves reported apart. kind "flops" (the
    recurrent design): the recurrent algorithm's flops, 7 Dk Dv per token and value head forward, 15 backward
    (recompute not credited)."""
    s = _sizes(w, nc)
    BT, Hv, Dk, Dv = w.B * w.T, w.Hv, w.Dk, w.Dv
    if kernel in KERNEL_IO:
        design = {"tiles": tiles_bytes, "dsend": s["ckpt_read"]}
        return "bytes", sum(s[n] for n in KERNEL_IO[kernel]), sum(design[n] for n in DESIGN_IO[kernel])
    if kernel == "rec_fwd":
        return "flops", 7.0 * Dk * Dv * BT * Hv, 0
    if kernel == "rec_bwd":
        return "flops", 15.0 * Dk * Dv * BT * Hv, 0
    if kernel == "rec_reduce":
        nblk = (Dv + 15) // 16
        return "bytes", sum(s[n] for n in ("g", "dq", "dk", "dg", "dbeta")), 2 * BT * Hv * nblk * (Dk + 1) * 4
    raise KeyError(kernel)


def step_roof_us(w, nc):
    """The whole fwd+bwd step's roofline time: max(bytes_alg / HBM peak, flops_alg / MFMA peak), bytes_alg = the
    compulsory bf16/f32 I/O plus the 64-token fp32 checkpoints written once and read once, flops_alg = 22 Dk Dv per
    token and value head."""
    s = _sizes(w, nc)
    fwd = ("q", "k", "v", "g", "beta", "s0", "y", "s_out")
    bwd = ("q", "k", "v", "g", "beta", "dy", "ds_out", "dq", "dk", "dv", "dg", "dbeta", "ds0")
    nbytes = sum(s[n] for n in fwd) + sum(s[n] for n in bwd) + s["ckpt_write"] + s["ckpt_read"]
    if w.s0_std <= 0 and not w.ds_out:
        nbytes -= s["ds0"]  # no initial state and no final-state cotangent: dS0 is not asked for
    flops = 22.0 * w.Dk * w.Dv * w.B * w.T * w.Hv
    return max(nbytes / (HBM_PEAK_GBS * 1e9), flops / (BF16_MFMA_PEAK_TFLOPS * 1e12)) * 1e6, nbytes, flops


def roofline_of(kind, amount, ms):
    if kind == "bytes":
        achieved = amount / (ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS}
    achieved = amount / (ms * 1e-3) / 1e12
    return {"bound": "valu", "achieved": achieved, "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": achieved / FP32_PEAK_TFLOPS}


def run_design(torch, hip, lib, w, dev, design, steps, warmup):
    """Times `steps` fwd+bwd steps after PREWARM_MS of untimed steps and `warmup` more, then runs as many with the
    library's trace events for each
    kernel's duration, then as many again with the caches flushed before the forward and before the backward;
    returns wall ms/step (of the uninstrumented steps), per-kernel mean ms, and the cold-cache step and kernels."""
    B, T, Hk, Hv, Dk, Dv = w.B, w.T, w.Hk, w.Hv, w.Dk, w.Dv
    cu = w.cu_seqlens
    dt = lib.BF16 if w.dtype == "bf16" else lib.F32
    desc_f, keep_f = lib.make_desc(B, T, Hk, Hv, Dk, Dv, dtype=dt, design=design, cu_seqlens=cu)
    desc_b, keep_b = lib.make_desc(B, T, Hk, Hv, Dk, Dv, dtype=dt, design=design, cu_seqlens=cu)
    why = lib.validate(desc_f)
    if why:
        return None, why
    fnames, bnames = lib.launches(desc_f, 0), lib.launches(desc_b, 1)
    N = w.n_states
    tdt = torch.bfloat16 if w.dtype == "bf16" else torch.float32
    y = torch.empty(B, T, Hv, Dv, dtype=tdt, device="cuda")
    s_out = torch.empty(N, Hv, Dv, Dk, dtype=torch.float32, device="cuda")
    ckpt = torch.empty(lib.ckpt_bytes(desc_f) // 4, dtype=torch.float32, device="cuda")
    ws = torch.empty(max(lib.workspace_bytes(desc_f), 1), dtype=torch.uint8, device="cuda")
    dq, dk = torch.empty_like(dev["q"]), torch.empty_like(dev["k"])
    dv, dbeta = torch.empty_like(dev["v"]), torch.empty_like(dev["beta"])
    dg = torch.empty_like(dev["g"])
    ds0 = torch.empty(N, Hv, Dv, Dk, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    nf, nb = len(fnames) + 1, len(bnames) + 1
    evs = [[hip.event() for _ in range(nf + nb)] for _ in range(steps)]

    def step(i=None, flush=None, st=stream):
        if i is not None:
            keep1 = lib.set_trace(desc_f, evs[i][:nf])
            keep2 = lib.set_trace(desc_b, evs[i][nf:])
        else:
            desc_f.trace_events, desc_f.n_trace_events = None, 0
            desc_b.trace_events, desc_b.n_trace_events = None, 0
        if flush is not None:
            flush.sum()
        lib.fwd(desc_f, p(dev["q"]), p(dev["k"]), p(dev["v"]), p(dev["g"]), p(dev["beta"]), p(dev["s0"]), p(y),
                p(s_out), p(ckpt), p(ws), st)
        if flush is not None:
            flush.sum()
        lib.bwd(desc_b, p(dev["q"]), p(dev["k"]), p(dev["v"]), p(dev["g"]), p(dev["beta"]), p(ckpt), p(dev["dy"]),
                p(dev["ds_out"]), p(dq), p(dk), p(dv), p(dg), p(dbeta), p(ds0), p(ws), st)
        if i is not None:
            del keep1, keep2

    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < PREWARM_MS:  # the clocks' settling time, untimed
        for _ in range(4):
            step()
        torch.cuda.synchronize()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()  # the step as a caller runs it: no events between the kernels
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    # The same steps captured once into a HIP graph and replayed, timed with events: the GPU's time per step without
    # the host's launches (what a caller that replays captured steps sees; at short sequences the host's launch rate,
    # not the GPU, sets the wall time above).
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _ in range(steps):
            step(st=side.cuda_stream)
    graph.replay()
    torch.cuda.synchronize()
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g0.record()
    for _ in range(3):
        graph.replay()
    g1.record()
    torch.cuda.synchronize()
    graph_ms = g0.elapsed_time(g1) / (3 * steps)
    del graph
    for i in range(steps):  # the same steps again with an event before and after each kernel, for their durations
        step(i)
    torch.cuda.synchronize()
    per = {}
    for i in range(steps):
        e = evs[i]
        for j, n in enumerate(fnames):
            per.setdefault(n, []).append(hip.elapsed_ms(e[j], e[j + 1]))
        for j, n in enumerate(bnames):
            per.setdefault(n, []).append(hip.elapsed_ms(e[nf + j], e[nf + j + 1]))
    fwd_ms = sum(hip.elapsed_ms(evs[i][0], evs[i][nf - 1]) for i in range(steps)) / steps
    bwd_ms = sum(hip.elapsed_ms(evs[i][nf], evs[i][nf + nb - 1]) for i in range(steps)) / steps
    # The same steps with the caches holding none of the step's data: a 512 MB read of an unrelated buffer before the
    # forward and before the backward (in training, other layers run between them). The kernels' spans, flushes
    # excluded.
    flush = torch.ones(128 << 20, dtype=torch.float32, device="cuda")
    for i in range(steps):
        step(i, flush)
    torch.cuda.synchronize()
    cold = {}
    for i in range(steps):
        e = evs[i]
        for j, n in enumerate(fnames):
            cold.setdefault(n, []).append(hip.elapsed_ms(e[j], e[j + 1]))
        for j, n in enumerate(bnames):
            cold.setdefault(n, []).append(hip.elapsed_ms(e[nf + j], e[nf + j + 1]))
    cold_ms = sum(hip.elapsed_ms(evs[i][0], evs[i][nf - 1]) + hip.elapsed_ms(evs[i][nf], evs[i][nf + nb - 1])
                  for i in range(steps)) / steps
    del flush
    for row in evs:
        for e in row:
            hip.lib.hipEventDestroy(ctypes.c_void_p(e))
    del keep_f, keep_b
    kernels = {n: sum(v) / len(v) for n, v in per.items()}
    nc = lib.num_chunks(desc_f)
    tiles = lib.ckpt_bytes(desc_f) - nc * Hv * Dv * Dk * 4
    return {"ms_per_step": wall_ms, "graph_ms_per_step": graph_ms, "fwd_ms": fwd_ms, "bwd_ms": bwd_ms,
            "kernels_ms": kernels,
            "cold_caches": {"ms_per_step": cold_ms, "kernels_ms": {n: sum(v) / len(v) for n, v in cold.items()}},
            "nc": nc,
            "tiles_bytes": tiles}, None


def run_decode(torch, lib, w, design, calls=200, warmup=20, graph_calls=64, replays=10):
    """The inference step: one-token forward calls at the workload's head shape, each carrying the state to the
    next (the reference's decode, src/deltanet.cpp:101-120). Returns microseconds per call, or None when the design
    rejects the shape: "host", the calls timed back to back on the host clock (launch included), and "graph", the
    same calls captured into a HIP graph and replayed, timed with events (the GPU's time per call, as a serving loop
    that replays captured steps sees it)."""
    from quotebound_amd.synthetic import Workload, make_inputs, to_device

    dw = Workload("decode", w.B, 1, w.Hk, w.Hv, w.Dk, w.Dv, seed=5, s0_std=0.02)
    dev = to_device(make_inputs(dw), "cuda")
    dt = lib.BF16 if w.dtype == "bf16" else lib.F32
    desc, keep = lib.make_desc(w.B, 1, w.Hk, w.Hv, w.Dk, w.Dv, dtype=dt, design=design)
    if lib.validate(desc):
        return None
    y = torch.empty_like(dev["v"])
    states = [dev["s0"].clone(), torch.empty_like(dev["s0"])]
    ws = torch.empty(max(lib.workspace_bytes(desc), 1), dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    def call(i):
        lib.fwd(desc, p(dev["q"]), p(dev["k"]), p(dev["v"]), p(dev["g"]), p(dev["beta"]), p(states[i & 1]), p(y),
                p(states[(i + 1) & 1]), None, p(ws), side.cuda_stream)

    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        for i in range(warmup):
            call(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(calls):
            call(i)
        torch.cuda.synchronize()
        host = (time.perf_counter() - t0) * 1e6 / calls
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for i in range(graph_calls):
            call(i)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph, keep
    return {"host": host, "graph": e0.elapsed_time(e1) * 1e3 / (replays * graph_calls)}


def run_neighbours(torch, lib, w, calls=50, warmup=5):
    """The layer's pointwise neighbours at the workload's shape (bf16 activations): each C-ABI entry point called
    back to back on one stream into preallocated outputs (so the host keeps ahead of the GPU), timed with events
    around the calls. Returns, per entry point, microseconds per call, the algorithmic HBM bytes (each activation
    read or written once) and their rate against the HBM peak."""
    if w.dtype != "bf16":
        return None
    g = torch.Generator(device="cuda").manual_seed(11)
    bt = w.B * w.T
    r = lambda *shape: torch.randn(*shape, device="cuda", generator=g).to(torch.bfloat16)  # noqa: E731
    qr, kr, dq, dk, q, k, dqr, dkr = (r(w.B, w.T, w.Hk, w.Dk) for _ in range(8))
    a, b, dbeta, beta, da, db = (r(w.B, w.T, w.Hv) for _ in range(6))
    dld, ld = (torch.randn(w.B, w.T, w.Hv, device="cuda", generator=g) for _ in range(2))
    a_log = torch.rand(w.Hv, device="cuda", generator=g) * 2.7
    dt_bias = torch.randn(w.Hv, device="cuda", generator=g) * 0.5
    da_log, ddt = torch.empty_like(a_log), torch.empty_like(dt_bias)
    y, z, dout, o, dy, dz = (r(w.B, w.T, w.Hv, w.Dv) for _ in range(6))
    nw, dnw = torch.ones(w.Dv, device="cuda"), torch.empty(w.Dv, device="cuda")
    desc, keep = lib.make_desc(w.B, w.T, w.Hk, w.Hv, w.Dk, w.Dv, dtype=lib.BF16)
    ws = torch.empty(max(lib.neighbours_workspace_bytes(desc), 1), dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    P = lambda *ts: [t.data_ptr() for t in ts]  # noqa: E731
    qk, gv, yz = bt * w.Hk * w.Dk * 2, bt * w.Hv, bt * w.Hv * w.Dv * 2
    cases = {
        "prologue_fwd": (lambda: lib.prologue_fwd(desc, *P(qr, kr, a, b, a_log, dt_bias, q, k, beta, ld), st),
                         4 * qk + 10 * gv),
        "prologue_bwd": (lambda: lib.prologue_bwd(desc, *P(qr, kr, a, b, a_log, dt_bias, dq, dk, dbeta, dld, dqr, dkr,
                                                         da, db, da_log, ddt, ws), st), 6 * qk + 14 * gv),
        "epilogue_fwd": (lambda: lib.epilogue_fwd(desc, y.data_ptr(), z.data_ptr(), nw.data_ptr(), 1e-6,
                                                  o.data_ptr(), st), 3 * yz),
        "epilogue_bwd": (lambda: lib.epilogue_bwd(desc, y.data_ptr(), z.data_ptr(), nw.data_ptr(), 1e-6,
                                                  *P(dout, dy, dz, dnw, ws), st), 5 * yz),
    }
    out = {"unit": "us per call (events around back-to-back calls on the launch stream)",
           "config": f"B={w.B} T={w.T} Hk={w.Hk} Hv={w.Hv} Dk={w.Dk} Dv={w.Dv}, bf16 activations"}
    for name, (fn, nbytes) in cases.items():
        for _ in range(warmup):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(calls):
            fn()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / calls
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"us": us, "bytes_alg": nbytes, "GB/s": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}
    del keep
    out["prologue_fusion"] = run_prologue_fusion(torch, lib, w, calls=20, warmup=warmup)
    return out


def run_prologue_fusion(torch, lib, w, calls=20, warmup=3):
    """The recurrence with its prologue, forward and backward, two ways at the workload's shape: the separate
    prologue pass, chunked forward, chunked backward and prologue backward (four entry points), and the two fused
    entry points (qb_gdn_fwd_prologue, qb_gdn_bwd_prologue). Microseconds per forward+backward, events around
    back-to-back calls."""
    g = torch.Generator(device="cuda").manual_seed(13)
    r = lambda *shape: torch.randn(*shape, device="cuda", generator=g).to(torch.bfloat16)  # noqa: E731
    qr, kr, q, k, dq, dk, dqr, dkr = (r(w.B, w.T, w.Hk, w.Dk) for _ in range(8))
    a, b, beta, dbeta, da, db = (r(w.B, w.T, w.Hv) for _ in range(6))
    v, dy, y, dv = (r(w.B, w.T, w.Hv, w.Dv) for _ in range(4))
    ld, dld = (torch.empty(w.B, w.T, w.Hv, device="cuda") for _ in range(2))
    a_log = torch.rand(w.Hv, device="cuda", generator=g) * 2.7
    dt_bias = torch.randn(w.Hv, device="cuda", generator=g) * 0.5
    da_log, ddt = torch.empty_like(a_log), torch.empty_like(dt_bias)
    desc, keep = lib.make_desc(w.B, w.T, w.Hk, w.Hv, w.Dk, w.Dv, dtype=lib.BF16, design=lib.CHUNKED,
                               cu_seqlens=w.cu_seqlens)
    nbd, keep2 = lib.make_desc(w.B, w.T, w.Hk, w.Hv, w.Dk, w.Dv, dtype=lib.BF16)
    N = w.n_states
    s_out, ds0 = (torch.empty(N, w.Hv, w.Dv, w.Dk, device="cuda") for _ in range(2))
    ckpt = torch.empty(lib.ckpt_bytes(desc) // 4, device="cuda")
    ws = torch.empty(max(lib.workspace_bytes(desc), lib.neighbours_workspace_bytes(nbd), 1), dtype=torch.uint8,
                     device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    P = lambda *ts: [None if t is None else t.data_ptr() for t in ts]  # noqa: E731

    def separate():
        lib.prologue_fwd(nbd, *P(qr, kr, a, b, a_log, dt_bias, q, k, beta, ld), st)
        lib.fwd(desc, *P(q, k, v, ld, beta, None, y, s_out, ckpt, ws), st)
        lib.bwd(desc, *P(q, k, v, ld, beta, ckpt, dy, None, dq, dk, dv, dld, dbeta, ds0, ws), st)
        lib.prologue_bwd(nbd, *P(qr, kr, a, b, a_log, dt_bias, dq, dk, dbeta, dld, dqr, dkr, da, db, da_log, ddt,
                                 ws), st)

    def fused():
        lib.fwd_prologue(desc, *P(qr, kr, v, a, b, a_log, dt_bias, None, q, k, beta, ld, y, s_out, ckpt, ws), st)
        lib.bwd_prologue(desc, *P(qr, kr, a, b, a_log, dt_bias, q, k, v, beta, ld, ckpt, dy, None, dqr, dkr, dv, da,
                                  db, da_log, ddt, ds0, ws), st)

    out = {"unit": "us per forward+backward (events around back-to-back calls)"}
    for name, fn in (("separate", separate), ("fused", fused)):
        for _ in range(warmup):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(calls):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = e0.elapsed_time(e1) * 1e3 / calls
    out["saved_frac"] = 1.0 - out["fused"] / out["separate"]
    del keep, keep2
    return out


def run_lora_step(torch, steps=5, warmup=2):
    """One LoRA training step of the tiny Qwen3.5-architecture model (quotebound_amd.lora.Config: 8 layers 3
    DeltaNet : 1 attention, hidden 1024, bf16 base, rank 16 on q/k/v/o and the DeltaNet in/out projections) on 4
    sequences of 1024 random tokens with the loss on the last half: forward, adapter gradients, AdamW. Timed with
    device synchronisations around `steps` steps, run eagerly and replayed from a captured HIP graph, with the
    DeltaNet layers' prologue fused into the recurrence (the default); `separate_prologue` replays the same step
    with the prologue as its own passes, and `prologue_fusion_ms` is what the fusion saves per step.
    `deltanet_path` times one DeltaNet layer's prologue and recurrence, forward and backward, at the layer's shape
    (B=4, T=1024, Hk=4, Hv=8, Dk=Dv=128) both ways, events around back-to-back calls."""
    import dataclasses

    from quotebound_amd import lora

    cfg = lora.Config()
    host = lora.init_weights(cfg, seed=31)
    w = lora.to_device(host, "cuda", torch.bfloat16)
    ads = lora.adapters_to(lora.init_adapters(cfg, host, seed=32, b_std=0.05), "cuda")
    batch = tuple(t.cuda() for t in lora.last_half_batch(4, 1024, cfg.vocab, seed=33))
    out = {"config": "8 layers (3 Gated DeltaNet : 1 attention), hidden 1024, DeltaNet Hk=4 Hv=8 D=128, vocab 32000,"
                     " bf16 base, LoRA rank 16 on q/k/v/o + in_proj_qkv/out_proj; batch 4 x 1024, loss on the last"
                     " half; forward + adapter gradients + AdamW"}
    for mode in ("eager", "graph"):
        step = lora.GraphStep(w, ads, lora.AdamW(lr=1e-4), cfg, batch, capture=(mode == "graph"))
        for _ in range(warmup):
            loss, _ = step(*batch)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            loss, _ = step(*batch)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        out[mode] = {"ms_per_step": ms, "tokens_per_s": 4 * 1024 / (ms * 1e-3), "loss": float(loss)}
        del step
    sep = dataclasses.replace(cfg, fused_prologue=False)
    step = lora.GraphStep(w, ads, lora.AdamW(lr=1e-4), sep, batch, capture=True)
    for _ in range(warmup):
        loss, _ = step(*batch)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss, _ = step(*batch)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    out["separate_prologue"] = {"graph_ms_per_step": ms, "loss": float(loss)}
    out["prologue_fusion_ms"] = ms - out["graph"]["ms_per_step"]
    del step
    from quotebound_amd import _lib
    from quotebound_amd.synthetic import Workload

    lw = Workload("lora_deltanet_layer", 4, 1024, cfg.lin_k_heads, cfg.lin_v_heads, cfg.lin_k_dim, cfg.lin_v_dim)
    out["deltanet_path"] = run_prologue_fusion(torch, _lib, lw, calls=20, warmup=warmup)
    out["deltanet_path"]["layers_per_step"] = sum(cfg.is_linear(i) for i in range(cfg.layers))
    return out


def traffic_of(w, kernel):
    """HBM bytes per launch of kernel from profiles/traffic.json (rocprofv3 FETCH_SIZE and WRITE_SIZE in KiB per
    dispatch, scaled by the copy calibration recorded with them), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    k = t.get("workloads", {}).get(w.name, {}).get(kernel)
    cal = t.get("calibration")
    if not k or not cal:
        return None
    return k["fetch_kib"] * 1024 * cal["fetch_factor"] + k["write_kib"] * 1024 * cal["write_factor"]


def copy_probe(torch, mib):
    """A plain device-to-device copy of mib MiB, three times: the calibration kernel of the traffic counters."""
    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def cpu_baseline(w, inp, budget_s=12.0, max_reps=60):
    """The oracle's float32 forward + backward on the host cores, repeated until about budget_s."""
    from oracle import gdn_ref

    f = inp.f32
    reps, total = 0, 0.0
    while reps < max_reps and (reps == 0 or total < budget_s):
        t0 = time.perf_counter()
        y, s, ck = gdn_ref.fwd(f["q"], f["k"], f["v"], f["g"], f["beta"], f["s0"], cu_seqlens=w.cu_seqlens,
                               dtype="float32")
        gdn_ref.bwd(f["q"], f["k"], f["v"], f["g"], f["beta"], ck, f["dy"], f["ds_out"], cu_seqlens=w.cu_seqlens,
                    dtype="float32")
        total += time.perf_counter() - t0
        reps += 1
    per = total / reps
    return {"value": w.tokens / per, "unit": "tokens/s", "cores": gdn_ref.threads(), "kind": "port",
            "sample": f"the full {w.name} workload ({w.tokens} tokens), float32 forward + backward, "
                      f"{reps} run(s), {per:.2f} s each"}


DESIGN_NAMES = {1: "recurrent", 2: "chunked"}


def measure_workload(torch, hip, lib, w, designs, steps, warmup):
    """Every design in `designs` on workload w: ms per step, per-kernel durations, and for the fastest the roofline
    of its dominant kernel and of the whole step. Returns (summary, inputs) or (None, reasons)."""
    from quotebound_amd.synthetic import make_inputs, to_device

    inp = make_inputs(w)
    dev = to_device(inp, "cuda")
    torch.cuda.synchronize()
    results = {}
    for d in designs:
        r, why = run_design(torch, hip, lib, w, dev, d, steps, warmup)
        if r is None:
            results[DESIGN_NAMES[d]] = {"unavailable": why}
            continue
        r["tokens_per_s"] = w.tokens / (r["ms_per_step"] * 1e-3)
        results[DESIGN_NAMES[d]] = r
    del dev
    ok = {k: v for k, v in results.items() if "ms_per_step" in v}
    if not ok:
        return None, results
    best = max(ok, key=lambda k: ok[k]["tokens_per_s"])
    r = ok[best]
    dom = max(r["kernels_ms"], key=r["kernels_ms"].get)
    kind, amount, design_bytes = algorithmic_work(w, dom, r["nc"], r["tiles_bytes"])
    roof = roofline_of(kind, amount, r["kernels_ms"][dom])
    roof.update({"kernel": dom, "mean_ms": r["kernels_ms"][dom], "algorithmic_" + kind + "_per_launch": amount,
                 "design_bytes_per_launch": design_bytes, "traffic": traffic_of(w, dom)})
    t_roof, nbytes, nflops = step_roof_us(w, r["nc"])
    summary = {
        "workload": f"{w.name}: B={w.B} T={w.T} Hk={w.Hk} Hv={w.Hv} Dk={w.Dk} Dv={w.Dv}"
                    + (f" ({len(w.seq_lens)} packed sequences)" if w.seq_lens else "")
                    + (", nonzero initial state" if w.s0_std > 0 else "")
                    + f", {w.dtype} I/O, fp32 state, 64-token checkpoints, fwd+bwd",
        "tokens": w.tokens, "design": best, "ms_per_step": r["ms_per_step"], "tokens_per_s": r["tokens_per_s"],
        "roofline": roof,
        "step_roofline": {"t_roof_us": t_roof, "bytes_alg": nbytes, "flops_alg": nflops,
                          "t_step_us": r["ms_per_step"] * 1e3, "frac": t_roof / (r["ms_per_step"] * 1e3)},
        "designs": {k: ({kk: vv for kk, vv in v.items() if kk not in ("nc", "tiles_bytes")} if "ms_per_step" in v
                        else v) for k, v in results.items()},
    }
    return summary, inp


def run_t_sweep(torch, hip, lib, design, steps=10, warmup=2):
    """The reference bench's sweep (reference tests/bench_grad.cpp:38-68, 124-130): the recurrence at the 4B head
    shape (B=1, Hk=16, Hv=32, Dk=Dv=128) for T in 128, 512, 1024, 2048, forward and forward + backward, with each
    kernel's time (what dominates at short T)."""
    from quotebound_amd.synthetic import make_inputs, to_device, workload

    out = {"unit": "ms: fwd_ms from HIP events around the forward's kernels, fwd_bwd_ms per step on the host clock "
                   "(launches from Python included), fwd_bwd_graph_ms per step from a replayed HIP graph",
           "design": DESIGN_NAMES[design]}
    for T in (128, 512, 1024, 2048):
        w = workload(f"qwen35_4b_t{T}")
        dev = to_device(make_inputs(w), "cuda")
        r, why = run_design(torch, hip, lib, w, dev, design, steps, warmup)
        if r is None:
            out[str(T)] = {"unavailable": why}
            continue
        out[str(T)] = {"fwd_ms": r["fwd_ms"], "fwd_bwd_ms": r["ms_per_step"],
                       "fwd_bwd_graph_ms": r["graph_ms_per_step"],
                       "tokens_per_s": T / (r["ms_per_step"] * 1e-3), "kernels_ms": r["kernels_ms"]}
    return out


def main():
    global PREWARM_MS
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--design", default="auto")
    ap.add_argument("--workload", default="qwen35_4b")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe-mib", type=int, default=0)
    ap.add_argument("--path-only", action="store_true",
                    help="time only the named workload's step (no other shapes, decode, neighbours or LoRA step), as "
                         "profiler counter passes need")
    ap.add_argument("--prologue-fusion", action="store_true",
                    help="time only the layer with its prologue, fused and as four separate entry points, at the "
                         "named workload's shape, and print that object (for kernel traces)")
    ap.add_argument("--prewarm-ms", type=float, default=PREWARM_MS,
                    help="wall time of each design's own step run untimed before its warm-up steps, for the device's "
                         "clocks to settle (0: none)")
    ap.add_argument("--decode-only", action="store_true",
                    help="time only the one-token inference step at the named workload's head shape, and print that "
                         "object (for kernel traces)")
    args = ap.parse_args()
    PREWARM_MS = args.prewarm_ms
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the recurrence shards "
              "by key-head groups with no exchange, so per-GPU work is the one-GPU run at Hk/N, Hv/N).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from quotebound_amd import _lib as lib
    from quotebound_amd.synthetic import workload

    if args.copy_probe_mib > 0:
        copy_probe(torch, args.copy_probe_mib)
    hip = Hip()
    if args.prologue_fusion:
        print(json.dumps(run_prologue_fusion(torch, lib, workload(args.workload), calls=args.steps,
                                             warmup=args.warmup)))
        return
    designs = [lib.RECURRENT, lib.CHUNKED] if args.design == "auto" else [int(args.design)]
    w = workload(args.workload)
    if args.decode_only:
        print(json.dumps({DESIGN_NAMES[d]: run_decode(torch, lib, w, d, calls=args.steps) for d in designs}))
        return
    head, inp = measure_workload(torch, hip, lib, w, designs, args.steps, args.warmup)
    if head is None:
        print(json.dumps({"metric": METRIC, "error": inp}))
        sys.exit(1)
    out = {
        "metric": METRIC,
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm_ms": PREWARM_MS,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if head["design"] == "recurrent" else "bf16x3-mfma/f32",
        "data": "synthetic (seeded numpy: unit-norm q/k, N(0,1) v, log-decay -softplus(N) clipped to [-8,0], "
                "beta sigmoid(N), dy N(0,1))",
        "config": {"workload": head["workload"], "design": head["design"], "io_dtype": w.dtype},
        "roofline": head["roofline"],
        "step_roofline": head["step_roofline"],
        "designs": head["designs"],
    }
    if not args.path_only:
        # The other layer shapes of the same metric, each with its own rooflines.
        out["workloads"] = {}
        for name in ("qwen35_9b", "qwen35_4b_varlen", "qwen35_4b_f32"):
            summary, _ = measure_workload(torch, hip, lib, workload(name), designs, args.steps, args.warmup)
            out["workloads"][name] = summary
        best = lib.CHUNKED if head["design"] == "chunked" else lib.RECURRENT
        out["t_sweep"] = run_t_sweep(torch, hip, lib, best)
        out["decode"] = {"unit": "us per one-token call (state carried): host clock with launch, and graph replay",
                         "config": f"B={w.B} Hk={w.Hk} Hv={w.Hv} Dk={w.Dk} Dv={w.Dv}, {w.dtype} I/O, fp32 state"}
        for d in designs:
            out["decode"][DESIGN_NAMES[d]] = run_decode(torch, lib, w, d)
        out["neighbours"] = run_neighbours(torch, lib, w)
        out["lora_step"] = run_lora_step(torch)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(w, inp)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
