"""Benchmark of the exact-fusions-v1 per-token layer path on one MI355X.

Headline workload: one launch of the fused residual-add +
RMSNorm + Q/K RMSNorm + NeoX RoPE + BF16 KV-store over a 2048-token prefill chunk
(hidden 2048, 16 Q heads, 4 KV heads, head_dim 128, KV capacity 131072, positions 0..2047
from a device PrefillState).  A step is one such launch.  Inputs are synthetic (seed 0,
1% outlier channels x20), resident in HBM before timing.  Launches rotate over `--sets`
independent buffer sets (50 by default, each with its own KV cache: about 3 GB touched per
graph replay) so the 256 MB Infinity Cache cannot serve them; K launches are captured in
one HIP graph.  The launch updates x, q and k in place, so every timed replay starts from
inputs restored by the library's streaming copy (clean in HBM, not dirty in a cache), and
ms_per_step is the median of `--replays` timed replays (p10 and p90
beside it).

Output: one JSON line (rank 0).  value = achieved algorithmic HBM GB/s of the launch;
roofline.frac = value / 8000 GB/s; cpu_baseline = the C oracle (a scalar port of the
reference arithmetic) timed on a bounded sample of the same workload on the host.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
TOKENS, HIDDEN, HQ, HKV, D, CAPACITY = 2048, 2048, 16, 4, 128, 131072


def chain_bytes(fmt: str) -> int:
    """Algorithmic HBM bytes per token of the fused chain (BF16 device I/O):
    residual-norm: read x, r; write x, y (4 * 2H);
    Q/K: read q, k, v; write q, k in place; one cos|sin table row (2D);
    cache: the K and V rows in `fmt` (BF16 2*1024; q8 1024 codes + 32 B scales;
    q8_0 2*544)."""
    norm = 4 * 2 * HIDDEN
    qk = 2 * (2 * HQ * D) + 2 * (2 * HKV * D) + 2 * HKV * D + 2 * D
    cache = {"bf16": 2 * 2 * HKV * D, "q8": 2 * HKV * D + 8 * HKV, "q8_0": 2 * 544,
             "q8_0_norot": 2 * 544}[fmt]
    return norm + qk + cache


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sets", type=int, default=50,
                    help="independent buffer sets of the headline workload (each with its own "
                         "KV cache); a 200-launch graph uses each set 4 times")
    ap.add_argument("--replays", type=int, default=11,
                    help="timed graph replays of the headline workload, each from restored "
                         "inputs; ms_per_step is their median")
    ap.add_argument("--positions", choices=("prefill", "base"), default="prefill",
                    help="headline positions from the chunk's device PrefillState (default) "
                         "or host-known (base + t)")
    ap.add_argument("--restore", choices=("stream", "torch"), default="stream",
                    help="how the untimed restore copies the inputs back: the library's "
                         "streaming copy (clean in HBM, like the copy ceiling's source) or "
                         "torch's copy_ (its written lines still dirty in the caches when "
                         "the timed replay starts)")
    ap.add_argument("--no-compare", action="store_true",
                    help="skip the 8-set (Infinity-Cache-assisted) comparison leg, so that a "
                         "profiled run's kernel averages are of cold launches")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the config 0/3/4 measurements (headline only)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--formats", default="bf16,q8_0,q8_0_norot,q8",
                    help="KV formats measured (the first is the headline)")
    return ap.parse_args()


class ChainSet:
    """One independent buffer set of the config-1 workload (`tokens` rows of host's)."""

    def __init__(self, torch, host, table, fmt, tokens=TOKENS, base_positions=False):
        if tokens != len(host["x"]):
            host = {k: (v[:tokens] if k in ("x", "residual", "q", "k", "v") else v)
                    for k, v in host.items()}
        from padra_amd import abi, ops
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()
        self.x, self.r = dev(host["x"]), dev(host["residual"])
        self.y = torch.empty_like(self.x)
        self.q, self.k, self.v = dev(host["q"]), dev(host["k"]), dev(host["v"])
        self.g, self.qn, self.kn = dev(host["gamma"]), dev(host["qn"]), dev(host["kn"])
        self.table = table
        code = {"bf16": abi.KV_BF16, "q8": abi.KV_Q8, "q8_0": abi.KV_Q8_0,
                "q8_0_norot": abi.KV_Q8_0_NOROT}[fmt]
        if fmt == "bf16":
            self.kc = torch.empty((CAPACITY, HKV * D), dtype=torch.int16, device="cuda")
            self.vc = torch.empty_like(self.kc)
            self.sc = None
        elif fmt == "q8":
            self.kc = torch.empty((CAPACITY, HKV * D), dtype=torch.int8, device="cuda")
            self.vc = torch.empty_like(self.kc)
            self.sc = torch.empty((CAPACITY, HKV, 2), dtype=torch.float32, device="cuda")
        else:
            self.kc = torch.empty((CAPACITY, 544), dtype=torch.uint8, device="cuda")
            self.vc = torch.empty_like(self.kc)
            self.sc = None
        self.state = torch.tensor([0, 0, tokens, CAPACITY, 0, 1, 1, 1], dtype=torch.int32,
                                  device="cuda")
        self.bad = torch.zeros(1, dtype=torch.int32, device="cuda")
        self.pos = ops.positions_base(0) if base_positions else \
            ops.positions_prefill(self.state, maximum=CAPACITY)
        self.kv = ops.kv_cache(code, self.kc, self.vc, CAPACITY, scales=self.sc)
        self.ops = ops
        # The launch updates x, q and k in place; restore() puts the synthetic inputs back
        # so that a timed replay sees the config's data, not data that earlier replays have
        # driven away from it (x accumulating r, q and k rescaled by qn, kn every launch).
        self.pristine = [(t, t.clone()) for t in (self.x, self.q, self.k)]

    def restore(self, mode="stream"):
        """Copies the pristine inputs back.  "stream" uses the library's streaming copy,
        whose non-temporal stores leave the inputs clean in HBM, as the copy ceiling's
        source is; "torch" uses copy_, whose written lines are still dirty in the caches when
        the timed launches start, and the launches pay for their write-back (config-1 BF16
        chunk: 13.24 against 12.58 us)."""
        from padra_amd import abi
        import torch
        stream = torch.cuda.current_stream().cuda_stream
        for t, p in self.pristine:
            if mode == "torch":
                t.copy_(p)
            else:
                abi.call("padra_StreamCopy", stream, t.data_ptr(), p.data_ptr(),
                         t.numel() * t.element_size())

    def launch(self):
        self.ops.ResidualNormQKRopeStore(self.x, self.r, self.y, self.g, self.q, self.k, self.v,
                                         self.qn, self.kn, self.table, self.pos, self.kv, self.bad)


def time_graph_fresh(torch, sets, steps, warmup, replays=11, restore="stream"):
    """Captures `steps` launches (rotating over sets) into one graph, warms it up, then
    times `replays` replays, each after every set's inputs are restored (untimed): returns
    the ms/launch of each timed replay, sorted."""
    for i in range(warmup):
        sets[i % len(sets)].launch()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                sets[i % len(sets)].launch()
    torch.cuda.synchronize()
    warm_graph(torch, graph)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = []
    for _ in range(replays):
        for s in sets:
            s.restore(restore)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            lead_in(torch)
            start.record(stream)
            graph.replay()
            end.record(stream)
        torch.cuda.synchronize()
        out.append(start.elapsed_time(end) / steps)
    return sorted(out)


def time_graph(torch, sets, steps, warmup, replays=None):
    """Captures `steps` launches (rotating over sets) into one graph; returns ms/launch of
    one timed replay.  With `replays` (a list), that many further replays are timed the
    same way and their ms/launch appended to it (for the spread of the figure)."""
    for i in range(warmup):
        sets[i % len(sets)].launch()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                sets[i % len(sets)].launch()
    torch.cuda.synchronize()
    warm_graph(torch, graph)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        lead_in(torch)
        start.record(stream)
        graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    if replays is not None:
        for _ in range(9):
            with torch.cuda.stream(stream):
                lead_in(torch)
                start.record(stream)
                graph.replay()
                end.record(stream)
            torch.cuda.synchronize()
            replays.append(start.elapsed_time(end) / steps)
    return ms


def lead_in(torch, cycles=2_000_000):
    """An untimed spin kernel on the current stream just before a start event: while it
    runs, the host submits the event, the graph and the end event, so the timed region
    does not hold the host's submission of the graph to an idle GPU.  (Config-1 BF16 chunk
    at K = 20: 12.93-12.95 us per launch with it, 12.96-13.06 without; at K = 200 12.52-12.58
    either way.  The rest of the K = 20 excess is a fixed cost of about 7 us per replay,
    not per launch.)"""
    torch.cuda._sleep(cycles)


def warm_graph(torch, graph, seconds=0.2, most=400):
    """Untimed replays of the captured graph for about `seconds` (at most `most` replays)
    before the timed one: on a fresh process the GPU clocks are still ramping during the
    first milliseconds of work (measured: the first 32-launch replay runs 4% slower than
    later ones), so the timed replay starts from the steady state a busy server runs in."""
    t0 = time.perf_counter()
    for _ in range(most):
        graph.replay()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            break


def time_eager(torch, sets, steps):
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        sets[i % len(sets)].launch()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


COPY_BYTES = 2 * 32 * 1024 * 1024  # bytes moved (read + write) per copy-ceiling launch


def copy_ceiling(torch, nbytes=COPY_BYTES, reps=50):
    """Device-to-device copy (torch copy_) moving `nbytes` in total (read + write), rotating
    over 8 buffer pairs; also the calibration kernel of the traffic counters."""
    n = nbytes // 2 // 2
    bufs = [(torch.empty(n, dtype=torch.int16, device="cuda").fill_(1),
             torch.empty(n, dtype=torch.int16, device="cuda")) for _ in range(8)]
    for s, d in bufs:
        d.copy_(s)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(reps):
        s, d = bufs[i % 8]
        d.copy_(s)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    return 2 * n * 2 / (ms * 1e-3) / 1e9


def stream_copy_ceiling(torch, nbytes, steps=200, sets=50):
    """The practical HBM ceiling at the chain's own size: the library's streaming copy
    (padra_StreamCopy) moving `nbytes` in total (read + write) per launch, rotating over
    `sets` buffer pairs, timed as the chain is (graph of `steps` launches)."""
    from padra_amd import abi
    n = nbytes // 2 // 16 * 16
    bufs = [(torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1),
             torch.empty(n, dtype=torch.uint8, device="cuda")) for _ in range(sets)]

    class Copy:
        def __init__(self, s, d):
            self.s, self.d = s, d

        def launch(self):
            abi.call("padra_StreamCopy", torch.cuda.current_stream().cuda_stream,
                     self.d.data_ptr(), self.s.data_ptr(), n)
    ms = time_graph(torch, [Copy(s, d) for s, d in bufs], steps, 20)
    return 2 * n / (ms * 1e-3) / 1e9, ms


def cpu_chain_rate(host, seconds, threads):
    """Seconds per 2048-token config-1 chunk of the C oracle on the host: residual-norm
    (128-thread tree), Q/K norm + RoPE and the BF16 store, with the chunk's tokens split
    into `threads` contiguous slices run concurrently (ctypes releases the GIL during each
    oracle call).  Repeats whole chunks until `seconds` have elapsed; returns (s, chunks)."""
    from concurrent.futures import ThreadPoolExecutor

    from oracle import oracle
    from padra_amd import synth
    table = synth.bf16_bits(oracle.rope_table(TOKENS, D, 1e6))
    kc = np.zeros((TOKENS, HKV * D), np.uint16)
    vc = np.zeros_like(kc)
    bounds = np.linspace(0, TOKENS, threads + 1).astype(int)

    def piece(i):
        lo, hi = bounds[i], bounds[i + 1]
        pos = np.arange(lo, hi, dtype=np.int32)
        oracle.residual_rmsnorm(host["x"][lo:hi], host["residual"][lo:hi], host["gamma"], 1e-6,
                                128)
        _, k, _ = oracle.qk_norm_rope(host["q"][lo:hi], host["k"][lo:hi], host["qn"],
                                      host["kn"], table, pos)
        oracle.kv_store_bf16(k, host["v"][lo:hi], kc, vc, pos, TOKENS)

    oracle.lib()
    reps, t0 = 0, time.perf_counter()
    with ThreadPoolExecutor(threads) as pool:
        while True:
            list(pool.map(piece, range(threads)))
            reps += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
    return el / reps, reps


def cpu_baseline(host, seconds, threads):
    """The oracle (kind "port") on the GPU box's host cores, single-threaded and on
    `threads` threads; the threaded figure is the reported value."""
    one, reps1 = cpu_chain_rate(host, seconds / 2, 1)
    many, reps = cpu_chain_rate(host, seconds / 2, threads)
    rate = lambda per_chunk: round(chain_bytes("bf16") * TOKENS / per_chunk / 1e9, 3)
    return {
        "value": rate(many),
        "unit": "GB/s",
        "cores": threads,
        "host_cpus": os.cpu_count(),
        "host_cpus_usable": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"{reps} full 2048-token config-1 chunks (BF16 KV) on {threads} threads and "
                  f"{reps1} on one thread, about {seconds / 2:.0f} s each",
        "tokens_per_s": round(TOKENS / many, 1),
        "us_per_token": round(many / TOKENS * 1e6, 3),
        "single_thread": {"value": rate(one), "tokens_per_s": round(TOKENS / one, 1)},
    }


COLD_BYTES = 1.5e9  # distinct bytes per graph replay: about six times the Infinity Cache


def cold_sets(nbytes, least=4):
    """Buffer sets for a kernel moving `nbytes` per launch so that one replay of a graph
    rotating over them touches COLD_BYTES: its inputs then come from HBM, not from the
    256 MB Infinity Cache, as the streaming copy it is compared with does."""
    return max(least, -(-int(COLD_BYTES) // int(nbytes)))


def graph_time(torch, step, steps, warmup=3, replays=5):
    """Median over `replays` timed replays of the ms per call of step(i), captured `steps`
    times in one HIP graph."""
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                step(i)
    torch.cuda.synchronize()
    warm_graph(torch, graph)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = []
    for _ in range(replays):
        with torch.cuda.stream(stream):
            lead_in(torch)
            start.record(stream)
            graph.replay()
            end.record(stream)
        torch.cuda.synchronize()
        out.append(start.elapsed_time(end) / steps)
    return float(np.median(out))


def bench_swiglu(torch, steps):
    """Config 3: SwiGLU over 2048 tokens x top-8 = 16384 expert-permuted rows of 1024."""
    from padra_amd import ops, synth
    d = synth.swiglu_inputs(tokens=2048, top_k=8, width=1024, experts=64, sigma=2.0, seed=0)
    table = torch.empty(65536, dtype=torch.int16, device="cuda")
    ops.SiluTableBuild(table)
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()
    nbytes = 6 * d["gate"].size
    sets = cold_sets(nbytes)
    bufs = [(dev(d["gate"]), dev(d["up"]), torch.empty(d["gate"].shape, dtype=torch.int16,
                                                         device="cuda")) for _ in range(sets)]
    ms = graph_time(torch, lambda i: ops.SwiGLU(bufs[i % sets][0], bufs[i % sets][1],
                                                bufs[i % sets][2], table, bad), max(steps, sets))
    if bad.item():
        raise SystemExit("device error flag set in the SwiGLU benchmark")
    return {"workload": "config3: SwiGLU 16384 rows x 1024, expert-permuted (64 experts)",
            "us_per_launch": round(ms * 1e3, 3), "bytes_per_launch": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "rows_per_s": round(d["gate"].shape[0] / (ms * 1e-3), 1)}


def bench_f32_layer(torch, steps):
    """The config-1 chunk in the reference's own activation form (fp32 buffers holding
    BF16-exact values, PADRA_ACT_F32): launched as the reference launches it (the residual
    + RMSNorm, then the Q/K norm + RoPE + BF16 KV store, each timed alone), and through
    the one chain entry point (padra_ResidualNormQKRopeStore)."""
    from padra_amd import abi, ops, synth
    host = synth.chain_inputs(TOKENS, HIDDEN, HQ, HKV, D, outliers=True, seed=0)
    f32 = lambda a: torch.from_numpy(synth.bf16_to_f32(a)).cuda()
    b16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()
    table = torch.from_numpy(ops.RopeTable(TOKENS, D, 1e6).view(torch.int16).numpy()).cuda()
    g, qn, kn = b16(host["gamma"]), b16(host["qn"]), b16(host["kn"])
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    norm_bytes = TOKENS * HIDDEN * 4 * 4
    qk_bytes = TOKENS * (((HQ + 2 * HKV) + (HQ + HKV)) * D * 4 + 2 * HKV * D * 2 + 2 * D)
    sets = cold_sets(min(norm_bytes, qk_bytes))
    steps = max(steps, sets)
    bufs = []
    for _ in range(sets):
        x = f32(host["x"])
        kc = torch.empty((CAPACITY, HKV * D), dtype=torch.int16, device="cuda")
        bufs.append((x, f32(host["residual"]), torch.empty_like(x), f32(host["q"]),
                     f32(host["k"]), f32(host["v"]), ops.kv_cache(abi.KV_BF16, kc, torch.empty_like(kc),
                                                                  CAPACITY), kc))
    norm_ms = graph_time(torch, lambda i: ops.ResidualPostNorm(*bufs[i % sets][:3], g, bad), steps)
    qk_ms = graph_time(torch, lambda i: ops.QKNormRopeStore(
        bufs[i % sets][3], bufs[i % sets][4], qn, kn, table, ops.positions_base(0), bad,
        v=bufs[i % sets][5], kv=bufs[i % sets][6]), steps)
    fused_ms = graph_time(torch, lambda i: ops.ResidualNormQKRopeStore(
        *bufs[i % sets][:3], g, *bufs[i % sets][3:6], qn, kn, table, ops.positions_base(0),
        bufs[i % sets][6], bad), steps)
    if bad.item():
        raise SystemExit("device error flag set in the fp32-activation benchmark")
    rate = lambda b, ms: round(b / (ms * 1e-3) / 1e9, 2)
    return {"workload": "config1 chunk with fp32 activations: residual+RMSNorm, then "
                        "QK-norm+RoPE+BF16 KV store (two entry points, and the one chain "
                        "entry point)",
            "fused_us": round(fused_ms * 1e3, 3),
            "fused_gbs": rate(norm_bytes + qk_bytes, fused_ms),
            "fused_frac": round((norm_bytes + qk_bytes) / (fused_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "norm_us": round(norm_ms * 1e3, 3), "norm_bytes": norm_bytes,
            "norm_gbs": rate(norm_bytes, norm_ms),
            "qk_us": round(qk_ms * 1e3, 3), "qk_bytes": qk_bytes, "qk_gbs": rate(qk_bytes, qk_ms),
            "gbs": rate(norm_bytes + qk_bytes, norm_ms + qk_ms),
            "frac": round((norm_bytes + qk_bytes) / ((norm_ms + qk_ms) * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_chain_sizes(torch, sizes=(2048, 4096, 8192, 16384), steps=50):
    """The BF16 chain at several token counts, each beside a streaming copy of the same bytes
    timed the same way: how much of a launch is its fixed cost and how fast the chain
    streams once the launch is large.  Host-known positions (PADRA_POS_BASE) at every
    size, since a prefill chunk holds at most 2048 tokens."""
    from padra_amd import ops, synth
    host = synth.chain_inputs(max(sizes), HIDDEN, HQ, HKV, D, outliers=True, seed=0)
    table = torch.from_numpy(ops.RopeTable(max(sizes), D, 1e6).view(torch.int16).numpy()).cuda()
    out = {}
    for t in sizes:
        nbytes = chain_bytes("bf16") * t
        sets = cold_sets(nbytes)
        chain_sets = [ChainSet(torch, host, table, "bf16", tokens=t, base_positions=True)
                      for _ in range(sets)]
        ms = time_graph(torch, chain_sets, max(steps, sets), 5)
        if any(int(c.bad.item()) for c in chain_sets):
            raise SystemExit(f"device error flag set in the chain at {t} tokens")
        del chain_sets
        torch.cuda.empty_cache()
        _, copy_ms = stream_copy_ceiling(torch, nbytes, steps=max(steps, sets), sets=sets)
        out[str(t)] = {"us_per_launch": round(ms * 1e3, 3), "bytes_per_launch": nbytes,
                       "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                       "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                       "copy_us": round(copy_ms * 1e3, 3),
                       "frac_of_copy": round(copy_ms / ms, 4)}
    return out


def bench_norm_fp8(torch, steps):
    """The input RMSNorm with its FP8 E4M3 row encoding (the QKV GEMM's input) over the
    config-1 chunk: 2048 rows of 2048; reads x, writes normalized (BF16) and codes."""
    from padra_amd import ops, synth
    host = synth.chain_inputs(TOKENS, HIDDEN, HQ, HKV, D, outliers=True, seed=0)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()
    g = dev(host["gamma"])
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    nbytes = TOKENS * (HIDDEN * (2 + 2 + 1) + 4)
    norm_bytes = TOKENS * HIDDEN * 2 * 2
    sets = cold_sets(norm_bytes)
    steps = max(steps, sets)
    bufs = []
    for _ in range(sets):
        x = dev(host["x"])
        bufs.append((x, torch.empty_like(x),
                     torch.empty((TOKENS, HIDDEN), dtype=torch.uint8, device="cuda"),
                     torch.empty(TOKENS, dtype=torch.float32, device="cuda")))
    ms = graph_time(torch, lambda i: ops.NormFP8(bufs[i % sets][0], bufs[i % sets][1], g,
                                                 bufs[i % sets][2], bufs[i % sets][3], bad),
                    steps)
    # The same RMSNorm without the encoding (padra_ResidualPostNorm with no residual, the
    # reference's Norm): reads x, writes normalized.
    norm_ms = graph_time(torch, lambda i: ops.ResidualPostNorm(bufs[i % sets][0], None,
                                                               bufs[i % sets][1], g, bad), steps)
    if bad.item():
        raise SystemExit("device error flag set in the FP8 norm benchmark")
    return {"workload": "RMSNorm + FP8 E4M3 row encoding, 2048 rows x 2048 (BF16 in/out)",
            "us_per_launch": round(ms * 1e3, 3), "bytes_per_launch": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "norm_only": {"us_per_launch": round(norm_ms * 1e3, 3), "bytes_per_launch": norm_bytes,
                          "gbs": round(norm_bytes / (norm_ms * 1e-3) / 1e9, 2),
                          "frac": round(norm_bytes / (norm_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}}


def bench_kv_neighbours(torch, steps=100):
    """The cache writers and readers next to the chain, on the config-1/2 chunk (2048
    tokens, 4 KV heads of 128): the store-only encode of a chunk buffer (padra_KVStore,
    cap = 2048), its commit into a 131072-row ring (padra_KVCommit), the q8_0 decode of a
    1024-row local ring's prefix (padra_KvQ8_0DequantizePrefix), the in-place K rotation
    of the chunk's K rows (padra_RotateRows) and the 1024-row local-ring snapshot
    (padra_KVCheckpointCapture).  Bytes: what each reads and writes once.  Each kernel
    rotates over cold_sets(its bytes) sets of its own buffers; the commits go to four
    rings, each set into its own 2048-row range of one of them (its own PrefillState)."""
    from padra_amd import abi, ops, synth
    T, F = TOKENS, HKV * D
    host = synth.chain_inputs(T, HIDDEN, HQ, HKV, D, outliers=True, seed=0)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    hk, hv = dev(host["k"]), dev(host["v"])
    row_bytes = {abi.KV_BF16: 2 * F, abi.KV_Q8: F, abi.KV_Q8_0: ops.q8_0_row_bytes(F)}

    def planes(fmt, rows):
        if fmt == abi.KV_BF16:
            return (torch.zeros((rows, F), dtype=torch.int16, device="cuda"),
                    torch.zeros((rows, F), dtype=torch.int16, device="cuda"), None)
        if fmt == abi.KV_Q8:
            return (torch.zeros((rows, F), dtype=torch.int8, device="cuda"),
                    torch.zeros((rows, F), dtype=torch.int8, device="cuda"),
                    torch.zeros((rows, HKV, 2), dtype=torch.float32, device="cuda"))
        rb = row_bytes[fmt]
        return (torch.zeros((rows, rb), dtype=torch.uint8, device="cuda"),
                torch.zeros((rows, rb), dtype=torch.uint8, device="cuda"), None)

    def prefill_state(base, tokens):
        return torch.tensor([base, base, tokens, CAPACITY, base, 1, 1, 1], dtype=torch.int32,
                            device="cuda")

    def timed(name, nbytes, make, launch):
        sets = cold_sets(nbytes)
        bufs = [make(j) for j in range(sets)]
        ms = graph_time(torch, lambda i: launch(bufs[i % sets]), max(steps, sets))
        del bufs
        torch.cuda.empty_cache()
        out[name] = {"us_per_launch": round(ms * 1e3, 3), "bytes_per_launch": nbytes,
                     "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2),
                     "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "buffer_sets": sets}

    out = {}
    names = {abi.KV_BF16: "bf16", abi.KV_Q8: "q8", abi.KV_Q8_0: "q8_0"}
    rings_per_fmt = 4
    for fmt in (abi.KV_BF16, abi.KV_Q8, abi.KV_Q8_0):
        scale_bytes = T * HKV * 8 if fmt == abi.KV_Q8 else 0
        timed(f"store_{names[fmt]}", 2 * T * F * 2 + 2 * T * row_bytes[fmt] + scale_bytes,
              lambda j: (hk.clone(), hv.clone(), planes(fmt, T)),
              lambda b: ops.KVStore(b[0], b[1], ops.positions_base(0),
                                    ops.kv_cache(fmt, *b[2][:2], T, scales=b[2][2]), bad))
        rings = [planes(fmt, CAPACITY) for _ in range(rings_per_fmt)]
        timed(f"commit_{names[fmt]}", 2 * (2 * T * row_bytes[fmt] + scale_bytes),
              lambda j: (planes(fmt, T), rings[j % rings_per_fmt],
                         prefill_state((j // rings_per_fmt) * T % CAPACITY, T)),
              lambda b: ops.KVCommit(
                  ops.kv_cache(fmt, *b[0][:2], T, scales=b[0][2]),
                  ops.kv_cache(fmt, *b[1][:2], CAPACITY, scales=b[1][2]),
                  ops.positions_prefill(b[2], maximum=CAPACITY), T, HKV, bad))
        del rings

    # q8_0 prefix decode of a 1024-row local ring whose chunk starts at base 4096
    def prefix_bufs(j):
        rk, rv, _ = planes(abi.KV_Q8_0, 1024)
        rk.view(torch.int16)[:, :16].fill_(0x2400)
        rv.view(torch.int16)[:, :16].fill_(0x2400)
        ok = torch.empty((1024, F), dtype=torch.int16, device="cuda")
        return rk, rv, ok, torch.empty_like(ok)
    ring_state = prefill_state(4096, T)
    timed("q8_0_dequantize_prefix_1024", 2 * 1024 * row_bytes[abi.KV_Q8_0] + 2 * 1024 * F * 2,
          prefix_bufs,
          lambda b: ops.KvQ8_0DequantizePrefix(*b, ops.positions_prefill(ring_state, maximum=CAPACITY),
                                               T, bad))
    timed("rotate_rows_k", 2 * T * F * 2, lambda j: hk.clone(), lambda b: ops.RotateRows(b, bad))
    # snapshot of a 1024-row BF16 local ring before the chunk at base 700, anchor 1250
    snap_state = torch.tensor([700, 700, 600, CAPACITY, 700, 1, 1, 1], dtype=torch.int32,
                              device="cuda")
    timed("checkpoint_capture_bf16_1024", 2 * 2 * 1024 * F * 2,
          lambda j: (planes(abi.KV_BF16, 1024), planes(abi.KV_BF16, 600), planes(abi.KV_BF16, 1024)),
          lambda b: ops.KVCheckpointCapture(
              ops.kv_cache(abi.KV_BF16, b[0][0], b[0][1], 1024),
              ops.kv_cache(abi.KV_BF16, b[1][0], b[1][1], 600),
              ops.kv_cache(abi.KV_BF16, b[2][0], b[2][1], 1024),
              ops.positions_prefill(snap_state, maximum=CAPACITY), 600, 1250, bad))
    torch.cuda.synchronize()
    if bad.item():
        raise SystemExit("device error flag set in the cache neighbour benchmarks")
    for name, e in out.items():
        gbs, cms = stream_copy_ceiling(torch, e["bytes_per_launch"],
                                       steps=max(steps, e["buffer_sets"]), sets=e["buffer_sets"])
        e["copy_us"] = round(cms * 1e3, 3)
        e["frac_of_copy"] = round(e["gbs"] / gbs, 4)
    return {"workload": "cache neighbours of the 2048-token chunk: store-only encode, commit "
                        "into a 131072-row ring, q8_0 prefix decode, K rotation, local-ring "
                        "snapshot", **out}


def bench_combine_norm(torch, steps):
    """The step after the expert down projection over the config-1 chunk: the ordered BF16
    combine of 8 expert rows into the residual, the RMSNorm and its FP8 encoding; 2048 rows
    of 2048.  Reads down (8 rows) and x, writes x, normalized and codes."""
    from padra_amd import ops, synth
    rng = np.random.default_rng(0)
    host = synth.chain_inputs(TOKENS, HIDDEN, HQ, HKV, D, outliers=True, seed=0)
    down_h = synth.bf16_bits((rng.standard_normal((TOKENS, 8, HIDDEN)) * 0.5).astype(np.float32))
    w = torch.from_numpy(rng.dirichlet(np.ones(8), TOKENS).astype(np.float32)).cuda()
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()
    g = dev(host["gamma"])
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    nbytes = TOKENS * (HIDDEN * (8 * 2 + 2 + 2 + 2 + 1) + 8 * 4 + 4)
    sets = cold_sets(nbytes)
    bufs = []
    for _ in range(sets):
        x = dev(host["x"])
        bufs.append((x, dev(down_h), torch.empty_like(x),
                     torch.empty((TOKENS, HIDDEN), dtype=torch.uint8, device="cuda"),
                     torch.empty(TOKENS, dtype=torch.float32, device="cuda")))

    def step(i):
        x, down, y, packed, scales = bufs[i % sets]
        ops.CombineNorm(x, down, w, y, g, bad, packed=packed, scales=scales)

    ms = graph_time(torch, step, max(steps, sets))
    if bad.item():
        raise SystemExit("device error flag set in the combine + norm benchmark")
    return {"workload": "expert combine (8 rows) + residual + RMSNorm + FP8, 2048 rows x 2048",
            "us_per_launch": round(ms * 1e3, 3), "bytes_per_launch": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_attention(torch, steps, seqs=64, capacity=CAPACITY, fill_seed=0, fmt="bf16",
                    local=False, splits=0):
    """Decode attention over BF16 caches (the consumer of the stored rows), one step of
    `seqs` sequences at ragged positions U[0, capacity) with per-sequence caches of
    `capacity` rows: the split-K pass and the per-head merge.  With `local`, each
    sequence's cache is the 1024-row local ring and the window its last 1024 keys (a local
    layer).  `splits` as padra_DecodeAttention takes it (0: the reference's count, -1: the
    MI355X-tuned count); a non-zero value also times the reference's count for comparison.
    Bytes: every key and value row of the window (4 KV heads x 256 B each) plus q and the
    output."""
    from padra_amd import abi, ops, synth
    rng = np.random.default_rng(fill_seed)
    positions = rng.integers(0, capacity, seqs).astype(np.int32)
    states = np.zeros((seqs, 8), np.int32)
    for i, p in enumerate(positions):
        states[i] = [1, p, capacity, 1 << 20, p, min(int(p), 1024), 0, 0]
    st = torch.from_numpy(states).cuda()
    gen = torch.Generator(device="cuda").manual_seed(fill_seed)
    rows_per_seq = 1024 if local else capacity
    code = {"bf16": abi.KV_BF16, "q8": abi.KV_Q8, "q8_0": abi.KV_Q8_0}[fmt]
    # every K and V row of the window (a q8_0 row holds all 4 KV heads: each KV head's
    # split reads its 128 codes and 8 scale bytes of it), plus q and the output
    per_row = {"bf16": HKV * D * 2, "q8": HKV * (D + 4), "q8_0": HKV * (D + 8)}[fmt]
    window = np.minimum(positions.astype(np.int64) + 1, 1024 if local else capacity)
    nbytes = int(window.sum()) * per_row * 2 + 2 * seqs * HQ * D * 2
    # Local rings (70-134 MB per step) would sit in the Infinity Cache if one set of caches
    # were replayed: each step reads its own set, as each layer of a model has its own.
    sets = cold_sets(nbytes, least=1) if local else 1

    def cache():
        if fmt == "q8_0":
            # valid rows: random codes, block scales 1/64 (fp16 0x2400)
            def rows():
                r = torch.randint(-127, 128, (seqs * rows_per_seq, 544), generator=gen,
                                  device="cuda", dtype=torch.int8)
                r[:, :32].view(torch.int16).fill_(0x2400)
                return r
            return rows(), rows(), None
        if fmt == "q8":
            return (torch.randint(-127, 128, (seqs * rows_per_seq, HKV * D), generator=gen,
                                  device="cuda", dtype=torch.int8),
                    torch.randint(-127, 128, (seqs * rows_per_seq, HKV * D), generator=gen,
                                  device="cuda", dtype=torch.int8),
                    torch.full((seqs * rows_per_seq, HKV, 2), 1.0 / 64, device="cuda"))
        return ((torch.randn((seqs * rows_per_seq, HKV * D), generator=gen, device="cuda"))
                .to(torch.bfloat16).view(torch.int16),
                (torch.randn((seqs * rows_per_seq, HKV * D), generator=gen, device="cuda"))
                .to(torch.bfloat16).view(torch.int16), None)
    planes = [cache() for _ in range(sets)]
    kvs = [ops.kv_cache(code, kc, vc, rows_per_seq, scales=sc, seq_stride=rows_per_seq)
           for kc, vc, sc in planes]
    q = (torch.randn((seqs, HQ, D), generator=gen, device="cuda") * 0.1).to(
        torch.bfloat16).view(torch.int16)
    out = torch.empty_like(q)
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    pos = ops.positions_decode(st, maximum=capacity)
    used = abi.lib().padra_DecodeAttentionSplits(ctypes.byref(kvs[0]), seqs, HKV, int(local),
                                                 splits)

    def timed(s):
        scratch = ops.DecodeAttention(q, kvs[0], out, pos, bad, local=local, splits=s)  # allocates
        return graph_time(torch, lambda i: ops.DecodeAttention(q, kvs[i % sets], out, pos, bad,
                                                               local=local, splits=s,
                                                               scratch=scratch),
                          max(steps, sets))
    ms = timed(splits)
    ms_reference = timed(0) if splits else None
    if bad.item():
        raise SystemExit("device error flag set in the decode attention benchmark")
    del planes, kvs
    torch.cuda.empty_cache()
    return {"workload": f"decode attention, {seqs} sequences at ragged positions < {capacity}, "
                        f"{fmt} caches{', 1024-row local rings' if local else ''} "
                        "(split-K + merge)",
            "splits": used, "us_per_step": round(ms * 1e3, 3), "bytes_per_step": nbytes,
            "buffer_sets": sets,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            **({"reference_splits_us_per_step": round(ms_reference * 1e3, 3)}
               if ms_reference else {})}


def bench_decode(torch, steps, seqs, vocab=131072, capacity=CAPACITY, fmt="bf16"):
    """Config 4 (seqs=64) and the GPU side of config 0 (seqs=1): embedding gather, then the
    fused residual-norm (256-thread decode tree) + Q/K norm + RoPE + KV store (BF16, or the
    q8 / q8_0 formats with fmt) at each sequence's own position (DecodeState per sequence,
    per-sequence caches)."""
    from padra_amd import abi, ops, synth
    rng = np.random.default_rng(0)
    gen = torch.Generator(device="cuda").manual_seed(0)
    table = (torch.randn((vocab, HIDDEN), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    ids = synth.zipf_ids(seqs, vocab, s=1.1, seed=0)
    positions = rng.integers(0, capacity, seqs).astype(np.int32) if seqs > 1 else \
        np.array([4097], np.int32)
    host = synth.chain_inputs(seqs, HIDDEN, HQ, HKV, D, outliers=False, seed=0)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()
    states = np.zeros((seqs, 8), np.int32)
    for i, p in enumerate(positions):
        states[i] = [ids[i], p, capacity, 1 << 20, p, min(int(p), 1024), 0, 0]
    st = torch.from_numpy(states).cuda()
    rope = torch.from_numpy(ops.RopeTable(capacity, D, 1e6).view(torch.int16).numpy()).cuda()
    code = {"bf16": abi.KV_BF16, "q8": abi.KV_Q8, "q8_0": abi.KV_Q8_0}[fmt]
    width = {"bf16": HKV * D, "q8": HKV * D, "q8_0": ops.q8_0_row_bytes(HKV * D)}[fmt]
    dtype = torch.int16 if fmt == "bf16" else torch.uint8
    kc = torch.zeros((seqs * capacity, width), dtype=dtype, device="cuda")
    vc = torch.zeros_like(kc)
    sc = torch.zeros((seqs * capacity, HKV, 2), dtype=torch.float32, device="cuda") \
        if fmt == "q8" else None
    x = torch.empty((seqs, HIDDEN), dtype=torch.int16, device="cuda")
    r, y = dev(host["residual"]), torch.empty_like(x)
    q, k, v = dev(host["q"]), dev(host["k"]), dev(host["v"])
    g, qn, kn = dev(host["gamma"]), dev(host["qn"]), dev(host["kn"])
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    pos = ops.positions_decode(st, maximum=capacity, vocab=vocab)
    kv = ops.kv_cache(code, kc, vc, capacity, scales=sc, seq_stride=capacity)
    tbl = table.view(torch.int16)

    def step(i):
        ops.Embed(tbl, x, bad, positions=pos)
        ops.ResidualNormQKRopeStore(x, r, y, g, q, k, v, qn, kn, rope, pos, kv, bad, tree=256)

    def fused_step(i):
        ops.EmbedResidualNormQKRopeStore(tbl, None, x, r, y, g, q, k, v, qn, kn, rope, pos, kv,
                                         bad, tree=256)
    # The chain alone on the reference's own activation form (fp32 buffers holding
    # BF16-exact values), at the same positions into the same caches.
    f32 = lambda a: torch.from_numpy(synth.bf16_to_f32(a)).cuda()
    x32, r32, q32, k32, v32 = (f32(host[n]) for n in ("x", "residual", "q", "k", "v"))
    y32 = torch.empty_like(x32)

    def f32_step(i):
        ops.ResidualNormQKRopeStore(x32, r32, y32, g, q32, k32, v32, qn, kn, rope, pos, kv, bad,
                                    tree=256)
    ms = graph_time(torch, step, steps)
    fused_ms = graph_time(torch, fused_step, steps)
    f32_ms = graph_time(torch, f32_step, steps)
    if bad.item():
        raise SystemExit("device error flag set in the decode benchmark")
    nbytes = seqs * (2 * 2 * HIDDEN + chain_bytes(fmt))
    return {"workload": f"{'config4' if seqs > 1 else 'config0'}: decode step of {seqs} "
                        f"sequence(s): gather + fused chain (256-thread tree), ragged positions, "
                        f"{fmt} KV",
            "us_per_step": round(ms * 1e3, 3), "tokens_per_s": round(seqs / (ms * 1e-3), 1),
            "fused_us_per_step": round(fused_ms * 1e3, 3),
            "fused_tokens_per_s": round(seqs / (fused_ms * 1e-3), 1),
            "f32_chain_us_per_step": round(f32_ms * 1e3, 3),
            "bytes_per_step": nbytes, "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2)}


def cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the box's CPU share for one GPU (16), or fewer
    where fewer cores exist."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return max(1, min(16, avail))


def cpu_decode_token(seconds=2.0):
    """Config 0 on the host: the oracle's single-token decode chain (256-thread tree,
    position 4097, capacity 8192), repeated for `seconds`."""
    from oracle import oracle
    from padra_amd import synth
    host = synth.chain_inputs(1, HIDDEN, HQ, HKV, D, outliers=False, seed=0)
    table = synth.bf16_bits(oracle.rope_table(4098, D, 1e6))
    pos = np.array([4097], np.int32)
    kc = np.zeros((8192, HKV * D), np.uint16)
    vc = np.zeros_like(kc)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.residual_rmsnorm(host["x"], host["residual"], host["gamma"], 1e-6, 256)
        _, k, _ = oracle.qk_norm_rope(host["q"], host["k"], host["qn"], host["kn"], table, pos)
        oracle.kv_store_bf16(k, host["v"], kc, vc, pos, 8192)
        reps += 1
    el = time.perf_counter() - t0
    return {"us_per_token": round(el / reps * 1e6, 3), "tokens_per_s": round(reps / el, 1),
            "cores": 1, "kind": "port"}

def _cpu_repeat(work, pieces, threads, seconds):
    """Runs work(i) for i in range(pieces) on `threads` threads (ctypes releases the GIL in
    each oracle call), repeated until `seconds` have elapsed; returns (s per pass, passes)."""
    from concurrent.futures import ThreadPoolExecutor
    reps, t0 = 0, time.perf_counter()
    with ThreadPoolExecutor(threads) as pool:
        while True:
            list(pool.map(work, range(pieces)))
            reps += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                return el / reps, reps


def cpu_configs(host, threads, seconds=2.0):
    """The oracle on the host for configs 2-4, each a bounded sample of about `seconds` on
    `threads` threads (work split into contiguous slices): the config-2 chunk with q8 and
    rotated q8_0 caches, the config-3 SwiGLU (16384 rows of 1024), and the config-4 decode
    step (64 sequences: gather from a 4096-row slice of the embedding table, ids mod 4096,
    then the 256-thread-tree chain at ragged positions into a 131072-row cache)."""
    from oracle import oracle
    from padra_amd import synth
    oracle.lib()
    out = {}
    table = synth.bf16_bits(oracle.rope_table(TOKENS, D, 1e6))
    bounds = np.linspace(0, TOKENS, threads + 1).astype(int)
    for fmt in ("q8", "q8_0"):
        if fmt == "q8":
            ck, cv = np.zeros((TOKENS, HKV * D), np.int8), np.zeros((TOKENS, HKV * D), np.int8)
            sc = np.zeros((TOKENS, HKV, 2), np.float32)
        else:
            ck, cv = np.zeros((TOKENS, 544), np.uint8), np.zeros((TOKENS, 544), np.uint8)

        def piece(i, fmt=fmt, ck=ck, cv=cv):
            lo, hi = bounds[i], bounds[i + 1]
            pos = np.arange(lo, hi, dtype=np.int32)
            oracle.residual_rmsnorm(host["x"][lo:hi], host["residual"][lo:hi], host["gamma"],
                                    1e-6, 128)
            _, k, _ = oracle.qk_norm_rope(host["q"][lo:hi], host["k"][lo:hi], host["qn"],
                                          host["kn"], table, pos)
            if fmt == "q8":
                oracle.kv_q8_encode(k, host["v"][lo:hi], ck, cv, sc, pos, TOKENS)
            else:
                oracle.kv_q8_0_encode(k, host["v"][lo:hi], ck, cv, pos, TOKENS)
        per, reps = _cpu_repeat(piece, threads, threads, seconds)
        out[f"config2_{fmt}"] = {"us_per_chunk": round(per * 1e6, 1),
                                 "tokens_per_s": round(TOKENS / per, 1),
                                 "gbs": round(chain_bytes(fmt) * TOKENS / per / 1e9, 3),
                                 "cores": threads, "kind": "port",
                                 "sample": f"{reps} full 2048-token chunks"}
    d = synth.swiglu_inputs(tokens=2048, top_k=8, width=1024, experts=64, sigma=2.0, seed=0)
    rows = d["gate"].shape[0]
    sb = np.linspace(0, rows, threads + 1).astype(int)
    per, reps = _cpu_repeat(lambda i: oracle.swiglu(d["gate"][sb[i]:sb[i + 1]],
                                                    d["up"][sb[i]:sb[i + 1]]),
                            threads, threads, seconds)
    out["config3"] = {"us_per_launch": round(per * 1e6, 1),
                      "rows_per_s": round(rows / per, 1),
                      "gbs": round(6 * rows * 1024 / per / 1e9, 3), "cores": threads,
                      "kind": "port", "sample": f"{reps} passes over {rows} rows"}
    seqs, vocab_slice, cap = 64, 4096, CAPACITY
    emb = synth.chain_inputs(vocab_slice, HIDDEN, HQ, HKV, D, outliers=False, seed=1)["x"]
    dec = synth.chain_inputs(seqs, HIDDEN, HQ, HKV, D, outliers=False, seed=0)
    ids = synth.zipf_ids(seqs, 131072, s=1.1, seed=0) % vocab_slice
    positions = np.random.default_rng(0).integers(0, cap, seqs).astype(np.int32)
    dtable = synth.bf16_bits(oracle.rope_table(cap, D, 1e6))
    kc = np.zeros((cap, HKV * D), np.uint16)
    vc = np.zeros_like(kc)
    db = np.linspace(0, seqs, threads + 1).astype(int)

    def step(i):
        lo, hi = db[i], db[i + 1]
        if hi <= lo:
            return
        x, _ = oracle.embed(emb, ids[lo:hi].astype(np.int32))
        oracle.residual_rmsnorm(x, dec["residual"][lo:hi], dec["gamma"], 1e-6, 256)
        _, k, _ = oracle.qk_norm_rope(dec["q"][lo:hi], dec["k"][lo:hi], dec["qn"], dec["kn"],
                                      dtable, positions[lo:hi])
        oracle.kv_store_bf16(k, dec["v"][lo:hi], kc, vc, positions[lo:hi], cap)
    per, reps = _cpu_repeat(step, threads, threads, seconds)
    out["config4"] = {"us_per_step": round(per * 1e6, 1), "tokens_per_s": round(seqs / per, 1),
                      "cores": threads, "kind": "port", "sample": f"{reps} steps of {seqs} sequences"}
    return out


def main():
    if len(sys.argv) > 2 and sys.argv[1] == "--summarize":
        summarize(sys.argv[2], " ".join(sys.argv[3:]) or "(see profiles/README)")
        return
    if len(sys.argv) > 5 and sys.argv[1] == "--summarize-kernels":
        # --summarize-kernels <outdir> <outfile> <title> <command> [name substrings...]
        summarize_kernels(sys.argv[2], sys.argv[5], sys.argv[3], sys.argv[4], sys.argv[6:] or None)
        return
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this path runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)
    import torch

    from padra_amd import abi, ops, synth

    abi.lib()
    host = synth.chain_inputs(TOKENS, HIDDEN, HQ, HKV, D, outliers=True, seed=0)
    table = torch.from_numpy(ops.RopeTable(TOKENS, D, 1e6).view(torch.int16).numpy()).cuda()
    formats = args.formats.split(",")
    results = {}
    for fmt in formats:
        sets = [ChainSet(torch, host, table, fmt, base_positions=args.positions == "base")
                for _ in range(args.sets)]
        spread = time_graph_fresh(torch, sets, args.steps, args.warmup, args.replays,
                                  args.restore)
        ms = float(np.median(spread))
        for st in sets:
            st.restore()
        eager = time_eager(torch, sets, min(args.steps, 50))
        # The earlier rounds' method, for comparison only: 8 sets rotating with no restore,
        # about 490 MB touched per cycle, partly served by the 256 MB Infinity Cache.
        warm8 = None
        if not args.no_compare:
            for st in sets:
                st.restore()
            warm8 = time_graph(torch, sets[:8], args.steps, args.warmup)
        nbytes = chain_bytes(fmt) * TOKENS
        results[fmt] = {"ms": ms, "eager_ms": eager, "bytes": nbytes, "warm8_ms": warm8,
                        "gbs": nbytes / (ms * 1e-3) / 1e9, "spread": spread}
        bad = sum(int(s.bad.item()) for s in sets)
        if bad:
            raise SystemExit(f"device error flag set for format {fmt}")
        del sets
        torch.cuda.empty_cache()
    head = results[formats[0]]
    ceiling = copy_ceiling(torch)
    stream_gbs, stream_ms = stream_copy_ceiling(torch, head["bytes"])
    achieved = head["gbs"]
    line = {
        "metric": "achieved HBM GB/s (% of peak) fused norm+RoPE+KV-store; tokens/s per layer",
        "value": round(achieved, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 5),
        "replays_ms_p10_median_p90": [round(float(np.percentile(head["spread"], q)), 5)
                                      for q in (10, 50, 90)],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seed 0, N(0,1) with 1% outlier channels x20; gamma U(0.5,1.5)); "
                "every timed replay starts from these inputs, restored untimed before it (restore: "
                + args.restore + ")",
        "config": {"workload": "config1: fused residual+RMSNorm+QK-norm+RoPE+BF16 KV store, "
                               "2048-token prefill chunk, 1 layer",
                   "tokens": TOKENS, "hidden": HIDDEN, "q_heads": HQ, "kv_heads": HKV,
                   "head_dim": D, "kv_capacity": CAPACITY, "kv_format": formats[0],
                   "norm_tree": 128, "buffer_sets": args.sets, "timed_replays": args.replays,
                   "restore": args.restore},
        "tokens_per_s": round(TOKENS / (head["ms"] * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles(formats[0]),
                     "traffic_source": "profiles/chain_config1_traffic.json: rocprofv3 --pmc "
                                       "request counts of this kernel (profiles/chain_config1.md)",
                     "kernel": chain_kernel(formats[0]), "bytes_per_launch": head["bytes"]},
        "copy_ceiling_gbs": round(stream_gbs, 1),
        "copy_ceiling": {"kernel": "padra_StreamCopy", "bytes_per_launch": 2 * (head["bytes"] // 2 // 16 * 16),
                         "us_per_launch": round(stream_ms * 1e3, 3), "gbs": round(stream_gbs, 1),
                         "chain_frac_of_copy": round(achieved / stream_gbs, 4),
                         "torch_copy_64MB_gbs": round(ceiling, 1)},
        "formats": {f: {"gbs": round(r["gbs"], 2), "us_per_launch": round(r["ms"] * 1e3, 3),
                        "eager_us_per_launch": round(r["eager_ms"] * 1e3, 3),
                        "cache_assisted_8_sets_us_per_launch":
                            None if r["warm8_ms"] is None else round(r["warm8_ms"] * 1e3, 3),
                        "replays_us_p10_median_p90": [
                            round(float(np.percentile(r["spread"], q)) * 1e3, 3)
                            for q in (10, 50, 90)],
                        "bytes_per_launch": r["bytes"],
                        "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                        "traffic": traffic_from_profiles(f)} for f, r in results.items()},
    }
    if not args.no_configs:
        torch.cuda.empty_cache()
        line["configs"] = {"config3": bench_swiglu(torch, 50),
                           "config4": bench_decode(torch, 100, 64),
                           "config0_gpu": bench_decode(torch, 200, 1, capacity=8192),
                           "config4_q8": bench_decode(torch, 100, 64, fmt="q8"),
                           "config4_q8_0": bench_decode(torch, 100, 64, fmt="q8_0"),
                           "config1_f32_activations": bench_f32_layer(torch, 200),
                           "norm_fp8": bench_norm_fp8(torch, 200),
                           "combine_norm": bench_combine_norm(torch, 100),
                           "attention": bench_attention(torch, 10),
                           "attention_q8_0": bench_attention(torch, 10, fmt="q8_0"),
                           "attention_q8": bench_attention(torch, 10, fmt="q8"),
                           "attention_local": bench_attention(torch, 10, local=True, splits=-1),
                           "attention_local_q8": bench_attention(torch, 10, fmt="q8",
                                                                 local=True, splits=-1),
                           "attention_local_q8_0": bench_attention(torch, 10, fmt="q8_0",
                                                                   local=True, splits=-1),
                           "kv_neighbours": bench_kv_neighbours(torch),
                           "config1_chunk_sizes": bench_chain_sizes(torch)}
        # The streaming copy of each memory-bound kernel's own byte count, timed the same
        # way: how far a launch of that size is from the copy, apart from the HBM peak.
        for key in ("config3", "norm_fp8", "norm_fp8.norm_only", "combine_norm",
                    "config1_f32_activations"):
            entry = line["configs"]
            for part in key.split("."):
                entry = entry[part]
            nbytes = entry.get("bytes_per_launch") or (entry["norm_bytes"] + entry["qk_bytes"])
            sets = cold_sets(nbytes)
            gbs, ms = stream_copy_ceiling(torch, nbytes, steps=max(100, sets), sets=sets)
            entry["copy_us"] = round(ms * 1e3, 3)
            entry["frac_of_copy"] = round(entry["gbs"] / gbs, 4)
            if "fused_gbs" in entry:
                entry["fused_frac_of_copy"] = round(entry["fused_gbs"] / gbs, 4)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(host, args.cpu_seconds, cpu_threads())
        if not args.no_configs:
            line["configs"]["config0_cpu"] = cpu_decode_token()
            line["configs"]["cpu_configs"] = cpu_configs(host, cpu_threads())
    print(json.dumps(line), flush=True)


FORMAT_CODES = {"bf16": 0, "q8": 1, "q8_0": 2, "q8_0_norot": 3}
SHADER_ENGINES, SIMDS = 32, 1024  # MI355X (rocminfo: 32 shader engines, 256 CUs x 4 SIMDs)


def chain_kernel(fmt: str) -> str:
    """Kernel-trace name of the config-1 chain launch (tree 128, H 2048, no gather)."""
    return f"k_chain<128, 16, {FORMAT_CODES[fmt]}, false, unsigned short>"


def hbm_bytes(c: dict) -> dict:
    """HBM bytes of one dispatch from the TCC-to-memory request counts.  Reads: on gfx950
    every read request to memory that is not a 32-byte one moves a 128-byte line (reading
    a 32 MiB buffer issues 262,144 of them and TCC_BUBBLE, the 128-byte request counter the
    FETCH_SIZE formula relies on, stays 0, so FETCH_SIZE counts those lines as 64 bytes:
    half the bytes).  Writes: 64-byte requests plus 32-byte ones (WRITE_SIZE's formula,
    exact: a 32 MiB write issues 524,288 64-byte requests)."""
    r, r32 = c["TCC_EA0_RDREQ_sum"], c["TCC_EA0_RDREQ_32B_sum"]
    w, w64 = c["TCC_EA0_WRREQ_sum"], c["TCC_EA0_WRREQ_64B_sum"]
    read = 128 * (r - r32) + 32 * r32
    write = 64 * w64 + 32 * (w - w64)
    return {"read": read, "write": write, "total": read + write}


def _grid(r: dict):
    """A dispatch's grid size from a rocprofv3 CSV row (None if the row has none)."""
    for key in ("Grid_Size", "Grid_Size_X"):
        if r.get(key):
            return int(float(r[key]))
    return None


def _largest_copy_grid(rows) -> int | None:
    """The streaming copy runs both as the copy ceiling and as the restore of the chain's
    inputs between timed replays (smaller buffers): the ceiling's dispatches are the ones
    with the largest grid."""
    grids = [_grid(r) for r in rows if "k_stream_copy" in r.get("Kernel_Name", "")]
    grids = [g for g in grids if g is not None]
    return max(grids) if grids else None


def _copy_trace_avg_ns(outdir: str, sub: str) -> float | None:
    """Average duration of the copy ceiling's dispatches (largest grid) from kernel_trace.csv."""
    import csv
    import glob
    files = glob.glob(os.path.join(outdir, sub, "**", "*kernel_trace.csv"), recursive=True)
    rows = [r for path in files for r in csv.DictReader(open(path))]
    big = _largest_copy_grid(rows)
    ns = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rows
          if "k_stream_copy" in r.get("Kernel_Name", "") and _grid(r) == big]
    return sum(ns) / len(ns) if ns else None


def _pmc(outdir: str, sub: str) -> dict:
    """{short kernel name: {counter: median value per dispatch}} of one --pmc pass."""
    import csv
    import glob
    import statistics
    files = glob.glob(os.path.join(outdir, sub, "**", "*counter_collection.csv"), recursive=True)
    vals: dict = {}
    rows = [r for path in files for r in csv.DictReader(open(path))]
    big = _largest_copy_grid(rows)
    for r in rows:
        name = r["Kernel_Name"].replace("void ", "").replace("(anonymous namespace)::", "")
        name = name.split("(")[0]
        if name.startswith("k_stream_copy") and big is not None and _grid(r) != big:
            continue
        vals.setdefault(name, {}).setdefault(r["Counter_Name"], []).append(
            float(r["Counter_Value"]))
    return {k: {c: statistics.median(v) for c, v in d.items()} for k, d in vals.items()}


def summarize(outdir: str, command: str) -> None:
    """Digests rocprofv3 CSV output of this script into profiles/ (text only):
    <outdir>/trace (--kernel-trace --stats), <outdir>/rd (--pmc TCC_EA0_RDREQ_sum
    TCC_EA0_RDREQ_32B_sum TCC_BUBBLE_sum), <outdir>/wr (--pmc TCC_EA0_WRREQ_sum
    TCC_EA0_WRREQ_64B_sum) and <outdir>/sq (--pmc of the SQ wave and instruction counters
    with GRBM_GUI_ACTIVE).  HBM traffic per launch comes from the request counts (hbm_bytes);
    the streaming copy of known size is listed as the check of that arithmetic."""
    import csv
    import glob
    prof = os.path.join(ROOT, "profiles")
    os.makedirs(prof, exist_ok=True)
    lines = ["# rocprofv3 summary: fused chain, config 1 (2048-token prefill chunk), every KV format",
             "", "Command (from the repository root):", "", "```", command, "```", ""]
    stats = glob.glob(os.path.join(outdir, "trace", "**", "*kernel_stats.csv"), recursive=True)
    avg_ns = {}
    if stats:
        lines += ["## Kernel trace (--kernel-trace --stats)", "",
                  "| kernel | calls | average us | min us | max us |", "|---|---:|---:|---:|---:|"]
        for r in csv.DictReader(open(stats[0])):
            short = r["Name"].replace("void ", "").replace("(anonymous namespace)::", "").split("(")[0]
            avg_ns[short] = float(r["AverageNs"])
            lines.append(f"| `{short[:70]}` | {r['Calls']} | {float(r['AverageNs'])/1e3:.2f} | "
                         f"{float(r['MinNs'])/1e3:.2f} | {float(r['MaxNs'])/1e3:.2f} |")
        lines.append("")
    rd, wr, sq = _pmc(outdir, "rd"), _pmc(outdir, "wr"), _pmc(outdir, "sq")
    copy_ns = _copy_trace_avg_ns(outdir, "trace")
    for k in avg_ns:
        if k.startswith("k_stream_copy") and copy_ns:
            avg_ns[k] = copy_ns
            lines += [f"The copy ceiling's own dispatches (largest grid; the smaller ones restore "
                      f"the chain's inputs between timed replays) average {copy_ns / 1e3:.2f} us.", ""]
    traffic = {}
    rows = []
    kernels = [(f, chain_kernel(f), chain_bytes(f) * TOKENS) for f in FORMAT_CODES]
    copy_name = next((k for k in rd if k.startswith("k_stream_copy")), None)
    if copy_name:
        kernels.append(("copy", copy_name, None))
    for fmt, name, alg in kernels:
        if name not in rd or name not in wr:
            continue
        b = hbm_bytes({**rd[name], **wr[name]})
        if fmt == "copy":
            alg = b["write"] * 2  # the copy writes exactly what it reads
        traffic[fmt] = {"kernel": name, "bytes_per_launch": int(b["total"]), "read": int(b["read"]),
                        "write": int(b["write"]), "algorithmic_bytes": alg,
                        "ratio": round(b["total"] / alg, 4),
                        "counters": {**rd[name], **wr[name]}}
        us = avg_ns.get(name, float("nan")) / 1e3
        rows.append(f"| {fmt} | `{name}` | {b['read']:.0f} | {b['write']:.0f} | {b['total']:.0f} | "
                    f"{alg} | {b['total'] / alg:.3f} | {us:.2f} | {alg / (us * 1e3):.0f} |")
    if rows:
        lines += ["## HBM traffic per launch (--pmc request counts, no calibration factor)", "",
                  "Read bytes = 128 x (TCC_EA0_RDREQ_sum - TCC_EA0_RDREQ_32B_sum) + 32 x "
                  "TCC_EA0_RDREQ_32B_sum; write bytes = 64 x TCC_EA0_WRREQ_64B_sum + 32 x the "
                  "other write requests (see bench.hbm_bytes).  The copy's read bytes equal its "
                  "written bytes: the check of the arithmetic.", "",
                  "| format | kernel | read B | write B | traffic B | algorithmic B | traffic / alg | "
                  "trace avg us | alg GB/s |", "|---|---|---:|---:|---:|---:|---:|---:|---:|"] + rows + [""]
        with open(os.path.join(prof, "chain_config1_traffic.json"), "w") as f:
            json.dump(traffic, f, indent=1)
    sq_rows = []
    for fmt, name, _ in kernels:
        c = sq.get(name)
        if not c or not c.get("SQ_WAVES"):
            continue
        waves = c["SQ_WAVES"]
        sq_rows.append(f"| {fmt} | {waves:.0f} | {c.get('SQ_INSTS_VALU', 0) / waves:.0f} | "
                       f"{c.get('SQ_INSTS_SALU', 0) / waves:.0f} | {c.get('SQ_INSTS_LDS', 0) / waves:.1f} | "
                       f"{c.get('SQ_INSTS_VMEM_RD', 0) / waves:.1f} | {c.get('SQ_INSTS_VMEM_WR', 0) / waves:.1f} | "
                       f"{c.get('SQ_INSTS_VALU', 0):.0f} | {c.get('SQ_WAVE_CYCLES', 0) / waves:.0f} | "
                       f"{c.get('SQ_BUSY_CYCLES', 0):.0f} | {c.get('GRBM_GUI_ACTIVE', 0):.0f} |")
    derived = []
    for fmt, name, _ in kernels:
        c = sq.get(name)
        us = avg_ns.get(name, 0.0) / 1e3
        if not c or not c.get("SQ_BUSY_CYCLES") or not us:
            continue
        ghz = c["SQ_BUSY_CYCLES"] / SHADER_ENGINES / (us * 1e3)
        valu_us = c.get("SQ_INSTS_VALU", 0) * 4 / SIMDS / (ghz * 1e3)
        derived.append(f"| {fmt} | {us:.2f} | {ghz:.2f} | {valu_us:.2f} | {valu_us / us:.2f} |")
    if sq_rows:
        lines += ["## Wave and instruction counters (--pmc SQ_*, GRBM_GUI_ACTIVE)", "",
                  "Per-wave figures are totals over the dispatch divided by SQ_WAVES.", "",
                  "| format | waves | VALU / wave | SALU / wave | LDS / wave | VMEM rd / wave | "
                  "VMEM wr / wave | VALU total | wave cycles / wave | SQ busy cycles | GRBM GUI active |",
                  "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"] + sq_rows + [""]
    if derived:
        lines += ["## Derived: clock and VALU issue time", "",
                  f"Clock = SQ_BUSY_CYCLES / {SHADER_ENGINES} shader engines (rocminfo) / the "
                  "kernel-trace average.  VALU issue time = SQ_INSTS_VALU x 4 cycles (a wave64 "
                  f"VALU instruction on a 16-lane SIMD) / {SIMDS} SIMDs / clock: the time the "
                  "arithmetic alone occupies the SIMDs, against the kernel's duration.", "",
                  "| format | trace avg us | clock GHz | VALU issue us | VALU issue / duration |",
                  "|---|---:|---:|---:|---:|"] + derived + [""]
    with open(os.path.join(prof, "chain_config1.md"), "w") as f:
        f.write("\n".join(lines))
    print("\n".join(lines))


KERNEL_ROLES = {
    "k_kv_store<unsigned short, 0>": "store-only BF16 cache rows (KVStore)",
    "k_kv_store<unsigned short, 1>": "store-only q8 encode (KVStore)",
    "k_kv_store<unsigned short, 2>": "store-only q8_0 encode, rotated (KVStore)",
    "k_kv_commit": "encoded chunk rows into the ring (KVCommit)",
    "k_q8_0_dequant<unsigned short>": "q8_0 rows to BF16 (KvQ8_0DequantizePrefix / Dequantize)",
    "k_rotate_rows<unsigned short, false>": "K-transform rotation of 128-wide rows (RotateRows)",
    "k_kv_checkpoint": "1024-row local-ring snapshot (KVCheckpointCapture)",
    "k_silu_table": "SiLU table build (once)",
    "k_attn_order": "decode attention: windows ranked longest first (dispatch order)",
    "k_chain<128, 16, 0, false, unsigned short>": "config 1 chain, BF16 KV",
    "k_chain<128, 16, 1, false, unsigned short>": "config 2 chain, q8 KV",
    "k_chain<128, 16, 2, false, unsigned short>": "config 2 chain, q8_0 KV (rotated)",
    "k_chain<128, 16, 3, false, unsigned short>": "config 2 chain, q8_0 KV (unrotated)",
    "k_chain_small<256, 8, 0, true>": "config 4/0 decode step: gather + chain, one launch",
    "k_chain_small<256, 8, 0, false>": "config 4/0 decode chain after a separate gather",
    "k_chain_heads<256, 8, 0, false, float>": "config 4/0 decode chain on fp32 activations, BF16 KV",
    "k_chain_heads<256, 8, 1, false, float>": "config 4 decode chain on fp32 activations, q8 KV",
    "k_chain_heads<256, 8, 2, false, float>": "config 4 decode chain on fp32 activations, q8_0 KV",
    "k_chain_small<256, 8, 1, true>": "config 4 decode step, q8 KV: gather + chain (pair waves)",
    "k_chain_small<256, 8, 1, false>": "config 4 decode chain, q8 KV, after a separate gather",
    "k_chain_small<256, 8, 2, true>": "config 4 decode step, q8_0 KV: gather + chain (pair waves)",
    "k_chain_small<256, 8, 2, false>": "config 4 decode chain, q8_0 KV, after a separate gather",
    "k_embed": "embedding gather (separate launch)",
    "k_swiglu": "config 3 SwiGLU",
    "k_norm<128, 16, float, true>": "residual + RMSNorm (fp32 activations)",
    "k_norm<128, 16, unsigned short, false>": "RMSNorm alone (no residual; BF16)",
    "k_norm": "residual + RMSNorm",
    "k_qk": "Q/K norm + RoPE + store (fp32 activations)",
    "k_norm_fp8": "RMSNorm + FP8 E4M3",
    "k_combine_norm": "expert combine + residual + RMSNorm + FP8",
    "k_combine_norm_wide": "expert combine + residual + RMSNorm + FP8 (BF16 rows)",
    "k_attn_mx": "decode attention split (BF16 / q8 cache)",
    "k_attn_merge": "decode attention merge",
    "k_q8_0_query": "decode attention, q8_0 query coding",
    "k_q8_0_mx": "decode attention split (q8_0 cache)",
    "k_q8_0_mx_merge": "decode attention merge (q8_0)",
    "k_stream_copy": "streaming copy: the ceilings at each leg's byte count (mixed sizes)",
}


def summarize_kernels(outdir: str, command: str, outfile: str, title: str, only=None) -> None:
    """Every kernel of a profiled run (torch's own set-up kernels left out): calls and
    average / min / max duration from <outdir>/trace, and read / write HBM bytes per dispatch
    (medians) from the request counters of <outdir>/rd and <outdir>/wr (hbm_bytes).
    `only`: substrings of the kernel names to keep."""
    import csv
    import glob
    stats = glob.glob(os.path.join(outdir, "trace", "**", "*kernel_stats.csv"), recursive=True)
    rd, wr = _pmc(outdir, "rd"), _pmc(outdir, "wr")
    lines = [f"# {title}", "", "Command (from the repository root):", "", "```", command, "```",
             "", "Durations: averages over every dispatch of the run (graph replays, warm-up and "
             "eager launches), so they sit a little above the bench's graph-timed figures.  "
             "Bytes: HBM read and write bytes per dispatch from the TCC-to-memory request "
             "counts (128 bytes per read request that is not a 32-byte one, 64 or 32 bytes per "
             "write request; bench.hbm_bytes), medians over the dispatches.", "",
             "| kernel | role | calls | average us | min us | max us | read B | write B |",
             "|---|---|---:|---:|---:|---:|---:|---:|"]
    rows = []
    for r in csv.DictReader(open(stats[0])):
        short = r["Name"].replace("void ", "").replace("(anonymous namespace)::", "").split("(")[0]
        if short.startswith(("at::", "__amd_rocclr")) or (only and not any(o in short for o in only)):
            continue
        role = KERNEL_ROLES.get(short) or next((v for k, v in KERNEL_ROLES.items()
                                                if short.split("<")[0] == k), "")
        b = hbm_bytes({**rd[short], **wr[short]}) if short in rd and short in wr else None
        rows.append((float(r["AverageNs"]), f"| `{short[:60]}` | {role} | {r['Calls']} | "
                     f"{float(r['AverageNs'])/1e3:.2f} | {float(r['MinNs'])/1e3:.2f} | "
                     f"{float(r['MaxNs'])/1e3:.2f} | "
                     + (f"{b['read']:,.0f} | {b['write']:,.0f} |" if b else "— | — |")))
    lines += [r for _, r in sorted(rows, key=lambda t: -t[0])] + [""]
    with open(os.path.join(ROOT, "profiles", outfile), "w") as f:
        f.write("\n".join(lines))
    print("\n".join(lines))


def traffic_from_profiles(fmt):
    """HBM bytes per launch of the chain in `fmt`, from the rocprofv3 request counters
    (hbm_bytes), read from the committed profile summary if present."""
    path = os.path.join(ROOT, "profiles", "chain_config1_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        data = json.load(f)
    return data.get(fmt, {}).get("bytes_per_launch")


if __name__ == "__main__":
    main()
