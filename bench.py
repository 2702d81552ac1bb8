"""Benchmark of the 4-bit quantized matmul path on one MI355X.

Headline (`value`): the decode GEMV at M = 1, K = 4096, N = 14336 (BASELINE config 1's gate/up shape), MLX affine
4-bit group 64, bf16 activations ~ N(0, 1), in GB/s of algorithmic bytes (N K 0.5625 + 2 M K + 2 M N) per step. A
step is one dispatch of the projection through the C ABI (sq_linear_add) over weights already resident in HBM; a
ring of weight copies larger than the 256 MB Infinity Cache makes every step read HBM. The K timed steps are
captured once in a HIP graph and replayed (a serving loop's form: no host work between dispatches), bracketed by
HIP events on the launching stream.

`stream_floor`: a read-only streaming kernel (sq_diag_stream_read, several launch shapes) over the same number of
bytes from a ring of copies, timed the same way: what one dispatch of that size reaches on this machine's HBM.

`roofline.achieved`: the same bytes over the column tile's average launch duration, the HIP-event timed region
on the launching stream divided by its K launches (one dispatch per step; rocprofv3's kernel trace of the same
command, profiles/decode_column_gemv_m1_4096x14336.txt, agrees to within the dispatch gaps); `roofline.traffic`:
HBM bytes per launch from rocprofv3's FETCH_SIZE and WRITE_SIZE counters (profiles/decode_column_traffic.txt), scaled
by the counters' reading for a plain copy of known size (`--calibrate-copy` runs one).

Also reported on the same line: the config-1 sweep (M in 1..16 over the four 8B projection shapes), the config-2
prefill GEMM at M = 2048 (TFLOPS), the config-3 Q4_K shapes, the config-4 MoE block and the CPU baseline (the
oracle's threaded C implementation of the same quantized matmul on this host's cores, over a bounded sample).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--sections LIST] [--sweep-points LIST]
[--calibrate-copy]
(--sections: a comma list of sweep, prefill, q4k, formats, moe, cpu; the headline always runs, and every section runs
by default. It picks which benchmarks run, for profiling one of them; it changes nothing inside any timed region.)
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "splash-desktop_amd"))

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
RING_BYTES = 1 << 30


COPY_BYTES = 1 << 29
TRAFFIC_FILE = ROOT / "profiles" / "decode_column_traffic.txt"


def traffic_bytes():
    """HBM bytes per launch of the headline kernel, from the committed counter summary (None when absent)."""
    try:
        fields = dict(line.split(":", 1) for line in TRAFFIC_FILE.read_text().splitlines() if ":" in line)
        return int(fields["fetch_bytes_per_launch"]) + int(fields["write_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gemv_bytes(m: int, n: int, k: int) -> float:
    return n * k * 0.5625 + 2 * m * k + 2 * m * n


def weight_bytes(sq, fmt: int, n: int, k: int) -> int:
    """Plane bytes of an n x k tensor: plane0, meta and plane1 (the format's native bits per weight)."""
    p0, meta = sq.plane_bytes(fmt, n, k)
    return p0 + meta + n * (k // 32) * sq.FORMATS[fmt][5]


class Projection:
    """An n x k weight tensor in `copies` ring slots on the device, prepared through the library's repack."""

    def __init__(self, torch, sq, synthetic, fmt: int, n: int, k: int, seed: int, copies: int = 1):
        rng = np.random.default_rng(seed)
        self.fmt, self.n, self.k = fmt, n, k
        p0_bytes, meta_bytes = sq.plane_bytes(fmt, n, k)
        p1_bytes = n * (k // 32) * sq.FORMATS[fmt][5]
        self.plane0 = [torch.empty(p0_bytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
        self.meta = [torch.empty(meta_bytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
        self.plane1 = [torch.empty(p1_bytes, dtype=torch.uint8, device="cuda") if p1_bytes else None
                       for _ in range(copies)]
        if fmt in (sq.FMT_Q4K, sq.FMT_Q5K, sq.FMT_Q6K, sq.FMT_Q80):
            native = synthetic.q4k_native(rng, n, k) if fmt == sq.FMT_Q4K else synthetic.gguf_native(rng, fmt, n, k)
            src = torch.from_numpy(native.reshape(-1)).cuda()
            dst = torch.empty(p0_bytes + meta_bytes + p1_bytes, dtype=torch.uint8, device="cuda")
            sq.gguf_repack(src, dst, n, k, fmt, native.shape[1], p0_bytes, dst_plane1=p0_bytes + meta_bytes)
            for c in range(copies):
                self.plane0[c].copy_(dst[:p0_bytes])
                self.meta[c].copy_(dst[p0_bytes:p0_bytes + meta_bytes])
                if p1_bytes:
                    self.plane1[c].copy_(dst[p0_bytes + meta_bytes:])
            del src, dst
        else:
            group, bits = {sq.FMT_AF4G32: (32, 4), sq.FMT_AF4G64: (64, 4), sq.FMT_AF4G128: (128, 4),
                           sq.FMT_AF8G64: (64, 8)}[fmt]
            _, weight, scales, biases = synthetic.mlx_affine(rng, n, k, group, bits=bits)
            w = torch.from_numpy(weight.view(np.int32)).cuda()
            s = torch.from_numpy(scales.view(np.int16)).cuda()
            b = torch.from_numpy(biases.view(np.int16)).cuda()
            for c in range(copies):
                sq.mlx_repack(fmt, n, k, w, s, b, self.plane0[c], self.meta[c])
        torch.cuda.synchronize()

    def projection(self, sq, copy: int = 0):
        return sq.projection(sq.segment(self.fmt, self.n, self.k, self.plane0[copy], self.meta[copy],
                                        plane1=self.plane1[copy]))

    def bytes(self) -> int:
        return self.plane0[0].numel() + self.meta[0].numel() + (self.plane1[0].numel() if self.plane1[0] is not None else 0)


def time_steps(torch, fn, steps: int, warmup: int) -> float:
    """Seconds per step: `warmup` untimed steps, then `steps` timed with HIP events on the launching stream."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / steps


def time_graph(torch, launch, steps: int, warmup: int) -> float:
    """Seconds per step: `warmup` untimed eager steps, then `steps` launches captured in one HIP graph, replayed once
    untimed and once between HIP events on the replaying stream. launch(i, stream_handle) issues step i."""
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        launch(i, stream.cuda_stream)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        handle = torch.cuda.current_stream().cuda_stream
        for i in range(steps):
            launch(i, handle)
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    del graph
    return start.elapsed_time(end) / 1e3 / steps


def stream_floor(torch, sq, nbytes: int, steps: int, warmup: int) -> dict:
    """The read-only streaming kernel (sq_diag_stream_read) over `nbytes` from a ring of copies larger than the
    Infinity Cache, timed like the headline GEMV: the HBM read rate one dispatch of that size reaches here, best of
    several launch shapes. Beside it, the dispatch floor: the same kernel over one 16-byte vector on the GEMV's grid
    (224 x 1024), graph-replayed: the time a dispatch costs with nothing to read."""
    span = (nbytes + 4095) // 4096 * 4096
    copies = max(2, -(-RING_BYTES // span))
    ring = torch.empty(copies * span, dtype=torch.uint8, device="cuda").fill_(1)
    sink = torch.zeros(8192, dtype=torch.int32, device="cuda")
    results = {}
    for workgroups, threads in ((224, 1024), (512, 256), (1024, 256), (2048, 256), (2048, 512), (4096, 512)):
        def launch(i, stream, workgroups=workgroups, threads=threads):
            copy = ring[(i % copies) * span:]
            sq.stream_read(copy, sink, workgroups, threads, nbytes=nbytes, stream=sq.c_void_p(stream))
        sec = time_graph(torch, launch, steps, warmup)
        results[f"{workgroups}x{threads}"] = round(nbytes / sec / 1e9, 1)
    best = max(results, key=results.get)

    # The empty dispatch on several grids (the GEMV's 224 x 1024, 256 x 256 and 4096 x 512, and one wave): the
    # kernel over one 16-byte vector, graph-replayed; the lowest is the floor the bound takes.
    dispatch = {}
    for workgroups, threads in ((224, 1024), (256, 256), (4096, 512), (1, 64)):
        def empty(i, stream, workgroups=workgroups, threads=threads):
            sq.stream_read(ring, sink, workgroups, threads, nbytes=16, stream=sq.c_void_p(stream))
        dispatch[f"{workgroups}x{threads}"] = round(time_graph(torch, empty, steps, warmup) * 1e6, 3)
    dispatch_us = min(dispatch.values())
    del ring, sink
    torch.cuda.empty_cache()
    return {"GB/s": results[best], "launch": best, "bytes": nbytes, "by_launch": results,
            "dispatch_floor_us": dispatch_us, "dispatch_floor_by_grid_us": dispatch,
            "bound_us": round(dispatch_us + nbytes / (HBM_PEAK_GBS * 1e3), 3)}


def mfma_ceiling(torch, sq, steps: int, warmup: int) -> dict:
    """The sustained f16 MFMA rate of this device (sq_diag_mfma_peak): one and two waves a SIMD on every compute
    unit, eight independent 16x16x32 chains a wave, graph-replayed like the GEMM; in TFLOP/s."""
    sink = torch.zeros(1024, dtype=torch.float32, device="cuda")
    iterations, out = 4096, {}
    for waves in (1, 2):
        workgroups = 256 * waves

        def launch(i, stream, workgroups=workgroups, waves=waves):
            sq.call("sq_diag_mfma_peak", sq.c_void_p(stream), sq.view(sink), workgroups, waves, iterations)
        sec = time_graph(torch, launch, max(4, steps // 4), max(1, warmup // 4))
        flops = workgroups * 4 * iterations * 8 * 16384
        out[f"{waves}_wave_per_simd"] = round(flops / sec / 1e12, 1)
    out["best"] = max(out.values())
    return out


class Gemv:
    """A decode projection over a weight ring; launch(i, stream) dispatches step i on ring copy i % copies. With
    `gate_up`, each step is the one-pass gate/up pair of the reference's decode FFN (LinearGguf.cpp:686-694): a gate
    and an up tensor of the shape, bf16(up) silu(bf16(gate)) out."""

    def __init__(self, torch, sq, synthetic, fmt, m, n, k, seed=1, gate_up=False):
        one = weight_bytes(sq, fmt, n, k) * (2 if gate_up else 1)
        self.copies = max(1, -(-RING_BYTES // one))
        self.weights = Projection(torch, sq, synthetic, fmt, n, k, seed, self.copies)
        self.projs = [self.weights.projection(sq, c) for c in range(self.copies)]
        self.gates = [None] * self.copies
        epilogue = sq.EPILOGUE_NONE
        if gate_up:
            self.gate_weights = Projection(torch, sq, synthetic, fmt, n, k, seed + 100, self.copies)
            self.gates = [self.gate_weights.projection(sq, c) for c in range(self.copies)]
            epilogue = sq.EPILOGUE_GATE_UP
        self.plan = sq.plan_for(sq.decode_workload(n, k, m, epilogue), self.projs[0], self.gates[0])
        self.scratch = sq.Scratch(self.plan)
        self.x = torch.from_numpy(synthetic.activations(np.random.default_rng(seed + 1), m, k).view(np.int16)).cuda()
        self.out = torch.empty((m, n), dtype=torch.int16, device="cuda")
        self.bufs = sq.LinearBuffers(sq.view(self.x), sq.view(self.out), sq.view(None), sq.view(self.scratch.gate),
                                     self.scratch.struct())
        self.sq = sq

    def launch(self, i, stream):
        sq = self.sq
        gate = self.gates[i % self.copies]
        sq.call("sq_linear_add", sq.c_void_p(stream), sq.byref(self.bufs), sq.byref(self.projs[i % self.copies]),
                sq.byref(self.plan), sq.byref(gate) if gate is not None else None)


def bench_gemv(torch, sq, synthetic, fmt, m, n, k, steps, warmup, seed=1):
    g = Gemv(torch, sq, synthetic, fmt, m, n, k, seed)
    sec = time_graph(torch, g.launch, steps, warmup)
    plan = g.plan
    del g
    return sec, plan


def bench_prefill(torch, sq, synthetic, m, n, k, steps, warmup, fmt=None):
    fmt = sq.FMT_AF4G64 if fmt is None else fmt
    w = Projection(torch, sq, synthetic, fmt, n, k, 7)
    proj = w.projection(sq)
    plan = sq.plan_for(sq.prefill_workload(n, k, m), proj)
    scratch = sq.Scratch(plan)
    x = torch.from_numpy(synthetic.activations(np.random.default_rng(8), m, k).view(np.int16)).cuda()
    out = torch.empty((plan.storage_rows, n), dtype=torch.int16, device="cuda")
    handle = sq.stream_handle()
    bufs = sq.LinearBuffers(sq.view(x), sq.view(out), sq.view(None), sq.view(None), scratch.struct())

    def step(i):
        sq.call("sq_linear_add", handle, sq.byref(bufs), sq.byref(proj), sq.byref(plan), None)

    sec = time_steps(torch, step, steps, warmup)
    return sec


def bench_moe(torch, sq, synthetic, steps, warmup, rows=512, experts=128, top_k=8, hidden=2048, inter=768,
              fmt=None, formats=None, shared=0, gated=False, router=False):
    """One MoE layer (sq_moe_add) per step: routing from the caller's scores (copied each step into the
    grouped-input scratch, where the router's scores live), or with `router` the block's F32 router rows projected
    first; routed experts in `fmt` unless `formats` names a projection's own ("gate", "up", "down", "shared_gate",
    ...). Returns (seconds, bytes of planes + router + activations in and out, flops)."""
    fmt = sq.FMT_AF4G64 if fmt is None else fmt
    formats = formats or {}
    plan_parts = [("gate", experts * inter, hidden), ("up", experts * inter, hidden), ("down", experts * hidden, inter)]
    if shared:
        plan_parts += [("shared_gate", shared * inter, hidden), ("shared_up", shared * inter, hidden),
                       ("shared_down", shared * hidden, inter)]
    parts = {name: Projection(torch, sq, synthetic, formats.get(name, fmt), n, kk, 20 + i)
             for i, (name, n, kk) in enumerate(plan_parts)}
    seg = lambda name: (sq.segment(parts[name].fmt, parts[name].n, parts[name].k, parts[name].plane0[0],
                                   parts[name].meta[0], plane1=parts[name].plane1[0]) if name in parts else sq.Segment())
    slots = torch.arange(experts, dtype=torch.int32, device="cuda")
    rng = np.random.default_rng(30)
    scalar_gate = torch.from_numpy(rng.normal(0, 0.05, hidden).astype(np.float32)).cuda() if gated else None
    router_rows, router_seg = None, sq.Segment()
    if router:
        router_rows = torch.from_numpy(rng.normal(0, 0.05, (experts, hidden)).astype(np.float32)).cuda()
        router_seg = sq.Segment(sq.view(router_rows), sq.view(None), sq.view(None), experts, hidden, 0,
                                sq.FLOAT32_ROWS)
    weights = sq.MoeWeights(seg("gate"), seg("up"), seg("down"), sq.view(slots), experts, seg("shared_gate"),
                            seg("shared_up"), seg("shared_down"), sq.view(scalar_gate), router_seg)
    shape = sq.MoeShape(hidden, experts, top_k, inter, formats.get("gate", fmt), 0, shared, int(gated))
    plan = sq.MoePlan()
    sq.call("sq_moe_prefill_plan", sq.byref(shape), rows, None, sq.byref(plan))
    x = torch.from_numpy(synthetic.activations(rng, rows, hidden).view(np.int16)).cuda()
    width = sq.lib().sq_moe_router_width(sq.byref(shape))
    scores = np.zeros((rows, width), np.float32)
    scores[:, :experts] = synthetic.router_logits(rng, rows, experts)
    out = torch.empty((rows, hidden), dtype=torch.int16, device="cuda")
    held = {}
    for name in sq._MOE_WORKSPACE:
        nbytes = getattr(plan.workspace, name)
        held[name] = torch.zeros(max(nbytes, 4) // 4 + 1, dtype=torch.int32, device="cuda") if nbytes else None
    # The routed work overwrites the grouped input (the scores' home) with the input rows, so a step without router
    # rows starts with the caller writing its scores there, as a router projection would: a 16-byte-vector copy of
    # rows x router width fp32 on the same stream, inside the timed step.
    score_dev = torch.from_numpy(scores.reshape(-1)).cuda()
    score_dst = held["grouped_input"].view(torch.float32)[:score_dev.numel()]
    buffers = sq.MoeBuffers(sq.view(x), sq.view(None), sq.view(out),
                            sq.MoeScratch(*[sq.view(held[n]) for n in sq._MOE_WORKSPACE]), sq.view(None))
    handle = sq.stream_handle()

    def step(i):
        if not router:
            score_dst.copy_(score_dev)
        sq.call("sq_moe_add", handle, sq.byref(buffers), sq.byref(weights), sq.byref(plan))

    sec = time_steps(torch, step, steps, warmup)
    planes = sum(p.bytes() for p in parts.values()) + (experts * hidden * 4 if router else 0)
    flops = 2 * rows * (top_k + shared) * 3 * inter * hidden + (2 * rows * experts * hidden if router else 0)
    return sec, planes + 2 * rows * hidden * 2, flops


def cpu_baseline(sq, synthetic, budget_s: float) -> dict:
    """The CPU baseline (oracle/sq_cpu.c: a persistent pool of this host's threads running the best kernel the CPU
    has, bf16 dot products (AVX512_BF16), AVX-512F or AVX2, buffers reserved outside the timed calls) on the BASELINE
    configs, each over a bounded sample: c0 and
    the c1 headline at M = 1 and 16, c2 and c3's prefill points on 64 rows of their chunk, c3's Q4_K decode points,
    and c4's expert projections for 8 of the 128 experts at the block's mean 32 rows each (scaled to 128). Returns
    the headline figure as `value` and every config beside it."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import sq_oracle as oracle
    # A one-GPU box hands its GPU 16 of the host's hardware threads (its CPU share, the thread pools' limit there);
    # the pool takes all the threads this process may use, up to that share.
    host_threads = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host_threads
    threads = min(usable, 16)
    pool = oracle.CpuPool(threads)
    rng = np.random.default_rng(1)
    weights = {}

    def planes(fmt, n, k, seed):
        key = (fmt, n, k)
        if key not in weights:
            r = np.random.default_rng(seed)
            if fmt == oracle.FMT_Q4K:
                native = synthetic.q4k_native(r, n, k).ravel()
            else:
                _, w, sc, bi = synthetic.mlx_affine(r, n, k, 64)
                native = oracle.mlx_native(fmt, w, sc, bi, n, k)
            weights[key] = oracle.repack(fmt, native, n, k)[:2]
        return weights[key]

    # The kernels this CPU runs; each config reports the fastest of them (which one wins depends on the CPU and the
    # rows: on a Zen 5 host the fp32 kernel leads at M = 1, the bf16 dot products at more rows).
    isas = [isa for isa in ("avx512bf16", "avx512f", "avx2+fma") if pool.set_isa(isa)] or [pool.isa]
    fastest = {}

    def timed(fmt, m, n, k, seed=3, reps=None, key=None):
        p0, meta = planes(fmt, n, k, seed)
        x = synthetic.activations(rng, m, k)
        pool.reserve(m, k)
        out = np.zeros((m, n), np.uint16)
        best_all, count_all = float("inf"), 0
        for isa in isas:
            pool.set_isa(isa)
            pool.matmul(fmt, x, p0, meta, n, out)   # warm-up: pages and caches
            best, total, count = float("inf"), 0.0, 0
            while count < (reps or 50) and (total < budget_s / 10 / len(isas) or count < 2):
                _, sec = pool.matmul(fmt, x, p0, meta, n, out)
                best, total, count = min(best, sec), total + sec, count + 1
            if key is not None:
                fastest.setdefault(key, {})[isa] = best
            if best < best_all:
                best_all, count_all = best, count
        return best_all, count_all

    configs = {}
    af4 = oracle.FMT_AF4G64
    for name, (fmt, m, n, k) in {"c0_M1_K4096xN4096": (af4, 1, 4096, 4096),
                                 "c1_M1_K4096xN14336": (af4, 1, 14336, 4096),
                                 "c1_M16_K4096xN14336": (af4, 16, 14336, 4096),
                                 "c3_q4k_M1_K5120xN27648": (oracle.FMT_Q4K, 1, 27648, 5120),
                                 "c3_q4k_M16_K5120xN27648": (oracle.FMT_Q4K, 16, 27648, 5120)}.items():
        sec, count = timed(fmt, m, n, k, key=name)
        isa = min(fastest[name], key=fastest[name].get)
        configs[name] = {"ms": round(sec * 1e3, 3), "GB/s": round(gemv_bytes(m, n, k) / sec / 1e9, 2), "runs": count,
                         "isa": isa}
    for name, (fmt, rows, n, k) in {"c2_M2048_K4096xN14336": (af4, 2048, 14336, 4096),
                                    "c2_M2048_K14336xN4096": (af4, 2048, 4096, 14336),
                                    "c2_M2048_K5120xN27648": (af4, 2048, 27648, 5120),
                                    "c3_q4k_M512_K5120xN27648": (oracle.FMT_Q4K, 512, 27648, 5120)}.items():
        sec, count = timed(fmt, 64, n, k, reps=2, key=name)
        gflops = 2 * 64 * n * k / sec / 1e9
        configs[name] = {"sample": "64 of the chunk's rows", "GFLOPS": round(gflops, 1),
                         "ms_for_whole_chunk": round(2 * rows * n * k / gflops / 1e6, 1), "runs": count,
                         "isa": min(fastest[name], key=fastest[name].get)}
    # c4: gate, up (768 x 2048) and down (2048 x 768) of 8 experts on 32 routed rows each.
    expert_sec = 0.0
    for e in range(8):
        for n, k in ((768, 2048), (768, 2048), (2048, 768)):
            sec, _ = timed(af4, 32, n, k, seed=100 + e, reps=2)
            expert_sec += sec
        weights.clear()
    block_sec = expert_sec * 128 / 8
    expert_bytes = 128 * 3 * 768 * 2048 * 0.5625
    configs["c4_moe_T512_E128_top8"] = {"sample": "8 of 128 experts' projections on 32 rows each, scaled to 128",
                                        "ms": round(block_sec * 1e3, 2),
                                        "GB/s": round(expert_bytes / block_sec / 1e9, 2)}
    head = configs["c1_M1_K4096xN14336"]
    # The headline on every kernel the CPU runs (value: the fastest).
    by_isa = {isa: round(gemv_bytes(1, 14336, 4096) / sec / 1e9, 2)
              for isa, sec in fastest["c1_M1_K4096xN14336"].items()}
    pool.set_isa(head["isa"])
    out = {"value": head["GB/s"], "unit": "GB/s", "cores": pool.threads, "kind": "port",
           "sample": f"best of {head['runs']} runs of the M=1 K4096xN14336 af4g64 GEMV (BASELINE config 1) on "
                     f"{pool.threads} threads ({head['isa']}, the fastest of {', '.join(isas)}); oracle/sq_cpu.c",
           "isa": head["isa"], "headline_GB/s_by_isa": by_isa, "cpu": _cpu_model(), "host_threads": host_threads,
           "usable_threads": usable, "threads_used": pool.threads, "configs": configs}
    pool.close()
    return out


def _cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it: model name, family/model/stepping, and whether it reports AVX-512
    BF16."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                key, value = (part.strip() for part in line.split(":", 1))
                fields.setdefault(key, value)
            elif fields:
                break
    except OSError:
        return "unknown"
    flags = fields.get("flags", "").split()
    return (f"{fields.get('model name', 'unknown')} (family {fields.get('cpu family', '?')}, model "
            f"{fields.get('model', '?')}, stepping {fields.get('stepping', '?')}; "
            f"avx512_bf16 {'yes' if 'avx512_bf16' in flags else 'no'})")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline only (no sweep, prefill, MoE or CPU baseline)")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--calibrate-copy", action="store_true", help="also run a plain copy of known size (counters)")
    ap.add_argument("--sections", default="sweep,prefill,q4k,formats,moe,cpu",
                    help="benchmarks beside the headline: sweep, prefill, q4k, formats, moe, cpu")
    ap.add_argument("--sweep-points", default="",
                    help="restrict the sweep to these points (a comma list of its keys, e.g. K4096xN1024_M8), for a "
                         "profiler run of one shape")
    args = ap.parse_args()
    sections = set() if args.quick else {v.strip() for v in args.sections.split(",") if v.strip()}
    unknown = sections - {"sweep", "prefill", "q4k", "formats", "moe", "cpu"}
    if unknown:
        print(f"bench.py: unknown sections {sorted(unknown)}", file=sys.stderr)
        return 2
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    import torch

    import splash_q4 as sq
    from splash_q4 import synthetic
    torch.cuda.set_device(0)
    m, n, k = 1, 14336, 4096
    log(f"headline: decode GEMV M={m} K={k} N={n} af4g64, {args.steps} steps")
    headline = Gemv(torch, sq, synthetic, sq.FMT_AF4G64, m, n, k)
    plan = headline.plan
    sec = time_graph(torch, headline.launch, args.steps, args.warmup)
    gbs = gemv_bytes(m, n, k) / sec / 1e9
    log(f"  {sec * 1e6:.2f} us/step, {gbs:.1f} GB/s, splits {plan.config.splits}")
    ring_copies = headline.copies
    del headline
    torch.cuda.empty_cache()
    floor = stream_floor(torch, sq, int(gemv_bytes(m, n, k)), args.steps, args.warmup)
    log(f"  stream floor over the same bytes: {floor['GB/s']} GB/s ({floor['launch']}); empty dispatch "
        f"{floor['dispatch_floor_by_grid_us']} us")
    # The reference's decode form of this shape: gate and up in one pass (LinearGguf.cpp:686-694), two tensors'
    # planes (66 MB) a launch, bf16(up) silu(bf16(gate)) out.
    pair = Gemv(torch, sq, synthetic, sq.FMT_AF4G64, m, n, k, gate_up=True)
    pair_sec = time_graph(torch, pair.launch, args.steps, args.warmup)
    pair_bytes = 2 * n * k * 0.5625 + 2 * m * k + 2 * m * n
    pair_floor = stream_floor(torch, sq, int(pair_bytes), args.steps, args.warmup)
    gate_up_pair = {"us": round(pair_sec * 1e6, 2), "GB/s": round(pair_bytes / pair_sec / 1e9, 1),
                    "hbm_frac": round(pair_bytes / pair_sec / 1e9 / HBM_PEAK_GBS, 4), "bytes": int(pair_bytes),
                    "one_pass": bool(pair.plan.config.one_gate_up_pass), "splits": pair.plan.config.splits,
                    "stream_floor_GB/s": pair_floor["GB/s"],
                    "frac_of_floor": round(pair_bytes / pair_sec / 1e9 / pair_floor["GB/s"], 3)}
    log(f"  gate/up pair K{k} N{n}: {pair_sec * 1e6:.2f} us, {gate_up_pair['GB/s']} GB/s")
    del pair
    # The reference's published decode point: the 27B model's gate/up pair (N 17408, K 5120) for one lane of 8 rows,
    # 245 us in two passes and 333 us in one on a 32-core M5 Max (docs/internals.md:498-500,
    # LinearGguf.cpp:176-178); af4g64, the format of its sweeps, under this library's own plan.
    lane = Gemv(torch, sq, synthetic, sq.FMT_AF4G64, 8, 17408, 5120, seed=27, gate_up=True)
    lane_sec = time_graph(torch, lane.launch, args.steps, args.warmup)
    lane_bytes = 2 * 17408 * 5120 * 0.5625 + 2 * 8 * 5120 + 2 * 8 * 17408
    gate_up_lane = {"us": round(lane_sec * 1e6, 2), "GB/s": round(lane_bytes / lane_sec / 1e9, 1),
                    "hbm_frac": round(lane_bytes / lane_sec / 1e9 / HBM_PEAK_GBS, 4),
                    "one_pass": bool(lane.plan.config.one_gate_up_pass), "splits": lane.plan.config.splits,
                    "reference_us": {"two_passes": 245.0, "one_pass": 333.0},
                    "reference_device": "32-core M5 Max (docs/internals.md:498-500)",
                    "speedup_vs_reference": round(245e-6 / lane_sec, 1)}
    log(f"  27B gate/up pair, one lane (8 rows, K5120 N17408): {lane_sec * 1e6:.2f} us (reference 245 us on M5 Max)")
    del lane
    torch.cuda.empty_cache()
    if args.calibrate_copy:
        # A plain device copy of known size for scaling the FETCH_SIZE / WRITE_SIZE counters.
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"  calibration copy: 5 x {COPY_BYTES} bytes")
        del src, dst
    extra = {}
    if "sweep" in sections:
        sweep = {}
        points = {v.strip() for v in args.sweep_points.split(",") if v.strip()}
        for (kk, nn) in ((4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)):
            for mm in (1, 2, 4, 8, 16):
                if points and f"K{kk}xN{nn}_M{mm}" not in points:
                    continue
                s, p = bench_gemv(torch, sq, synthetic, sq.FMT_AF4G64, mm, nn, kk, max(50, args.steps // 2), 10)
                g = gemv_bytes(mm, nn, kk) / s / 1e9
                sweep[f"K{kk}xN{nn}_M{mm}"] = {"us": round(s * 1e6, 2), "GB/s": round(g, 1),
                                               "hbm_frac": round(g / HBM_PEAK_GBS, 3), "splits": p.config.splits}
                log(f"  sweep K{kk} N{nn} M{mm}: {s * 1e6:.2f} us, {g:.0f} GB/s")
        # The small shapes' floors: the streaming kernel over each M=1 point's own bytes (best launch shape) and the
        # empty dispatch, timed alike. Below ~10 MB a dispatch's fixed cost is most of its time.
        for (kk, nn) in ((4096, 4096), (4096, 1024)):
            if any(f"K{kk}xN{nn}_M{mm}" not in sweep for mm in (1, 8, 16)):
                continue
            f = stream_floor(torch, sq, int(gemv_bytes(1, nn, kk)), max(50, args.steps // 2), 10)
            for mm in (1, 8, 16):
                # Each point's own bytes at the rate the streaming kernel reaches over this shape's.
                point = sweep[f"K{kk}xN{nn}_M{mm}"]
                point["stream_floor_us"] = round(gemv_bytes(mm, nn, kk) / f["GB/s"] / 1e3, 2)
                point["dispatch_floor_us"] = f["dispatch_floor_us"]
                point["frac_of_floor"] = round(point["stream_floor_us"] / point["us"], 3)
            log(f"  stream floor K{kk} N{nn}: {sweep[f'K{kk}xN{nn}_M1']['stream_floor_us']} us ({f['launch']}), "
                f"dispatch {f['dispatch_floor_by_grid_us']} us")
        extra["c1_decode_sweep_af4g64"] = sweep
    if "prefill" in sections:
        ceiling = mfma_ceiling(torch, sq, args.steps, args.warmup)
        log(f"  MFMA ceiling: {ceiling}")
        extra["mfma_ceiling_tflops"] = ceiling
        prefill = {}
        for (kk, nn) in ((4096, 14336), (14336, 4096), (5120, 27648)):
            s = bench_prefill(torch, sq, synthetic, 2048, nn, kk, 10, 3)
            tf = 2 * 2048 * nn * kk / s / 1e12
            # The vendor library's unquantized bf16 GEMM on the same shape (torch.matmul: hipBLASLt), for scale.
            xa = torch.randn(2048, kk, device="cuda", dtype=torch.bfloat16)
            wb = torch.randn(kk, nn, device="cuda", dtype=torch.bfloat16)
            blas = time_steps(torch, lambda i: torch.matmul(xa, wb), 10, 3)
            del xa, wb
            prefill[f"M2048_K{kk}xN{nn}"] = {"us": round(s * 1e6, 1), "TFLOPS": round(tf, 1),
                                             "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 3),
                                             "frac_of_measured_ceiling": round(tf / ceiling["best"], 3),
                                             "hipblaslt_bf16_unquantized_us": round(blas * 1e6, 1)}
            log(f"  prefill K{kk} N{nn}: {s * 1e6:.0f} us, {tf:.0f} TFLOPS (hipBLASLt bf16 unquantized: "
                f"{blas * 1e6:.0f} us)")
        extra["c2_prefill_af4g64"] = prefill
    if "q4k" in sections:
        q4k = {}
        for mm in (1, 16):
            s, p = bench_gemv(torch, sq, synthetic, sq.FMT_Q4K, mm, 27648, 5120, max(50, args.steps // 2), 10)
            g = gemv_bytes(mm, 27648, 5120) / s / 1e9
            q4k[f"M{mm}_K5120xN27648"] = {"us": round(s * 1e6, 2), "GB/s": round(g, 1), "hbm_frac": round(g / HBM_PEAK_GBS, 3)}
            log(f"  q4k M{mm}: {s * 1e6:.2f} us, {g:.0f} GB/s")
        s = bench_prefill(torch, sq, synthetic, 512, 27648, 5120, 10, 3, fmt=sq.FMT_Q4K)
        tf = 2 * 512 * 27648 * 5120 / s / 1e12
        q4k["M512_K5120xN27648"] = {"us": round(s * 1e6, 1), "TFLOPS": round(tf, 1), "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 3)}
        log(f"  q4k M512: {s * 1e6:.0f} us, {tf:.0f} TFLOPS")
        # The reference's gguf-projection-benchmark: one Q4_K 17408x5120 projection on 2048 rows
        # (dev/benchmarks/prefill-m3max.md:38-41: 30.68 ms on a 40-core M3 Max).
        s = bench_prefill(torch, sq, synthetic, 2048, 17408, 5120, 10, 3, fmt=sq.FMT_Q4K)
        tf = 2 * 2048 * 17408 * 5120 / s / 1e12
        q4k["M2048_K5120xN17408"] = {"us": round(s * 1e6, 1), "TFLOPS": round(tf, 1),
                                     "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 3), "reference_ms": 30.68,
                                     "speedup_vs_reference": round(30.68e-3 / s, 1)}
        log(f"  q4k M2048 17408x5120: {s * 1e6:.0f} us, {tf:.0f} TFLOPS (reference 30.68 ms on M3 Max)")
        extra["c3_q4k"] = q4k
    if "formats" in sections:
        # The adjacent formats on the BASELINE config-1 shape, in GB/s of their own plane bytes plus activations
        # and outputs.
        formats = {}
        for fmt, name in ((sq.FMT_Q5K, "q5_k"), (sq.FMT_Q6K, "q6_k"), (sq.FMT_Q80, "q8_0"), (sq.FMT_AF8G64, "af8g64")):
            for mm in (1, 16):
                s, p = bench_gemv(torch, sq, synthetic, fmt, mm, 14336, 4096, max(50, args.steps // 2), 10)
                g = (weight_bytes(sq, fmt, 14336, 4096) + 2 * mm * (4096 + 14336)) / s / 1e9
                formats[f"{name}_M{mm}_K4096xN14336"] = {"us": round(s * 1e6, 2), "GB/s": round(g, 1),
                                                          "hbm_frac": round(g / HBM_PEAK_GBS, 3),
                                                          "splits": p.config.splits}
                log(f"  {name} M{mm}: {s * 1e6:.2f} us, {g:.0f} GB/s")
            s = bench_prefill(torch, sq, synthetic, 2048, 14336, 4096, 10, 3, fmt=fmt)
            tf = 2 * 2048 * 14336 * 4096 / s / 1e12
            formats[f"{name}_M2048_K4096xN14336"] = {"us": round(s * 1e6, 1), "TFLOPS": round(tf, 1),
                                                       "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 3)}
            log(f"  {name} prefill M2048: {s * 1e6:.0f} us, {tf:.0f} TFLOPS")
        extra["c5_formats"] = formats
    if "moe" in sections:
        s, moe_bytes, moe_flops = bench_moe(torch, sq, synthetic, 50, 5)
        g = moe_bytes / s / 1e9
        extra["c4_moe_af4g64"] = {"us": round(s * 1e6, 1), "GB/s": round(g, 1), "hbm_frac": round(g / HBM_PEAK_GBS, 3),
                                  "TFLOPS": round(moe_flops / s / 1e12, 2)}
        log(f"  moe: {s * 1e6:.0f} us, {g:.0f} GB/s")
        # The reference's own MoE benchmark layer (gguf_moe_benchmark.mm, 35B shape: hidden 2048, 256 experts, top 8,
        # intermediate 512, Q4_K gate/up and Q5_K down experts, a gated Q8_0 shared expert, an F32 router) on a
        # 2048-row prefill chunk, the whole layer: router projection, routing, expert passes and combine.
        s, moe_bytes, moe_flops = bench_moe(torch, sq, synthetic, 20, 3, rows=2048, experts=256, top_k=8, hidden=2048,
                                            inter=512, fmt=sq.FMT_Q4K,
                                            formats={"down": sq.FMT_Q5K, "shared_gate": sq.FMT_Q80,
                                                     "shared_up": sq.FMT_Q80, "shared_down": sq.FMT_Q80},
                                            shared=1, gated=True, router=True)
        extra["c6_moe_35b_gguf_2048_rows"] = {
            "ms": round(s * 1e3, 3), "TFLOPS": round(moe_flops / s / 1e12, 2), "GB/s": round(moe_bytes / s / 1e9, 1),
            "reference_ms": 11.7, "reference_device": "40-core M3 Max (dev/benchmarks/prefill-m3max.md:44-50)",
            "speedup_vs_reference": round(11.7e-3 / s, 1)}
        log(f"  moe 35b gguf 2048 rows: {s * 1e3:.3f} ms (reference 11.7 ms on M3 Max)")
    result = {
        "metric": "4-bit GEMV GB/s (% HBM peak) at M=1; prefill q-GEMM TFLOPS at M=2048",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded: bf16 N(0,1) activations, uint4 codes, bf16 |N(0,0.02)| scales, biases -8s)",
        "config": {"workload": "decode GEMV M=1 K=4096 N=14336 (BASELINE config 1, gate/up shape)", "M": m, "K": k,
                   "N": n, "format": "af4g64", "weights": "4-bit MLX affine group 64", "tile": "column",
                   "splits": plan.config.splits, "weight_ring_copies": ring_copies, "timing": "HIP graph replay"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_bytes(),
                     "kernel": "column_kernel<af4g64, 1 row>", "launch_us": round(sec * 1e6, 3),
                     "algorithmic_bytes": int(gemv_bytes(m, n, k))},
        "stream_floor": dict(floor, frac_of_floor=round(gbs / floor["GB/s"], 3)),
        "c1_gate_up_pair": gate_up_pair,
        "c1_gate_up_pair_27b_lane": gate_up_lane,
    }
    result.update(extra)
    if "cpu" in sections:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(sq, synthetic, args.cpu_budget)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
