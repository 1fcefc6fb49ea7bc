#!/usr/bin/env python3
"""Benchmark of the MI355X decode hot path (one GPU).

Workload (the configuration the headline metric is quoted on): Llama-3-8B
decode, int4 group-64 linear layers. One step = one token through the 7
projections of all 32 transformer layers (q, k, v, o 4096x4096 / 1024x4096,
gate, up 14336x4096, down 4096x14336), every layer with its own weights, so
the 3.93 GB of distinct weights defeat L2 and the 256 MB MALL. The step is
captured once as a HIP graph (224 kernel launches) and replayed.

`value` = algorithmic bytes per step / time (GB/s), algorithmic bytes =
W + (scale, bias) + x + y(fp16) per GEMV. Also reported: per-shape GB/s, the
roofline of the dominant kernel (the 4096x14336 GEMV), the gpt-oss-120b MoE
block (36 layers x 128 experts resident, batch 1 and 8), VQ GEMV, the
skinny-GEMM VALU/MFMA sweep, the fixed cost of a launch inside a graph, and
the CPU baseline (the reference's CPU int4 path restated for x86, timed on
this host).

Timing protocol (the reference's, int4-gemv/src/main.mm:417-438,496-521):
every kernel section warms all its variants, then times them round-robin
(one span each per round, 7 rounds, median and best reported), and the
streaming read of each kernel's own byte count -- the best launch shape of
the reference's unroll x threads sweep at that size -- rides in the same
rotation, so every kernel carries its "% of same-size ceiling".

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--sections ...]
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
WARM_S = 0.2  # seconds of replays before each timed kernel section
ROUNDS = 7  # round-robin rounds per timed section (best and median reported)
LLAMA = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
         ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
N_LAYERS = 32
G = 64


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def int4_bytes(M, K, batch=1, G=G):
    return M * K // 2 + M * (K // G) * 4 + 2 * batch * K + 2 * batch * M


class Timer:
    """HIP events on torch's current stream (where every libkq launch goes)."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, fn, iters, warmup, warm_s=0.0):
        return self.spans(fn, iters, warmup, 1, warm_s)[0]

    def spans(self, fn, iters, warmup, n, warm_s=0.0):
        """n back-to-back timed spans of iters calls each (ms per call). The
        warm-up repeats batches of `warmup` calls until warm_s seconds have
        passed (one batch at least): right after large allocations and their
        initialisation a kernel runs several percent slower for the first
        ~10 ms of replays. The last warm-up batch and every span are enqueued
        without a host wait in between, so the GPU never idles (and drops
        its clock) before or between the timed spans."""
        t = self.torch
        t.cuda.synchronize()
        t0, k = time.perf_counter(), 0
        while True:
            for _ in range(warmup):
                fn(k)
                k += 1
            if time.perf_counter() - t0 >= warm_s:
                break
            t.cuda.synchronize()
        ev = [t.cuda.Event(enable_timing=True) for _ in range(n + 1)]
        ev[0].record()
        for s in range(n):
            for _ in range(iters):
                fn(k)
                k += 1
            ev[s + 1].record()
        t.cuda.synchronize()
        return [ev[s].elapsed_time(ev[s + 1]) / iters for s in range(n)]  # ms

    def round_robin(self, variants, rounds=ROUNDS, warm_s=WARM_S):
        """The reference's interleaved timing (int4-gemv/src/main.mm:496-521):
        every variant is warmed, then timed once per round, round-robin, so
        clock and thermal drift land on all of them alike. variants: name ->
        (fn, calls per span, launches per call). Every warm-up batch and
        span is enqueued with no host wait before or between the spans.
        Returns name -> {"us": median per launch, "us_best": best per
        launch, "spans": rounds} (microseconds)."""
        t = self.torch
        names = list(variants)
        t.cuda.synchronize()
        t0 = time.perf_counter()
        while True:
            for nm in names:
                fn, calls, _ = variants[nm]
                for _ in range(calls):
                    fn()
            if time.perf_counter() - t0 >= warm_s:
                break
            t.cuda.synchronize()
        ev = [[t.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
              for _ in range(rounds)]
        for r in range(rounds):
            ev[r][0].record()
            for i, nm in enumerate(names):
                fn, calls, _ = variants[nm]
                for _ in range(calls):
                    fn()
                ev[r][i + 1].record()
        t.cuda.synchronize()
        out = {}
        for i, nm in enumerate(names):
            _, calls, launches = variants[nm]
            per = sorted(ev[r][i].elapsed_time(ev[r][i + 1]) * 1e3 / (calls * launches)
                         for r in range(rounds))
            out[nm] = {"us": round(per[rounds // 2], 3), "us_best": round(per[0], 3),
                       "spans": rounds}
        return out


def graph_of(torch, fn):
    """Capture fn() (a sequence of libkq launches) as a HIP graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm (first-launch code object loading) outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


# ---------------------------------------------------------------------------
def make_int4_layers(torch, dev, n_layers, shapes, seed=1234):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    layers = []
    for _ in range(n_layers):
        L = {}
        for name, M, K in shapes:
            W = torch.randint(-2**31, 2**31 - 1, (M, K // 8), dtype=torch.int32, device=dev,
                              generator=gen)
            S = (torch.randn((M, K // G), device=dev, generator=gen) * 0.02).abs()
            B = torch.randn((M, K // G), device=dev, generator=gen) * 0.02
            SB = torch.stack([S, B], -1).half().contiguous()
            L[name] = (W, SB, M, K)
        layers.append(L)
    return layers


def bench_int4_step(torch, kq, dev, args, timer, ceil, res):
    layers = make_int4_layers(torch, dev, N_LAYERS, LLAMA)
    x = {K: (torch.randn((1, K), device=dev)).half() for K in (4096, 14336)}
    y = {M: torch.empty((1, M), dtype=torch.float16, device=dev) for M in (1024, 4096, 14336)}
    step_bytes = sum(int4_bytes(M, K) for _, M, K in LLAMA) * N_LAYERS

    def step():
        for L in layers:
            for name, _, _ in LLAMA:
                W, SB, M, K = L[name]
                kq.int4_gemv(W, SB, x[K], y[M], kq.GemvParams(M, K, G))

    # eager (Python launch loop) for reference
    eager_ms = timer.run(lambda i: step(), 3, 1)
    g = graph_of(torch, step)
    # settle after the 3.93 GB of allocations and their initialisation (the
    # first ~10 ms of replays run several percent slow), then W warm-up steps,
    # then exactly K timed steps between host synchronisations
    timer.run(lambda i: g.replay(), 1, 1, WARM_S)
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    res["step"] = dict(ms=ms, bytes=step_bytes, gbs=step_bytes / ms / 1e6, eager_ms=eager_ms)

    # per shape: one graph per shape over the 32 layer copies, timed
    # round-robin with the streaming read of each shape's byte count over
    # 32 buffers
    variants, holds, shapes = {}, [], {}
    for name, M, K in LLAMA:
        if name in ("k", "o", "up"):
            continue  # same shape as v, q, gate

        def one(name=name, M=M, K=K):
            for L in layers:
                W, SB, _, _ = L[name]
                kq.int4_gemv(W, SB, x[K], y[M], kq.GemvParams(M, K, G))
        gs = graph_of(torch, one)
        holds.append(gs)
        b = int4_bytes(M, K)
        sh = f"{M}x{K}"
        shapes[sh] = b
        variants[sh] = (gs.replay, 5 if b > 20e6 else 10, N_LAYERS)
        clabel = f"int4_{b / 1e6:.2f}MB"
        if clabel not in variants:
            cv, hold = ceil.variant(clabel, b, N_LAYERS)
            holds.append(hold)
            variants[clabel] = cv
        cv, hold = ceil.variant_out(clabel, b, N_LAYERS, M)
        holds.append(hold)
        variants[f"out_{sh}"] = cv
    r = timer.round_robin(variants)
    per = {}
    for sh, b in shapes.items():
        k = r[sh]
        per[sh] = dict(us=k["us"], us_best=k["us_best"], gbs=round(b / k["us"] / 1e3, 1),
                       frac=round(b / k["us"] / 1e3 / HBM_PEAK_GBS, 4), bytes=b,
                       **vs_ceiling(k, r[f"int4_{b / 1e6:.2f}MB"], r[f"out_{sh}"]))
    # the step's own ceilings: its 224 reads at the per-shape ceilings, and
    # the same with each GEMV's y stored
    step_ceil_us = N_LAYERS * sum(r[f"int4_{int4_bytes(M, K) / 1e6:.2f}MB"]["us"]
                                  for _, M, K in LLAMA)
    step_ceil_out_us = N_LAYERS * sum(r[f"out_{M}x{K}"]["us"] for _, M, K in LLAMA)
    res["step"]["ceiling_ms"] = round(step_ceil_us / 1e3, 4)
    res["step"]["of_ceiling"] = round(step_ceil_us / 1e3 / ms, 4)
    res["step"]["ceiling_out_ms"] = round(step_ceil_out_us / 1e3, 4)
    res["step"]["of_ceiling_out"] = round(step_ceil_out_us / 1e3 / ms, 4)
    res["per_shape"] = per
    del holds, variants

    # The same weights with the projections that share an input stored as one
    # matrix, as inference engines keep them: q, k and v rows stacked
    # (6144x4096), gate and up rows stacked (28672x4096); o and down as they
    # are. 4 launches a layer instead of 7, the same weight and metadata
    # bytes (x is read once per launch). Timed round-robin with the 7-GEMV
    # step.
    fused = []
    for L in layers:
        F = {}
        for name, parts in (("qkv", ("q", "k", "v")), ("gateup", ("gate", "up"))):
            W = torch.cat([L[p][0] for p in parts])
            SB = torch.cat([L[p][1] for p in parts])
            F[name] = (W, SB, W.shape[0], L[parts[0]][3])
        F["o"], F["down"] = L["o"], L["down"]
        fused.append(F)
    yf = {M: torch.empty((1, M), dtype=torch.float16, device=dev) for M in (4096, 6144, 28672)}
    order = ("qkv", "o", "gateup", "down")
    fused_bytes = sum(int4_bytes(fused[0][n][2], fused[0][n][3]) for n in order) * N_LAYERS

    def fstep():
        for F in fused:
            for name in order:
                W, SB, M, K = F[name]
                kq.int4_gemv(W, SB, x[K], yf[M], kq.GemvParams(M, K, G))

    gf = graph_of(torch, fstep)
    r = timer.round_robin({"step": (g.replay, 2, 1), "fused": (gf.replay, 2, 1)})
    fms = r["fused"]["us"] / 1e3
    res["step"]["round_robin_ms"] = round(r["step"]["us"] / 1e3, 4)
    res["step"]["round_robin_ms_best"] = round(r["step"]["us_best"] / 1e3, 4)
    res["step_fused"] = dict(ms=round(fms, 4), ms_best=round(r["fused"]["us_best"] / 1e3, 4),
                             launches=len(order) * N_LAYERS, bytes=fused_bytes,
                             gbs=round(fused_bytes / fms / 1e6, 1),
                             frac=round(fused_bytes / fms / 1e6 / HBM_PEAK_GBS, 4),
                             shapes="6144x4096 (q|k|v), 4096x4096 (o), 28672x4096 (gate|up), "
                                    "4096x14336 (down)")
    del fused, gf, g, layers
    torch.cuda.empty_cache()


def settle_clocks(torch, kq, dev, timer):
    """The reference's clock settle (int4-gemv/src/main.mm:262-292): hold the
    memory system at a sustained 1 GiB streaming read until the achieved rate
    stops improving -- at least 20 rounds and 8 in a row within +0.5% of the
    best, at most 120 -- so no section times a DVFS ramp."""
    big = 1 << 30
    bb = torch.empty(big, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    best, stable, rounds = 0.0, 0, 0
    while rounds < 120 and (rounds < 20 or stable < 8):
        rounds += 1
        us = timer.run(lambda i: kq.stream_read(bb, big, sink), 4, 0) * 1e3
        gbs = big / us / 1e3
        stable = stable + 1 if gbs < best * 1.005 else 0
        best = max(best, gbs)
    del bb
    return {"rounds": rounds, "plateau_gbs": round(best, 1)}


SWEEP = [(u, q) for u in (1, 2, 4, 8) for q in (1, 2, 4, 8, 16, 32)] + [(1, 0)]


class Ceilings:
    """The streaming-read ceiling at each timed kernel's own byte count, as
    the reference measures it: a sweep of unroll {1, 2, 4, 8} x quads per
    thread {1 .. 32} (threads = quads / (qpt * unroll), rounded down to 256,
    at least 1024), plus this library's default shape (unroll 1 over 2048 x
    256 threads, qpt reported as 0), keeps the best -- "the best this
    machine can do on a pure read, or it is not a ceiling"
    (int4-gemv/src/main.mm:294-334). The chosen shape then rides in the
    kernel's own timing rotation, over as many buffers as the kernel has
    weight copies, so "% of ceiling" compares two numbers measured under the
    same clock and thermal state (int4-gemv/src/main.mm:417-438)."""

    def __init__(self, torch, kq, dev, timer):
        self.torch, self.kq, self.dev, self.timer = torch, kq, dev, timer
        self.sink = torch.zeros(4, dtype=torch.int32, device=dev)
        self.best = {}

    @staticmethod
    def threads(nbytes, U, qpt):
        if qpt == 0:
            return 2048 * 256
        thr = (nbytes // 16) // (qpt * U) // 256 * 256
        return thr if thr >= 1024 else None

    def _bufs(self, nbytes, copies):
        return [self.torch.empty(nbytes, dtype=self.torch.uint8, device=self.dev)
                for _ in range(copies)]

    def _graph(self, bufs, nbytes, U, thr, out=None, nout=0):
        kq, sink = self.kq, self.sink

        def one():
            for b in bufs:
                if out is None:
                    kq.stream_read(b, nbytes, sink, unroll=U, threads=thr)
                else:
                    kq.stream_read_out(b, nbytes, out, nout, U, thr)
        return graph_of(self.torch, one)

    @staticmethod
    def calls(nbytes, copies):
        """Replays per span so that a span lasts about a millisecond."""
        est_us = copies * (1.8 + nbytes / 7.0e6)
        return max(1, int(1000.0 / est_us))

    def sweep(self, label, nbytes, copies):
        nbytes = nbytes // 16 * 16
        if label in self.best:
            return self.best[label]
        bufs = self._bufs(nbytes, copies)
        graphs, variants = [], {}
        for U, q in SWEEP:
            thr = self.threads(nbytes, U, q)
            if thr is None:
                continue
            g = self._graph(bufs, nbytes, U, thr)
            graphs.append(g)
            variants[(U, thr, q)] = (g.replay, self.calls(nbytes, copies), copies)
        r = self.timer.round_robin(variants, rounds=3, warm_s=0.05)
        key = min(r, key=lambda k: r[k]["us_best"])
        self.best[label] = {"bytes": nbytes, "copies": copies, "unroll": key[0],
                            "threads": key[1], "qpt": key[2], "us_best": r[key]["us_best"],
                            "gbs": round(nbytes / r[key]["us_best"] / 1e3, 1),
                            "configs": len(variants)}
        del graphs, bufs
        return self.best[label]

    def variant(self, label, nbytes, copies):
        """(fn, calls, launches) of the best shape at this size over its own
        `copies` buffers, and the holder that keeps them alive."""
        c = self.sweep(label, nbytes, copies)
        bufs = self._bufs(c["bytes"], copies)
        g = self._graph(bufs, c["bytes"], c["unroll"], c["threads"])
        return (g.replay, self.calls(c["bytes"], copies), copies), (bufs, g)

    def variant_out(self, label, nbytes, copies, out_elems):
        """The same best read shape, then out_elems 2-byte values stored
        across the grid (kq_stream_read_out): the ceiling of a kernel that
        must also store its y. A launch that stores from every XCD pays for
        the write-back of each XCD's dirty L2 lines at its end (measured:
        +0.37-0.47 us at 2.4-33 MB; +0.26-0.31 us even with every store
        issued before the reads; plain stores cheaper than sc0, sc1 or nt)."""
        c = self.sweep(label, nbytes, copies)
        bufs = self._bufs(c["bytes"], copies)
        out = self.torch.empty(out_elems, dtype=self.torch.int16, device=self.dev)
        g = self._graph(bufs, c["bytes"], c["unroll"], c["threads"], out, out_elems)
        return (g.replay, self.calls(c["bytes"], copies), copies), (bufs, out, g)

    def fit(self):
        """Least-squares t = fixed + bytes / rate over the best reads of
        every size swept (the fixed part is what one launch costs beyond
        its bytes)."""
        pts = [(c["bytes"], c["us_best"]) for c in self.best.values()]
        if len(pts) < 2:
            return None
        n = len(pts)
        mx = sum(b for b, _ in pts) / n
        my = sum(t for _, t in pts) / n
        sxx = sum((b - mx) ** 2 for b, _ in pts)
        slope = sum((b - mx) * (t - my) for b, t in pts) / sxx
        return {"fixed_us": round(my - slope * mx, 3), "rate_gbs": round(1e-3 / slope, 1),
                "sizes": n}


def rot_copies(nbytes):
    """Buffers a rotation needs: 32 (the GEMV protocol) up to 64 MB, else
    enough that a replay streams more than 1 GB (beyond the 256 MB MALL)."""
    return N_LAYERS if nbytes <= 64e6 else max(2, -(-int(1.1e9) // int(nbytes)))


def vs_ceiling(kern, ceil, out=None):
    """A kernel's timing against the same-size read timed in its rotation
    and, given `out`, against that read followed by the kernel's output
    store (the same number of 2-byte values)."""
    d = {"ceiling_us": ceil["us"], "ceiling_us_best": ceil["us_best"],
         "of_ceiling": round(ceil["us"] / kern["us"], 4),
         "of_ceiling_best": round(ceil["us_best"] / kern["us_best"], 4)}
    if out is not None:
        d.update({"ceiling_out_us": out["us"], "ceiling_out_us_best": out["us_best"],
                  "of_ceiling_out": round(out["us"] / kern["us"], 4)})
    return d


def bench_floor(torch, kq, dev, timer, res):
    """The fixed cost of one launch inside a HIP graph: 32 launches a replay
    of a kernel with (almost) nothing to do -- the streaming-read kernel over
    one 16-byte quad, so one thread loads and every other thread exits --
    on 1, 256 and 2048 workgroups of 256 threads. Timed round-robin like
    every other section."""
    buf = torch.zeros(16, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    graphs, variants = [], {}
    for name, thr in (("1_workgroup", 256), ("256_workgroups", 256 * 256),
                      ("2048_workgroups", 2048 * 256)):
        def one(thr=thr):
            for _ in range(N_LAYERS):
                kq.stream_read(buf, 16, sink, unroll=1, threads=thr)
        g = graph_of(torch, one)
        graphs.append(g)
        variants[name] = (g.replay, 10, N_LAYERS)
    r = timer.round_robin(variants)
    res["launch_floor"] = {"what": "us per launch, 32 launches of a one-quad streaming read per "
                                   "graph replay, 10 replays a span, median and best of "
                                   f"{ROUNDS} round-robin spans", **r}
    del graphs


def bench_ceiling(torch, kq, dev, timer, ceil, res):
    """1 GiB read (the machine's streaming rate, one buffer re-read) and the
    fit of every size swept so far."""
    c = ceil.sweep("1GiB", 1 << 30, 1)
    res["ceiling_1GiB"] = c
    res["ceiling_sizes"] = {k: v for k, v in ceil.best.items()}
    res["ceiling_fit"] = ceil.fit()


def bench_roofline(torch, kq, dev, timer, ceil, res):
    """The dominant kernel: int4 GEMV at 4096 x 14336 (33 MB per launch),
    launched back to back over 32 weight copies on torch's current stream,
    timed round-robin with the streaming read of the same 33 MB over 32
    buffers: spans of 5 graph replays (160 launches), the median span's
    average launch time is the figure, the fastest span beside it."""
    M, K = 4096, 14336
    layers = make_int4_layers(torch, dev, N_LAYERS, [("down", M, K)], seed=99)
    x = torch.randn((1, K), device=dev).half()
    y = torch.empty((1, M), dtype=torch.float16, device=dev)

    def one():
        for L in layers:
            W, SB, _, _ = L["down"]
            kq.int4_gemv(W, SB, x, y, kq.GemvParams(M, K, G))
    g = graph_of(torch, one)
    b = int4_bytes(M, K)
    cv, hold = ceil.variant(f"int4_{b / 1e6:.2f}MB", b, N_LAYERS)
    cvo, hold_o = ceil.variant_out(f"int4_{b / 1e6:.2f}MB", b, N_LAYERS, M)
    r = timer.round_robin({"gemv": (g.replay, 5, N_LAYERS), "ceiling": cv, "ceiling_out": cvo})
    us = r["gemv"]["us"]
    res["roofline"] = {"bound": "hbm", "achieved": round(b / us / 1e3, 1), "peak": HBM_PEAK_GBS,
                       "unit": "GB/s", "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                       "traffic": measured_traffic(), "kernel": "int4_valu (vector path), 4096x14336, batch 1",
                       "bytes_per_launch": b, "us_per_launch": us,
                       "us_per_launch_best_span": r["gemv"]["us_best"],
                       "launches_timed": 5 * ROUNDS * N_LAYERS,
                       **vs_ceiling(r["gemv"], r["ceiling"], r["ceiling_out"])}
    del layers, hold, hold_o


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "int4_gemv_4096x14336_traffic.json")


def measured_traffic():
    """HBM bytes per launch of the roofline kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs over the `traffic` section (each
    counter scaled by what it reads for a torch copy kernel of known size).
    Counters cannot be read live, so this is the recorded figure (or None)."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["traffic_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def bench_traffic(torch, kq, dev, res):
    """Eager launches for the counter runs (rocprofv3 --pmc FETCH_SIZE, then
    WRITE_SIZE, each a run of its own): the roofline GEMV over its 32 weight
    copies; the MoE block at 1 and 8 tokens over 8 layers of 128 experts
    each (distinct experts per layer recorded, for the bytes actually read);
    the VQ GEMV 14336 x 4096 over 8 copies; the matrix-core skinny GEMM
    28672 x 8192 at 16 tokens over 4 copies; then a plain copy kernel
    (int32 -> fp32 elementwise, COPY_BYTES read and COPY_BYTES written; a
    same-dtype copy_ would be a DMA memcpy with no kernel) that calibrates
    FETCH_SIZE and WRITE_SIZE."""
    out = {}
    M, K = 4096, 14336
    layers = make_int4_layers(torch, dev, N_LAYERS, [("down", M, K)], seed=99)
    x = torch.randn((1, K), device=dev).half()
    y = torch.empty((1, M), dtype=torch.float16, device=dev)
    for L in layers:
        W, SB, _, _ = L["down"]
        kq.int4_gemv(W, SB, x, y, kq.GemvParams(M, K, G))
    torch.cuda.synchronize()
    del layers
    out["gemv"] = {"launches": N_LAYERS, "bytes": int4_bytes(M, K)}
    # MoE block
    d = kq.moe_default_desc()
    nl = 8
    pools = make_moe_pools(torch, dev, nl, d)
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    Rs = [(torch.randn((d.n_experts, d.hidden), device=dev, generator=gen) * 0.02).half()
          for _ in range(nl)]
    per_exp = 3 * (d.hidden * d.inter // 2 + 2 * 2 * d.inter * (d.hidden // 64) + 2 * d.inter)
    for batch in (1, 8):
        xs = [torch.randn((batch, d.hidden), device=dev, generator=gen).half() for _ in range(nl)]
        idx = torch.zeros((nl, batch, d.top_k), dtype=torch.int32, device=dev)
        wgt = torch.zeros((nl, batch, d.top_k), dtype=torch.float32, device=dev)
        H = torch.zeros((batch, d.top_k, d.inter), dtype=torch.float16, device=dev)
        Y = torch.zeros((batch, d.hidden), dtype=torch.float32, device=dev)
        nws = kq.moe_workspace_size(d, batch)
        ws = torch.empty(nws, dtype=torch.uint8, device=dev)
        kq.moe_workspace_init(ws, nws)
        for l in range(nl):
            kq.moe_block(pools[l], d, Rs[l], xs[l], idx[l], wgt[l], H, Y, ws, nws, batch=batch)
        torch.cuda.synchronize()
        ids = idx.cpu().numpy()
        uniq = [len(set(ids[l].ravel().tolist())) for l in range(nl)]
        out[f"moe_batch{batch}"] = {"blocks": nl, "unique_experts": uniq,
                                    "bytes_per_block": int(sum(uniq) / nl * per_exp
                                                           + d.n_experts * d.hidden * 2)}
    del pools
    torch.cuda.empty_cache()
    # VQ GEMV
    M, K = 14336, 4096
    mats = []
    for _ in range(8):
        mats.append((torch.randint(0, 256, (M, K // 2), dtype=torch.uint8, device=dev),
                     (torch.randn((M // 256, 256, 2), device=dev) * 0.02).half(),
                     (torch.randn((M, 1), device=dev) * 0.1 + 1).abs().half()))
    x = torch.randn((1, K), device=dev).half()
    y = torch.empty((1, M), dtype=torch.float16, device=dev)
    for IDX, C, S in mats:
        kq.vq_gemv(IDX, C, S, x, y, kq.VQParams(M, K, 256, K))
    torch.cuda.synchronize()
    out["vq"] = {"launches": 8, "bytes": M * K // 2 + 2 * M + (M // 256) * 1024 + 2 * K + 2 * M}
    del mats
    # matrix-core skinny GEMM, 16 tokens
    M, K = 28672, 8192
    layers = make_int4_layers(torch, dev, 4, [("w", M, K)], seed=M)
    x = torch.randn((16, K), device=dev).half()
    y = torch.empty((16, M), dtype=torch.float16, device=dev)
    for L in layers:
        W, SB, _, _ = L["w"]
        kq.int4_gemv(W, SB, x, y, kq.GemvParams(M, K, G), batch=16, path=kq.PATH_MFMA)
    torch.cuda.synchronize()
    out["mfma_b16"] = {"launches": 4, "bytes": int4_bytes(M, K, 16)}
    del layers
    torch.cuda.empty_cache()
    src = torch.ones(COPY_BYTES // 4, dtype=torch.int32, device=dev)
    dst = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    out["copy"] = {"launches": 4, "bytes": COPY_BYTES}
    res["traffic_run"] = out


COPY_BYTES = 256 << 20


# ---------------------------------------------------------------------------
def make_moe_pools(torch, dev, n_layers, d, seed=7):
    """n_layers x n_experts expert blobs (gpt-oss layout) generated on the
    GPU: uniform nibbles, bf16 scale ~ |N(0.0064, 0.001)|, bias ~ N(-0.048,
    0.004), output bias ~ N(0, 0.02) (the statistics of int4-quantised
    N(0, 0.02) weights)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    ne = d.n_experts
    pools = []
    for _ in range(n_layers):
        p = torch.randint(0, 256, (ne, d.blob), dtype=torch.uint8, device=dev, generator=gen)
        for off, rows, cols in ((d.off_gate, d.inter, d.hidden), (d.off_up, d.inter, d.hidden),
                                (d.off_down, d.hidden, d.inter)):
            ng = rows * (cols // 64)
            s = (torch.randn((ne, ng), device=dev, generator=gen) * 0.001 + 0.0064).abs()
            b = torch.randn((ne, ng), device=dev, generator=gen) * 0.004 - 0.048
            bi = torch.randn((ne, rows), device=dev, generator=gen) * 0.02
            for sub, t in ((d.sub_s, s), (d.sub_b, b), (d.sub_bi, bi)):
                raw = t.bfloat16().contiguous().view(torch.uint8)
                p[:, off + sub: off + sub + raw.shape[1]] = raw
        pools.append(p)
    return pools


def bench_moe(torch, kq, dev, args, timer, ceil, res, n_layers=36):
    """The gpt-oss-120b MoE block over 36 resident layers of 128 experts,
    one HIP graph per launch structure, timed round-robin with the streaming
    read of the bytes actually read per block (32 buffers)."""
    d = kq.moe_default_desc()
    pools = make_moe_pools(torch, dev, n_layers, d)
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    Rs = [(torch.randn((d.n_experts, d.hidden), device=dev, generator=gen) * 0.02).half()
          for _ in range(n_layers)]
    per_exp = 3 * (d.hidden * d.inter // 2 + 2 * 2 * d.inter * (d.hidden // 64) + 2 * d.inter)
    router = d.n_experts * d.hidden * 2
    out = {}
    for batch in (1, 8):
        xs = [torch.randn((batch, d.hidden), device=dev, generator=gen).half()
              for _ in range(n_layers)]
        idx = torch.zeros((n_layers, batch, d.top_k), dtype=torch.int32, device=dev)
        wgt = torch.zeros((n_layers, batch, d.top_k), dtype=torch.float32, device=dev)
        H = torch.zeros((batch, d.top_k, d.inter), dtype=torch.float16, device=dev)
        Y = torch.zeros((batch, d.hidden), dtype=torch.float32, device=dev)
        nws = kq.moe_workspace_size(d, batch)
        ws = torch.empty(nws, dtype=torch.uint8, device=dev)
        kq.moe_workspace_init(ws, nws)

        def step(path=kq.MOE_PATH_AUTO):
            for l in range(n_layers):
                kq.moe_block(pools[l], d, Rs[l], xs[l], idx[l], wgt[l], H, Y, ws, nws,
                             batch=batch, path=path)
        g = graph_of(torch, step)
        # bytes actually read: the distinct selected experts' 3 projections
        # + router, per layer
        ids = idx.cpu().numpy()
        uniq = sum(len(set(ids[l].ravel().tolist())) for l in range(n_layers))
        b = uniq * per_exp + n_layers * router
        bpb = b // n_layers
        holds = [g]
        variants = {"block": (g.replay, 2, n_layers)}
        if batch == 1:
            # the other launch structures of the same block, same layers:
            # one launch (KQ_MOE_PATH_ONE) and the reference's atomic sum(h)
            # form (KQ_MOE_PATH_ATOMIC); skipped where the library refuses one
            skipped = {}
            for pname, path in (("one_launch", kq.MOE_PATH_ONE), ("atomic", kq.MOE_PATH_ATOMIC)):
                try:
                    gp = graph_of(torch, lambda path=path: step(path))
                except kq.KQError as e:
                    skipped[pname] = str(e)
                    continue
                holds.append(gp)
                variants[pname] = (gp.replay, 2, n_layers)
            # the same layers one operation per launch (encodeUnfused,
            # moe-fused/src/main.mm:208-284), also replayed from a graph
            nuw = kq.moe_unfused_workspace_size(d)
            uws = torch.empty(nuw, dtype=torch.uint8, device=dev)
            nl = [0]

            def ustep():
                for l in range(n_layers):
                    nl[0] = kq.moe_block_unfused(pools[l], d, Rs[l], xs[l], idx[l], wgt[l], H, Y,
                                                 uws, nuw)
            gu = graph_of(torch, ustep)
            holds.append(gu)
            variants["unfused"] = (gu.replay, 1, n_layers)
        cv, hold = ceil.variant(f"moe_b{batch}_{bpb / 1e6:.1f}MB", bpb, rot_copies(bpb))
        holds.append(hold)
        variants["ceiling"] = cv
        r = timer.round_robin(variants)
        us_block = r["block"]["us"]
        row = dict(us_per_block=us_block, us_per_block_best=r["block"]["us_best"],
                   us_per_token_per_block=round(us_block / batch, 3),
                   unique_experts_per_block=round(uniq / n_layers, 2),
                   bytes_per_block=bpb,
                   gbs=round(bpb / us_block / 1e3, 1),
                   frac=round(bpb / us_block / 1e3 / HBM_PEAK_GBS, 4),
                   **vs_ceiling(r["block"], r["ceiling"]))
        if batch == 1:
            for pname in ("one_launch", "atomic"):
                if pname in r:
                    row[pname] = dict(us_per_block=r[pname]["us"],
                                      us_per_block_best=r[pname]["us_best"])
                else:
                    row[pname] = dict(skipped=skipped.get(pname))
            row["unfused"] = dict(launches=nl[0], us_per_block=r["unfused"]["us"],
                                  us_per_block_best=r["unfused"]["us_best"],
                                  over_fused=round(r["unfused"]["us"] / us_block, 3))
        out[f"batch{batch}"] = row
        del holds, variants, g
    res["moe"] = out
    del pools
    torch.cuda.empty_cache()


def bench_vq(torch, kq, dev, args, timer, ceil, res):
    """VQ GEMV at both config-3 shapes over 32 matrices each, timed
    round-robin with the int4 GEMV at the same shapes (the reference's
    equal-bytes comparison, vq-gemv/src/main.mm) and the streaming read of
    each kernel's byte count."""
    out = {}
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    variants, holds, nbytes = {}, [], {}
    for M, K in ((14336, 4096), (4096, 14336)):
        mats = []
        for _ in range(N_LAYERS):
            IDX = torch.randint(0, 256, (M, K // 2), dtype=torch.uint8, device=dev, generator=gen)
            C = (torch.randn((M // 256, 256, 2), device=dev, generator=gen) * 0.02).half()
            S = (torch.randn((M, 1), device=dev, generator=gen) * 0.1 + 1).abs().half()
            mats.append((IDX, C, S))
        x = torch.randn((1, K), device=dev).half()
        y = torch.empty((1, M), dtype=torch.float16, device=dev)

        def one(mats=mats, x=x, y=y, M=M, K=K):
            for IDX, C, S in mats:
                kq.vq_gemv(IDX, C, S, x, y, kq.VQParams(M, K, 256, K))
        g = graph_of(torch, one)
        layers = make_int4_layers(torch, dev, N_LAYERS, [("w", M, K)], seed=M + K)
        yi = torch.empty((1, M), dtype=torch.float16, device=dev)

        def ione(layers=layers, x=x, yi=yi, M=M, K=K):
            for L in layers:
                W, SB, _, _ = L["w"]
                kq.int4_gemv(W, SB, x, yi, kq.GemvParams(M, K, G))
        gi = graph_of(torch, ione)
        holds += [mats, g, layers, gi]
        b = M * K // 2 + 2 * M + (M // 256) * 1024 + 2 * K + 2 * M
        sh = f"{M}x{K}"
        nbytes[sh] = b
        variants[sh] = (g.replay, 5, N_LAYERS)
        variants[f"int4_{sh}"] = (gi.replay, 5, N_LAYERS)
        cv, hold = ceil.variant(f"vq_{b / 1e6:.2f}MB", b, N_LAYERS)
        holds.append(hold)
        variants[f"ceiling_{sh}"] = cv
        cv, hold = ceil.variant_out(f"vq_{b / 1e6:.2f}MB", b, N_LAYERS, M)
        holds.append(hold)
        variants[f"ceiling_out_{sh}"] = cv
    r = timer.round_robin(variants)
    for sh, b in nbytes.items():
        k, ki = r[sh], r[f"int4_{sh}"]
        M, K = (int(v) for v in sh.split("x"))
        bi = int4_bytes(M, K)
        out[sh] = dict(us=k["us"], us_best=k["us_best"], gbs=round(b / k["us"] / 1e3, 1),
                       frac=round(b / k["us"] / 1e3 / HBM_PEAK_GBS, 4), bytes=b,
                       int4_us=ki["us"], int4_bytes=bi,
                       time_per_byte_vs_int4=round((k["us"] / b) / (ki["us"] / bi), 3),
                       **vs_ceiling(k, r[f"ceiling_{sh}"], r[f"ceiling_out_{sh}"]))
    del holds, variants
    # the quantiser that makes this format (vq-gemv/quant/pq_quantize.py:28-83)
    # from dense N(0, 0.02) weights: 14336 x 4096, reference defaults (25
    # iterations, 200000-point sample), both formats
    M, K = 14336, 4096
    W = torch.randn((M, K), device=dev, generator=gen) * 0.02
    for name, R, Gq in (("cb256_rowscale", 256, K), ("reference_cb1_g32", M, 32)):
        nblk = (M + R - 1) // R
        IDX = torch.empty((M, K // 2), dtype=torch.uint8, device=dev)
        C = torch.empty((nblk, 256, 2), dtype=torch.float16, device=dev)
        S = torch.empty((M, K // Gq), dtype=torch.float16, device=dev)
        wsb = kq.vq_quantize_workspace_size(M, K, R, Gq)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        kq.vq_quantize(W, IDX, C, S, M, K, R, Gq, ws, wsb)
        ms = timer.run(lambda i: kq.vq_quantize(W, IDX, C, S, M, K, R, Gq, ws, wsb), 3, 1)
        out[f"quantize_{M}x{K}_{name}"] = dict(ms=round(ms, 3), iters=25, sample=200_000,
                                               launches=3 + 2 * 25)
    del W
    res["vq"] = out


def bench_skinny(torch, kq, dev, args, timer, ceil, res):
    """Each of --skinny-shapes (default: both config-2 shapes) at each of
    --skinny-batches tokens through the vector path, the matrix cores and
    AUTO's choice, each a HIP graph over enough weight copies (8 for the
    config-2 shapes, at most 256) that ~940 MB of weights stream per replay,
    so every byte comes from HBM. The token counts of one path form one
    rotation, round-robin with the streaming read of the weights' bytes over
    as many buffers, as the reference rotates the variants of one kernel
    (int4-gemv/src/main.mm:496-521): in one rotation of every path, the
    vector path's long passes at 8-16 tokens (0.1-0.2 ms a launch) left the
    matrix-core spans after them 4-10% slower than in a rotation of their
    own, measured on one box."""
    out = {}
    batches = [int(b) for b in args.skinny_batches.split(",")]
    shapes = [tuple(int(v) for v in sh.split("x")) for sh in args.skinny_shapes.split(",")]
    paths = (("valu", kq.PATH_VALU), ("mfma", kq.PATH_MFMA), ("auto", kq.PATH_AUTO))
    for M, K in shapes:
        ncopy = max(8, min(256, int(940e6 // (M * K // 2))))
        layers = make_int4_layers(torch, dev, ncopy, [("w", M, K)], seed=M)
        wb = int4_bytes(M, K, 0)
        cv, chold = ceil.variant(f"skinny_{M}x{K}", wb, ncopy)
        xs = {batch: torch.randn((batch, K), device=dev).half() for batch in batches}
        ys = {batch: torch.empty((batch, M), dtype=torch.float16, device=dev) for batch in batches}
        rows = {batch: {} for batch in batches}
        ceil_us = []
        for pname, path in paths:
            variants, holds = {}, []
            for batch in batches:
                def one(path=path, x=xs[batch], y=ys[batch], batch=batch):
                    for L in layers:
                        W, SB, _, _ = L["w"]
                        kq.int4_gemv(W, SB, x, y, kq.GemvParams(M, K, G), batch=batch, path=path)
                try:
                    one()
                except kq.KQError:
                    continue
                g = graph_of(torch, one)
                holds.append(g)
                variants[batch] = (g.replay, 2, ncopy)
            variants["ceiling"] = cv
            r = timer.round_robin(variants, rounds=5)
            ceil_us.append(r["ceiling"])
            for batch in batches:
                if batch not in r:
                    rows[batch][pname] = None
                    continue
                k = r[batch]
                b = int4_bytes(M, K, batch)
                rows[batch][pname] = dict(us=k["us"], us_best=k["us_best"],
                                          gbs=round(b / k["us"] / 1e3, 1),
                                          of_ceiling=round(r["ceiling"]["us"] / k["us"], 4))
            del variants, holds
        for batch in batches:
            out[f"{M}x{K}_b{batch}"] = rows[batch]
        out[f"{M}x{K}_ceiling"] = dict(us=statistics.median(c["us"] for c in ceil_us),
                                       us_best=min(c["us_best"] for c in ceil_us),
                                       bytes=wb, copies=ncopy)
        del layers, chold, xs, ys
        torch.cuda.empty_cache()
    res["skinny"] = out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds):
    """The reference's CPU int4 GEMV paths (cpu_gemv_neon16 and cpu_gemv_neon,
    hetero-gemv/src/cpu_gemv.h:55-103, restated for x86 in oracle/cpu_fast.c)
    over the same Llama layer shapes, on this host's cores, for a bounded
    sample of about `seconds` of CPU work. Every path the CPU supports is
    probed on one pass over the layers and the fastest is timed; the rows run
    on a persistent pool of `cores` threads (all cores of this process's
    affinity, at most 16: the host share of one GPU on the GPU boxes)."""
    import numpy as np

    import oracle
    from kernels_amd import gen
    if not oracle.cpu_fast_supported():
        return None
    affinity = len(os.sched_getaffinity(0))
    cores = max(1, min(affinity, 16))
    ncopy = 3  # 369 MB of distinct weights per pass, beyond the host LLC
    mats = []
    for c in range(ncopy):
        L = []
        for name, M, K in LLAMA:
            p = gen.int4_problem(M, K, G, seed=c * 10 + len(L))
            L.append((p["W"], p["SB"], p["X"][0], M, K))
        mats.append(L)
    step_bytes = sum(int4_bytes(M, K) for _, M, K in LLAMA)

    def timed(path, budget, min_passes):
        n, t0 = 0, time.perf_counter()
        while True:
            for W, SB, X, M, K in mats[n % ncopy]:
                oracle.int4_gemv_cpu_fast(W, SB, X, M, K, G, nthreads=cores, path=path)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget and n >= min_passes:
                return n, el

    best = oracle.cpu_fast_path_name(0)
    paths, probes = [], {}
    for path in (oracle.CPU_AVX2, oracle.CPU_AVX512, oracle.CPU_FP16):
        paths.append(path)
        if oracle.cpu_fast_path_name(path) == best:
            break
    timed(paths[-1], 0.0, 1)  # thread pool start, first touch
    for path in paths:
        n, el = timed(path, 0.5, ncopy)
        probes[oracle.cpu_fast_path_name(path)] = round(step_bytes * n / el / 1e9, 2)
    path = max(paths, key=lambda q: probes[oracle.cpu_fast_path_name(q)])
    n, el = timed(path, seconds, ncopy)
    layer_s = el / n
    # the fp64 oracle (the reference's host check, int4-gemv/src/main.mm:64-92)
    # on the same cores, over a shorter sample of the same layers
    n64, t0 = 0, time.perf_counter()
    while True:
        W, SB, X, M, K = mats[n64 % ncopy][n64 % len(LLAMA)]
        oracle.int4_gemv(W, SB, None, X, M, K, G, True, nthreads=cores)
        n64 += 1
        el64 = time.perf_counter() - t0
        if el64 >= seconds / 3 and n64 >= len(LLAMA):
            break
    b64 = sum(int4_bytes(*LLAMA[i % len(LLAMA)][1:]) for i in range(n64))
    fp64 = {"value": round(b64 / el64 / 1e9, 3), "unit": "GB/s", "cores": cores,
            "sample": f"{n64} GEMVs of the Llama layer shapes in {el64:.1f} s"}
    name = oracle.cpu_fast_path_name(path)
    return {"value": round(step_bytes / layer_s / 1e9, 2), "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": f"{n} Llama-3-8B layers (7 int4 GEMVs each, {step_bytes / 1e6:.1f} MB) "
                      f"over {ncopy} weight copies in {el:.1f} s; {name}, restating "
                      f"hetero-gemv/src/cpu_gemv.h:55-103, on a persistent pool of {cores} "
                      f"threads ({affinity} cores in this process's affinity)",
            "cpu": cpu_model(),
            "path": name,
            "path_probe_gbs": probes,
            "ms_per_layer": round(layer_s * 1e3, 3),
            "ms_per_step_32_layers": round(layer_s * 1e3 * N_LAYERS, 2),
            "fp64_oracle": fp64}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sections", default="floor,roofline,step,moe,vq,skinny,ceiling,cpu")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--skinny-batches", default="1,2,3,4,8,16")
    ap.add_argument("--skinny-shapes", default="28672x8192,8192x28672",
                    help="MxK list for the skinny section")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (GEMV "
              "weights would shard by output rows, MoE experts by expert); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    sections = set(args.sections.split(","))

    import torch
    from kernels_amd import kq
    kq.lib()
    dev = torch.device("cuda:0")
    timer = Timer(torch)
    res = {}
    t_start = time.time()
    timed = {"floor", "step", "ceiling", "roofline", "moe", "vq", "skinny"}
    if sections & timed:
        log("[bench] clock settle (1 GiB streaming reads until the rate plateaus)")
        res["settle"] = settle_clocks(torch, kq, dev, timer)
        log(f"[bench] settle {res['settle']}")
    ceil = Ceilings(torch, kq, dev, timer)
    if "floor" in sections:
        log("[bench] launch floor (near-empty kernel, 32 launches per graph replay)")
        bench_floor(torch, kq, dev, timer, res)
        log(f"[bench] floor {res['launch_floor']}")
    if "roofline" in sections:
        log("[bench] roofline kernel 4096x14336 (round-robin with its same-size read)")
        bench_roofline(torch, kq, dev, timer, ceil, res)
        log(f"[bench] roofline {res['roofline']}")
    if "step" in sections:
        log("[bench] int4 decode step (Llama-3-8B, 32 layers)")
        bench_int4_step(torch, kq, dev, args, timer, ceil, res)
        log(f"[bench] step {res['step']} per shape {res['per_shape']} "
            f"fused projections {res.get('step_fused')}")
    if "traffic" in sections:
        log("[bench] counter-run launches (roofline kernel + calibration copy)")
        bench_traffic(torch, kq, dev, res)
        log(f"[bench] traffic {res['traffic_run']}")
    if "moe" in sections:
        log("[bench] MoE block, 36 layers x 128 experts")
        bench_moe(torch, kq, dev, args, timer, ceil, res)
        log(f"[bench] moe {res['moe']}")
    if "vq" in sections:
        log("[bench] VQ GEMV")
        bench_vq(torch, kq, dev, args, timer, ceil, res)
        log(f"[bench] vq {res['vq']}")
    if "skinny" in sections:
        log("[bench] skinny GEMM sweep")
        bench_skinny(torch, kq, dev, args, timer, ceil, res)
        log(f"[bench] skinny {res['skinny']}")
    if "ceiling" in sections:
        log("[bench] stream-read ceiling (1 GiB) and the fit over every size swept")
        bench_ceiling(torch, kq, dev, timer, ceil, res)
        log(f"[bench] ceiling 1GiB {res['ceiling_1GiB']} fit {res['ceiling_fit']}")
    cpu = None
    if "cpu" in sections:
        log("[bench] CPU baseline")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"[bench] cpu {cpu}")

    st = res.get("step", {})
    line = {
        "metric": "int4 GEMV achieved HBM GB/s & % of 8 TB/s; fused MoE block us/token",
        "value": round(st.get("gbs", 0.0), 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(st.get("ms", 0.0), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 x f16 -> f32 acc, f16 out",
        "data": "synthetic (seeded, generated on the GPU)",
        "config": {"workload": "Llama-3-8B decode int4 g64 linear layers: 32 layers x 7 GEMVs "
                               "(4096x4096 x2, 1024x4096 x2, 14336x4096 x2, 4096x14336), batch 1, "
                               "HIP graph of one token step",
                   "bytes_per_step": st.get("bytes"), "frac_of_8TBs": round(st.get("gbs", 0) /
                                                                            HBM_PEAK_GBS, 4)},
        "roofline": res.get("roofline"),
        "cpu_baseline": cpu,
        "step": {k: st[k] for k in ("ceiling_ms", "of_ceiling", "ceiling_out_ms", "of_ceiling_out",
                                    "round_robin_ms", "round_robin_ms_best") if k in st} or None,
        "per_shape": res.get("per_shape"),
        "step_fused_projections": res.get("step_fused"),
        "launch_floor": res.get("launch_floor"),
        "ceiling_1GiB": res.get("ceiling_1GiB"),
        "ceiling_sizes": res.get("ceiling_sizes"),
        "ceiling_fit": res.get("ceiling_fit"),
        "settle": res.get("settle"),
        "moe": res.get("moe"),
        "vq": res.get("vq"),
        "skinny": res.get("skinny"),
        "eager_ms_per_step": round(st.get("eager_ms", 0.0), 3) if st else None,
        "wall_s": round(time.time() - t_start, 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
