"""Re-entrancy across streams and host threads, through the C ABI: the same
calls issued on two default-priority streams at once (interleaved from one
thread, and from two host threads each with its own stream) give, bit for
bit, what they give one after another on one stream. Covers the int4 vector
and matrix-core paths, VQ, and the MoE block (three launches, each stream
with its own workspace) -- the library keeps no mutable state a call could
share with another."""
import threading

import numpy as np
import pytest
import torch

from kernels_amd import gen, kq
from tests._util import dev

pytestmark = pytest.mark.gpu


class Work:
    """One independent set of calls with its own inputs and outputs."""

    def __init__(self, gpu, seed, pool, d):
        p = gen.int4_problem(4096, 4096, 64, batch=1, seed=seed)
        self.gemv = (dev(p["W"], gpu), dev(p["SB"], gpu), dev(p["X"], gpu))
        pm = gen.int4_problem(2048, 4096, 64, batch=8, seed=seed + 1)
        self.mfma = (dev(pm["W"], gpu), dev(pm["SB"], gpu), dev(pm["X"], gpu))
        q = gen.vq_problem(4096, 4096, rows_per_cb=256, seed=seed + 2)
        self.vq = tuple(dev(q[k], gpu) for k in ("IDX", "C", "S", "X"))
        R, X = gen.moe_inputs(d.n_experts, batch=3, seed=seed + 3)
        self.moe_in = (dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16))
        self.pool, self.d = pool, d
        self.y1 = torch.empty((1, 4096), dtype=torch.float16, device=gpu)
        self.y8 = torch.empty((8, 2048), dtype=torch.float16, device=gpu)
        self.yv = torch.empty((1, 4096), dtype=torch.float16, device=gpu)
        self.idx = torch.zeros((3, d.top_k), dtype=torch.int32, device=gpu)
        self.wgt = torch.zeros((3, d.top_k), dtype=torch.float32, device=gpu)
        self.H = torch.zeros((3, d.top_k, d.inter), dtype=torch.float16, device=gpu)
        self.ym = torch.zeros((3, d.hidden), dtype=torch.float32, device=gpu)
        self.wsb = kq.moe_workspace_size(d, 3)
        self.ws = torch.empty(self.wsb, dtype=torch.uint8, device=gpu)
        kq.moe_workspace_init(self.ws, self.wsb)

    def outs(self):
        return (self.y1, self.y8, self.yv, self.idx, self.wgt, self.H, self.ym)

    def clear(self):
        for o in self.outs():
            o.zero_()

    def run(self, stream, reps=3):
        with torch.cuda.stream(stream):
            for _ in range(reps):
                W, SB, X = self.gemv
                kq.int4_gemv(W, SB, X, self.y1, kq.GemvParams(4096, 4096, 64), stream=stream)
                W, SB, X = self.mfma
                kq.int4_gemv(W, SB, X, self.y8, kq.GemvParams(2048, 4096, 64), batch=8,
                             path=kq.PATH_MFMA, stream=stream)
                I, C, S, X = self.vq
                kq.vq_gemv(I, C, S, X, self.yv, kq.VQParams(4096, 4096, 256, 4096), stream=stream)
                R, X = self.moe_in
                kq.moe_block(self.pool, self.d, R, X, self.idx, self.wgt, self.H, self.ym, self.ws,
                             self.wsb, batch=3, stream=stream)


@pytest.fixture(scope="module")
def works(gpu):
    host = gen.moe_pool(16, seed=91, quantize=True)
    pool = dev(host, gpu)
    d = kq.moe_default_desc()
    d.n_experts = 16
    return [Work(gpu, 1000 * (i + 1), pool, d) for i in range(2)]


def reference(works):
    """Every set one after another on one stream."""
    s = torch.cuda.current_stream()
    refs = []
    for w in works:
        w.clear()
        w.run(s, reps=1)
        torch.cuda.synchronize()
        refs.append([o.clone() for o in w.outs()])
    return refs


def check(works, refs, what):
    for i, (w, ref) in enumerate(zip(works, refs)):
        for j, (o, r) in enumerate(zip(w.outs(), ref)):
            assert torch.equal(o, r), f"{what}: set {i} output {j} differs"


def test_two_streams_interleaved(gpu, works):
    refs = reference(works)
    streams = [torch.cuda.Stream() for _ in works]
    for w in works:
        w.clear()
    torch.cuda.synchronize()
    for rep in range(3):  # the two sets' launches interleaved call by call
        for w, s in zip(works, streams):
            w.run(s, reps=1)
    torch.cuda.synchronize()
    check(works, refs, "interleaved streams")


def test_two_host_threads(gpu, works):
    refs = reference(works)
    streams = [torch.cuda.Stream() for _ in works]
    for w in works:
        w.clear()
    torch.cuda.synchronize()
    errors = []

    def body(w, s):
        try:
            torch.cuda.set_device(gpu)
            w.run(s, reps=4)
            s.synchronize()
        except Exception as e:  # reported below, in the test's thread
            errors.append(repr(e))

    threads = [threading.Thread(target=body, args=(w, s)) for w, s in zip(works, streams)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a host thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    check(works, refs, "two host threads")
    ids = works[0].idx.cpu().numpy()
    assert ((ids >= 0) & (ids < 16)).all()
