"""The GEMV kernels inside HIP graphs, the way bench.py times them: a graph of
several launches (the int4 vector and matrix-core paths, K parts, the VQ
GEMV) replayed several times, with eager work and synchronisations between
the replays. Every replay must equal the eager result bit for bit (the
kernels are deterministic and keep no state between calls), and the eager
result is checked against the fp64 oracle."""
import numpy as np
import pytest
import torch

import oracle
from kernels_amd import gen, kq
from tests._util import assert_close, dev, to_f64

pytestmark = pytest.mark.gpu


def replay_check(fn, outs, reps=4):
    fn()
    torch.cuda.synchronize()
    ref = [o.clone() for o in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for rep in range(reps):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i, (o, r) in enumerate(zip(outs, ref)):
            assert torch.equal(o, r), f"replay {rep} output {i}"
        fn()  # eager work between replays
        torch.cuda.synchronize()
    return ref


def test_int4_paths_in_one_graph(gpu):
    """A vector-path GEMV (batch 1), a forced K-part plan, and a matrix-core
    GEMM (batch 8), captured together."""
    a = gen.int4_problem(4096, 14336, 64, batch=1, seed=1)
    b = gen.int4_problem(2048, 8192, 64, batch=8, seed=2)
    Wa, SBa, Xa = dev(a["W"], gpu), dev(a["SB"], gpu), dev(a["X"], gpu)
    Wb, SBb, Xb = dev(b["W"], gpu), dev(b["SB"], gpu), dev(b["X"], gpu)
    Ya = torch.empty((1, 4096), dtype=torch.float16, device=gpu)
    Yk = torch.empty((1, 4096), dtype=torch.float32, device=gpu)
    Yb = torch.empty((8, 2048), dtype=torch.float16, device=gpu)

    def fn():
        kq.int4_gemv(Wa, SBa, Xa, Ya, kq.GemvParams(4096, 14336, 64))
        kq.int4_gemv(Wa, SBa, Xa, Yk, kq.GemvParams(4096, 14336, 64), path=kq.PATH_VALU, rows=7,
                     unroll=2)
        kq.int4_gemv(Wb, SBb, Xb, Yb, kq.GemvParams(2048, 8192, 64), batch=8,
                     path=kq.PATH_MFMA)
    ya, yk, yb = replay_check(fn, [Ya, Yk, Yb])
    ra = oracle.int4_gemv(a["W"], a["SB"], None, a["X"], 4096, 14336, 64, 1)
    rb = oracle.int4_gemv(b["W"], b["SB"], None, b["X"], 2048, 8192, 64, 1)
    assert_close(to_f64(ya), ra, what="vector")
    assert_close(to_f64(yk), ra, what="vector, 7 K parts")
    assert_close(to_f64(yb), rb, what="matrix cores")


def test_vq_in_a_graph(gpu):
    p = gen.vq_problem(14336, 4096, rows_per_cb=256, seed=3)
    IDX, C, S, X = (dev(p[k], gpu) for k in ("IDX", "C", "S", "X"))
    Y = torch.empty((1, 14336), dtype=torch.float16, device=gpu)

    def fn():
        kq.vq_gemv(IDX, C, S, X, Y, kq.VQParams(14336, 4096, 256, 4096))
    (y,) = replay_check(fn, [Y])
    ref = oracle.vq_gemv(p["IDX"], p["C"], p["S"], p["X"], 14336, 4096, 256, 4096)
    assert_close(to_f64(y), ref, what="vq")
