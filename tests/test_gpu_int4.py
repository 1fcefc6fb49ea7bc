"""int4 GEMV / skinny GEMM on the GPU through libkq's C ABI vs the fp64 oracle.

Bar: fp16 (or fp32) outputs with fp32 accumulation within
|got - ref| <= 1e-2 + 1e-3 |ref|; the reference harness's own metric
max|d| / max|ref| < 2e-3 (int4-gemv/src/main.mm:475-479) is asserted too.
"""
import numpy as np
import pytest
import torch

import oracle
from kernels_amd import gen, kq
from tests._util import assert_close, dev, inf_rel, to_f64

pytestmark = pytest.mark.gpu


def run_int4(p, device, layout="sb", sb_dtype=kq.F16, y_dtype=torch.float16, path=kq.PATH_AUTO,
             rows=0, unroll=0, S=None, B=None):
    M, K, G, batch = p["M"], p["K"], p["G"], p["batch"]
    W = dev(p["W"], device)
    X = dev(p["X"], device)
    if layout == "sb":
        Sd, Bd = dev(p["SB"] if S is None else S, device), None
    else:
        Sd, Bd = dev(p["S"] if S is None else S, device), dev(p["B"] if B is None else B, device)
    Y = torch.full((batch, M), float("nan"), dtype=y_dtype, device=device)
    kq.int4_gemv(W, Sd, X, Y, kq.GemvParams(M, K, G), B=Bd, batch=batch, sb_dtype=sb_dtype,
                 path=path, rows=rows, unroll=unroll)
    torch.cuda.synchronize()
    return to_f64(Y)


def ref_int4(p, layout="sb", sb_dtype=oracle.F16, S=None, B=None):
    if layout == "sb":
        return oracle.int4_gemv(p["W"], p["SB"] if S is None else S, None, p["X"], p["M"], p["K"],
                                p["G"], 1, sb_dtype)
    return oracle.int4_gemv(p["W"], p["S"] if S is None else S, p["B"] if B is None else B, p["X"],
                            p["M"], p["K"], p["G"], 0, sb_dtype)


def check(got, ref, what):
    assert_close(got, ref, what=what)
    assert inf_rel(got, ref) < 2e-3, what


def test_config0_4096x4096(gpu):
    p = gen.int4_problem(4096, 4096, 64, seed=12345)
    ref = ref_int4(p)
    got = run_int4(p, gpu)
    check(got, ref, "4096x4096 fp16 y")
    print(f"config0 inf-rel err {inf_rel(got, ref):.2e}")


PATHS = [kq.PATH_VALU, kq.PATH_MFMA]


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("M,K", [(1024, 4096), (14336, 4096), (4096, 14336)])
def test_llama_layer_shapes(gpu, M, K, path):
    p = gen.int4_problem(M, K, 64, seed=M + K)
    check(run_int4(p, gpu, path=path), ref_int4(p), f"{M}x{K} path {path}")


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("layout", ["sb", "split"])
@pytest.mark.parametrize("ydt", [torch.float16, torch.float32])
def test_layouts_and_output_dtype(gpu, layout, ydt, path):
    p = gen.int4_problem(1000, 2048, 64, seed=7, dist="ref")
    check(run_int4(p, gpu, layout=layout, y_dtype=ydt, path=path), ref_int4(p, layout),
          f"{layout} {ydt} path {path}")


@pytest.mark.parametrize("path", PATHS)
def test_bf16_metadata(gpu, path):
    p = gen.int4_problem(512, 1024, 64, seed=3)
    rng = np.random.default_rng(0)
    S = gen.bf16_bits(np.abs(rng.normal(0, 0.02, (512, 16))))
    B = gen.bf16_bits(rng.normal(0, 0.02, (512, 16)))
    SB = np.ascontiguousarray(np.stack([S, B], -1))
    ref = oracle.int4_gemv(p["W"], S, B, p["X"], 512, 1024, 64, 0, oracle.BF16)
    check(run_int4(p, gpu, layout="split", sb_dtype=kq.BF16, S=S, B=B, path=path), ref,
          "bf16 split")
    check(run_int4(p, gpu, layout="sb", sb_dtype=kq.BF16, S=SB, path=path), ref, "bf16 sb")


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("G", [32, 64, 128])
@pytest.mark.parametrize("M,K", [(1, 512), (7, 4096), (4097, 1024), (300, 2880), (65, 32 * 64),
                                 (33, 28672), (2, 32)])
def test_edge_shapes_and_groups(gpu, M, K, G, path):
    if K % G:
        pytest.skip("K % G")
    if path == kq.PATH_MFMA and K % 128:
        pytest.skip("matrix-core path needs K % 128 == 0")
    p = gen.int4_problem(M, K, G, seed=M * 31 + K + G)
    check(run_int4(p, gpu, path=path), ref_int4(p), f"M={M} K={K} G={G} path {path}")


@pytest.mark.parametrize("batch", [2, 3, 4, 5, 8, 16])
def test_batched_valu(gpu, batch):
    p = gen.int4_problem(777, 4096, 64, batch=batch, seed=batch)
    check(run_int4(p, gpu, path=kq.PATH_VALU), ref_int4(p), f"valu batch {batch}")


# (K parts, ring depth) per K: parts divide the 1 KiB steps of a row
# (8192: 4 steps; 2880: 2 steps, the last one partial; 28672: 14 steps)
VALU_PLANS = [(8192, 1, 2), (8192, 1, 8), (8192, 2, 4), (8192, 4, 2), (8192, 4, 8),
              (8192, 1, 16), (2880, 1, 4), (2880, 2, 2), (2880, 2, 8), (2880, 1, 16),
              (28672, 1, 8), (28672, 2, 4), (28672, 7, 2), (28672, 14, 8), (28672, 1, 16)]


@pytest.mark.parametrize("K,parts,depth", VALU_PLANS)
@pytest.mark.parametrize("M,batch", [(1031, 1), (70, 2), (257, 4)])
def test_forced_launch_shapes_agree(gpu, K, parts, depth, M, batch):
    """Every (K parts, ring depth) plan of the vector path gives the oracle's
    answer: split-K with the LDS reduction, padding items, a partial last
    step (zero-padded x) and idle row lanes included. At 4 tokens a ring
    deeper than 4 takes passes of fewer tokens."""
    p = gen.int4_problem(M, K, 64, batch=batch, seed=11 + K + parts)
    got = run_int4(p, gpu, path=kq.PATH_VALU, rows=parts, unroll=depth)
    check(got, ref_int4(p), f"P={parts} D={depth} K={K} M={M} b={batch}")


@pytest.mark.parametrize("parts,depth,batch", [(2, 2, 1), (2, 4, 2), (4, 2, 1), (1, 16, 1),
                                               (2, 16, 1), (1, 8, 2), (2, 2, 3), (2, 4, 4),
                                               (4, 2, 4), (1, 4, 3), (4, 4, 7)])
def test_forced_kparts_many_rounds(gpu, parts, depth, batch):
    """K parts over several rounds of row groups per workgroup: every
    round's partial sums wait in LDS until the one reduction at the end."""
    p = gen.int4_problem(9000, 8192, 64, batch=batch, seed=5 + parts + depth)
    got = run_int4(p, gpu, path=kq.PATH_VALU, rows=parts, unroll=depth)
    check(got, ref_int4(p), f"P={parts} D={depth} M=9000 b={batch}")


# (K parts P, 10 * tiles per wave T + ring depth: 2 at T = 1 and 4, 4 at T = 2; 0 = automatic T)
MFMA_PLANS = [(16, 12), (1, 12), (8, 24), (2, 24), (4, 42), (8, 42), (1, 42), (4, 0)]


@pytest.mark.parametrize("parts,unroll", MFMA_PLANS)
@pytest.mark.parametrize("M,batch", [(1000, 1), (257, 5), (9600, 3)])
def test_mfma_forced_plans_agree(gpu, parts, unroll, M, batch):
    """Every (K parts, tiles per wave) plan of the matrix-core path gives the
    oracle's result: parts padded to whole scale/bias windows (P = 16: 2
    spans per part, 6 padding steps), clamped rows, idle lanes and several
    rounds per workgroup (M = 9600: 600 tiles) included (K = 4096: 32
    spans)."""
    p = gen.int4_problem(M, 4096, 64, batch=batch, seed=parts * 100 + unroll + M)
    got = run_int4(p, gpu, path=kq.PATH_MFMA, rows=parts, unroll=unroll)
    check(got, ref_int4(p), f"mfma P={parts} T,D={unroll} M={M} b={batch}")


@pytest.mark.parametrize("G", [32, 128])
@pytest.mark.parametrize("layout", ["sb", "split"])
@pytest.mark.parametrize("parts", [1, 8])
def test_mfma_two_tiles_deep_ring(gpu, G, layout, parts):
    """Two tiles a wave stream through a 4-deep ring (two span pairs ahead,
    the scale/bias window loaded 4 steps before its first span): other group
    sizes, both scale/bias layouts, 16 tokens, padding steps (P = 8: 4 spans
    per part, padded to 8) and two rounds per workgroup (P = 8: one row-group
    lane)."""
    p = gen.int4_problem(9000, 4096, G, batch=16, seed=G + parts)
    got = run_int4(p, gpu, layout=layout, path=kq.PATH_MFMA, rows=parts, unroll=24)
    check(got, ref_int4(p, layout), f"mfma T=2 G={G} {layout} P={parts}")


def test_mfma_forced_plan_unsupported(gpu):
    p = gen.int4_problem(64, 4096, 64, seed=3)
    with pytest.raises(kq.KQError) as e:
        run_int4(p, gpu, path=kq.PATH_MFMA, rows=3, unroll=12)  # 3 does not divide 32 spans
    assert e.value.status == kq.KQ_EUNSUPPORTED
    with pytest.raises(kq.KQError) as e:
        run_int4(p, gpu, path=kq.PATH_MFMA, rows=16, unroll=42)  # T = 4 has 8 waves
    assert e.value.status == kq.KQ_EUNSUPPORTED
    with pytest.raises(kq.KQError) as e:
        run_int4(p, gpu, path=kq.PATH_MFMA, rows=4, unroll=13)  # ring depth is 2
    assert e.value.status == kq.KQ_EUNSUPPORTED
    with pytest.raises(kq.KQError) as e:
        run_int4(p, gpu, path=kq.PATH_MFMA, rows=4, unroll=22)  # T = 2 has ring depth 4
    assert e.value.status == kq.KQ_EUNSUPPORTED


@pytest.mark.parametrize("layout,sb", [("sb", kq.F16), ("split", kq.F16), ("split", kq.BF16)])
@pytest.mark.parametrize("M,K,G,batch", [(777, 4096, 64, 1), (129, 2880, 32, 3), (64, 32768, 128, 2),
                                         (4096, 14336, 64, 1)])
def test_scalar_debug_path(gpu, layout, sb, M, K, G, batch):
    """The debug scalar kernel (v0's one-thread-per-row loop) against the
    oracle, and the vector path against it (K = 32768: past the vector
    path's LDS bound, which only the scalar kernel takes)."""
    p = gen.int4_problem(M, K, G, batch=batch, seed=M + K + G)
    if sb == kq.BF16:
        rng = np.random.default_rng(M)
        S = gen.bf16_bits(np.abs(rng.normal(0, 0.02, (M, K // G))))
        B = gen.bf16_bits(rng.normal(0, 0.02, (M, K // G)))
        ref = oracle.int4_gemv(p["W"], S, B, p["X"], M, K, G, 0, oracle.BF16)
        got = run_int4(p, gpu, layout="split", sb_dtype=kq.BF16, S=S, B=B, path=kq.PATH_SCALAR)
    else:
        ref = ref_int4(p, layout)
        got = run_int4(p, gpu, layout=layout, path=kq.PATH_SCALAR)
    check(got, ref, f"scalar {layout} {M}x{K} G{G} b{batch}")
    if K <= 29120 and sb == kq.F16:
        fast = run_int4(p, gpu, layout=layout, path=kq.PATH_VALU)
        assert_close(fast, got, what="vector path vs scalar")
