"""VQ (d=2, 256-entry codebook) dequant-GEMV on the GPU vs the fp64 oracle.
Index lookup is integer work and is pinned bit-exactly by the read-back case;
outputs are held to |d| <= 1e-2 + 1e-3 |ref|."""
import numpy as np
import pytest
import torch

import oracle
from kernels_amd import gen, kq
from tests._util import assert_close, dev, inf_rel, to_f64

pytestmark = pytest.mark.gpu


def run_vq(p, device, y_dtype=torch.float16):
    M, K, batch = p["M"], p["K"], p["batch"]
    Y = torch.full((batch, M), float("nan"), dtype=y_dtype, device=device)
    kq.vq_gemv(dev(p["IDX"], device), dev(p["C"], device), dev(p["S"], device),
               dev(p["X"], device), Y, kq.VQParams(M, K, p["rows_per_cb"], p["scale_group"]),
               batch=batch)
    torch.cuda.synchronize()
    return to_f64(Y)


def ref_vq(p):
    return oracle.vq_gemv(p["IDX"], p["C"], p["S"], p["X"], p["M"], p["K"], p["rows_per_cb"],
                          p["scale_group"])


@pytest.mark.parametrize("M,K", [(14336, 4096), (4096, 14336)])
def test_config3_shapes(gpu, M, K):
    p = gen.vq_problem(M, K, rows_per_cb=256, scale_group=K, seed=M ^ K)
    got, ref = run_vq(p, gpu), ref_vq(p)
    assert_close(got, ref, what=f"vq {M}x{K}")
    assert inf_rel(got, ref) < 2e-3


def test_reference_format(gpu):
    """One codebook per matrix and one scale per 32 weights (the reference's
    layout, vq-gemv/src/kernels.metal:15-19) with its U(-1,1) data."""
    p = gen.vq_problem(2048, 4096, rows_per_cb=2048, scale_group=32, seed=1, dist="ref")
    got, ref = run_vq(p, gpu, torch.float32), ref_vq(p)
    assert_close(got, ref, what="vq ref format")
    assert inf_rel(got, ref) < 2e-3


def test_index_readback_exact(gpu):
    M, K = 300, 512
    rng = np.random.default_rng(0)
    IDX = rng.integers(0, 256, (M, K // 2), dtype=np.uint8)
    C = np.zeros((2, 256, 2), np.uint16)
    C[:, :, 0] = gen.f16_bits(np.arange(256))
    C[1, :, 0] = gen.f16_bits(np.arange(256) + 1000)  # second block offset by 1000
    S = np.full((M, K // 32), gen.f16_bits(1.0), np.uint16)
    for i in (0, 5, 255):
        X = np.zeros((1, K), np.uint16)
        X[0, 2 * i] = gen.f16_bits(1.0)
        p = dict(IDX=IDX, C=C, S=S, X=X, M=M, K=K, rows_per_cb=256, scale_group=32, batch=1)
        got = run_vq(p, gpu, torch.float32)[0]
        want = IDX[:, i].astype(np.float64) + np.where(np.arange(M) >= 256, 1000, 0)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("M,K,rpc,sg,batch", [(1, 512, 1, 32, 1), (257, 1024, 256, 64, 2),
                                              (1000, 2880, 7, 32, 1), (513, 4096, 256, 4096, 3),
                                              (100, 8192, 100, 128, 4),
                                              # short and long: split K over waves + LDS sum
                                              (64, 28672, 64, 32, 1), (130, 14336, 256, 14336, 2),
                                              # scale groups longer than a 2048-weight step
                                              (200, 8192, 256, 4096, 1), (96, 16384, 64, 8192, 2)])
def test_edge_shapes(gpu, M, K, rpc, sg, batch):
    p = gen.vq_problem(M, K, rows_per_cb=rpc, scale_group=sg, batch=batch, seed=M + sg)
    assert_close(run_vq(p, gpu), ref_vq(p), what=f"vq M={M} K={K} rpc={rpc} sg={sg} b={batch}")
