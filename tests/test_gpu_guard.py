"""Out-of-bounds guard for the GEMV kernels on the GPU through the C ABI.

y (and xsum32's output) sits between 4 KiB guard bands of 0xA5; after the
call the bands must be untouched and every output element written (no NaN
left of the NaN fill), across the int4 vector, matrix-core, scalar and
automatic paths, forced launch plans, short and ragged shapes, 1-16 tokens,
and the VQ kernel in both formats."""
import numpy as np
import pytest
import torch

from kernels_amd import gen, kq
from tests._util import dev
from tests.test_gpu_moe_guard import Guarded

pytestmark = pytest.mark.gpu

SHAPES = [(33, 4096), (1024, 4096), (70, 14336), (1031, 2048), (4096, 14336), (100, 320)]


@pytest.mark.parametrize("path", [kq.PATH_AUTO, kq.PATH_VALU, kq.PATH_MFMA, kq.PATH_SCALAR])
@pytest.mark.parametrize("M,K", SHAPES)
@pytest.mark.parametrize("batch", [1, 3, 16])
def test_int4_guard(gpu, path, M, K, batch):
    if path == kq.PATH_MFMA and K % 128:
        pytest.skip("the matrix-core path needs K % 128 == 0")
    if path == kq.PATH_SCALAR and M * K > 1024 * 4096:
        pytest.skip("the debug scalar path is exercised on the small shapes")
    p = gen.int4_problem(M, K, 64, batch=batch, seed=M + K + batch)
    y = Guarded((batch, M), torch.float16, gpu, float("nan"))
    kq.int4_gemv(dev(p["W"], gpu), dev(p["SB"], gpu), dev(p["X"], gpu), y.t,
                 kq.GemvParams(M, K, 64), batch=batch, path=path)
    torch.cuda.synchronize()
    assert y.intact(), f"y guard band written ({M}x{K}, batch {batch}, path {path})"
    assert torch.isfinite(y.t).all(), f"y element not written ({M}x{K}, batch {batch})"


@pytest.mark.parametrize("rows,unroll", [(1, 2), (1, 4), (1, 8), (7, 2), (7, 4)])
def test_int4_guard_forced_plans(gpu, rows, unroll):
    """Forced vector-path plans at 4096x14336, 2 tokens: K parts (a divisor of
    the 7 steps of 2048 k) x ring depth."""
    M, K, batch = 4096, 14336, 2
    p = gen.int4_problem(M, K, 64, batch=batch, seed=5)
    y = Guarded((batch, M), torch.float32, gpu, float("nan"))
    kq.int4_gemv(dev(p["W"], gpu), dev(p["SB"], gpu), dev(p["X"], gpu), y.t,
                 kq.GemvParams(M, K, 64), batch=batch, path=kq.PATH_VALU, rows=rows, unroll=unroll)
    torch.cuda.synchronize()
    assert y.intact() and torch.isfinite(y.t).all()


@pytest.mark.parametrize("K,batch", [(32, 1), (4096, 3), (14336, 2)])
def test_xsum32_guard(gpu, K, batch):
    x = torch.randn((batch, K), device=gpu).half()
    xs = Guarded((batch, K // 32), torch.float32, gpu, float("nan"))
    kq.xsum32(x, xs.t, K, batch)
    torch.cuda.synchronize()
    assert xs.intact() and torch.isfinite(xs.t).all()


@pytest.mark.parametrize("M,K,rows_per_cb,sg", [(14336, 4096, 256, 4096), (4096, 14336, 256, 14336),
                                                (300, 2048, 300, 32), (1000, 512, 256, 32)])
@pytest.mark.parametrize("batch", [1, 4])
def test_vq_guard(gpu, M, K, rows_per_cb, sg, batch):
    q = gen.vq_problem(M, K, rows_per_cb=rows_per_cb, scale_group=sg, batch=batch, seed=M + K)
    y = Guarded((batch, M), torch.float16, gpu, float("nan"))
    kq.vq_gemv(dev(q["IDX"], gpu), dev(q["C"], gpu), dev(q["S"], gpu), dev(q["X"], gpu), y.t,
               kq.VQParams(M, K, rows_per_cb, sg), batch=batch)
    torch.cuda.synchronize()
    assert y.intact(), f"VQ y guard band written ({M}x{K}, batch {batch})"
    assert torch.isfinite(y.t).all()
