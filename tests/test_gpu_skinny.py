"""Config 2: the batched skinny int4 GEMM at its own shapes, W 28672 x 8192
(70B-class FFN up) and 8192 x 28672 (down), group 64, X fp16 [B][K] ~ N(0, 1),
for B in {1, 2, 3, 4, 8, 16}, on the vector path, the matrix-core path and AUTO,
each against the fp64 oracle through the C ABI.

The batch-B oracle is the batch-1 oracle applied per row of X (no reference
kernel takes a batch), so the fp64 result at B = 16 is computed once per
shape and its first B rows are the expected output at B.

Bar: |got - ref| <= 1e-2 + 1e-3 |ref| (fp16 y, fp32 accumulation) and the
reference harness's max|d| / max|ref| < 2e-3 (int4-gemv/src/main.mm:475-479).
"""
import numpy as np
import pytest
import torch

import oracle
from kernels_amd import gen, kq
from tests._util import assert_close, dev, inf_rel, to_f64

pytestmark = pytest.mark.gpu

SHAPES = [(28672, 8192), (8192, 28672)]
BATCHES = [1, 2, 3, 4, 8, 16]
PATHS = {"valu": kq.PATH_VALU, "mfma": kq.PATH_MFMA, "auto": kq.PATH_AUTO}


@pytest.fixture(scope="module", params=SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def problem(request, gpu):
    M, K = request.param
    p = gen.int4_problem(M, K, 64, batch=16, seed=M // 7 + K)
    ref = oracle.int4_gemv(p["W"], p["SB"], None, p["X"], M, K, 64, 1)  # [16][M]
    bufs = dict(W=dev(p["W"], gpu), SB=dev(p["SB"], gpu), X=dev(p["X"], gpu))
    yield M, K, bufs, ref
    del bufs
    torch.cuda.empty_cache()


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("batch", BATCHES)
def test_config2_skinny(problem, batch, path):
    M, K, b, ref = problem
    Y = torch.full((batch, M), float("nan"), dtype=torch.float16, device=b["W"].device)
    kq.int4_gemv(b["W"], b["SB"], b["X"][:batch], Y, kq.GemvParams(M, K, 64), batch=batch,
                 path=PATHS[path])
    torch.cuda.synchronize()
    got = to_f64(Y)
    what = f"{M}x{K} batch {batch} path {path}"
    assert_close(got, ref[:batch], what=what)
    assert inf_rel(got, ref[:batch]) < 2e-3, what
