"""The one-launch MoE block (KQ_MOE_PATH_ONE, one token) on the GPU through
the C ABI: bit-identical to the three-launch block (idx, wgt, H, xh and y
compared as bits), against the fp64 oracle (routing exact, y within the
block tests' bar), with the workspace's error word still 0 after every call
(no grid-barrier wait gave up)."""
import numpy as np
import pytest
import torch

import oracle
from kernels_amd import gen, kq
from tests._util import assert_close, dev, inf_rel, to_f64
from tests.test_gpu_moe import Block, _compact_desc, _pool_desc, odesc, routing_margin

pytestmark = pytest.mark.gpu


def err_word(b):
    return kq.moe_workspace_error(b.ws, b.wsb)


def test_workspace_error_query(gpu):
    """kq_moe_workspace_error reads the word a give-up would set and clears
    it on request; the word is set here from the host (no wait is made to
    give up)."""
    d = kq.moe_default_desc()
    b = Block(gpu, d, 1)
    assert kq.moe_workspace_error(b.ws, b.wsb) == 0
    b.ws[kq.MOE_WS_ERR_OFFSET:kq.MOE_WS_ERR_OFFSET + 4].copy_(
        torch.from_numpy(np.array([0x1234], np.uint32).view(np.uint8)).to(gpu))
    assert kq.moe_workspace_error(b.ws, b.wsb) == 0x1234  # read, not cleared
    assert kq.moe_workspace_error(b.ws, b.wsb, clear=True) == 0x1234
    assert kq.moe_workspace_error(b.ws, b.wsb) == 0
    with pytest.raises(kq.KQError):
        kq.moe_workspace_error(b.ws, 64)


def run(pool, d, Rd, Xd, b, path, xh=True):
    b.y.fill_(float("nan"))
    b.H.zero_()
    b.idx.fill_(-1)
    kq.moe_block(pool, d, Rd, Xd, b.idx, b.wgt, b.H, b.y, b.ws, b.wsb, batch=1,
                 xh=b.xh if xh else None, path=path)
    torch.cuda.synchronize()
    out = {"idx": b.idx.clone(), "wgt": b.wgt.clone(), "H": b.H.clone(), "y": b.y.clone()}
    if b.xh is not None:
        out["xh"] = b.xh.clone()
    return out


def assert_same(a, b, what):
    for k in a:
        assert torch.equal(a[k], b[k]), f"{what}: {k} differs"


@pytest.fixture(scope="module")
def pool16(gpu):
    host = gen.moe_pool(16, seed=31, quantize=True)
    return host, dev(host, gpu)


def test_one_launch_full_pool(gpu):
    """128 experts of gpt-oss-120b shape, fp16 router and x, three calls in a
    row on one workspace (the barrier counters carry over)."""
    host = gen.moe_pool(128, seed=55, quantize=False)
    pool = dev(host, gpu)
    d = kq.moe_default_desc()
    R, X = gen.moe_inputs(128, batch=1, seed=10)
    oidx, owgt, lg = oracle.moe_router(R, oracle.F16, X, oracle.F16, 1, odesc(d))
    assert routing_margin(lg, 4) > 1e-4
    _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F16, X, oracle.F16, 1)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    b3, b1 = Block(gpu, d, 1), Block(gpu, d, 1)
    ref = run(pool, d, Rd, Xd, b3, kq.MOE_PATH_LAUNCHES)
    for rep in range(3):
        got = run(pool, d, Rd, Xd, b1, kq.MOE_PATH_ONE)
        assert err_word(b1) == 0
        assert_same(got, ref, f"rep {rep}")
        assert np.array_equal(got["idx"].cpu().numpy().astype(np.uint32), oidx)
        assert np.allclose(got["wgt"].cpu().numpy(), owgt, atol=1e-6)
        y = to_f64(got["y"])
        assert_close(y, Yref, what=f"one-launch rep {rep}")
        assert inf_rel(y, Yref) < 2e-3
    del pool


def test_one_launch_fp32_inputs_fp16_out(gpu, pool16):
    """fp32 router and x (xh = half(x) written), fp16 y."""
    host, pool = pool16
    d = _pool_desc(16)
    rng = np.random.default_rng(21)
    R = rng.normal(0, 0.02, (16, 2880)).astype(np.float32)
    X = rng.normal(0, 1, (1, 2880)).astype(np.float32)
    oidx, _, lg = oracle.moe_router(R, oracle.F32, X, oracle.F32, 1, odesc(d))
    assert routing_margin(lg, 4) > 1e-4
    Rd, Xd = torch.from_numpy(R).to(gpu), torch.from_numpy(X).to(gpu)
    b3 = Block(gpu, d, 1, x_f32=True, y_dtype=torch.float16)
    b1 = Block(gpu, d, 1, x_f32=True, y_dtype=torch.float16)
    ref = run(pool, d, Rd, Xd, b3, kq.MOE_PATH_LAUNCHES)
    got = run(pool, d, Rd, Xd, b1, kq.MOE_PATH_ONE)
    assert err_word(b1) == 0
    assert_same(got, ref, "fp32 inputs")
    assert np.array_equal(got["idx"].cpu().numpy().astype(np.uint32), oidx)
    _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F32, X, oracle.F32, 1)
    assert inf_rel(to_f64(got["y"]), Yref) < 2e-3


# every chunk count of the kernel (J = 1..4), partial chunks, top-2..4
@pytest.mark.parametrize("hidden,inter,top_k", [(1024, 1024, 3), (1536, 1536, 4), (2048, 2048, 2),
                                                (3072, 3072, 4), (2880, 2816, 4), (4096, 4096, 2)])
def test_one_launch_other_shapes(gpu, hidden, inter, top_k):
    d, off = _compact_desc(hidden, inter, 16, top_k)
    host = gen.moe_pool(16, seed=hidden + inter + top_k, quantize=True, hidden=hidden, inter=inter,
                        blob=d.blob, off=off)
    pool = dev(host, gpu)
    R, X = gen.moe_inputs(16, hidden=hidden, batch=1, seed=inter + top_k)
    oidx, _, lg = oracle.moe_router(R, oracle.F16, X, oracle.F16, 1, odesc(d))
    assert routing_margin(lg, top_k) > 1e-5
    _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F16, X, oracle.F16, 1)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    b3, b1 = Block(gpu, d, 1), Block(gpu, d, 1)
    ref = run(pool, d, Rd, Xd, b3, kq.MOE_PATH_LAUNCHES)
    got = run(pool, d, Rd, Xd, b1, kq.MOE_PATH_ONE)
    assert err_word(b1) == 0
    assert_same(got, ref, f"{hidden}x{inter} top-{top_k}")
    assert np.array_equal(got["idx"].cpu().numpy().astype(np.uint32), oidx)
    assert_close(to_f64(got["y"]), Yref, what=f"one-launch {hidden}x{inter}")


def test_one_launch_graph_replays(gpu, pool16):
    """Captured in a HIP graph: every replay, with eager one-launch and
    three-launch blocks on the same workspace in between, equals the eager
    result bit for bit."""
    host, pool = pool16
    d = _pool_desc(16)
    R, X = gen.moe_inputs(16, batch=1, seed=81)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    b = Block(gpu, d, 1)
    ref = run(pool, d, Rd, Xd, b, kq.MOE_PATH_ONE)

    def block():
        kq.moe_block(pool, d, Rd, Xd, b.idx, b.wgt, b.H, b.y, b.ws, b.wsb, batch=1,
                     path=kq.MOE_PATH_ONE)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        block()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        block()
    for rep in range(4):
        b.y.fill_(float("nan"))
        b.idx.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(b.idx, ref["idx"]) and torch.equal(b.y, ref["y"]), f"replay {rep}"
        got = run(pool, d, Rd, Xd, b, kq.MOE_PATH_ONE if rep % 2 else kq.MOE_PATH_LAUNCHES)
        assert_same(got, ref, f"eager after replay {rep}")
    assert err_word(b) == 0


def test_one_launch_workspace_shared_with_larger_batches(gpu, pool16):
    """A workspace sized for 8 tokens: one-launch single tokens and 8-token
    blocks in turn, each against the oracle."""
    host, pool = pool16
    d = _pool_desc(16)
    b8 = Block(gpu, d, 8)
    for rep, batch in enumerate([1, 8, 1, 8, 1]):
        R, X = gen.moe_inputs(16, batch=batch, seed=90 + rep)
        oidx, _, _ = oracle.moe_router(R, oracle.F16, X, oracle.F16, batch, odesc(d))
        _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F16, X, oracle.F16, batch)
        y = torch.full((batch, d.hidden), float("nan"), dtype=torch.float32, device=gpu)
        kq.moe_block(pool, d, dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16),
                     b8.idx[:batch], b8.wgt[:batch], b8.H[:batch], y, b8.ws, b8.wsb, batch=batch,
                     path=kq.MOE_PATH_ONE if batch == 1 else kq.MOE_PATH_AUTO)
        torch.cuda.synchronize()
        assert np.array_equal(b8.idx[:batch].cpu().numpy().astype(np.uint32), oidx)
        assert_close(to_f64(y), Yref, what=f"shared workspace rep {rep} batch {batch}")
    assert err_word(b8) == 0


def test_one_launch_unsupported(gpu, pool16):
    _, pool = pool16
    d = _pool_desc(16)
    R, X = gen.moe_inputs(16, batch=2, seed=5)
    b = Block(gpu, d, 2)
    with pytest.raises(kq.KQError) as e:
        kq.moe_block(pool, d, dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16),
                     b.idx, b.wgt, b.H, b.y, b.ws, b.wsb, batch=2, path=kq.MOE_PATH_ONE)
    assert e.value.status == kq.KQ_EUNSUPPORTED
    dd, _ = _compact_desc(1024, 2048, 16, 3)  # hidden and inter of different step counts
    b1 = Block(gpu, dd, 1)
    R, X = gen.moe_inputs(16, hidden=1024, batch=1, seed=6)
    with pytest.raises(kq.KQError) as e:
        kq.moe_block(pool, dd, dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16),
                     b1.idx, b1.wgt, b1.H, b1.y, b1.ws, b1.wsb, batch=1, path=kq.MOE_PATH_ONE)
    assert e.value.status == kq.KQ_EUNSUPPORTED
