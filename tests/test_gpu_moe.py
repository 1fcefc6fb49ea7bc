"""MoE block (router top-k, gathered gate/up + SwiGLU, gathered down +
combine) on the GPU through libkq's C ABI vs the fp64 oracle.

Routing is held bit-exact (indices equal, and order); softmax weights within
1e-6; h and y within |d| <= 1e-2 + 1e-3 |ref|, plus the reference's own
max|d| / max|y| < 2e-3 (moe-fused/src/main.mm:356-375)."""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from kernels_amd import gen, kq
from tests._util import assert_close, dev, host_bits, inf_rel, to_f64

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def odesc(d):
    o = oracle.MoEDesc()
    for f, _ in kq.MoEDesc._fields_:
        setattr(o, f, getattr(d, f))
    return o


class Block:
    """Device buffers for one block call."""

    def __init__(self, device, d, batch, x_f32=False, y_dtype=torch.float32):
        self.d, self.batch = d, batch
        self.idx = torch.zeros((batch, d.top_k), dtype=torch.int32, device=device)
        self.wgt = torch.zeros((batch, d.top_k), dtype=torch.float32, device=device)
        self.H = torch.zeros((batch, d.top_k, d.inter), dtype=torch.float16, device=device)
        self.y = torch.full((batch, d.hidden), float("nan"), dtype=y_dtype, device=device)
        self.xh = torch.zeros((batch, d.hidden), dtype=torch.float16, device=device) if x_f32 else None
        self.wsb = kq.moe_workspace_size(d, batch)
        self.ws = torch.empty(self.wsb, dtype=torch.uint8, device=device)
        kq.moe_workspace_init(self.ws, self.wsb)


@pytest.fixture(scope="module")
def pool16(gpu):
    """16 experts of real gpt-oss shape, weights quantised from N(0, 0.02)."""
    host = gen.moe_pool(16, seed=31, quantize=True)
    return host, dev(host, gpu)


def routing_margin(lg, k):
    s = np.sort(lg, axis=-1)[..., ::-1]
    return float(np.min(s[..., k - 1] - s[..., k]))


def test_router_golden_lcg(gpu):
    """moe-fused/results/topk.txt reproduced on the GPU (fp32 R and x)."""
    spec = json.load(open(os.path.join(GOLD, "moe_topk_lcg.json")))
    d = kq.moe_default_desc()
    R, X = gen.moe_lcg_inputs()
    b = Block(gpu, d, 1, x_f32=True)
    Rd = torch.from_numpy(R).to(gpu)
    Xd = torch.from_numpy(X).to(gpu)
    kq.moe_router_topk(Rd, Xd, b.idx, b.wgt, d, b.ws, b.wsb, batch=1, xh=b.xh)
    torch.cuda.synchronize()
    assert b.idx.cpu().tolist()[0] == spec["expected_idx"]
    assert np.allclose(b.wgt.cpu().numpy()[0], spec["expected_wgt"], atol=1e-6, rtol=0)
    assert np.array_equal(host_bits(b.xh, np.uint16), X.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("batch", [1, 3, 8, 16])
def test_router_fp16_exact(gpu, batch):
    d = kq.moe_default_desc()
    R, X = gen.moe_inputs(128, batch=batch, seed=100 + batch)
    idx, wgt, lg = oracle.moe_router(R, oracle.F16, X, oracle.F16, batch, odesc(d))
    assert routing_margin(lg, 4) > 1e-4, "test data too close to a tie"
    b = Block(gpu, d, batch)
    kq.moe_router_topk(dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16), b.idx,
                       b.wgt, d, b.ws, b.wsb, batch=batch)
    torch.cuda.synchronize()
    assert np.array_equal(b.idx.cpu().numpy().astype(np.uint32), idx)
    assert np.allclose(b.wgt.cpu().numpy(), wgt, atol=1e-6, rtol=0)


def test_router_ties_lowest_index(gpu):
    """Exactly tied logits: the lowest expert index wins (strict > scan)."""
    d = kq.moe_default_desc()
    d.n_experts, d.top_k = 16, 4
    R = np.zeros((16, 2880), np.float32)
    R[[3, 9, 12], 0] = 2.0          # three-way tie for first
    R[[5, 6], 0] = 1.0              # tie for fourth: 5 wins
    X = np.zeros((1, 2880), np.float32)
    X[0, 0] = 1.0
    b = Block(gpu, d, 1, x_f32=True)
    kq.moe_router_topk(torch.from_numpy(R).to(gpu), torch.from_numpy(X).to(gpu), b.idx, b.wgt, d,
                       b.ws, b.wsb, batch=1, xh=b.xh)
    torch.cuda.synchronize()
    oidx, owgt, _ = oracle.moe_router(R, oracle.F32, X, oracle.F32, 1, odesc(d))
    assert b.idx.cpu().tolist()[0] == [3, 9, 12, 5] == oidx[0].tolist()
    assert np.allclose(b.wgt.cpu().numpy()[0], owgt[0], atol=1e-6)


NAN, NINF = float("nan"), float("-inf")
# (experts, top-k, base logit of expert e, logits set apart, the expected picks):
# ties across the four 64-expert columns (7 / 135, 64 / 200: the lower index
# first), NaN and -inf never picked, -0 tying +0 (expert 2 before 3); only
# two candidates in columns 2 and 3 (experts 128, 129); fewer candidates than
# picks (the passes past them give expert 0 and weight 0)
TOPK_EDGE = {
    "wide": (256, 8, lambda e: -1.0 - e / 512,
             {7: 5.0, 135: 5.0, 255: 4.5, 64: 4.0, 200: 4.0, 130: 3.0, 131: 3.0, 2: -0.0, 3: 0.0,
              0: NAN, 1: NINF},
             [7, 135, 255, 64, 200, 130, 131, 2]),
    "ragged": (130, 4, lambda e: -e / 256, {129: 2.0, 128: 1.5, 5: 1.5}, [129, 5, 128, 0]),
    "unselectable": (16, 8, lambda e: NAN, {10: NINF, 11: NINF, 12: NINF, 13: 1.0, 14: 3.0, 15: 2.0},
                     [14, 15, 13, 0, 0, 0, 0, 0]),
}


def edge_router(ne, base, special):
    """fp32 router weights whose logits for x = e_0 are exactly the given values."""
    R = np.zeros((ne, 2880), np.float32)
    R[:, 0] = [base(e) for e in range(ne)]
    for e, v in special.items():
        R[e, 0] = v
    X = np.zeros((1, 2880), np.float32)
    X[0, 0] = 1.0
    return R, X


@pytest.mark.parametrize("case", list(TOPK_EDGE))
def test_router_topk_edge_logits(gpu, case):
    """The wave top-k's columns, ties, NaN / -inf / -0 and passes with nothing
    left to pick, against the oracle's strict-greater scan."""
    ne, tk, base, special, want = TOPK_EDGE[case]
    d = kq.moe_default_desc()
    d.n_experts, d.top_k = ne, tk
    R, X = edge_router(ne, base, special)
    oidx, owgt, _ = oracle.moe_router(R, oracle.F32, X, oracle.F32, 1, odesc(d))
    assert oidx[0].tolist() == want
    b = Block(gpu, d, 1, x_f32=True)
    kq.moe_router_topk(torch.from_numpy(R).to(gpu), torch.from_numpy(X).to(gpu), b.idx, b.wgt, d,
                       b.ws, b.wsb, batch=1, xh=b.xh)
    torch.cuda.synchronize()
    assert b.idx.cpu().tolist()[0] == want
    assert np.allclose(b.wgt.cpu().numpy()[0], owgt[0], atol=1e-6, rtol=0)


@pytest.mark.parametrize("path", [kq.MOE_PATH_AUTO, kq.MOE_PATH_ONE, kq.MOE_PATH_ATOMIC])
def test_block_topk_edge_logits(gpu, pool16, path):
    """The block's own top-k (in the gate/up launch, or in the one-launch
    kernel) on tied, NaN and -inf logits: routing and y as the oracle's."""
    host, pool = pool16
    d = _pool_desc(16)
    R, X = edge_router(16, lambda e: -e / 64, {0: NAN, 1: NINF, 4: NAN, 9: 2.0, 12: 2.0, 10: 1.0, 15: 1.0})
    oidx, owgt, Yref = oracle.moe_block(host, odesc(d), R, oracle.F32, X, oracle.F32, 1)
    assert oidx[0].tolist() == [9, 12, 10, 15]
    b = Block(gpu, d, 1, x_f32=True)
    kq.moe_block(pool, d, torch.from_numpy(R).to(gpu), torch.from_numpy(X).to(gpu), b.idx, b.wgt,
                 b.H, b.y, b.ws, b.wsb, batch=1, xh=b.xh, path=path)
    torch.cuda.synchronize()
    assert b.idx.cpu().tolist()[0] == [9, 12, 10, 15]
    assert np.allclose(b.wgt.cpu().numpy()[0], owgt[0], atol=1e-6, rtol=0)
    assert_close(to_f64(b.y), Yref, what=f"edge-logit block path {path}")


def unfused_ws(device, d):
    wsb = kq.moe_unfused_workspace_size(d)
    return torch.empty(wsb, dtype=torch.uint8, device=device), wsb


def _pool_desc(n):
    d = kq.moe_default_desc()
    d.n_experts = n
    return d


@pytest.mark.parametrize("batch", [1, 2, 5, 8, 16])
def test_gate_up_and_down_vs_oracle(gpu, pool16, batch):
    host, pool = pool16
    d = _pool_desc(16)
    rng = np.random.default_rng(batch)
    idx = np.stack([rng.choice(16, 4, replace=False) for _ in range(batch)]).astype(np.uint32)
    wgt = rng.dirichlet(np.ones(4), batch)
    X = gen.f16_bits(rng.normal(0, 1, (batch, 2880)))
    b = Block(gpu, d, batch)
    idx_d = dev(idx, gpu)
    wgt_d = torch.from_numpy(wgt.astype(np.float32)).to(gpu)
    kq.moe_gate_up_swiglu(pool, d, idx_d, dev(X, gpu), b.H, b.ws, b.wsb, batch=batch)
    torch.cuda.synchronize()
    Href = oracle.moe_gate_up(host, odesc(d), idx, X, oracle.F16, batch)
    Hgot = to_f64(b.H)
    assert_close(Hgot, Href, what="h")
    # down from the GPU's own fp16 h, weights as fp32 exactly as the GPU sees them
    kq.moe_down_combine(pool, d, idx_d, wgt_d, b.H, b.y, b.ws, b.wsb, batch=batch)
    torch.cuda.synchronize()
    Yref = oracle.moe_down(host, odesc(d), idx, wgt.astype(np.float32).astype(np.float64),
                           host_bits(b.H, np.uint16), batch)
    assert_close(to_f64(b.y), Yref, atol=1e-4, rtol=1e-4, what="down+combine")


def test_duplicate_and_shared_experts(gpu, pool16):
    """Slots that select the same expert (within and across tokens) read its
    rows once and still land in their own h / y slots."""
    host, pool = pool16
    d = _pool_desc(16)
    idx = np.array([[3, 3, 7, 1], [7, 3, 2, 15], [1, 1, 1, 1]], np.uint32)
    wgt = np.array([[0.4, 0.3, 0.2, 0.1], [0.25] * 4, [0.1, 0.2, 0.3, 0.4]])
    batch = 3
    X = gen.f16_bits(np.random.default_rng(4).normal(0, 1, (batch, 2880)))
    b = Block(gpu, d, batch)
    kq.moe_gate_up_swiglu(pool, d, dev(idx, gpu), dev(X, gpu), b.H, b.ws, b.wsb, batch=batch)
    kq.moe_down_combine(pool, d, dev(idx, gpu), torch.from_numpy(wgt.astype(np.float32)).to(gpu),
                        b.H, b.y, b.ws, b.wsb, batch=batch)
    torch.cuda.synchronize()
    Href = oracle.moe_gate_up(host, odesc(d), idx, X, oracle.F16, batch)
    assert_close(to_f64(b.H), Href, what="h dup")
    Yref = oracle.moe_down(host, odesc(d), idx, wgt.astype(np.float32).astype(np.float64),
                           host_bits(b.H, np.uint16), batch)
    assert_close(to_f64(b.y), Yref, atol=1e-4, rtol=1e-4, what="y dup")


@pytest.mark.parametrize("batch", [1, 8])
def test_block_full_pool(gpu, batch):
    """Config 4: 128 experts of gpt-oss-120b shape (1.8 GB resident), top-4,
    fp16 router and x; the block vs the fp64 block reference."""
    host = gen.moe_pool(128, seed=55, quantize=False)
    pool = dev(host, gpu)
    d = kq.moe_default_desc()
    R, X = gen.moe_inputs(128, batch=batch, seed=9 + batch)
    oidx, owgt, lg = oracle.moe_router(R, oracle.F16, X, oracle.F16, batch, odesc(d))
    assert routing_margin(lg, 4) > 1e-4
    _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F16, X, oracle.F16, batch)
    b = Block(gpu, d, batch)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    for rep in range(3):  # workspace counters must reset between calls
        b.y.fill_(float("nan"))
        kq.moe_block(pool, d, Rd, Xd, b.idx, b.wgt, b.H, b.y, b.ws, b.wsb, batch=batch)
        torch.cuda.synchronize()
        assert np.array_equal(b.idx.cpu().numpy().astype(np.uint32), oidx)
        assert np.allclose(b.wgt.cpu().numpy(), owgt, atol=1e-6)
        got = to_f64(b.y)
        assert_close(got, Yref, what=f"block batch {batch} rep {rep}")
        assert inf_rel(got, Yref) < 2e-3
    if batch == 1:
        # the same block one operation per launch: same routing, same result
        u = Block(gpu, d, 1)
        ws, wsb = unfused_ws(gpu, d)
        n = kq.moe_block_unfused(pool, d, Rd, Xd, u.idx, u.wgt, u.H, u.y, ws, wsb)
        torch.cuda.synchronize()
        assert n == 3 + 5 * d.top_k == 23
        assert np.array_equal(u.idx.cpu().numpy().astype(np.uint32), oidx)
        assert np.allclose(u.wgt.cpu().numpy(), owgt, atol=1e-6)
        Href = oracle.moe_gate_up(host, odesc(d), oidx, X, oracle.F16, 1)
        assert_close(to_f64(u.H), Href, what="unfused h")
        got = to_f64(u.y)
        assert_close(got, Yref, what="unfused block")
        assert inf_rel(got, Yref) < 2e-3
    del pool


@pytest.mark.parametrize("batch", [3, 5, 6, 16])
def test_block_expert_partitioned_down(gpu, pool16, batch):
    """From 3 tokens gate/up runs partitioned by expert. At 3-5 tokens the
    streaming down reads the plan and weights from the workspace; from 6
    tokens the slots' h vectors no longer fit one workgroup's LDS, so down
    runs partitioned by expert too (per-slot products to the workspace, then
    the combine launch). 16 experts, top-4: tokens share experts, so plan
    entries carry several slots."""
    host, pool = pool16
    d = _pool_desc(16)
    R, X = gen.moe_inputs(16, batch=batch, seed=40 + batch)
    oidx, owgt, lg = oracle.moe_router(R, oracle.F16, X, oracle.F16, batch, odesc(d))
    assert routing_margin(lg, 4) > 1e-5
    _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F16, X, oracle.F16, batch)
    b = Block(gpu, d, batch)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    for rep in range(2):
        b.y.fill_(float("nan"))
        kq.moe_block(pool, d, Rd, Xd, b.idx, b.wgt, b.H, b.y, b.ws, b.wsb, batch=batch)
        torch.cuda.synchronize()
        assert np.array_equal(b.idx.cpu().numpy().astype(np.uint32), oidx)
        got = to_f64(b.y)
        assert_close(got, Yref, what=f"block batch {batch} rep {rep}")
        assert inf_rel(got, Yref) < 2e-3


def _atomic_vs_default(gpu, pool, host, d, R, X, batch, k, what):
    """The atomic sum(h) block against the default block and the oracle:
    routing bit for bit; h within one fp16 ulp (the default kernel rounds the
    SwiGLU's last product straight to fp16, the atomic one also needs it as
    a float and rounds twice, as the reference's half(hv) does); y to the
    block's tolerance (its sums of h are fp32 atomics in no fixed order).
    Two calls on one workspace: the router zeroes the sums every call."""
    oidx, owgt, lg = oracle.moe_router(R, oracle.F16, X, oracle.F16, batch, odesc(d))
    assert routing_margin(lg, k) > 1e-5
    _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F16, X, oracle.F16, batch)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    ref, at = Block(gpu, d, batch), Block(gpu, d, batch)
    kq.moe_block(pool, d, Rd, Xd, ref.idx, ref.wgt, ref.H, ref.y, ref.ws, ref.wsb, batch=batch)
    torch.cuda.synchronize()
    for rep in range(2):
        at.y.fill_(float("nan"))
        at.H.zero_()
        kq.moe_block(pool, d, Rd, Xd, at.idx, at.wgt, at.H, at.y, at.ws, at.wsb, batch=batch,
                     path=kq.MOE_PATH_ATOMIC)
        torch.cuda.synchronize()
        assert np.array_equal(at.idx.cpu().numpy().astype(np.uint32), oidx), f"{what} rep {rep}"
        assert torch.equal(at.wgt, ref.wgt), f"{what} rep {rep}"
        ulp = (at.H.view(torch.int16).int() - ref.H.view(torch.int16).int()).abs()
        assert int(ulp.max()) <= 1, f"{what} rep {rep}: h {int(ulp.max())} ulp from the default block"
        assert float((ulp != 0).float().mean()) < 0.01, f"{what} rep {rep}"
        got = to_f64(at.y)
        assert_close(got, Yref, what=f"{what} rep {rep}")
        assert inf_rel(got, Yref) < 2e-3
        assert inf_rel(got, to_f64(ref.y)) < 1e-3, f"{what} rep {rep}: far from the default block"


@pytest.mark.parametrize("batch", [1, 2])
def test_block_atomic_sum_h(gpu, pool16, batch):
    """KQ_MOE_PATH_ATOMIC at gpt-oss shapes (16 experts, top-4), 1 and 2
    tokens (moe-fused/src/kernels.metal:400-487)."""
    host, pool = pool16
    d = _pool_desc(16)
    R, X = gen.moe_inputs(16, batch=batch, seed=60 + batch)
    _atomic_vs_default(gpu, pool, host, d, R, X, batch, 4, f"atomic batch {batch}")


@pytest.mark.parametrize("hidden,inter,batch", [(1024, 2048, 1), (4096, 512, 2), (2048, 4096, 1)])
def test_block_atomic_sum_h_other_shapes(gpu, hidden, inter, batch):
    """KQ_MOE_PATH_ATOMIC on other descriptors (chunk counts 1-4 of both
    streaming kernels, partial chunks, top-3)."""
    d, off = _compact_desc(hidden, inter, 16, 3)
    host = gen.moe_pool(16, seed=hidden + inter + 7, quantize=True, hidden=hidden, inter=inter,
                        blob=d.blob, off=off)
    R, X = gen.moe_inputs(16, hidden=hidden, batch=batch, seed=inter + batch + 7)
    _atomic_vs_default(gpu, dev(host, gpu), host, d, R, X, batch, 3, f"atomic {hidden}x{inter} b{batch}")


def test_block_atomic_unsupported(gpu, pool16):
    """Three tokens: the streaming gate/up does not run, so the atomic path is
    refused (KQ_EUNSUPPORTED) rather than run in another form."""
    host, pool = pool16
    d = _pool_desc(16)
    R, X = gen.moe_inputs(16, batch=3, seed=70)
    b = Block(gpu, d, 3)
    with pytest.raises(kq.KQError) as e:
        kq.moe_block(pool, d, dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16), b.idx,
                     b.wgt, b.H, b.y, b.ws, b.wsb, batch=3, path=kq.MOE_PATH_ATOMIC)
    assert e.value.status == kq.KQ_EUNSUPPORTED


def test_workspace_reused_across_batches(gpu, pool16):
    """One workspace sized for 16 tokens serves calls at 8, 3, 16 and 1 tokens
    in turn (every block form: streaming, expert-partitioned gate/up and
    down, the combine launch): the router's counter and the plan sit at fixed
    offsets, so no call's logits or products overwrite them."""
    host, pool = pool16
    d = _pool_desc(16)
    wsb = kq.moe_workspace_size(d, 16)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    kq.moe_workspace_init(ws, wsb)
    for batch in (8, 3, 16, 1, 8):
        R, X = gen.moe_inputs(16, batch=batch, seed=500 + batch)
        oidx, owgt, lg = oracle.moe_router(R, oracle.F16, X, oracle.F16, batch, odesc(d))
        assert routing_margin(lg, 4) > 1e-5
        _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F16, X, oracle.F16, batch)
        b = Block(gpu, d, batch)
        kq.moe_block(pool, d, dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16),
                     b.idx, b.wgt, b.H, b.y, ws, wsb, batch=batch)
        torch.cuda.synchronize()
        assert np.array_equal(b.idx.cpu().numpy().astype(np.uint32), oidx), f"batch {batch}"
        assert np.allclose(b.wgt.cpu().numpy(), owgt, atol=1e-6)
        assert_close(to_f64(b.y), Yref, what=f"shared workspace, batch {batch}")


def test_block_fp32_inputs_and_fp16_out(gpu, pool16):
    """Reference-fidelity inputs: fp32 router and x (xh written by the router)."""
    host, pool = pool16
    d = _pool_desc(16)
    rng = np.random.default_rng(12)
    R = (rng.normal(0, 0.02, (16, 2880))).astype(np.float32)
    X = rng.normal(0, 1, (2, 2880)).astype(np.float32)
    oidx, owgt, lg = oracle.moe_router(R, oracle.F32, X, oracle.F32, 2, odesc(d))
    assert routing_margin(lg, 4) > 1e-4
    b = Block(gpu, d, 2, x_f32=True, y_dtype=torch.float16)
    kq.moe_block(pool, d, torch.from_numpy(R).to(gpu), torch.from_numpy(X).to(gpu), b.idx, b.wgt,
                 b.H, b.y, b.ws, b.wsb, batch=2, xh=b.xh)
    torch.cuda.synchronize()
    assert np.array_equal(b.idx.cpu().numpy().astype(np.uint32), oidx)
    # the reference CPU block uses x unrounded; the GPU projections use half(x)
    _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F32, X, oracle.F32, 2)
    got = to_f64(b.y)
    assert inf_rel(got, Yref) < 2e-3
    assert_close(got, Yref, atol=2e-2, rtol=2e-3, what="fp32-in block")


@pytest.mark.parametrize("batch", [1, 8, 16])
def test_block_graph_replays(gpu, pool16, batch):
    """The block captured in a HIP graph: every replay (with eager block calls
    and synchronisations between replays, and the router's completion counter
    carried in the workspace across all of them) equals the eager result bit
    for bit -- the kernels are deterministic."""
    host, pool = pool16
    d = _pool_desc(16)
    R, X = gen.moe_inputs(16, batch=batch, seed=70 + batch)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    b = Block(gpu, d, batch)

    def block():
        kq.moe_block(pool, d, Rd, Xd, b.idx, b.wgt, b.H, b.y, b.ws, b.wsb, batch=batch)

    block()
    torch.cuda.synchronize()
    ref_idx, ref_y = b.idx.clone(), b.y.clone()
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
        assert torch.equal(b.idx, ref_idx), f"replay {rep} idx"
        assert torch.equal(b.y, ref_y), f"replay {rep} y"
        block()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(b.y, ref_y), f"eager after replay {rep}"


def _compact_desc(hidden, inter, n_experts, top_k):
    """A blob layout for other shapes: gate, up, down one after another, each
    W, S, B, BI (256-byte aligned); returns (kq desc, offsets for gen)."""
    def al(v):
        return (v + 255) // 256 * 256
    # every projection shares the sub-offsets, so size them for the largest
    rows_cols = [(inter, hidden), (inter, hidden), (hidden, inter)]
    wmax = max(r * c // 2 for r, c in rows_cols)
    smax = max(r * (c // 64) * 2 for r, c in rows_cols)
    bimax = max(r * 2 for r, c in rows_cols)
    sub = dict(sub_w=0, sub_s=al(wmax), sub_b=al(wmax) + al(smax), sub_bi=al(wmax) + 2 * al(smax))
    proj = al(sub["sub_bi"] + bimax)
    off = dict(off_gate=0, off_up=proj, off_down=2 * proj, **sub)
    d = kq.moe_default_desc()
    d.hidden, d.inter, d.n_experts, d.top_k = hidden, inter, n_experts, top_k
    d.blob = 3 * proj
    for k, v in off.items():
        setattr(d, k, v)
    return d, off


@pytest.mark.parametrize("hidden,inter,batch", [(1024, 2048, 1), (4096, 512, 2), (2048, 4096, 1),
                                                (1536, 1024, 3), (2048, 2048, 4), (2048, 4096, 3),
                                                (1024, 2048, 8), (2048, 1024, 12), (4096, 512, 16),
                                                (1536, 4096, 7)])
def test_other_shapes(gpu, hidden, inter, batch):
    """Descriptors other than gpt-oss's (every chunk count of the streaming
    kernels, partial chunks, 16 experts, top-3): the block and the
    standalone projections against the oracle, routing exact. From 6 tokens
    both projections run partitioned by expert with their items handed out
    in the workgroup, here at every chunk count (hidden 1024 / 1536 / 2048 /
    4096 for gate/up, inter 512 / 1024 / 2048 / 4096 for down) and with
    experts shared by several tokens."""
    d, off = _compact_desc(hidden, inter, 16, 3)
    host = gen.moe_pool(16, seed=hidden + inter, quantize=True, hidden=hidden, inter=inter,
                        blob=d.blob, off=off)
    pool = dev(host, gpu)
    R, X = gen.moe_inputs(16, hidden=hidden, batch=batch, seed=inter + batch)
    oidx, owgt, lg = oracle.moe_router(R, oracle.F16, X, oracle.F16, batch, odesc(d))
    assert routing_margin(lg, 3) > 1e-5
    _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F16, X, oracle.F16, batch)
    b = Block(gpu, d, batch)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    kq.moe_block(pool, d, Rd, Xd, b.idx, b.wgt, b.H, b.y, b.ws, b.wsb, batch=batch)
    torch.cuda.synchronize()
    assert np.array_equal(b.idx.cpu().numpy().astype(np.uint32), oidx)
    assert np.allclose(b.wgt.cpu().numpy(), owgt, atol=1e-6)
    assert_close(to_f64(b.y), Yref, what=f"block {hidden}x{inter} b{batch}")
    # the standalone projections from the same routing
    kq.moe_gate_up_swiglu(pool, d, b.idx, Xd, b.H, b.ws, b.wsb, batch=batch)
    torch.cuda.synchronize()
    Href = oracle.moe_gate_up(host, odesc(d), oidx, X, oracle.F16, batch)
    assert_close(to_f64(b.H), Href, what=f"h {hidden}x{inter} b{batch}")
    kq.moe_down_combine(pool, d, b.idx, b.wgt, b.H, b.y, b.ws, b.wsb, batch=batch)
    torch.cuda.synchronize()
    Yd = oracle.moe_down(host, odesc(d), oidx, b.wgt.cpu().numpy().astype(np.float64),
                         host_bits(b.H, np.uint16), batch)
    assert_close(to_f64(b.y), Yd, atol=1e-4, rtol=1e-4, what=f"down {hidden}x{inter} b{batch}")


# (experts, top-k, tokens): the most slots a call can have, 16 tokens x top-8
# of 256 experts (128 slots, over 100 distinct experts: plan entries past 64,
# slots in both words of the masks), and one slot a token (top-1), at every
# token count form of the block (streaming 1, whole-entry split 5, equal-cost
# ranges 8 and 16)
SLOT_EXTREMES = [(256, 8, 1), (256, 8, 5), (256, 8, 8), (256, 8, 16),
                 (64, 1, 1), (64, 1, 5), (64, 1, 8), (64, 1, 16)]


@pytest.fixture(scope="module")
def slot_pools(gpu):
    """Pools of 256 x top-8 and 64 x top-1 experts, hidden = inter = 256."""
    out = {}
    for ne, tk in sorted({(e, k) for e, k, _ in SLOT_EXTREMES}):
        d, off = _compact_desc(256, 256, ne, tk)
        host = gen.moe_pool(ne, seed=ne + tk, quantize=True, hidden=256, inter=256, blob=d.blob,
                            off=off)
        out[(ne, tk)] = (d, host, dev(host, gpu))
    return out


@pytest.mark.parametrize("ne,tk,batch", SLOT_EXTREMES)
def test_block_slot_extremes(gpu, slot_pools, ne, tk, batch):
    """The block, and the standalone projections from its routing, against
    the oracle at the slot extremes (routing exact); at one token also the
    one-launch, atomic sum(h) and unfused forms."""
    d, host, pool = slot_pools[(ne, tk)]
    R, X = gen.moe_inputs(ne, hidden=256, batch=batch, seed=1000 * tk + 10 * batch)
    oidx, owgt, lg = oracle.moe_router(R, oracle.F16, X, oracle.F16, batch, odesc(d))
    assert routing_margin(lg, tk) > 1e-5
    _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F16, X, oracle.F16, batch)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    paths = [None] + ([kq.MOE_PATH_ONE, kq.MOE_PATH_ATOMIC] if batch == 1 else [])
    for path in paths:
        b = Block(gpu, d, batch)
        kq.moe_block(pool, d, Rd, Xd, b.idx, b.wgt, b.H, b.y, b.ws, b.wsb, batch=batch, path=path)
        torch.cuda.synchronize()
        what = f"{ne} experts top-{tk} b{batch} path {path}"
        assert np.array_equal(b.idx.cpu().numpy().astype(np.uint32), oidx), what
        assert np.allclose(b.wgt.cpu().numpy(), owgt, atol=1e-6), what
        assert_close(to_f64(b.y), Yref, what=what)
    kq.moe_gate_up_swiglu(pool, d, b.idx, Xd, b.H, b.ws, b.wsb, batch=batch)
    torch.cuda.synchronize()
    Href = oracle.moe_gate_up(host, odesc(d), oidx, X, oracle.F16, batch)
    assert_close(to_f64(b.H), Href, what=f"h {ne} experts top-{tk} b{batch}")
    kq.moe_down_combine(pool, d, b.idx, b.wgt, b.H, b.y, b.ws, b.wsb, batch=batch)
    torch.cuda.synchronize()
    Yd = oracle.moe_down(host, odesc(d), oidx, b.wgt.cpu().numpy().astype(np.float64),
                         host_bits(b.H, np.uint16), batch)
    assert_close(to_f64(b.y), Yd, atol=1e-4, rtol=1e-4, what=f"down {ne} experts top-{tk} b{batch}")
    if batch == 1:
        b = Block(gpu, d, 1)
        ws, wsb = unfused_ws(gpu, d)
        kq.moe_block_unfused(pool, d, Rd, Xd, b.idx, b.wgt, b.H, b.y, ws, wsb)
        torch.cuda.synchronize()
        assert np.array_equal(b.idx.cpu().numpy().astype(np.uint32), oidx)
        assert_close(to_f64(b.y), Yref, what=f"unfused {ne} experts top-{tk}")


def test_unfused_fp32_inputs_and_fp16_out(gpu, pool16):
    """The one-op-per-launch block with fp32 router and x (xh written by its
    router launch) and an fp16 output, against the oracle and the fused
    block's routing."""
    host, pool = pool16
    d = _pool_desc(16)
    rng = np.random.default_rng(13)
    R = (rng.normal(0, 0.02, (16, 2880))).astype(np.float32)
    X = rng.normal(0, 1, (1, 2880)).astype(np.float32)
    oidx, owgt, lg = oracle.moe_router(R, oracle.F32, X, oracle.F32, 1, odesc(d))
    assert routing_margin(lg, 4) > 1e-4
    b = Block(gpu, d, 1, x_f32=True, y_dtype=torch.float16)
    ws, wsb = unfused_ws(gpu, d)
    n = kq.moe_block_unfused(pool, d, torch.from_numpy(R).to(gpu), torch.from_numpy(X).to(gpu),
                             b.idx, b.wgt, b.H, b.y, ws, wsb, xh=b.xh)
    torch.cuda.synchronize()
    assert n == 23
    assert np.array_equal(b.idx.cpu().numpy().astype(np.uint32), oidx)
    assert np.allclose(b.wgt.cpu().numpy(), owgt, atol=1e-6)
    assert np.array_equal(host_bits(b.xh, np.uint16), X.astype(np.float16).view(np.uint16))
    _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F32, X, oracle.F32, 1)
    got = to_f64(b.y)
    assert inf_rel(got, Yref) < 2e-3
    assert_close(got, Yref, atol=2e-2, rtol=2e-3, what="fp32-in unfused block")


@pytest.mark.parametrize("hidden,inter", [(1024, 2048), (4096, 512), (2048, 4096)])
def test_unfused_other_shapes(gpu, hidden, inter):
    """The one-op-per-launch block on other descriptors (16 experts, top-3:
    3 + 5 * 3 = 18 launches) against the oracle."""
    d, off = _compact_desc(hidden, inter, 16, 3)
    host = gen.moe_pool(16, seed=hidden + 2 * inter, quantize=True, hidden=hidden, inter=inter,
                        blob=d.blob, off=off)
    pool = dev(host, gpu)
    R, X = gen.moe_inputs(16, hidden=hidden, batch=1, seed=inter + 7)
    oidx, owgt, lg = oracle.moe_router(R, oracle.F16, X, oracle.F16, 1, odesc(d))
    assert routing_margin(lg, 3) > 1e-5
    _, _, Yref = oracle.moe_block(host, odesc(d), R, oracle.F16, X, oracle.F16, 1)
    b = Block(gpu, d, 1)
    ws, wsb = unfused_ws(gpu, d)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    n = kq.moe_block_unfused(pool, d, Rd, Xd, b.idx, b.wgt, b.H, b.y, ws, wsb)
    torch.cuda.synchronize()
    assert n == 18
    assert np.array_equal(b.idx.cpu().numpy().astype(np.uint32), oidx)
    assert np.allclose(b.wgt.cpu().numpy(), owgt, atol=1e-6)
    Href = oracle.moe_gate_up(host, odesc(d), oidx, X, oracle.F16, 1)
    assert_close(to_f64(b.H), Href, what=f"unfused h {hidden}x{inter}")
    assert_close(to_f64(b.y), Yref, what=f"unfused block {hidden}x{inter}")


def test_unfused_graph_replays(gpu, pool16):
    """The 23 launches captured in a HIP graph: every replay, with eager calls
    and synchronisations between replays, equals the eager result bit for
    bit."""
    host, pool = pool16
    d = _pool_desc(16)
    R, X = gen.moe_inputs(16, batch=1, seed=77)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    b = Block(gpu, d, 1)
    ws, wsb = unfused_ws(gpu, d)

    def block():
        kq.moe_block_unfused(pool, d, Rd, Xd, b.idx, b.wgt, b.H, b.y, ws, wsb)

    block()
    torch.cuda.synchronize()
    ref_idx, ref_y = b.idx.clone(), b.y.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        block()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        block()
    for rep in range(3):
        b.y.fill_(float("nan"))
        b.idx.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(b.idx, ref_idx), f"replay {rep} idx"
        assert torch.equal(b.y, ref_y), f"replay {rep} y"
        block()
        torch.cuda.synchronize()
        assert torch.equal(b.y, ref_y), f"eager after replay {rep}"
