"""kq_moe_block_noalloc: the MoE block on libkq's per-GPU static workspace
(no allocation) against kq_moe_block on a caller workspace, through the C
ABI. The kernels are the same and deterministic, so routing, h and y must
match bit for bit; routing is also checked against the fp64 oracle.

Three calls in a row on the shared array, each smaller than the one before
(8 tokens: expert-partitioned gate/up and down with the per-slot products
in the workspace and the combine launch; 3 tokens: partitioned gate/up,
streaming down from the workspace plan; 1 token: streaming with the
in-kernel top-k), so a later call runs on what an earlier one left behind.
A fresh process whose first no-allocation call is made under stream capture
records only the block's kernels: its graph's replays equal the eager block.
"""
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest
import torch

import oracle
from kernels_amd import gen, kq
from tests._util import dev

pytestmark = pytest.mark.gpu


def _odesc(d):
    o = oracle.MoEDesc()
    for f, _ in kq.MoEDesc._fields_:
        setattr(o, f, getattr(d, f))
    return o


def _bufs(device, d, batch):
    return dict(idx=torch.full((batch, d.top_k), -1, dtype=torch.int32, device=device),
                wgt=torch.full((batch, d.top_k), float("nan"), dtype=torch.float32, device=device),
                H=torch.zeros((batch, d.top_k, d.inter), dtype=torch.float16, device=device),
                y=torch.full((batch, d.hidden), float("nan"), dtype=torch.float32, device=device))


def test_noalloc_block_matches_block(gpu):
    host = gen.moe_pool(16, seed=61, quantize=True)
    pool = dev(host, gpu)
    d = kq.moe_default_desc()
    d.n_experts = 16
    for batch in (8, 3, 1):
        R, X = gen.moe_inputs(16, batch=batch, seed=900 + batch)
        Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
        oidx, _, _ = oracle.moe_router(R, oracle.F16, X, oracle.F16, batch, _odesc(d))
        a = _bufs(gpu, d, batch)
        wsb = kq.moe_workspace_size(d, batch)
        ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
        kq.moe_workspace_init(ws, wsb)
        kq.moe_block(pool, d, Rd, Xd, a["idx"], a["wgt"], a["H"], a["y"], ws, wsb, batch=batch)
        b = _bufs(gpu, d, batch)
        kq.moe_block_noalloc(pool, d, Rd, Xd, b["idx"], b["wgt"], b["H"], b["y"], batch=batch)
        torch.cuda.synchronize()
        assert np.array_equal(b["idx"].cpu().numpy().astype(np.uint32), oidx), f"batch {batch}"
        for k in ("idx", "wgt", "H", "y"):
            assert torch.equal(a[k], b[k]), f"batch {batch}: {k} differs"
        assert torch.isfinite(b["y"]).all()


CAPTURE_FIRST = textwrap.dedent("""
    import sys
    sys.path.insert(0, sys.argv[1])
    import numpy as np
    import torch
    from kernels_amd import gen, kq
    from tests._util import dev
    gpu = torch.device("cuda:0")
    kq.lib()
    host = gen.moe_pool(16, seed=62, quantize=True)
    pool = dev(host, gpu)
    d = kq.moe_default_desc()
    d.n_experts = 16
    R, X = gen.moe_inputs(16, batch=1, seed=77)
    Rd, Xd = dev(R, gpu).view(torch.float16), dev(X, gpu).view(torch.float16)
    def bufs():
        return dict(idx=torch.full((1, d.top_k), -1, dtype=torch.int32, device=gpu),
                    wgt=torch.full((1, d.top_k), float("nan"), dtype=torch.float32, device=gpu),
                    H=torch.zeros((1, d.top_k, d.inter), dtype=torch.float16, device=gpu),
                    y=torch.full((1, d.hidden), float("nan"), dtype=torch.float32, device=gpu))
    # the block on a caller workspace first: the library's kernels are then
    # loaded, and what the capture below meets is the no-allocation call's own
    # per-GPU set-up
    a = bufs()
    wsb = kq.moe_workspace_size(d, 1)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    kq.moe_workspace_init(ws, wsb)
    kq.moe_block(pool, d, Rd, Xd, a["idx"], a["wgt"], a["H"], a["y"], ws, wsb, batch=1)
    torch.cuda.synchronize()
    g_out = bufs()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):  # the process's first kq_moe_block_noalloc call
        kq.moe_block_noalloc(pool, d, Rd, Xd, g_out["idx"], g_out["wgt"], g_out["H"],
                             g_out["y"], batch=1)
    torch.cuda.synchronize()
    for rep in range(4):
        for t in g_out.values():
            t.fill_(7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for k in ("idx", "wgt", "H", "y"):
            assert torch.equal(a[k], g_out[k]), f"replay {rep}: {k} differs"
        # eager work of the program's own between replays
        b = bufs()
        kq.moe_block_noalloc(pool, d, Rd, Xd, b["idx"], b["wgt"], b["H"], b["y"], batch=1)
        torch.cuda.synchronize()
        assert torch.equal(a["y"], b["y"]), f"eager call after replay {rep}: y differs"
    print("CAPTURE_FIRST_OK", flush=True)
""")


def test_noalloc_first_call_captured():
    """A fresh process makes its first kq_moe_block_noalloc call inside a
    torch CUDA graph capture (the per-GPU set-up then happens under
    capture), replays the graph four times with eager calls and host
    synchronisations between, and compares every replay with kq_moe_block
    on a caller workspace, bit for bit."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("[noalloc] capture-first subprocess, 16 experts, batch 1", flush=True)
    r = subprocess.run([sys.executable, "-c", CAPTURE_FIRST, root], capture_output=True,
                       text=True, timeout=110)
    assert r.returncode == 0 and "CAPTURE_FIRST_OK" in r.stdout, (r.stdout[-2000:],
                                                                  r.stderr[-3000:])
