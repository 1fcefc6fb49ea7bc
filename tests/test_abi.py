"""libkq's C ABI on the CPU: it loads, exports every symbol include/kq.h
declares, and rejects malformed calls on the host before any launch (these
calls never reach the GPU, so they run without one)."""
import ctypes as C
import os
import re

import pytest

from kernels_amd import kq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = 0x10000  # 64 KiB-aligned non-null address; never dereferenced by these calls


def header_symbols():
    text = open(os.path.join(ROOT, "include", "kq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_exactly_the_exports():
    assert header_symbols() == sorted(kq.EXPORTS)


def test_library_exports_every_symbol():
    L = kq.lib()
    for name in header_symbols():
        assert hasattr(L, name), name


def test_status_strings_and_version():
    L = kq.lib()
    assert L.kq_status_str(kq.KQ_OK) == b"ok"
    assert b"null" in L.kq_status_str(kq.KQ_ENULL)
    assert L.kq_version().startswith(b"kq ")
    assert L.kq_last_hip_error() == 0


def _int4(W=FAKE, S=FAKE, B=None, sbdt=kq.F16, X=FAKE, Y=FAKE, ydt=kq.F16, M=64, K=512, G=64,
          batch=1):
    return kq.lib().kq_int4_gemv(W, S, B, sbdt, X, Y, ydt, M, K, G, batch, None)


@pytest.mark.parametrize("kw,status", [
    (dict(W=None), kq.KQ_ENULL), (dict(X=None), kq.KQ_ENULL), (dict(Y=None), kq.KQ_ENULL),
    (dict(K=100), kq.KQ_EINVAL), (dict(K=0), kq.KQ_EINVAL), (dict(M=0), kq.KQ_EINVAL),
    (dict(G=48), kq.KQ_EINVAL), (dict(G=256), kq.KQ_EINVAL), (dict(K=96, G=64), kq.KQ_EINVAL),
    (dict(batch=0), kq.KQ_EINVAL), (dict(batch=17), kq.KQ_EINVAL),
    (dict(sbdt=kq.F32), kq.KQ_EUNSUPPORTED), (dict(ydt=kq.BF16), kq.KQ_EUNSUPPORTED),
    (dict(W=FAKE + 4), kq.KQ_EALIGN), (dict(X=FAKE + 8), kq.KQ_EALIGN),
    (dict(S=FAKE + 2), kq.KQ_EALIGN), (dict(Y=FAKE + 2, ydt=kq.F32), kq.KQ_EALIGN),
])
def test_int4_rejects_on_host(kw, status):
    assert _int4(**kw) == status


def test_int4_path_and_cfg_reject_on_host():
    L = kq.lib()
    assert L.kq_int4_gemv_path(FAKE, FAKE, None, kq.F16, FAKE, FAKE, kq.F16, 64, 512, 64, 1, 7,
                               None) == kq.KQ_EINVAL
    assert L.kq_int4_gemv_cfg(FAKE, FAKE, None, kq.F16, FAKE, FAKE, kq.F16, 64, 512, 64, 1,
                              kq.PATH_VALU, 3, 1, None) == kq.KQ_EUNSUPPORTED
    assert L.kq_int4_gemv_cfg(FAKE, FAKE, None, kq.F16, FAKE, FAKE, kq.F16, 64, 512, 64, 1,
                              kq.PATH_AUTO, 1, 1, None) == kq.KQ_EINVAL


def test_vq_rejects_on_host():
    L = kq.lib()
    ok = dict(IDX=FAKE, C=FAKE, S=FAKE, X=FAKE, Y=FAKE, ydt=kq.F16, M=256, K=512, rpc=256,
              sg=32, batch=1)

    def call(**kw):
        a = dict(ok, **kw)
        return L.kq_vq_gemv(a["IDX"], a["C"], a["S"], a["X"], a["Y"], a["ydt"], a["M"], a["K"],
                            a["rpc"], a["sg"], a["batch"], None)
    assert call(IDX=None) == kq.KQ_ENULL
    assert call(K=100) == kq.KQ_EINVAL
    assert call(sg=48) == kq.KQ_EINVAL
    assert call(sg=16) == kq.KQ_EINVAL
    assert call(rpc=0) == kq.KQ_EINVAL
    assert call(batch=0) == kq.KQ_EINVAL
    assert call(IDX=FAKE + 1) == kq.KQ_EALIGN


def test_moe_desc_and_workspace():
    d = kq.moe_default_desc()
    assert (d.hidden, d.inter, d.n_experts, d.top_k, d.blob) == (2880, 2880, 128, 4, 14024704)
    assert (d.off_up, d.off_down, d.sub_s, d.sub_b, d.sub_bi) == (4671360, 9342720, 4147200,
                                                                  4406400, 4665600)
    n1 = kq.moe_workspace_size(d, 1)
    n8 = kq.moe_workspace_size(d, 8)
    assert 0 < n1 < n8
    bad = kq.moe_default_desc()
    bad.top_k = 0
    assert kq.lib().kq_moe_workspace_size(C.byref(bad), 1) == 0
    bad = kq.moe_default_desc()
    bad.sub_bi = bad.blob  # output bias would run past the blob
    assert kq.lib().kq_moe_workspace_size(C.byref(bad), 1) == 0
    assert kq.lib().kq_moe_workspace_size(C.byref(d), 17) == 0


def test_moe_workspace_head_is_batch_independent():
    """The workspace is [counter + plan head][logits][per-slot products][sums
    of h for the atomic block]: the batch-dependent parts are exactly those
    three, so the head (the router's completion counter and the plan, which
    must survive between calls) sits at the same offsets for every batch and
    descriptor, and a workspace sized for one batch can serve another."""
    def al(v):
        return (v + 255) // 256 * 256

    heads = set()
    for ne, tk in ((128, 4), (16, 3), (256, 8)):
        d = kq.moe_default_desc()
        d.n_experts, d.top_k = ne, tk
        for b in range(1, 17):
            n = kq.moe_workspace_size(d, b)
            heads.add(n - al(4 * b * ne) - al(4 * b * tk * d.hidden) - al(4 * b * tk * ((d.inter + 31) // 32)))
    assert len(heads) == 1, heads


def test_moe_noalloc_rejects_on_host():
    """kq_moe_block_noalloc refuses, before any launch, a (desc, batch) whose
    workspace exceeds its static array, and validates like kq_moe_block."""
    L = kq.lib()
    d = kq.moe_default_desc()
    assert kq.moe_workspace_size(d, 16) <= kq.MOE_NOALLOC_WS_BYTES  # gpt-oss fits at 16 tokens
    big = kq.moe_default_desc()
    big.hidden, big.inter, big.top_k = 4096, 4096, 8
    big.off_up = big.off_down = big.sub_s = big.sub_b = big.sub_bi = 0
    big.blob = 4096 * 4096
    assert kq.moe_workspace_size(big, 16) > kq.MOE_NOALLOC_WS_BYTES

    def call(desc, batch, **kw):
        a = dict(pool=FAKE, R=FAKE, X=FAKE, idx=FAKE, wgt=FAKE, xh=None, H=FAKE, Y=FAKE)
        a.update(kw)
        return L.kq_moe_block_noalloc(a["pool"], C.byref(desc), a["R"], kq.F16, a["X"], kq.F16,
                                      batch, a["idx"], a["wgt"], a["xh"], a["H"], a["Y"], kq.F32,
                                      None)
    assert call(big, 16) == kq.KQ_EWORKSPACE
    assert call(d, 17) == kq.KQ_EINVAL
    assert call(d, 1, pool=None) == kq.KQ_ENULL
    assert call(d, 1, H=FAKE + 2) == kq.KQ_EALIGN


def test_moe_rejects_on_host():
    L = kq.lib()
    d = kq.moe_default_desc()
    n = kq.moe_workspace_size(d, 1)
    r = L.kq_moe_router_topk(FAKE, kq.F16, FAKE, kq.F16, 1, C.byref(d), FAKE, FAKE, None, FAKE,
                             n - 1, None)
    assert r == kq.KQ_EWORKSPACE
    r = L.kq_moe_router_topk(FAKE, kq.F16, FAKE, kq.F16, 1, C.byref(d), FAKE, FAKE, None, None,
                             n, None)
    assert r == kq.KQ_EWORKSPACE
    r = L.kq_moe_router_topk(FAKE, kq.BF16, FAKE, kq.F16, 1, C.byref(d), FAKE, FAKE, None, FAKE,
                             n, None)
    assert r == kq.KQ_EUNSUPPORTED
    r = L.kq_moe_gate_up_swiglu(None, C.byref(d), FAKE, FAKE, FAKE, 1, FAKE, n, None)
    assert r == kq.KQ_ENULL
    r = L.kq_moe_down_combine(FAKE, C.byref(d), FAKE, FAKE, FAKE, FAKE, kq.BF16, 1, FAKE, n, None)
    assert r == kq.KQ_EUNSUPPORTED
    r = L.kq_moe_block(FAKE, C.byref(d), FAKE, kq.F16, FAKE, kq.F32, 1, FAKE, FAKE, None, FAKE,
                       FAKE, kq.F32, FAKE, n, None)
    assert r == kq.KQ_ENULL  # fp32 x needs an xh buffer
    assert L.kq_moe_workspace_init(FAKE + 4, 64, None) == kq.KQ_EALIGN


def test_moe_block_path_rejects_on_host():
    """kq_moe_block_path: an unknown path is KQ_EINVAL, the one-launch path
    outside its limits (here two tokens) and the atomic sum(h) path outside
    its (here three tokens) KQ_EUNSUPPORTED, before any launch."""
    L = kq.lib()
    d = kq.moe_default_desc()
    n = kq.moe_workspace_size(d, 2)

    def call(batch, path):
        return L.kq_moe_block_path(FAKE, C.byref(d), FAKE, kq.F16, FAKE, kq.F16, batch, FAKE, FAKE,
                                   None, FAKE, FAKE, kq.F32, FAKE, n, path, None)
    assert call(1, 4) == kq.KQ_EINVAL
    assert call(1, -1) == kq.KQ_EINVAL
    assert call(2, kq.MOE_PATH_ONE) == kq.KQ_EUNSUPPORTED
    n3 = kq.moe_workspace_size(d, 3)
    assert L.kq_moe_block_path(FAKE, C.byref(d), FAKE, kq.F16, FAKE, kq.F16, 3, FAKE, FAKE, None, FAKE,
                               FAKE, kq.F32, FAKE, n3, kq.MOE_PATH_ATOMIC, None) == kq.KQ_EUNSUPPORTED


def test_moe_unfused_rejects_on_host():
    L = kq.lib()
    d = kq.moe_default_desc()
    n = kq.moe_unfused_workspace_size(d)
    assert n >= 4 * (128 + 2 * 2880 + 2 * 2880)
    cnt = C.c_uint32(7)

    def call(batch=1, ws=FAKE, wsb=n, pool=FAKE, xdt=kq.F16, xh=None):
        return L.kq_moe_block_unfused(pool, C.byref(d), FAKE, kq.F16, FAKE, xdt, batch, FAKE,
                                      FAKE, xh, FAKE, FAKE, kq.F32, ws, wsb, C.byref(cnt), None)
    assert call(batch=2) == kq.KQ_EUNSUPPORTED  # one token, like the reference's unfused path
    assert call(batch=0) == kq.KQ_EINVAL
    assert call(wsb=n - 1) == kq.KQ_EWORKSPACE
    assert call(ws=None) == kq.KQ_EWORKSPACE
    assert call(ws=FAKE + 16) == kq.KQ_EALIGN
    assert call(pool=None) == kq.KQ_ENULL
    assert call(xdt=kq.F32) == kq.KQ_ENULL  # fp32 x needs an xh buffer
    assert cnt.value == 7  # untouched by a rejected call
    bad = kq.moe_default_desc()
    bad.top_k = 9
    assert L.kq_moe_unfused_workspace_size(C.byref(bad)) == 0


def test_vq_quantize_rejects_on_host():
    L = kq.lib()
    n = kq.vq_quantize_workspace_size(14336, 4096, 256, 4096, 200_000)
    # scales + 56 blocks x 200000 sample points + centroids and their sums
    assert n >= 14336 * 4 + 56 * 200_000 * 8 + 56 * 256 * (8 + 24)
    assert L.kq_vq_quantize_workspace_size(64, 100, 64, 32, 1000) == 0    # K % 32
    assert L.kq_vq_quantize_workspace_size(64, 128, 64, 48, 1000) == 0    # group not 2^k
    assert L.kq_vq_quantize_workspace_size(64, 128, 64, 16, 1000) == 0    # group < 32
    assert L.kq_vq_quantize_workspace_size(64, 128, 0, 32, 1000) == 0     # rows_per_cb
    assert L.kq_vq_quantize_workspace_size(64, 128, 64, 32, 0) == 0       # sample
    assert L.kq_vq_quantize_workspace_size(70000, 128, 1, 32, 10) == 0    # > 65535 blocks
    m = kq.vq_quantize_workspace_size(64, 128, 64, 32, 1000)

    def call(ws=FAKE, wsb=m, W=FAKE, dt=kq.F32, iters=25, IDX=FAKE):
        return L.kq_vq_quantize(W, dt, 64, 128, 64, 32, iters, 1000, 0, IDX, FAKE, FAKE, ws, wsb,
                                None)
    assert call(wsb=m - 1) == kq.KQ_EWORKSPACE
    assert call(ws=None) == kq.KQ_EWORKSPACE
    assert call(W=None) == kq.KQ_ENULL
    assert call(dt=7) == kq.KQ_EUNSUPPORTED
    assert call(iters=1001) == kq.KQ_EINVAL
    assert call(IDX=FAKE + 2) == kq.KQ_EALIGN
    assert call(ws=FAKE + 64) == kq.KQ_EALIGN


def test_stream_read_and_xsum_reject_on_host():
    L = kq.lib()
    assert L.kq_stream_read(FAKE, 100, FAKE, None) == kq.KQ_EINVAL
    assert L.kq_stream_read(None, 1024, FAKE, None) == kq.KQ_ENULL
    assert L.kq_xsum32(FAKE, FAKE, 100, 1, None) == kq.KQ_EINVAL
    assert L.kq_stream_read_cfg(FAKE, 1024, FAKE, 3, 256, None) == kq.KQ_EINVAL  # unroll
    assert L.kq_stream_read_cfg(FAKE, 1024, FAKE, 4, 300, None) == kq.KQ_EINVAL  # threads % 256
    assert L.kq_stream_read_cfg(FAKE, 1024, FAKE, 4, 0, None) == kq.KQ_EINVAL
    assert L.kq_stream_read_cfg(FAKE + 4, 1024, FAKE, 4, 256, None) == kq.KQ_EALIGN
    assert L.kq_stream_read_cfg(None, 1024, FAKE, 4, 256, None) == kq.KQ_ENULL
    assert L.kq_stream_read_out(None, 1024, FAKE, 16, 1, 256, None) == kq.KQ_ENULL
    assert L.kq_stream_read_out(FAKE, 1024, None, 16, 1, 256, None) == kq.KQ_ENULL
    assert L.kq_stream_read_out(FAKE, 1000, FAKE, 16, 1, 256, None) == kq.KQ_EINVAL  # bytes % 16
    assert L.kq_stream_read_out(FAKE, 1024, FAKE, 0, 1, 256, None) == kq.KQ_EINVAL  # no outputs
    assert L.kq_stream_read_out(FAKE, 1024, FAKE, 16, 3, 256, None) == kq.KQ_EINVAL  # unroll
    assert L.kq_stream_read_out(FAKE, 1024, FAKE, 16, 1, 300, None) == kq.KQ_EINVAL  # threads
    assert L.kq_stream_read_out(FAKE, 1024, FAKE + 1, 16, 1, 256, None) == kq.KQ_EALIGN
