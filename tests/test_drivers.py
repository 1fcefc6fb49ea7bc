"""The C++ host drivers (int4gemv, vqgemv, moefused; the counterparts of the
reference's int4-gemv/src/main.mm, vq-gemv/src/main.mm and
moe-fused/src/main.mm).

CPU: the binaries are built and print their usage. GPU: each driver runs a
small configuration end to end (its own fp64 check must pass, exit 0), and
the tensors its --dump writes are checked against the CPU oracle:
int4/VQ outputs within |d| <= 1e-2 + 1e-3 |ref|; the MoE routing of the
reference's LCG inputs equal to the golden fixture moe-fused/results/topk.txt
(indices exact, weights within 1e-6) and y against the oracle's block."""
import json
import os
import subprocess

import numpy as np
import pytest

import oracle
from kernels_amd import gen
from tests._util import assert_close, inf_rel

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "kernels_amd", "_bin")
GOLD = os.path.join(os.path.dirname(__file__), "golden")
DRIVERS = ("int4gemv", "vqgemv", "moefused", "moepipe")


def _exe(name):
    path = os.path.join(BIN, name)
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (run __graft_entry__.build())")
    return path


def _run(name, *args, timeout=240):
    cmd = [_exe(name)] + [str(a) for a in args]
    print("running", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, f"{name} exited {r.returncode}"
    return r.stdout


@pytest.mark.parametrize("name", DRIVERS)
def test_driver_usage(name):
    r = subprocess.run([_exe(name), "--help"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0
    assert r.stdout.startswith(name)


def _f16(path):
    return np.fromfile(path, np.uint16)


def _ys(tmp, ext):
    out = {f: os.path.join(tmp, f) for f in os.listdir(tmp) if f.startswith("y_") and f.endswith(ext)}
    assert out, f"no y_*{ext} dumped"
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,G,batch,y", [(300, 1024, 64, 1, "f16"), (256, 2048, 32, 4, "f32"),
                                           (512, 4096, 128, 8, "f16")])
def test_int4gemv_driver(tmp_path, M, K, G, batch, y):
    out = _run("int4gemv", "--M", M, "--K", K, "--G", G, "--batch", batch, "--y", y,
               "--rot-mb", 16, "--iters", 3, "--warmup", 1, "--repeat", 2, "--dump", tmp_path)
    assert "all variants verified" in out
    W = np.fromfile(tmp_path / "W.u32", np.uint32)
    S, B, X = _f16(tmp_path / "S.f16"), _f16(tmp_path / "B.f16"), _f16(tmp_path / "x.f16")
    ref = oracle.int4_gemv(W, S, B, X, M, K, G, False)
    for name, path in _ys(tmp_path, "." + y).items():
        got = (np.fromfile(path, np.float32) if y == "f32"
               else _f16(path).view(np.float16)).astype(np.float64).reshape(batch, M)
        assert_close(got, ref, what=name)
        assert inf_rel(got, ref) < 2e-3


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,M,K,batch", [("ref", 384, 2048, 1), ("cfg", 512, 4096, 2)])
def test_vqgemv_driver(tmp_path, fmt, M, K, batch):
    out = _run("vqgemv", "--M", M, "--K", K, "--format", fmt, "--batch", batch, "--rot-mb", 16,
               "--iters", 3, "--warmup", 1, "--repeat", 2, "--dump", tmp_path)
    assert "all variants verified" in out
    M_, K_, rpc, sg, b_ = map(int, open(tmp_path / "shape.txt").read().split())
    assert (M_, K_, b_) == (M, K, batch)
    X = _f16(tmp_path / "x.f16")
    vq = oracle.vq_gemv(np.fromfile(tmp_path / "IDX.u8", np.uint8), _f16(tmp_path / "C.f16"),
                        _f16(tmp_path / "S.f16"), X, M, K, rpc, sg)
    SB = _f16(tmp_path / "SB.f16")
    i4 = oracle.int4_gemv(np.fromfile(tmp_path / "W.u32", np.uint32), SB, None, X, M, K, 64, True)
    ys = _ys(tmp_path, ".f32")
    for name, path in ys.items():
        got = np.fromfile(path, np.float32).astype(np.float64).reshape(batch, M)
        assert_close(got, i4 if "int4" in name else vq, what=name)


def _lcg_inputs(ne, hid, batch):
    """moe-fused/src/main.mm:160-171 (token b shifts the x pattern by 7b)."""
    i = np.arange(ne * hid, dtype=np.uint64)
    h = ((i * np.uint64(1103515245) + np.uint64(12345)) & np.uint64(0xFFFFFFFF)) >> np.uint64(16)
    R = (np.float32(0.02) * ((h % np.uint64(2001)).astype(np.int32) - 1000).astype(np.float32)
         / np.float32(1000.0)).astype(np.float32).reshape(ne, hid)
    k = np.arange(hid)
    X = np.stack([np.float32(0.05) * (((k + 7 * b) % 17) - 8).astype(np.float32)
                  for b in range(batch)]).astype(np.float32)
    return R, X


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [1, 3])
def test_moefused_driver(tmp_path, batch):
    out = _run("moefused", "--batch", batch, "--resident", 1, "--iters", 2, "--warmup", 1,
               "--repeat", 2, "--dump", tmp_path)
    assert "FAIL" not in out
    rows = [l.split() for l in open(tmp_path / "topk.txt").read().splitlines()]
    idx = np.array([int(r[0]) for r in rows], np.uint32).reshape(batch, -1)
    wgt = np.array([float(r[1]) for r in rows]).reshape(batch, -1)
    gold = json.load(open(os.path.join(GOLD, "moe_topk_lcg.json")))
    assert idx[0].tolist() == gold["expected_idx"]
    np.testing.assert_allclose(wgt[0], gold["expected_wgt"], atol=1e-6, rtol=0)

    d = oracle.MoEDesc(2880, 2880, 128, 4, 14024704, 0, 4671360, 9342720, 0, 4147200, 4406400,
                       4665600)
    R, X = _lcg_inputs(d.n_experts, d.hidden, batch)
    oidx, owgt, _ = oracle.moe_router(R, oracle.F32, X, oracle.F32, batch, d)
    assert np.array_equal(oidx, idx)
    np.testing.assert_allclose(wgt, owgt, atol=1e-6, rtol=0)
    # y from the dumped selected experts, packed into a small pool
    uniq = sorted(set(idx.ravel().tolist()))
    pool = np.concatenate([np.fromfile(tmp_path / f"expert_{e}.bin", np.uint8) for e in uniq])
    small = oracle.MoEDesc(*[getattr(d, f) for f, _ in oracle.MoEDesc._fields_])
    small.n_experts = len(uniq)
    sidx = np.vectorize(uniq.index)(idx).astype(np.uint32)
    Xh = X.astype(np.float16).view(np.uint16)  # the projections read half(x)
    H = oracle.moe_gate_up(pool, small, sidx, Xh, oracle.F16, batch)
    Hh = H.astype(np.float16).view(np.uint16)  # the kernels hand h over in fp16
    Y = oracle.moe_down(pool, small, sidx, owgt, Hh, batch)
    got = np.fromfile(tmp_path / "y.f32", np.float32).astype(np.float64).reshape(batch, -1)
    assert_close(got, Y, what="moefused y")
    assert inf_rel(got, Y) < 2e-3


@pytest.mark.gpu
def test_moefused_driver_store(tmp_path):
    """The real-weight path: an expert store in the reference's on-disk
    layout (n_experts blobs of 14,024,704 B, moe-fused/src/main.mm:129-149)
    written from gen.moe_pool, read back by moefused --store with pread. The
    dumped selected experts equal the store's bytes (the loader read the
    right blobs), routing equals the oracle's on the reference's LCG inputs,
    and y equals the oracle's block computed from the store. The reference's
    own real-weight golden (moe-fused/results/y_metal.f32) needs its
    experts.bin, which is not in this image: that output stays unpinned."""
    n = 16
    d = oracle.MoEDesc(2880, 2880, n, 4, 14024704, 0, 4671360, 9342720, 0, 4147200, 4406400,
                       4665600)
    host = gen.moe_pool(n, seed=4242, quantize=True)
    store = tmp_path / "experts.bin"
    host.tofile(store)
    dump = tmp_path / "dump"
    dump.mkdir()
    out = _run("moefused", "--store", store, "--experts", n, "--batch", 1, "--resident", 1,
               "--iters", 2, "--warmup", 1, "--repeat", 2, "--dump", dump)
    assert "FAIL" not in out and "loading 16 experts" in out
    rows = [l.split() for l in open(dump / "topk.txt").read().splitlines()]
    idx = np.array([int(r[0]) for r in rows], np.uint32).reshape(1, -1)
    wgt = np.array([float(r[1]) for r in rows]).reshape(1, -1)
    R, X = _lcg_inputs(n, d.hidden, 1)
    oidx, owgt, _ = oracle.moe_router(R, oracle.F32, X, oracle.F32, 1, d)
    assert np.array_equal(oidx, idx)
    np.testing.assert_allclose(wgt, owgt, atol=1e-6, rtol=0)
    blobs = host.reshape(n, d.blob)
    for e in idx.ravel().tolist():
        assert np.array_equal(np.fromfile(dump / f"expert_{e}.bin", np.uint8), blobs[e]), e
    Xh = X.astype(np.float16).view(np.uint16)
    H = oracle.moe_gate_up(host, d, oidx, Xh, oracle.F16, 1)
    Y = oracle.moe_down(host, d, oidx, owgt, H.astype(np.float16).view(np.uint16), 1)
    got = np.fromfile(dump / "y.f32", np.float32).astype(np.float64).reshape(1, -1)
    assert_close(got, Y, what="moefused --store y")
    assert inf_rel(got, Y) < 2e-3


@pytest.mark.gpu
def test_moepipe_store(tmp_path):
    """The expert streaming pipeline (moe-pipeline/src/main.mm): 12 experts
    of a store file streamed through 5 pinned slots (depth 3) and 2 HBM
    slots, every expert computed as it lands. The driver compares every
    expert's y of the pipelined run with the stop-and-wait run bit for bit
    (same kernels and inputs: a slot overwritten too early would show);
    expert 0's h and y, dumped by --verify, are checked against the oracle."""
    n = 12
    blob = 14024704
    host = gen.moe_pool(n, seed=777, quantize=False)
    store = tmp_path / "experts.bin"
    host.tofile(store)
    vd = tmp_path / "verify"
    vd.mkdir()
    out = _run("moepipe", "--store", store, "--experts", n, "--depth", 3, "--workers", 2,
               "--reps", 1, "--verify", vd)
    assert f"pipe outputs == seq outputs (bitwise, {n} experts): OK" in out
    off = int(open(vd / "meta.txt").read().split()[0])
    assert off % blob == 0
    e = off // blob
    d = oracle.MoEDesc(2880, 2880, n, 1, blob, 0, 4671360, 9342720, 0, 4147200, 4406400, 4665600)
    x = np.fromfile(vd / "x.f32", np.float32)
    k = np.arange(2880)
    assert np.array_equal(x, (np.float32(0.05) * ((k % 17) - 8)).astype(np.float32))
    Xh = x.reshape(1, -1).astype(np.float16).view(np.uint16)
    idx = np.array([[e]], np.uint32)
    H = oracle.moe_gate_up(host, d, idx, Xh, oracle.F16, 1)
    h = np.fromfile(vd / "h.f16", np.float16).astype(np.float64).reshape(H.shape)
    assert_close(h, H, what="moepipe h")
    Y = oracle.moe_down(host, d, idx, np.ones((1, 1)), h.astype(np.float16).view(np.uint16), 1)
    y = np.fromfile(vd / "y.f32", np.float32).astype(np.float64).reshape(1, -1)
    assert_close(y, Y, what="moepipe y")
    assert inf_rel(y, Y) < 2e-3
