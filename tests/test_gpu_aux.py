"""The two auxiliary kernels of the int4 project on the GPU through the C ABI:

* kq_xsum32 (int4-gemv/src/kernels.metal:54-65): per 32-chunk fp32 sums of
  x, bit-exact against the oracle's restatement of the reference's
  summation order;
* kq_stream_read (int4-gemv/src/kernels.metal:260-283): the streaming-read
  ceiling kernel. Its result is a sink written only when some thread's XOR
  fold of its loads is all ones, so a zero buffer with one marked 16-byte
  quad shows that the quad was read (sink set) and a marker just past the
  range shows that nothing beyond `bytes` was (sink untouched).
"""
import numpy as np
import pytest
import torch

import oracle
from kernels_amd import gen, kq
from tests._util import dev

pytestmark = pytest.mark.gpu

SENTINEL = 0x13572468


@pytest.mark.parametrize("batch", [1, 2, 3])
@pytest.mark.parametrize("K", [32, 4096, 14336])
def test_xsum32_bit_exact(gpu, K, batch):
    X = gen.f16_bits(np.random.default_rng(K + batch).normal(0, 1, (batch, K)))
    xs = torch.full((batch, K // 32), float("nan"), dtype=torch.float32, device=gpu)
    kq.xsum32(dev(X, gpu), xs, K, batch)
    torch.cuda.synchronize()
    want = oracle.xsum32(X, K)
    got = xs.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"K={K} batch={batch}: {np.flatnonzero(got != want)[:5]}"


def test_xsum32_order_sensitive_values(gpu):
    """Values whose fp32 sum depends on the association order: 2^24 + 1 - 2^24
    style cancellations inside a chunk (fp16 can hold +-65504 and 1/1024)."""
    K = 256
    v = np.tile(np.array([2048.0, 0.5, -2048.0, 0.25, 1024.0, 0.125, -1024.0, 0.0625],
                         np.float32), K // 8)
    v[::11] = 1.0 / 1024
    X = gen.f16_bits(v.reshape(1, K))
    xs = torch.zeros((1, K // 32), dtype=torch.float32, device=gpu)
    kq.xsum32(dev(X, gpu), xs, K, 1)
    torch.cuda.synchronize()
    want = oracle.xsum32(X, K)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), want.view(np.uint32))


def _sink(gpu):
    return torch.full((1,), SENTINEL, dtype=torch.int32, device=gpu)


# (unroll, threads): the default shape, and shapes of the reference's sweep
SHAPES = [(0, 0), (1, 256), (2, 1024 * 256), (4, 8192 * 256), (8, 2048 * 256)]


@pytest.mark.parametrize("unroll,threads", SHAPES)
@pytest.mark.parametrize("nbytes", [16, 4096, 33_067_008, 16 * 1_000_003])
def test_stream_read_reads_every_quad(gpu, nbytes, unroll, threads):
    nq = nbytes // 16
    buf = torch.zeros(nq * 4 + 4, dtype=torch.int32, device=gpu)  # one spare quad past the end
    sink = _sink(gpu)
    kq.stream_read(buf, nbytes, sink, unroll=unroll, threads=threads)
    torch.cuda.synchronize()
    assert sink.item() == SENTINEL, "all-zero buffer must not set the sink"
    for q in sorted({0, nq // 2, nq - 1, max(0, nq - 257)}):
        buf.zero_()
        buf[4 * q + (q % 4)] = -1  # one word of quad q all ones
        sink = _sink(gpu)
        kq.stream_read(buf, nbytes, sink, unroll=unroll, threads=threads)
        torch.cuda.synchronize()
        assert sink.item() == -1, f"quad {q} of {nq} not read"
    # a marker in the quad just past the range is never read
    buf.zero_()
    buf[4 * nq] = -1
    sink = _sink(gpu)
    kq.stream_read(buf, nbytes, sink, unroll=unroll, threads=threads)
    torch.cuda.synchronize()
    assert sink.item() == SENTINEL, "read past the range"


@pytest.mark.parametrize("nbytes,out_elems,threads", [(1 << 20, 4096, 2048 * 256),
                                                       (1 << 20, 20000, 2048 * 256),
                                                       (4096, 7, 256)])
def test_stream_read_out_writes_exactly_its_outputs(gpu, nbytes, out_elems, threads):
    """kq_stream_read_out writes out[0:out_elems] (each wave's fold: 0 over a
    zero buffer; 20000 outputs over 8192 waves: some waves write three) and
    nothing past it; an all-ones word in quad 0, read by lane 0 of wave 0,
    reaches wave 0's outputs (out[0], out[waves], ...) as 0xFFFF + 0xFFFF =
    0xFFFE (low 16 bits)."""
    buf = torch.zeros(nbytes // 4, dtype=torch.int32, device=gpu)
    out = torch.full((out_elems + 64,), 0x2468, dtype=torch.int16, device=gpu)
    kq.stream_read_out(buf, nbytes, out, out_elems, 1, threads)
    torch.cuda.synchronize()
    o = out.cpu().numpy().view(np.uint16)
    assert (o[:out_elems] == 0).all()
    assert (o[out_elems:] == 0x2468).all()
    buf[0] = -1
    kq.stream_read_out(buf, nbytes, out, out_elems, 1, threads)
    torch.cuda.synchronize()
    o = out.cpu().numpy().view(np.uint16)
    want = np.zeros(out_elems, dtype=np.uint16)
    want[::threads // 64] = 0xFFFE
    assert (o[:out_elems] == want).all() and (o[out_elems:] == 0x2468).all()


def test_stream_read_fold_cancels(gpu):
    """Two all-ones words in the same thread's loads cancel in the XOR fold:
    the sink stays untouched (the fold is really over the loaded values)."""
    nbytes = 4096
    buf = torch.zeros(nbytes // 4, dtype=torch.int32, device=gpu)
    buf[0] = -1
    buf[1] = -1  # same quad, same thread: x ^ y ^ ... = 0
    sink = _sink(gpu)
    kq.stream_read(buf, nbytes, sink)
    torch.cuda.synchronize()
    assert sink.item() == SENTINEL
