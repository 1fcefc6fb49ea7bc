"""VQ quantiser on the GPU (kq_vq_quantize through libkq's C ABI) against
the CPU oracle (oracle/vqquant.c): indices, codebooks and scales bit for bit
on small shapes of both formats and all input dtypes; at the benchmark shape
(14336 x 4096) the size-independent properties -- determinism, nearest
codeword, reconstruction error -- and the VQ GEMV on the quantised matrix
against the fp64 GEMV of its dequantisation."""
import numpy as np
import pytest
import torch

import oracle
from kernels_amd import kq
from tests._util import assert_close, dev, host_bits, to_f64

pytestmark = pytest.mark.gpu


def quantize_gpu(device, W, M, K, R, G, iters, sample, seed, w_dtype=None):
    nblk = (M + R - 1) // R
    IDX = torch.zeros((M, K // 2), dtype=torch.uint8, device=device)
    Cb = torch.zeros((nblk, 256, 2), dtype=torch.float16, device=device)
    S = torch.zeros((M, K // G), dtype=torch.float16, device=device)
    wsb = kq.vq_quantize_workspace_size(M, K, R, G, sample)
    ws = torch.empty(wsb, dtype=torch.uint8, device=device)
    kq.vq_quantize(W, IDX, Cb, S, M, K, R, G, ws, wsb, iters=iters, sample=sample, seed=seed,
                   w_dtype=w_dtype)
    torch.cuda.synchronize()
    return IDX, Cb, S


def weights(M, K, seed):
    rng = np.random.default_rng(seed)
    return rng.normal(0, 0.02, (M, K)).astype(np.float32)


# (M, K, rows_per_cb, scale_group, iters, sample, dtype)
CASES = [
    (256, 256, 256, 32, 25, 3000, "f32"),     # reference format, subsampled
    (512, 128, 256, 128, 5, 200_000, "f16"),  # per-row scale, every pair sampled
    (300, 64, 128, 32, 3, 100_000, "bf16"),   # partial last block
    (64, 2048, 16, 2048, 1, 5000, "f32"),     # one scale per row, 4 blocks
    (128, 96, 128, 32, 0, 777, "f16"),        # initial draws only
]


@pytest.mark.parametrize("M,K,R,G,iters,sample,dt", CASES)
def test_quantize_bit_exact_vs_oracle(gpu, M, K, R, G, iters, sample, dt):
    W = weights(M, K, M + K + G)
    if dt == "f32":
        Wh, odt, Wd = W, oracle.F32, torch.from_numpy(W).to(gpu)
    elif dt == "f16":
        Wh = W.astype(np.float16).view(np.uint16)
        odt, Wd = oracle.F16, torch.from_numpy(W).half().to(gpu)
    else:
        Wt = torch.from_numpy(W).bfloat16()
        Wh = Wt.view(torch.int16).numpy().view(np.uint16)
        odt, Wd = oracle.BF16, Wt.to(gpu)
    seed = 1234 + iters
    IDX, Cb, S = quantize_gpu(gpu, Wd, M, K, R, G, iters, sample, seed)
    oIDX, oCb, oS, _ = oracle.vq_quantize(Wh, odt, M, K, R, G, iters=iters, sample=sample,
                                          seed=seed)
    assert np.array_equal(host_bits(S, np.uint16), oS), "scales"
    assert np.array_equal(host_bits(Cb, np.uint16), oCb), "codebooks"
    got = IDX.cpu().numpy()
    assert np.array_equal(got, oIDX), f"indices: {np.mean(got != oIDX):.2e} differ"


def test_quantize_zero_and_constant_rows(gpu):
    """All-zero groups (scale 0, pairs divided by 1) and constant rows."""
    M, K = 64, 128
    W = weights(M, K, 7)
    W[0] = 0.0
    W[5, :32] = 0.01
    Wd = torch.from_numpy(W).to(gpu)
    IDX, Cb, S = quantize_gpu(gpu, Wd, M, K, 32, 32, 4, 900, 5)
    oIDX, oCb, oS, _ = oracle.vq_quantize(W, oracle.F32, M, K, 32, 32, iters=4, sample=900, seed=5)
    assert np.array_equal(host_bits(S, np.uint16), oS)
    assert np.array_equal(host_bits(Cb, np.uint16), oCb)
    assert np.array_equal(IDX.cpu().numpy(), oIDX)


def dequant(IDX, rows, Cb, S, R, G):
    """pq_quantize.dequantize (vq-gemv/quant/pq_quantize.py:79-84) of the
    given rows (IDX and S are those rows), with a codebook per block."""
    n, half = IDX.shape
    K = 2 * half
    C = Cb.astype(np.float64)
    cw = C[(np.asarray(rows) // R)[:, None], IDX.astype(np.int64)]  # [n, K/2, 2]
    return (cw.reshape(n, K // G, G) * S.astype(np.float64)[:, :, None]).reshape(n, K)


@pytest.mark.parametrize("R,G", [(256, 4096), (14336, 32)])
def test_quantize_benchmark_shape(gpu, R, G):
    """14336 x 4096 in the benchmark's format (codebook per 256 rows, one
    scale per row) and the reference's (one codebook, scale per 32): two
    runs are identical; sampled rows sit on their nearest codeword; the
    relative reconstruction error is that of the small cases; and the VQ
    GEMV over the output matches the fp64 GEMV of its dequantisation."""
    M, K = 14336, 4096
    Wd = (torch.randn((M, K), generator=torch.Generator(device=gpu).manual_seed(3),
                      device=gpu) * 0.02)
    a = quantize_gpu(gpu, Wd, M, K, R, G, 25, 200_000, 77)
    b = quantize_gpu(gpu, Wd, M, K, R, G, 25, 200_000, 77)
    assert all(torch.equal(x, y) for x, y in zip(a, b)), "not deterministic"
    IDX, Cb, S = (t.cpu().numpy() for t in a)
    Cb = Cb.astype(np.float32)
    S = S.astype(np.float32)
    rows = np.random.default_rng(0).choice(M, 24, replace=False)
    W = Wd[torch.from_numpy(rows).to(gpu)].cpu().numpy().astype(np.float64)
    g = W.reshape(len(rows), K // G, G)
    sc = np.abs(g).max(axis=2)
    U = (g / np.where(sc > 0, sc, 1)[:, :, None]).reshape(len(rows), K // 2, 2)
    for r, m in enumerate(rows):
        C = Cb[m // R].astype(np.float64)
        d2 = ((U[r][:, None, :] - C[None]) ** 2).sum(-1)
        got = d2[np.arange(K // 2), IDX[m]]
        # assignment used the fp32 centroids; the stored codebook is fp16
        assert np.mean(got <= d2.min(axis=1) + 2e-3) > 0.999, m
    Wq = dequant(IDX[rows], rows, Cb, S[rows], R, G)
    rel = np.sqrt(np.mean((Wq - W) ** 2) / np.mean(W ** 2))
    assert rel < 0.1, rel
    # the GEMV on the quantised matrix
    X = torch.randn((1, K), device=gpu).half()
    Y = torch.zeros((1, M), dtype=torch.float32, device=gpu)
    kq.vq_gemv(a[0], a[1], a[2], X, Y, kq.VQParams(M, K, R, G))
    torch.cuda.synchronize()
    Yref = oracle.vq_gemv(IDX, host_bits(a[1], np.uint16), host_bits(a[2], np.uint16),
                          host_bits(X, np.uint16), M, K, R, G)
    assert_close(to_f64(Y), Yref, what="vq gemv on quantised weights")
