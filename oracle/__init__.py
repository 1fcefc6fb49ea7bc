"""CPU oracle for the decode hot path -- TEST INFRASTRUCTURE ONLY.

ctypes bindings over oracle/_build/libkqref.so (built by oracle/build.py).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, as the checker or the timed CPU baseline. The product
(kernels_amd / libkq) never imports it.

All fp16/bf16 arrays are numpy uint16 bit patterns; results are float64.
"""
import ctypes as C
import os

import numpy as np

from . import build as _build

F16, BF16, F32 = 0, 1, 2

_lib = None


class MoEDesc(C.Structure):
    """Same field order as kq_moe_desc (include/kq.h) and MoEParams
    (moe-fused/src/kernels.metal:22-35, without the derived fields)."""
    _fields_ = [("hidden", C.c_uint32), ("inter", C.c_uint32), ("n_experts", C.c_uint32),
                ("top_k", C.c_uint32), ("blob", C.c_uint64), ("off_gate", C.c_uint64),
                ("off_up", C.c_uint64), ("off_down", C.c_uint64), ("sub_w", C.c_uint64),
                ("sub_s", C.c_uint64), ("sub_b", C.c_uint64), ("sub_bi", C.c_uint64)]


def lib():
    global _lib
    if _lib is None:
        path = _build.LIB
        if not os.path.exists(path):
            _build.build()
        L = C.CDLL(path)
        vp, u32, i32 = C.c_void_p, C.c_uint32, C.c_int
        L.kqref_f16_to_f64.argtypes = [C.c_uint16]
        L.kqref_f16_to_f64.restype = C.c_double
        L.kqref_bf16_to_f64.argtypes = [C.c_uint16]
        L.kqref_bf16_to_f64.restype = C.c_double
        L.kqref_f32_to_f16.argtypes = [C.c_float]
        L.kqref_f32_to_f16.restype = C.c_uint16
        L.kqref_int4_gemv_f64.argtypes = [vp, vp, vp, i32, i32, vp, vp, u32, u32, u32, u32, i32]
        L.kqref_xsum32.argtypes = [vp, vp, u32, u32]
        L.kqref_vq_gemv_f64.argtypes = [vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, i32]
        L.kqref_moe_router_f64.argtypes = [vp, i32, vp, i32, u32, C.POINTER(MoEDesc), vp, vp, vp]
        L.kqref_moe_proj_f64.argtypes = [vp, C.c_uint64, C.POINTER(MoEDesc), vp, vp, u32, u32, i32]
        L.kqref_swiglu_f64.argtypes = [C.c_double, C.c_double]
        L.kqref_swiglu_f64.restype = C.c_double
        L.kqref_moe_gate_up_f64.argtypes = [vp, C.POINTER(MoEDesc), vp, vp, i32, u32, vp, i32]
        L.kqref_moe_down_f64.argtypes = [vp, C.POINTER(MoEDesc), vp, vp, vp, i32, u32, vp, i32]
        L.kqref_moe_block_f64.argtypes = [vp, C.POINTER(MoEDesc), vp, i32, vp, i32, u32, vp, vp,
                                          vp, i32]
        L.kqref_int4_gemv_cpu_fast.argtypes = [vp, vp, vp, vp, u32, u32, u32, i32]
        L.kqref_int4_gemv_cpu_fast_path.argtypes = [vp, vp, vp, vp, u32, u32, u32, i32, i32]
        L.kqref_cpu_fast_path_name.argtypes = [i32]
        L.kqref_cpu_fast_path_name.restype = C.c_char_p
        L.kqref_cpu_fast_supported.restype = i32
        L.kqref_vq_quantize.argtypes = [vp, i32, u32, u32, u32, u32, u32, u32, C.c_uint64, vp,
                                        vp, vp, vp]
        L.kqref_vq_hash.argtypes = [C.c_uint64, u32, u32]
        L.kqref_vq_hash.restype = C.c_uint64
        L.kqref_vq_score.argtypes = [C.c_float] * 4
        L.kqref_vq_score.restype = C.c_float
        L.kqref_vq_fix.argtypes = [C.c_float]
        L.kqref_vq_fix.restype = C.c_int64
        L.kqref_vq_mean.argtypes = [C.c_int64, C.c_uint64]
        L.kqref_vq_mean.restype = C.c_float
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def _c(a, dtype):
    a = np.ascontiguousarray(a)
    assert a.dtype == dtype, (a.dtype, dtype)
    return a


def f16_to_f64(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


def int4_gemv(W, S, B, X, M, K, G, sb_interleaved, sb_dtype=F16, nthreads=0):
    """fp64 int4 GEMV; X is uint16 [batch][K] (fp16 bits). Returns [batch][M]."""
    W = _c(W, np.uint32)
    S = _c(S, np.uint16)
    B = _c(B, np.uint16) if B is not None else None
    X = _c(X, np.uint16).reshape(-1, K)
    batch = X.shape[0]
    Y = np.zeros((batch, M), np.float64)
    lib().kqref_int4_gemv_f64(_p(W), _p(S), _p(B), int(sb_interleaved), sb_dtype, _p(X), _p(Y),
                              M, K, G, batch, nthreads)
    return Y


def xsum32(X, K):
    X = _c(X, np.uint16).reshape(-1, K)
    xs = np.zeros((X.shape[0], K // 32), np.float32)
    lib().kqref_xsum32(_p(X), _p(xs), K, X.shape[0])
    return xs


def vq_gemv(IDX, Cb, S, X, M, K, rows_per_cb, scale_group, nthreads=0):
    IDX = _c(IDX, np.uint8)
    Cb = _c(Cb, np.uint16)
    S = _c(S, np.uint16)
    X = _c(X, np.uint16).reshape(-1, K)
    batch = X.shape[0]
    Y = np.zeros((batch, M), np.float64)
    lib().kqref_vq_gemv_f64(_p(IDX), _p(Cb), _p(S), _p(X), _p(Y), M, K, rows_per_cb, scale_group,
                            batch, nthreads)
    return Y


def moe_router(R, r_dtype, X, x_dtype, batch, desc):
    R = np.ascontiguousarray(R)
    X = np.ascontiguousarray(X)
    idx = np.zeros((batch, desc.top_k), np.uint32)
    wgt = np.zeros((batch, desc.top_k), np.float64)
    lg = np.zeros((batch, desc.n_experts), np.float64)
    lib().kqref_moe_router_f64(_p(R), r_dtype, _p(X), x_dtype, batch, C.byref(desc), _p(idx),
                               _p(wgt), _p(lg))
    return idx, wgt, lg


def moe_proj(blob, proj, desc, x, M, K, nthreads=0):
    blob = _c(blob, np.uint8)
    x = _c(x, np.float64)
    y = np.zeros(M, np.float64)
    lib().kqref_moe_proj_f64(_p(blob), proj, C.byref(desc), _p(x), _p(y), M, K, nthreads)
    return y


def swiglu(g, u):
    return lib().kqref_swiglu_f64(float(g), float(u))


def moe_gate_up(pool, desc, idx, X, x_dtype, batch, nthreads=0):
    pool = _c(pool, np.uint8)
    idx = _c(idx, np.uint32)
    X = np.ascontiguousarray(X)
    H = np.zeros((batch, desc.top_k, desc.inter), np.float64)
    lib().kqref_moe_gate_up_f64(_p(pool), C.byref(desc), _p(idx), _p(X), x_dtype, batch, _p(H),
                                nthreads)
    return H


def moe_down(pool, desc, idx, wgt, H, batch, nthreads=0):
    """H: float64 array, or uint16 fp16 bits."""
    pool = _c(pool, np.uint8)
    idx = _c(idx, np.uint32)
    wgt = _c(np.asarray(wgt, np.float64), np.float64)
    H = np.ascontiguousarray(H)
    hd = F16 if H.dtype == np.uint16 else F32
    if hd == F32:
        H = _c(H, np.float64)
    Y = np.zeros((batch, desc.hidden), np.float64)
    lib().kqref_moe_down_f64(_p(pool), C.byref(desc), _p(idx), _p(wgt), _p(H), hd, batch, _p(Y),
                             nthreads)
    return Y


def moe_block(pool, desc, R, r_dtype, X, x_dtype, batch, nthreads=0):
    pool = _c(pool, np.uint8)
    R = np.ascontiguousarray(R)
    X = np.ascontiguousarray(X)
    idx = np.zeros((batch, desc.top_k), np.uint32)
    wgt = np.zeros((batch, desc.top_k), np.float64)
    Y = np.zeros((batch, desc.hidden), np.float64)
    lib().kqref_moe_block_f64(_p(pool), C.byref(desc), _p(R), r_dtype, _p(X), x_dtype, batch,
                              _p(idx), _p(wgt), _p(Y), nthreads)
    return idx, wgt, Y


def cpu_fast_supported():
    return bool(lib().kqref_cpu_fast_supported())


CPU_AVX2, CPU_AVX512, CPU_FP16 = 1, 2, 3


def cpu_fast_path_name(path=0):
    return lib().kqref_cpu_fast_path_name(path).decode()


def int4_gemv_cpu_fast(W, SB, X, M, K, G, nthreads=0, path=0):
    """The reference's CPU int4 GEMV restated for x86 (path 0: the fastest
    this CPU has; CPU_FP16 = neon16, CPU_AVX512 / CPU_AVX2 = neon fp32)."""
    W = _c(W, np.uint32)
    SB = _c(SB, np.uint16)
    X = _c(X, np.uint16)
    Y = np.zeros(M, np.float32)
    lib().kqref_int4_gemv_cpu_fast_path(_p(W), _p(SB), _p(X), _p(Y), M, K, G, nthreads, path)
    return Y


def vq_quantize(W, w_dtype, M, K, rows_per_cb, scale_group, iters=25, sample=200_000, seed=0):
    """VQ quantiser (vq-gemv/quant/pq_quantize.py:28-83 as specified for the
    GPU). W: float32 [M][K] (w_dtype F32) or uint16 bits (F16 / BF16).
    Returns (IDX u8 [M][K/2], C fp16 bits [nblk][256][2], S fp16 bits
    [M][K/scale_group], fp32 centroids [nblk][256][2])."""
    W = np.ascontiguousarray(W)
    nblk = (M + rows_per_cb - 1) // rows_per_cb
    IDX = np.zeros((M, K // 2), np.uint8)
    Cb = np.zeros((nblk, 256, 2), np.uint16)
    S = np.zeros((M, K // scale_group), np.uint16)
    cent = np.zeros((nblk, 256, 2), np.float32)
    lib().kqref_vq_quantize(_p(W), w_dtype, M, K, rows_per_cb, scale_group, iters, sample, seed,
                            _p(IDX), _p(Cb), _p(S), _p(cent))
    return IDX, Cb, S, cent
