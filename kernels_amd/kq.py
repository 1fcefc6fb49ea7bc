"""Python host layer over libkq's C ABI (include/kq.h).

Mirrors the reference's per-kernel call surface: the parameter structs
(GemvParams int4-gemv/src/kernels.metal:42-49, VQParams
vq-gemv/src/kernels.metal:32-37, MoEParams moe-fused/src/kernels.metal:22-35)
and one call per hot-path kernel, taking device buffers. Buffers are torch
tensors on the GPU (torch is only the allocator/stream provider here) or raw
device addresses (int). Every call goes through libkq; there is no fallback:
if the library is missing or a call fails, a KQError is raised.
"""
import ctypes as C
import os
from dataclasses import dataclass

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_lib", "libkq.so")

KQ_OK, KQ_EINVAL, KQ_ENULL, KQ_EALIGN, KQ_EUNSUPPORTED, KQ_EWORKSPACE, KQ_EHIP = range(7)
F16, BF16, F32 = 0, 1, 2
PATH_AUTO, PATH_VALU, PATH_MFMA, PATH_SCALAR = 0, 1, 2, 3
MOE_PATH_AUTO, MOE_PATH_LAUNCHES, MOE_PATH_ONE, MOE_PATH_ATOMIC = 0, 1, 2, 3  # KQ_MOE_PATH_*
MOE_WS_ERR_OFFSET = 128  # KQ_MOE_WS_ERR_OFFSET

# every symbol include/kq.h declares
EXPORTS = ("kq_status_str", "kq_last_hip_error", "kq_version", "kq_int4_gemv",
           "kq_int4_gemv_path", "kq_int4_gemv_cfg", "kq_xsum32", "kq_stream_read",
           "kq_stream_read_cfg", "kq_stream_read_out",
           "kq_vq_gemv", "kq_moe_default_desc", "kq_moe_workspace_size",
           "kq_moe_workspace_init", "kq_moe_workspace_error", "kq_moe_router_topk", "kq_moe_gate_up_swiglu",
           "kq_moe_down_combine", "kq_moe_block", "kq_moe_block_path", "kq_moe_block_noalloc",
           "kq_moe_unfused_workspace_size",
           "kq_moe_block_unfused", "kq_vq_quantize_workspace_size", "kq_vq_quantize")


class KQError(RuntimeError):
    def __init__(self, status, where):
        self.status = status
        msg = lib().kq_status_str(status).decode()
        if status == KQ_EHIP:
            msg += f" (hipError {lib().kq_last_hip_error()})"
        super().__init__(f"{where}: {msg} [kq_status {status}]")


class MoEDesc(C.Structure):
    """kq_moe_desc: MoEParams without its derived fields."""
    _fields_ = [("hidden", C.c_uint32), ("inter", C.c_uint32), ("n_experts", C.c_uint32),
                ("top_k", C.c_uint32), ("blob", C.c_uint64), ("off_gate", C.c_uint64),
                ("off_up", C.c_uint64), ("off_down", C.c_uint64), ("sub_w", C.c_uint64),
                ("sub_s", C.c_uint64), ("sub_b", C.c_uint64), ("sub_bi", C.c_uint64)]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


_lib = None


def lib():
    """Load libkq.so. Raises if it was not built: there is no CPU fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libkq not built: {LIB_PATH} is missing "
                               "(run __graft_entry__.build() or kernels_amd/build.py)")
        L = C.CDLL(LIB_PATH)
        vp, u32, i32, sz = C.c_void_p, C.c_uint32, C.c_int, C.c_size_t
        L.kq_status_str.argtypes = [i32]
        L.kq_status_str.restype = C.c_char_p
        L.kq_last_hip_error.restype = i32
        L.kq_version.restype = C.c_char_p
        L.kq_int4_gemv.argtypes = [vp, vp, vp, i32, vp, vp, i32, u32, u32, u32, u32, vp]
        L.kq_int4_gemv_path.argtypes = [vp, vp, vp, i32, vp, vp, i32, u32, u32, u32, u32, i32, vp]
        L.kq_int4_gemv_cfg.argtypes = [vp, vp, vp, i32, vp, vp, i32, u32, u32, u32, u32, i32,
                                       i32, i32, vp]
        L.kq_xsum32.argtypes = [vp, vp, u32, u32, vp]
        L.kq_stream_read.argtypes = [vp, sz, vp, vp]
        L.kq_stream_read_cfg.argtypes = [vp, sz, vp, u32, u32, vp]
        L.kq_stream_read_out.argtypes = [vp, sz, vp, u32, u32, u32, vp]
        L.kq_vq_gemv.argtypes = [vp, vp, vp, vp, vp, i32, u32, u32, u32, u32, u32, vp]
        L.kq_moe_default_desc.argtypes = [C.POINTER(MoEDesc)]
        L.kq_moe_default_desc.restype = None
        L.kq_moe_workspace_size.argtypes = [C.POINTER(MoEDesc), u32]
        L.kq_moe_workspace_size.restype = sz
        L.kq_moe_workspace_init.argtypes = [vp, sz, vp]
        L.kq_moe_workspace_error.argtypes = [vp, sz, C.POINTER(u32), i32, vp]
        L.kq_moe_router_topk.argtypes = [vp, i32, vp, i32, u32, C.POINTER(MoEDesc), vp, vp, vp,
                                         vp, sz, vp]
        L.kq_moe_gate_up_swiglu.argtypes = [vp, C.POINTER(MoEDesc), vp, vp, vp, u32, vp, sz, vp]
        L.kq_moe_down_combine.argtypes = [vp, C.POINTER(MoEDesc), vp, vp, vp, vp, i32, u32, vp,
                                          sz, vp]
        L.kq_moe_block.argtypes = [vp, C.POINTER(MoEDesc), vp, i32, vp, i32, u32, vp, vp, vp, vp,
                                   vp, i32, vp, sz, vp]
        L.kq_moe_block_path.argtypes = [vp, C.POINTER(MoEDesc), vp, i32, vp, i32, u32, vp, vp, vp,
                                        vp, vp, i32, vp, sz, i32, vp]
        L.kq_moe_block_noalloc.argtypes = [vp, C.POINTER(MoEDesc), vp, i32, vp, i32, u32, vp, vp,
                                           vp, vp, vp, i32, vp]
        L.kq_moe_unfused_workspace_size.argtypes = [C.POINTER(MoEDesc)]
        L.kq_moe_unfused_workspace_size.restype = sz
        L.kq_moe_block_unfused.argtypes = [vp, C.POINTER(MoEDesc), vp, i32, vp, i32, u32, vp, vp,
                                           vp, vp, vp, i32, vp, sz, C.POINTER(u32), vp]
        L.kq_vq_quantize_workspace_size.argtypes = [u32, u32, u32, u32, u32]
        L.kq_vq_quantize_workspace_size.restype = sz
        L.kq_vq_quantize.argtypes = [vp, i32, u32, u32, u32, u32, u32, u32, C.c_uint64, vp, vp,
                                     vp, vp, sz, vp]
        for name in EXPORTS:
            if name not in ("kq_status_str", "kq_last_hip_error", "kq_version",
                            "kq_moe_default_desc", "kq_moe_workspace_size",
                            "kq_moe_unfused_workspace_size", "kq_vq_quantize_workspace_size"):
                getattr(L, name).restype = i32
        _lib = L
    return _lib


def _ptr(t):
    """Device address of a torch tensor (or an int address, or None)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _check(st, where):
    if st != KQ_OK:
        raise KQError(st, where)


def _dt(t):
    import torch
    return {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}[t.dtype]


# ---------------------------------------------------------------------------
# int4 GEMV
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class GemvParams:
    """GemvParams (int4-gemv/src/kernels.metal:42-49); derived fields are
    properties, validated by the library (K % 32, G in {32,64,128})."""
    M: int
    K: int
    G: int = 64

    @property
    def words_pr(self):
        return self.K // 8

    @property
    def groups_pr(self):
        return self.K // self.G

    @property
    def chunks_pg(self):
        return self.G // 32


def int4_gemv(W, SB, x, y, P: GemvParams, B=None, batch=1, sb_dtype=F16, path=PATH_AUTO,
              stream=None, rows=0, unroll=0):
    """y = dequant(W, SB[, B]) . x  (y: [batch][M], fp16 or fp32 by tensor dtype).

    SB alone = interleaved (scale, bias) pairs (the v4-v6 layout,
    int4-gemv/src/main.mm:198-199); SB and B = separate scale and bias arrays
    (the v0-v3 layout). rows/unroll > 0 forces the launch shape."""
    ydt = y if isinstance(y, int) else _dt(y)
    if isinstance(y, int):
        raise TypeError("pass y as a tensor so its dtype is known")
    s = _stream(stream)
    if rows or unroll:
        st = lib().kq_int4_gemv_cfg(_ptr(W), _ptr(SB), _ptr(B), sb_dtype, _ptr(x), _ptr(y), ydt,
                                    P.M, P.K, P.G, batch, path, rows, unroll, s)
    elif path != PATH_AUTO:
        st = lib().kq_int4_gemv_path(_ptr(W), _ptr(SB), _ptr(B), sb_dtype, _ptr(x), _ptr(y), ydt,
                                     P.M, P.K, P.G, batch, path, s)
    else:
        st = lib().kq_int4_gemv(_ptr(W), _ptr(SB), _ptr(B), sb_dtype, _ptr(x), _ptr(y), ydt,
                                P.M, P.K, P.G, batch, s)
    _check(st, "kq_int4_gemv")


def xsum32(x, xs, K, batch=1, stream=None):
    _check(lib().kq_xsum32(_ptr(x), _ptr(xs), K, batch, _stream(stream)), "kq_xsum32")


def stream_read(src, nbytes, sink, stream=None, unroll=0, threads=0):
    """Streaming-read ceiling; unroll/threads > 0 set the launch shape of the
    reference's sweep (int4-gemv/src/main.mm:294-334)."""
    if unroll or threads:
        _check(lib().kq_stream_read_cfg(_ptr(src), nbytes, _ptr(sink), unroll, threads,
                                        _stream(stream)), "kq_stream_read_cfg")
    else:
        _check(lib().kq_stream_read(_ptr(src), nbytes, _ptr(sink), _stream(stream)),
               "kq_stream_read")


def stream_read_out(src, nbytes, out, out_elems, unroll, threads, stream=None):
    """The streaming read, then out_elems 2-byte values written across the
    grid (a GEMV's output store): the ceiling of a kernel that stores y."""
    _check(lib().kq_stream_read_out(_ptr(src), nbytes, _ptr(out), out_elems, unroll, threads,
                                    _stream(stream)), "kq_stream_read_out")


# ---------------------------------------------------------------------------
# VQ GEMV
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class VQParams:
    """VQParams (vq-gemv/src/kernels.metal:32-37) plus the two format knobs:
    rows_per_cb (codebook block height; M = one codebook per matrix, the
    reference) and scale_group (32 = the reference; K = one scale per row)."""
    M: int
    K: int
    rows_per_cb: int
    scale_group: int = 32
    cb_size: int = 256

    @property
    def chunks_pr(self):
        return self.K // 32


def vq_gemv(IDX, Cb, S, x, y, P: VQParams, batch=1, stream=None):
    _check(lib().kq_vq_gemv(_ptr(IDX), _ptr(Cb), _ptr(S), _ptr(x), _ptr(y), _dt(y), P.M, P.K,
                            P.rows_per_cb, P.scale_group, batch, _stream(stream)), "kq_vq_gemv")


def vq_quantize_workspace_size(M, K, rows_per_cb, scale_group, sample=200_000):
    n = lib().kq_vq_quantize_workspace_size(M, K, rows_per_cb, scale_group, sample)
    if n == 0:
        raise KQError(KQ_EINVAL, "kq_vq_quantize_workspace_size")
    return n


def vq_quantize(W, IDX, Cb, S, M, K, rows_per_cb, scale_group, ws, ws_bytes, iters=25,
                sample=200_000, seed=0, w_dtype=None, stream=None):
    """quantize_matrix (vq-gemv/quant/pq_quantize.py:28-83) on the GPU: W
    [M][K] (float32, float16 or bfloat16 tensor) into IDX u8 [M][K/2], Cb
    fp16 [blocks][256][2] and S fp16 [M][K/scale_group]."""
    _check(lib().kq_vq_quantize(_ptr(W), _dt(W) if w_dtype is None else w_dtype, M, K,
                                rows_per_cb, scale_group, iters, sample, seed, _ptr(IDX),
                                _ptr(Cb), _ptr(S), _ptr(ws), ws_bytes, _stream(stream)),
           "kq_vq_quantize")


# ---------------------------------------------------------------------------
# MoE block
# ---------------------------------------------------------------------------
def moe_default_desc():
    d = MoEDesc()
    lib().kq_moe_default_desc(C.byref(d))
    return d


def moe_workspace_size(desc, batch):
    n = lib().kq_moe_workspace_size(C.byref(desc), batch)
    if n == 0:
        raise KQError(KQ_EINVAL, "kq_moe_workspace_size")
    return n


def moe_workspace_init(ws, nbytes, stream=None):
    _check(lib().kq_moe_workspace_init(_ptr(ws), nbytes, _stream(stream)), "kq_moe_workspace_init")


def moe_workspace_error(ws, nbytes, clear=False, stream=None):
    """The workspace's error word after the stream's earlier work (synchronises
    the stream); non-zero: a one-launch block on it gave up waiting."""
    v = C.c_uint32(0)
    _check(lib().kq_moe_workspace_error(_ptr(ws), nbytes, C.byref(v), int(bool(clear)),
                                        _stream(stream)), "kq_moe_workspace_error")
    return v.value


def moe_router_topk(R, x, idx, wgt, desc, ws, ws_bytes, batch=1, xh=None, stream=None):
    _check(lib().kq_moe_router_topk(_ptr(R), _dt(R), _ptr(x), _dt(x), batch, C.byref(desc),
                                    _ptr(idx), _ptr(wgt), _ptr(xh), _ptr(ws), ws_bytes,
                                    _stream(stream)), "kq_moe_router_topk")


def moe_gate_up_swiglu(pool, desc, idx, xh, H, ws, ws_bytes, batch=1, stream=None):
    _check(lib().kq_moe_gate_up_swiglu(_ptr(pool), C.byref(desc), _ptr(idx), _ptr(xh), _ptr(H),
                                       batch, _ptr(ws), ws_bytes, _stream(stream)),
           "kq_moe_gate_up_swiglu")


def moe_down_combine(pool, desc, idx, wgt, H, y, ws, ws_bytes, batch=1, stream=None):
    _check(lib().kq_moe_down_combine(_ptr(pool), C.byref(desc), _ptr(idx), _ptr(wgt), _ptr(H),
                                     _ptr(y), _dt(y), batch, _ptr(ws), ws_bytes, _stream(stream)),
           "kq_moe_down_combine")


def moe_block(pool, desc, R, x, idx, wgt, H, y, ws, ws_bytes, batch=1, xh=None, stream=None,
              path=None):
    """encodeFused (moe-fused/src/main.mm:176-206): router_topk ->
    gate_up_swiglu -> down_combine on one stream. path (MOE_PATH_*): the
    launch structure (None: kq_moe_block, the same as MOE_PATH_AUTO);
    MOE_PATH_ATOMIC is the reference's atomic sum(h) form at 1-2 tokens
    (moe-fused/src/kernels.metal:400-487)."""
    if path is None:
        _check(lib().kq_moe_block(_ptr(pool), C.byref(desc), _ptr(R), _dt(R), _ptr(x), _dt(x),
                                  batch, _ptr(idx), _ptr(wgt), _ptr(xh), _ptr(H), _ptr(y), _dt(y),
                                  _ptr(ws), ws_bytes, _stream(stream)), "kq_moe_block")
    else:
        _check(lib().kq_moe_block_path(_ptr(pool), C.byref(desc), _ptr(R), _dt(R), _ptr(x),
                                       _dt(x), batch, _ptr(idx), _ptr(wgt), _ptr(xh), _ptr(H),
                                       _ptr(y), _dt(y), _ptr(ws), ws_bytes, path,
                                       _stream(stream)), "kq_moe_block_path")


MOE_NOALLOC_WS_BYTES = 1 << 20  # KQ_MOE_NOALLOC_WS_BYTES


def moe_block_noalloc(pool, desc, R, x, idx, wgt, H, y, batch=1, xh=None, stream=None):
    """moe_block on libkq's per-GPU static workspace: no allocation, no
    workspace argument (no reference counterpart; for callers that cannot
    allocate). Calls that overlap on one GPU race."""
    _check(lib().kq_moe_block_noalloc(_ptr(pool), C.byref(desc), _ptr(R), _dt(R), _ptr(x), _dt(x),
                                      batch, _ptr(idx), _ptr(wgt), _ptr(xh), _ptr(H), _ptr(y),
                                      _dt(y), _stream(stream)), "kq_moe_block_noalloc")


def moe_unfused_workspace_size(desc):
    n = lib().kq_moe_unfused_workspace_size(C.byref(desc))
    if n == 0:
        raise KQError(KQ_EINVAL, "kq_moe_unfused_workspace_size")
    return n


def moe_block_unfused(pool, desc, R, x, idx, wgt, H, y, ws, ws_bytes, batch=1, xh=None,
                      stream=None):
    """encodeUnfused (moe-fused/src/main.mm:208-284): the block one operation
    per launch. Returns the number of kernel launches it made."""
    n = C.c_uint32(0)
    _check(lib().kq_moe_block_unfused(_ptr(pool), C.byref(desc), _ptr(R), _dt(R), _ptr(x), _dt(x),
                                      batch, _ptr(idx), _ptr(wgt), _ptr(xh), _ptr(H), _ptr(y),
                                      _dt(y), _ptr(ws), ws_bytes, C.byref(n), _stream(stream)),
           "kq_moe_block_unfused")
    return n.value
