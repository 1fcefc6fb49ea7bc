"""kernels_amd -- MI355X (gfx950) decode hot path: int4 GEMV / skinny GEMM,
VQ dequant-GEMV and the three-kernel MoE block, behind libkq's C ABI.

`kernels_amd.kq` is the host layer (ctypes over include/kq.h);
`kernels_amd.gen` builds the seeded synthetic inputs of the benchmark configs.
"""
from . import kq  # noqa: F401
from .kq import (GemvParams, KQError, MoEDesc, VQParams, int4_gemv, lib, moe_block,  # noqa: F401
                 moe_default_desc, moe_down_combine, moe_gate_up_swiglu, moe_router_topk,
                 moe_workspace_init, moe_workspace_size, stream_read, vq_gemv, xsum32)

__all__ = ["kq", "GemvParams", "VQParams", "MoEDesc", "KQError", "lib", "int4_gemv", "vq_gemv",
           "xsum32", "stream_read", "moe_default_desc", "moe_workspace_size",
           "moe_workspace_init", "moe_router_topk", "moe_gate_up_swiglu", "moe_down_combine",
           "moe_block"]
