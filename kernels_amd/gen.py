"""Seeded synthetic inputs for the decode-path configurations.

Distributions follow the benchmark configs: int4 nibbles uniform in [0, 15]
(uniform uint32 words), fp16 scale |N(0, 0.02)| and bias N(0, 0.02) per
(row, group), x ~ N(0, 1). `dist="ref"` gives the reference harness's
distributions instead (int4-gemv/src/main.mm:187-207: scale U(-1,1)*0.02,
bias U(-1,1)*0.15, x U(-1,1); vq-gemv/src/main.mm:158-172: codebook U(-1,1),
scale U(-1,1)*0.05), drawn from numpy rather than std::mt19937.

fp16/bf16 tensors are returned as uint16 bit patterns (numpy), so the same
arrays feed the oracle and, uploaded, the GPU.
"""
import numpy as np

MOE_BLOB = 14024704
MOE_OFF = dict(off_gate=0, off_up=4671360, off_down=9342720, sub_w=0, sub_s=4147200,
               sub_b=4406400, sub_bi=4665600)


def f16_bits(a):
    return np.asarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


def bf16_bits(a):
    """float32 -> bf16 bits, round to nearest even."""
    u = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def int4_problem(M, K, G=64, batch=1, seed=12345, dist="cfg", x_dist=None):
    """Returns dict W (uint32 [M][K/8]), S, B (uint16 [M][K/G]), SB (uint16
    [M][K/G][2] interleaved), X (uint16 [batch][K])."""
    rng = np.random.default_rng(seed)
    W = rng.integers(0, 2**32, size=(M, K // 8), dtype=np.uint32)
    ng = K // G
    if dist == "ref":
        S = f16_bits(rng.uniform(-1, 1, (M, ng)) * 0.02)
        B = f16_bits(rng.uniform(-1, 1, (M, ng)) * 0.15)
        X = f16_bits(rng.uniform(-1, 1, (batch, K)))
    else:
        S = f16_bits(np.abs(rng.normal(0.0, 0.02, (M, ng))))
        B = f16_bits(rng.normal(0.0, 0.02, (M, ng)))
        X = f16_bits(rng.normal(0.0, 1.0, (batch, K)))
    SB = np.stack([S, B], axis=-1)
    return dict(W=W, S=S, B=B, SB=np.ascontiguousarray(SB), X=X, M=M, K=K, G=G, batch=batch)


def vq_problem(M, K, rows_per_cb=256, scale_group=None, batch=1, seed=12345, dist="cfg"):
    """IDX uint8 [M][K/2], C uint16 [ceil(M/rows_per_cb)][256][2],
    S uint16 [M][K/scale_group], X uint16 [batch][K]."""
    if scale_group is None:
        scale_group = K
    rng = np.random.default_rng(seed)
    ncb = (M + rows_per_cb - 1) // rows_per_cb
    IDX = rng.integers(0, 256, size=(M, K // 2), dtype=np.uint8)
    ns = K // scale_group
    if dist == "ref":
        C = f16_bits(rng.uniform(-1, 1, (ncb, 256, 2)))
        S = f16_bits(rng.uniform(-1, 1, (M, ns)) * 0.05)
        X = f16_bits(rng.uniform(-1, 1, (batch, K)))
    else:
        C = f16_bits(rng.normal(0.0, 0.02, (ncb, 256, 2)))
        S = f16_bits(np.abs(rng.normal(1.0, 0.1, (M, ns))))
        X = f16_bits(rng.normal(0.0, 1.0, (batch, K)))
    return dict(IDX=IDX, C=C, S=S, X=X, M=M, K=K, rows_per_cb=rows_per_cb,
                scale_group=scale_group, batch=batch)


def quantize_affine_int4(w, group=64):
    """Group-affine 4-bit quantisation of float rows (the MLX/mlx.quantize
    format the blobs use): per group of `group` weights, bias = min,
    scale = (max - min) / 15, q = clip(round((w - bias) / scale), 0, 15).
    Scale and bias are rounded to bf16 first and q is computed against the
    rounded values. Returns (W uint32 [rows][cols/8], S bf16 bits, B bf16
    bits) with nibble j of a word = column 8*word + j."""
    rows, cols = w.shape
    g = w.reshape(rows, cols // group, group).astype(np.float32)
    mn = g.min(axis=2)
    mx = g.max(axis=2)
    S = bf16_bits((mx - mn) / 15.0)
    B = bf16_bits(mn)
    s = (S.astype(np.uint32) << 16).view(np.float32)
    b = (B.astype(np.uint32) << 16).view(np.float32)
    sd = np.where(s == 0, 1.0, s)
    q = np.clip(np.rint((g - b[..., None]) / sd[..., None]), 0, 15).astype(np.uint32)
    q = q.reshape(rows, cols // 8, 8)
    W = np.zeros((rows, cols // 8), np.uint32)
    for j in range(8):
        W |= q[:, :, j] << np.uint32(4 * j)
    return W, S, B


def moe_expert_blob(rng, hidden=2880, inter=2880, blob=MOE_BLOB, off=MOE_OFF, quantize=True):
    """One expert in the gpt-oss blob layout (moe-fused/src/main.mm:23-25):
    gate, up [inter][hidden] and down [hidden][inter], int4 group 64 with
    bf16 S/B and a bf16 output bias BI. quantize=True quantises N(0, 0.02)
    weights; quantize=False draws uniform nibbles and plausible S/B directly
    (same byte layout, much faster)."""
    out = np.zeros(blob, np.uint8)
    for name, rows, cols in (("off_gate", inter, hidden), ("off_up", inter, hidden),
                             ("off_down", hidden, inter)):
        base = off[name]
        if quantize:
            W, S, B = quantize_affine_int4(rng.normal(0.0, 0.02, (rows, cols)).astype(np.float32))
        else:
            W = rng.integers(0, 2**32, size=(rows, cols // 8), dtype=np.uint32)
            S = bf16_bits(np.abs(rng.normal(0.0064, 0.001, (rows, cols // 64))))
            B = bf16_bits(rng.normal(-0.048, 0.004, (rows, cols // 64)))
        BI = bf16_bits(rng.normal(0.0, 0.02, rows))
        for sub, arr in (("sub_w", W), ("sub_s", S), ("sub_b", B), ("sub_bi", BI)):
            raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
            o = base + off[sub]
            out[o:o + raw.size] = raw
    return out


def moe_pool(n_experts, seed=12345, quantize=True, hidden=2880, inter=2880, blob=MOE_BLOB,
             off=MOE_OFF):
    rng = np.random.default_rng(seed)
    return np.concatenate([moe_expert_blob(rng, hidden, inter, blob, off, quantize)
                           for _ in range(n_experts)])


def moe_inputs(n_experts, hidden=2880, batch=1, seed=777, r_dist="cfg"):
    """Router R (fp16 bits [n_experts][hidden], N(0, 0.02)) and x (fp16 bits
    [batch][hidden], N(0, 1))."""
    rng = np.random.default_rng(seed)
    R = f16_bits(rng.normal(0.0, 0.02, (n_experts, hidden)))
    X = f16_bits(rng.normal(0.0, 1.0, (batch, hidden)))
    return R, X


def moe_lcg_inputs(n_experts=128, hidden=2880):
    """The reference harness's closed-form router and input
    (moe-fused/src/main.mm:165-171), in fp32:
      h = uint32(i*1103515245 + 12345) >> 16, R[i] = 0.02f*((int)(h % 2001) - 1000)/1000.0f
      X[i] = 0.05f*((int)(i % 17) - 8)."""
    i = np.arange(n_experts * hidden, dtype=np.uint64)
    h = ((i * np.uint64(1103515245) + np.uint64(12345)) & np.uint64(0xFFFFFFFF)) >> np.uint64(16)
    v = (h % np.uint64(2001)).astype(np.int64) - 1000
    R = (np.float32(0.02) * v.astype(np.float32)) / np.float32(1000.0)
    R = R.astype(np.float32).reshape(n_experts, hidden)
    k = np.arange(hidden)
    X = (np.float32(0.05) * ((k % 17) - 8).astype(np.float32)).astype(np.float32)
    return R, X.reshape(1, hidden)
