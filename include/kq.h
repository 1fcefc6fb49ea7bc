/*
 * kq.h -- C ABI of libkq, the MI355X (gfx950) decode hot path:
 *   int4 group-affine GEMV / batched skinny GEMM, codebook (VQ) dequant-GEMV,
 *   and the three-kernel MoE block (router top-k, gathered gate/up + SwiGLU,
 *   gathered down + weighted combine).
 *
 * Every entry point is stream-ordered and asynchronous: it validates its
 * arguments on the host, enqueues kernels on `stream` and returns. Nothing
 * here allocates device memory, synchronises, prints or exits. All pointers
 * are caller-owned device pointers (W, IDX and X 16-byte aligned). Errors are
 * reported as kq_status; kq_last_hip_error() gives the HIP code behind
 * KQ_EHIP.
 *
 * The reference (Apple Metal) exposes this path only as per-kernel call
 * surfaces encoded by its Objective-C++ harnesses; each declaration below
 * cites the kernel and the encode site it replaces (paths are relative to the
 * reference repository root).
 */
#ifndef KQ_H
#define KQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same type as hipStream_t; NULL is the default stream. */
typedef struct ihipStream_t* kq_stream_t;

typedef enum kq_status {
    KQ_OK = 0,
    KQ_EINVAL = 1,        /* shape or argument violates the format contract */
    KQ_ENULL = 2,         /* a required pointer is NULL */
    KQ_EALIGN = 3,        /* a pointer is not aligned as required */
    KQ_EUNSUPPORTED = 4,  /* well-formed but not implemented (dtype, batch) */
    KQ_EWORKSPACE = 5,    /* workspace NULL or smaller than required */
    KQ_EHIP = 6           /* the HIP runtime rejected a launch */
} kq_status;

typedef enum kq_dtype { KQ_F16 = 0, KQ_BF16 = 1, KQ_F32 = 2 } kq_dtype;

/* Kernel family used by kq_int4_gemv_path (0 picks by batch size).
 * KQ_PATH_SCALAR: the debug scalar kernel, one thread per (row, token) with
 * a plain per-chunk loop and no staging, after gemv_int4_scalar (v0,
 * int4-gemv/src/kernels.metal:71-95) -- slow, for checking the fast paths
 * on the device; AUTO never picks it. */
typedef enum kq_int4_path {
    KQ_PATH_AUTO = 0,
    KQ_PATH_VALU = 1,
    KQ_PATH_MFMA = 2,
    KQ_PATH_SCALAR = 3
} kq_int4_path;

const char* kq_status_str(kq_status s);
/* hipError_t of the last KQ_EHIP returned on this host thread (0 if none). */
int kq_last_hip_error(void);
/* Library version string, e.g. "kq 0.1 gfx950". */
const char* kq_version(void);

/* ------------------------------------------------------------------------
 * int4 group-affine GEMV / skinny GEMM
 *
 *   Y[b, m] = sum_k (S[m, k/G] * q[m, k] + B[m, k/G]) * X[b, k]
 *   q[m, k] = (W[m, k/8] >> 4*(k%8)) & 0xF          (low nibble = lowest k)
 *
 * W  : uint32 [M][K/8], row-major.
 * S,B: per (row, group) scale and bias, dtype sb_dtype (KQ_F16 or KQ_BF16).
 *      B == NULL selects the interleaved layout: S points at SB[M][K/G][2]
 *      (scale, bias) pairs. B != NULL selects separate S[M][K/G], B[M][K/G].
 * X  : fp16 [batch][K].  Y: [batch][M] of y_dtype (KQ_F16 or KQ_F32).
 * Accumulation is fp32. Constraints: K % 32 == 0, G in {32, 64, 128},
 * K % G == 0, 1 <= batch <= 16, M >= 1. The activations are staged in LDS,
 * which bounds K (K <= 29120 on the VALU path); a shape no path takes
 * returns KQ_EUNSUPPORTED.
 *
 * Replaces: gemv_int4_wide_unroll (v6, interleaved SB)
 *   int4-gemv/src/kernels.metal:397-448, encoded by addGemv
 *   int4-gemv/src/main.mm:353-377,404-408; and the split-S/B layout of
 *   gemv_int4_scalar / gemv_int4_simd int4-gemv/src/kernels.metal:71-136.
 *   batch > 1 has no reference kernel (it is the per-row batch-1 op).
 * ------------------------------------------------------------------------ */
kq_status kq_int4_gemv(const uint32_t* W, const void* S, const void* B, kq_dtype sb_dtype,
                       const uint16_t* X, void* Y, kq_dtype y_dtype,
                       uint32_t M, uint32_t K, uint32_t G, uint32_t batch,
                       kq_stream_t stream);

/* kq_int4_gemv with the kernel family forced (VALU dot2 path, MFMA
 * 16x16x32 path, or the debug scalar kernel); used to measure the crossover
 * and to cross-check the paths. Same contract (the scalar kernel has no K
 * limit beyond it). */
kq_status kq_int4_gemv_path(const uint32_t* W, const void* S, const void* B, kq_dtype sb_dtype,
                            const uint16_t* X, void* Y, kq_dtype y_dtype,
                            uint32_t M, uint32_t K, uint32_t G, uint32_t batch,
                            kq_int4_path path, kq_stream_t stream);

/* Tuning entry point: kq_int4_gemv with the kernel family and launch shape
 * forced; 0 = automatic for either field.
 * VALU: rows = K parts P per workgroup (a divisor of the number of 2048-k
 * steps), unroll = ring depth D (2, 4, 8).
 * MFMA: rows = K parts P per workgroup (a divisor of K/128; at most 8 with
 * 2 or 4 tiles per wave, else 16), unroll = 10 * T + D with T the 16-row
 * tiles per wave and D its ring depth in steps: 12, 24 or 42.
 * Returns KQ_EUNSUPPORTED for a shape the family cannot run. Used by the
 * benchmark sweeps and the tests. */
kq_status kq_int4_gemv_cfg(const uint32_t* W, const void* S, const void* B, kq_dtype sb_dtype,
                           const uint16_t* X, void* Y, kq_dtype y_dtype,
                           uint32_t M, uint32_t K, uint32_t G, uint32_t batch,
                           kq_int4_path path, int rows, int unroll, kq_stream_t stream);

/* xs[b, j] = sum_{i<32} X[b, 32j + i] in fp32, for j < K/32.
 * Replaces: xsum32 int4-gemv/src/kernels.metal:54-65 (encoded at
 * int4-gemv/src/main.mm:247-258). kq_int4_gemv computes this itself. */
kq_status kq_xsum32(const uint16_t* X, float* xs, uint32_t K, uint32_t batch,
                    kq_stream_t stream);

/* Streaming read of `bytes` (multiple of 16) from src, XOR-folded; writes to
 * sink[0] only if the fold is all ones. The bandwidth ceiling.
 * Replaces: stream_read int4-gemv/src/kernels.metal:260-283. */
kq_status kq_stream_read(const void* src, size_t bytes, uint32_t* sink, kq_stream_t stream);

/* kq_stream_read with the launch shape of the reference's ceiling sweep:
 * `unroll` (1, 2, 4 or 8) independent loads in flight per thread, over
 * `threads` threads (a multiple of 256). kq_stream_read uses the best
 * shape measured on MI355X (unroll 1, 2048 x 256 threads).
 * Replaces: stream_read with function constant UNROLL and its dispatch
 * size int4-gemv/src/kernels.metal:260-283, swept by
 * int4-gemv/src/main.mm:294-334. */
kq_status kq_stream_read_cfg(const void* src, size_t bytes, uint32_t* sink, uint32_t unroll,
                             uint32_t threads, kq_stream_t stream);

/* kq_stream_read_cfg that then writes `out_elems` 2-byte values to out: lane
 * 0 of every wave of the grid writes its fold to out[w], out[w + waves], ...
 * -- a GEMV's output store (y of out_elems rows, written from every XCD)
 * after the same read. No counterpart in the reference: a measurement entry,
 * so that a kernel that must store its output is also compared with a read
 * that pays for the same store at the end of its launch. */
kq_status kq_stream_read_out(const void* src, size_t bytes, uint16_t* out, uint32_t out_elems,
                             uint32_t unroll, uint32_t threads, kq_stream_t stream);

/* ------------------------------------------------------------------------
 * Codebook (VQ, d = 2, 256 entries) dequant-GEMV
 *
 *   Y[b, m] = sum_i S[m, 2i / scale_group] *
 *             ( C[m / rows_per_cb][IDX[m, i]][0] * X[b, 2i]
 *             + C[m / rows_per_cb][IDX[m, i]][1] * X[b, 2i+1] )
 *
 * IDX: uint8 [M][K/2].  C: fp16 [ceil(M/rows_per_cb)][256][2].
 * S  : fp16 [M][K/scale_group].  X: fp16 [batch][K].  Y: [batch][M].
 * rows_per_cb = M and scale_group = 32 is the reference format;
 * rows_per_cb = 256 and scale_group = K is the per-row-scale format.
 * Constraints: K % 32 == 0, K <= 30000 (x is staged in LDS, else
 * KQ_EUNSUPPORTED), scale_group == K or a power of two >= 32 dividing K,
 * rows_per_cb >= 1, 1 <= batch <= 16.
 *
 * Replaces: gemv_vq_wide (v5) vq-gemv/src/kernels.metal:337-380, encoded by
 *   addVQ vq-gemv/src/main.mm:266-286,308-312.
 * ------------------------------------------------------------------------ */
kq_status kq_vq_gemv(const uint8_t* IDX, const uint16_t* C, const uint16_t* S,
                     const uint16_t* X, void* Y, kq_dtype y_dtype,
                     uint32_t M, uint32_t K, uint32_t rows_per_cb, uint32_t scale_group,
                     uint32_t batch, kq_stream_t stream);

/* ------------------------------------------------------------------------
 * VQ quantiser: a dense weight matrix into the format kq_vq_gemv reads
 *
 * W: [M][K] of w_dtype (KQ_F32, KQ_F16 or KQ_BF16; finite values).
 * Out: IDX u8 [M][K/2], C fp16 [ceil(M/rows_per_cb)][256][2] (one codebook
 * per block of rows_per_cb rows; rows_per_cb >= M is the reference's one
 * codebook per matrix), S fp16 [M][K/scale_group] (per-group abs-max;
 * scale_group = 32 is the reference format, = K one scale per row).
 * Per block: Lloyd's k-means with 256 codewords on the pairs normalised by
 * their group's scale -- all of the block's pairs, or `sample` of them drawn
 * with replacement when there are more -- 256 initial centroids drawn from
 * that sample, `iters` iterations, then every pair to its nearest centroid.
 * The draws are seeded (splitmix64 of seed, block and draw number) and the
 * cluster sums are exact integer sums, so the output is a function of the
 * arguments (the same on every run and device).
 * Constraints: K % 32 == 0; scale_group == K or a power of two >= 32
 * dividing K; 1 <= sample <= 2^24; iters <= 1000; K <= 2^18,
 * min(rows_per_cb, M) * K / 2 < 2^32 and ceil(M / rows_per_cb) <= 65535
 * (else KQ_EUNSUPPORTED).
 * ws: kq_vq_quantize_workspace_size bytes, 256-byte aligned (the scales,
 * the sample, the centroids and their sums); 0 means invalid arguments.
 * Launches: 3 + 2 * iters.
 *
 * Replaces: quantize_matrix / _kmeans vq-gemv/quant/pq_quantize.py:28-83
 *   (reference defaults: iters 25, sample 200000, scale_group 32,
 *   rows_per_cb = M).
 * ------------------------------------------------------------------------ */
size_t kq_vq_quantize_workspace_size(uint32_t M, uint32_t K, uint32_t rows_per_cb,
                                     uint32_t scale_group, uint32_t sample);
kq_status kq_vq_quantize(const void* W, kq_dtype w_dtype, uint32_t M, uint32_t K,
                         uint32_t rows_per_cb, uint32_t scale_group, uint32_t iters,
                         uint32_t sample, uint64_t seed, uint8_t* IDX, uint16_t* C, uint16_t* S,
                         void* ws, size_t ws_bytes, kq_stream_t stream);

/* ------------------------------------------------------------------------
 * MoE decode block (gpt-oss expert-blob format)
 *
 * pool: n_experts blobs of `blob` bytes. Within a blob, projection p (gate,
 * up, down) starts at off_p; within a projection, W (uint32 [rows][cols/8]),
 * S and B (bf16 [rows][cols/64]) and BI (bf16 [rows], output bias) start at
 * sub_w / sub_s / sub_b / sub_bi. gate and up are [inter][hidden], down is
 * [hidden][inter]. Group size is 64.
 * Mirrors MoEParams moe-fused/src/kernels.metal:22-35 and the blob constants
 * moe-fused/src/main.mm:23-25 (derived fields are computed, not passed).
 * ------------------------------------------------------------------------ */
typedef struct kq_moe_desc {
    uint32_t hidden, inter, n_experts, top_k;
    uint64_t blob;
    uint64_t off_gate, off_up, off_down;
    uint64_t sub_w, sub_s, sub_b, sub_bi;
} kq_moe_desc;

/* Fills the gpt-oss-120b values: hidden = inter = 2880, 128 experts, top-4,
 * blob 14,024,704 B, offsets as in moe-fused/src/main.mm:23-25. */
void kq_moe_default_desc(kq_moe_desc* d);

/* Bytes of workspace the MoE entry points need for `batch` tokens: the router
 * logits, a completion counter, the one-launch block's grid-barrier word, the
 * routing plan (distinct experts and their token slots) that the block's
 * gate/up and down kernels read, and the per-slot down products of the block
 * at 6 or more tokens. A new workspace must be zeroed once with
 * kq_moe_workspace_init (a kernel, not a memset, so it can sit in a captured
 * graph) before its first use; every call leaves it ready for the next.
 * Calls sharing one workspace must be stream-ordered. The uint32 at byte
 * KQ_MOE_WS_ERR_OFFSET stays 0 unless a one-launch block's barrier wait gave
 * up (all of its workgroups were not resident together, e.g. beside other
 * work on the GPU): that call's outputs are then invalid, and the word stays
 * set until the workspace is initialised again. The standalone gate_up and
 * down derive the plan from idx and accept a NULL workspace. */
#define KQ_MOE_WS_ERR_OFFSET 128
size_t kq_moe_workspace_size(const kq_moe_desc* d, uint32_t batch);
kq_status kq_moe_workspace_init(void* ws, size_t bytes, kq_stream_t stream);

/* Reads the workspace's error word into *err after the work already on
 * `stream` (this call synchronises the stream, the one entry point that
 * does); with `clear` non-zero a set word is reset to 0 by a kernel on
 * `stream` before the call returns. *err != 0 means a one-launch block on
 * this workspace gave up waiting and its outputs are invalid. ws_bytes must
 * cover the workspace head (at least 256 bytes). No counterpart in the
 * reference, whose Metal command buffers report a failed dispatch through
 * their status (int4-gemv/src/main.mm:109-113). */
kq_status kq_moe_workspace_error(void* ws, size_t ws_bytes, uint32_t* err, int clear,
                                 kq_stream_t stream);

/* Router logits (fp32 accumulation) for every token, top_k by repeated
 * argmax (strictly greater wins, so the lowest index wins ties), softmax over
 * the selected logits. idx: uint32 [batch][top_k] in descending-logit order;
 * wgt: fp32 [batch][top_k]. If X is fp32, xh (fp16 [batch][hidden]) receives
 * half(X) for the projections; xh may be NULL when X is fp16.
 * R: [n_experts][hidden] of r_dtype (KQ_F16 or KQ_F32).
 * Replaces: router_topk moe-fused/src/kernels.metal:121-163 (encoded at
 *   moe-fused/src/main.mm:178-185); batch > 1 is new. */
kq_status kq_moe_router_topk(const void* R, kq_dtype r_dtype, const void* X, kq_dtype x_dtype,
                             uint32_t batch, const kq_moe_desc* d,
                             uint32_t* idx, float* wgt, uint16_t* xh,
                             void* ws, size_t ws_bytes, kq_stream_t stream);

/* H[b][k][m] = fp16( swiglu(gate_e(xh_b)[m] + BIg[m], up_e(xh_b)[m] + BIu[m]) )
 * for e = idx[b][k], with swiglu(g, u) = min(g,7)*sigmoid(1.702*min(g,7)) *
 * (clamp(u,-7,7) + 1). Each selected expert's rows are read once for all the
 * tokens that chose it. H: fp16 [batch][top_k][inter].
 * Replaces: fused_gate_up_swiglu moe-fused/src/kernels.metal:177-215
 *   (encoded at moe-fused/src/main.mm:187-194). */
kq_status kq_moe_gate_up_swiglu(const uint8_t* pool, const kq_moe_desc* d,
                                const uint32_t* idx, const uint16_t* xh, uint16_t* H,
                                uint32_t batch, void* ws, size_t ws_bytes, kq_stream_t stream);

/* Y[b][m] = sum_k wgt[b][k] * (down_e(H[b][k])[m] + BId[m]), e = idx[b][k],
 * summed in k order. Y: [batch][hidden] of y_dtype (KQ_F32 or KQ_F16).
 * Replaces: fused_down_combine moe-fused/src/kernels.metal:224-265
 *   (encoded at moe-fused/src/main.mm:196-204). */
kq_status kq_moe_down_combine(const uint8_t* pool, const kq_moe_desc* d,
                              const uint32_t* idx, const float* wgt, const uint16_t* H,
                              void* Y, kq_dtype y_dtype, uint32_t batch,
                              void* ws, size_t ws_bytes, kq_stream_t stream);

/* The three passes back to back on one stream (encodeFused,
 * moe-fused/src/main.mm:176-206): three launches; from 6 tokens down writes
 * per-slot products to the workspace and a fourth, small launch sums them in
 * slot order. idx, wgt, xh (if X is fp32) and H are caller-provided
 * outputs/intermediates of the sizes above. */
kq_status kq_moe_block(const uint8_t* pool, const kq_moe_desc* d,
                       const void* R, kq_dtype r_dtype, const void* X, kq_dtype x_dtype,
                       uint32_t batch, uint32_t* idx, float* wgt, uint16_t* xh, uint16_t* H,
                       void* Y, kq_dtype y_dtype, void* ws, size_t ws_bytes,
                       kq_stream_t stream);

/* kq_moe_block with the launch structure chosen (bit-identical results on
 * every path). KQ_MOE_PATH_AUTO and KQ_MOE_PATH_LAUNCHES: what kq_moe_block
 * does, the three passes of encodeFused (moe-fused/src/main.mm:176-206).
 * KQ_MOE_PATH_ONE: one token, the whole block in one launch of one
 * workgroup per CU (router logits exchanged through tagged device-coherent
 * stores, h through one grid-wide barrier); inside a graph 0.3-0.6 us a
 * block faster than three launches (about 20.7 against 21.3 us at the
 * gpt-oss-120b shape), two launches fewer for eager callers. It stays an
 * option rather than the default for its residency demand. Every workgroup must
 * be resident at once: the path is refused (KQ_EUNSUPPORTED) when the
 * occupancy query says otherwise, and a wait that still gives up (the GPU
 * shared with other work) sets the workspace's error word (see
 * kq_moe_workspace_size). KQ_EUNSUPPORTED too unless batch is 1, hidden and
 * inter need the same number of 1024-element steps, and each wave's down
 * rows fit its registers (ceil(ceil(hidden / (2 x CUs)) / floor(8 / top_k))
 * <= 4, 2 when hidden > 3072). A PATH_ONE call needs every CU to itself:
 * it must not overlap any other work on the device, another PATH_ONE call
 * on another stream included (kq_moe_workspace_error reads the error word
 * a give-up sets). New: the reference always encodes three passes.
 * KQ_MOE_PATH_ATOMIC: the reference's atomic sum(h) block
 * (fused_gate_up_swiglu_at and fused_down_combine_at,
 * moe-fused/src/kernels.metal:400-487; encodeFused with atomicVar,
 * moe-fused/src/main.mm:176-206): three launches, the router zeroing a
 * workspace array of sum(h) per slot and 32-element chunk, gate/up adding
 * every h value to it (as a float, before its fp16 rounding) with a
 * device-scope atomic, down reading the sums instead of summing h. The sums'
 * order is not fixed, so y may differ in the last bits from call to call;
 * idx, wgt and h are those of the other paths. KQ_EUNSUPPORTED unless batch
 * <= 2 and the streaming kernels take the shapes (the block's default form
 * there). */
#define KQ_MOE_PATH_AUTO 0
#define KQ_MOE_PATH_LAUNCHES 1
#define KQ_MOE_PATH_ONE 2
#define KQ_MOE_PATH_ATOMIC 3
kq_status kq_moe_block_path(const uint8_t* pool, const kq_moe_desc* d,
                            const void* R, kq_dtype r_dtype, const void* X, kq_dtype x_dtype,
                            uint32_t batch, uint32_t* idx, float* wgt, uint16_t* xh, uint16_t* H,
                            void* Y, kq_dtype y_dtype, void* ws, size_t ws_bytes, int path,
                            kq_stream_t stream);

/* kq_moe_block without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). It has no counterpart in the reference.
 * The workspace is a fixed array of KQ_MOE_NOALLOC_WS_BYTES in libkq's own
 * device memory, one per GPU, held until the process ends; the call
 * allocates nothing. A (desc, batch) whose kq_moe_workspace_size exceeds
 * KQ_MOE_NOALLOC_WS_BYTES returns KQ_EWORKSPACE (gpt-oss-120b shapes fit up
 * to 16 tokens). The first call on a GPU looks the array's address up
 * (hipGetSymbolAddress) and enqueues nothing else: the array starts as zeros
 * (static storage), so a first call made under stream capture records only
 * the block's own kernels. Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (different streams, or different
 * host threads, without ordering between them) race and must not be made.
 * Otherwise the same arguments, results and launches as kq_moe_block. */
#define KQ_MOE_NOALLOC_WS_BYTES (1u << 20)
kq_status kq_moe_block_noalloc(const uint8_t* pool, const kq_moe_desc* d,
                               const void* R, kq_dtype r_dtype, const void* X, kq_dtype x_dtype,
                               uint32_t batch, uint32_t* idx, float* wgt, uint16_t* xh,
                               uint16_t* H, void* Y, kq_dtype y_dtype, kq_stream_t stream);

/* The same block with one operation per launch, one token: router logits,
 * top-k, softmax, then per slot gate GEMV, up GEMV, SwiGLU, and per slot
 * down GEMV, weighted accumulate -- 3 + 5 * top_k launches (23 at top-4),
 * every intermediate through `ws`. It exists to measure what the
 * three-launch block saves. Same arguments and results as kq_moe_block at
 * batch 1 (other batches: KQ_EUNSUPPORTED); ws needs
 * kq_moe_unfused_workspace_size bytes, 256-byte aligned, and no
 * initialisation. n_launches (may be NULL) receives the number of kernel
 * launches made.
 * Replaces: encodeUnfused moe-fused/src/main.mm:208-284 and its kernels
 *   u_router .. u_axpy moe-fused/src/kernels.metal:284-392 (the reference's
 *   28 launches include five x-sum passes that this GEMV does in-kernel). */
size_t kq_moe_unfused_workspace_size(const kq_moe_desc* d);
kq_status kq_moe_block_unfused(const uint8_t* pool, const kq_moe_desc* d,
                               const void* R, kq_dtype r_dtype, const void* X, kq_dtype x_dtype,
                               uint32_t batch, uint32_t* idx, float* wgt, uint16_t* xh,
                               uint16_t* H, void* Y, kq_dtype y_dtype, void* ws, size_t ws_bytes,
                               uint32_t* n_launches, kq_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* KQ_H */
