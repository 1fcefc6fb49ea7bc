/*
 * kqref.h -- CPU oracle for the decode hot path (TEST INFRASTRUCTURE ONLY).
 *
 * Plain-C, fp64-accumulating restatements of the reference's own CPU
 * implementations. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker or the
 * timed CPU baseline; the product path (libkq) never links or calls it.
 *
 * Every function cites the reference lines it restates (paths relative to the
 * reference repository root). Pinning of each function against golden
 * vectors, closed forms and brute force lives in tests/test_oracle.py.
 *
 * Conventions: fp16/bf16 tensors are passed as raw uint16 bit patterns;
 * outputs are double. nthreads <= 0 means "all online cores".
 */
#ifndef KQREF_H
#define KQREF_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { KQREF_F16 = 0, KQREF_BF16 = 1, KQREF_F32 = 2 };

double kqref_f16_to_f64(uint16_t h);
double kqref_bf16_to_f64(uint16_t h);
/* round-to-nearest-even float -> binary16 bits (used to build inputs) */
uint16_t kqref_f32_to_f16(float f);

/* int4 group-affine GEMV, fp64 accumulation in k order.
 * Restates cpuRefRows/cpuRef int4-gemv/src/main.mm:64-92 (separate S, B:
 * sb_interleaved = 0) and int4RefRows vq-gemv/src/main.mm:67-80 (interleaved
 * (scale, bias) pairs: sb_interleaved = 1; B ignored). sb_dtype selects fp16
 * or bf16 metadata. X: fp16 [batch][K]; Y: [batch][M]. */
void kqref_int4_gemv_f64(const uint32_t* W, const uint16_t* S, const uint16_t* B,
                         int sb_interleaved, int sb_dtype, const uint16_t* X, double* Y,
                         uint32_t M, uint32_t K, uint32_t G, uint32_t batch, int nthreads);

/* xs[b][j] = sum_{i<32} x[b][32j+i]  (fp32 sum in index order, as the kernel
 * int4-gemv/src/kernels.metal:54-65 defines it). */
void kqref_xsum32(const uint16_t* X, float* xs, uint32_t K, uint32_t batch);

/* VQ d=2 dequant-GEMV, fp64. Restates vqRefRows vq-gemv/src/main.mm:51-66,
 * generalised by rows_per_cb (codebook block per rows) and scale_group. */
void kqref_vq_gemv_f64(const uint8_t* IDX, const uint16_t* C, const uint16_t* S,
                       const uint16_t* X, double* Y, uint32_t M, uint32_t K,
                       uint32_t rows_per_cb, uint32_t scale_group, uint32_t batch,
                       int nthreads);

/* MoE blob description; same fields as kq_moe_desc in include/kq.h. */
typedef struct kqref_moe_desc {
    uint32_t hidden, inter, n_experts, top_k;
    uint64_t blob;
    uint64_t off_gate, off_up, off_down;
    uint64_t sub_w, sub_s, sub_b, sub_bi;
} kqref_moe_desc;

/* Router + top-k + softmax, fp64. Restates moe-fused/src/main.mm:303-319:
 * logits = R x (fp64), k passes of "strictly greater wins" over an ascending
 * scan starting from -1e300, winner set to -1e300; softmax over the chosen k
 * with max subtraction. R is r_dtype (F16 or F32) [n_experts][hidden]; X is
 * x_dtype (F16 or F32) [batch][hidden]. logits (optional) [batch][n_experts]. */
void kqref_moe_router_f64(const void* R, int r_dtype, const void* X, int x_dtype,
                          uint32_t batch, const kqref_moe_desc* d,
                          uint32_t* idx, double* wgt, double* logits);

/* One expert projection with output bias, fp64. Restates refProj
 * moe-fused/src/main.mm:46-62 (bf16 S/B/BI, group 64). y[m] for m < M. */
void kqref_moe_proj_f64(const uint8_t* blob, uint64_t proj, const kqref_moe_desc* d,
                        const double* x, double* y, uint32_t M, uint32_t K, int nthreads);

/* gpt-oss SwiGLU: g = min(g, 7), u = clamp(u, -7, 7),
 * h = g / (1 + exp(-1.702 g)) * (u + 1). Restates moe-fused/src/main.mm:327-330
 * (and swiglu_k moe-pipeline/src/kernels.metal:88-98). */
double kqref_swiglu_f64(double g, double u);

/* Gate/up + SwiGLU for every (token, slot): H[b][k][m], x as given (fp16 or
 * fp32 per x_dtype). Restates moe-fused/src/main.mm:323-330. */
void kqref_moe_gate_up_f64(const uint8_t* pool, const kqref_moe_desc* d, const uint32_t* idx,
                           const void* X, int x_dtype, uint32_t batch, double* H, int nthreads);

/* Down + weighted combine in slot order: Y[b][m] = sum_k wgt[b][k] *
 * (down_e(H[b][k])[m] + BI[m]). H is fp64 (h_dtype = F32 means a double
 * array) or fp16 bits (h_dtype = F16). Restates moe-fused/src/main.mm:331-333. */
void kqref_moe_down_f64(const uint8_t* pool, const kqref_moe_desc* d, const uint32_t* idx,
                        const double* wgt, const void* H, int h_dtype, uint32_t batch,
                        double* Y, int nthreads);

/* Whole block: router, top-k, softmax, gate/up, SwiGLU, down, combine.
 * Restates the block reference moe-fused/src/main.mm:302-334. */
void kqref_moe_block_f64(const uint8_t* pool, const kqref_moe_desc* d, const void* R, int r_dtype,
                         const void* X, int x_dtype, uint32_t batch, uint32_t* idx, double* wgt,
                         double* Y, int nthreads);

/* ---- timed CPU baseline (x86 restatements of the reference's CPU int4 paths) ----
 * path 3: cpu_gemv_neon16 hetero-gemv/src/cpu_gemv.h:55-84 (32-weight chunk
 * unpack, fp16 FMA against fp16 x in 8 lanes, fp32 fold per chunk) on
 * AVX-512-FP16; path 2 / 1: cpu_gemv_neon cpu_gemv.h:88-103 (fp32 FMA against
 * fp32 x) on AVX-512F / AVX2+FMA. path <= 0 picks the fastest the CPU has.
 * Row blocks over a persistent pool of nthreads threads.
 * SB interleaved fp16 (scale, bias); x fp16; y fp32. */
void kqref_int4_gemv_cpu_fast_path(const uint32_t* W, const uint16_t* SB, const uint16_t* X,
                                   float* Y, uint32_t M, uint32_t K, uint32_t G, int nthreads,
                                   int path);
void kqref_int4_gemv_cpu_fast(const uint32_t* W, const uint16_t* SB, const uint16_t* X,
                              float* Y, uint32_t M, uint32_t K, uint32_t G, int nthreads);
/* 1 if this CPU has at least AVX2, FMA and F16C (the slowest path's requirement). */
int kqref_cpu_fast_supported(void);
/* Name of a path (path <= 0: the fastest this CPU has). */
const char* kqref_cpu_fast_path_name(int path);

/* VQ quantiser (vqquant.c): quantize_matrix / _kmeans of
 * vq-gemv/quant/pq_quantize.py:28-83 as specified for the GPU quantiser
 * (kq_vq_quantize). W: [M][K] of w_dtype; IDX u8 [M][K/2]; Cb fp16
 * [ceil(M/rows_per_cb)][256][2]; S fp16 [M][K/scale_group]; centroids_out
 * (may be NULL) receives the fp32 centroids the assignment used. */
void kqref_vq_quantize(const void* W, int w_dtype, uint32_t M, uint32_t K, uint32_t rows_per_cb,
                       uint32_t scale_group, uint32_t iters, uint32_t sample, uint64_t seed,
                       uint8_t* IDX, uint16_t* Cb, uint16_t* S, float* centroids_out);
uint64_t kqref_vq_hash(uint64_t seed, uint32_t blk, uint32_t j);
float kqref_vq_score(float px, float py, float cx, float cy);
int64_t kqref_vq_fix(float v);
float kqref_vq_mean(int64_t sum, uint64_t cnt);

#ifdef __cplusplus
}
#endif
#endif
