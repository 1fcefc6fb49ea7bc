/*
 * vqquant.c -- CPU oracle of the VQ quantiser (TEST INFRASTRUCTURE ONLY).
 *
 * Restates quantize_matrix / _kmeans of vq-gemv/quant/pq_quantize.py:28-83
 * as this build specifies it for the GPU (kernels_amd/csrc/kq_vq_quant.hip),
 * step for step, so the GPU output can be checked bit for bit:
 *
 *   1. scale[m][g] = max |w| over the group (fp32); S = fp16(scale) (RNE);
 *      the pairs are normalised by the fp32 scale (1 where it is 0)
 *      (pq_quantize.py:59-62).
 *   2. per codebook block b (rows_per_cb rows; the reference has one block
 *      per matrix): the k-means sample is every pair of the block if there
 *      are at most `sample` of them, else `sample` pairs drawn with
 *      replacement (pq_quantize.py:38-39); the initial centroids are 256
 *      sample points drawn with replacement (pq_quantize.py:40). The draws
 *      use splitmix64 (MLX's generator is not available here).
 *   3. `iters` Lloyd iterations (pq_quantize.py:41-48): assign each sample
 *      point to argmax_c score(p, c), ties to the lowest c, with
 *      score = fmaf(p.x, c.x, fmaf(p.y, c.y, hc)), hc = -0.5f * fmaf(c.x, c.x, c.y * c.y)
 *      (the reference's p.c - |c|^2/2 argmax); the new centroid is the mean of
 *      its points, empty clusters keep theirs. The sums are taken in 2^-40
 *      fixed point (exact integer sums, so the order of accumulation -- the
 *      GPU's atomics -- cannot change the result): mean =
 *      (float)((double)sum * 2^-40 / count), coordinates truncated to the grid.
 *   4. every pair of the block is assigned with the fp32 centroids
 *      (pq_quantize.py:66-73); the codebook is stored as fp16 (RNE).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "kqref.h"

#define KQREF_CB 256

static float w_at(const void* W, int dt, size_t i) {
    if (dt == KQREF_F32) return ((const float*)W)[i];
    const uint16_t h = ((const uint16_t*)W)[i];
    return dt == KQREF_BF16 ? (float)kqref_bf16_to_f64(h) : (float)kqref_f16_to_f64(h);
}

uint64_t kqref_vq_hash(uint64_t seed, uint32_t blk, uint32_t j) {
    uint64_t x = seed + 0x9E3779B97F4A7C15ull * ((((uint64_t)blk) << 32) + (uint64_t)j + 1ull);
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

/* uniform index in [0, n) from draw j of block blk */
static uint32_t draw(uint64_t seed, uint32_t blk, uint32_t j, uint32_t n) {
    return (uint32_t)(((kqref_vq_hash(seed, blk, j) >> 32) * (uint64_t)n) >> 32);
}

float kqref_vq_score(float px, float py, float cx, float cy) {
    const float hc = -0.5f * fmaf(cx, cx, cy * cy);
    return fmaf(px, cx, fmaf(py, cy, hc));
}

static uint32_t nearest(float px, float py, const float* C) {
    uint32_t best = 0;
    float bs = kqref_vq_score(px, py, C[0], C[1]);
    for (uint32_t c = 1; c < KQREF_CB; ++c) {
        const float s = kqref_vq_score(px, py, C[2 * c], C[2 * c + 1]);
        if (s > bs) {
            bs = s;
            best = c;
        }
    }
    return best;
}

int64_t kqref_vq_fix(float v) { return (int64_t)(v * 0x1p40f); }

float kqref_vq_mean(int64_t sum, uint64_t cnt) {
    return (float)((double)sum * 0x1p-40 / (double)cnt);
}

void kqref_vq_quantize(const void* W, int w_dtype, uint32_t M, uint32_t K, uint32_t rows_per_cb,
                       uint32_t scale_group, uint32_t iters, uint32_t sample, uint64_t seed,
                       uint8_t* IDX, uint16_t* Cb, uint16_t* S, float* centroids_out) {
    const uint32_t G = scale_group, gpr = K / G, half = K / 2;
    const uint32_t nblk = (M + rows_per_cb - 1) / rows_per_cb;
    float* sc = (float*)malloc(sizeof(float) * (size_t)M * gpr);
    for (uint32_t m = 0; m < M; ++m)
        for (uint32_t g = 0; g < gpr; ++g) {
            float a = 0.0f;
            for (uint32_t k = 0; k < G; ++k) {
                const float v = fabsf(w_at(W, w_dtype, (size_t)m * K + (size_t)g * G + k));
                a = v > a ? v : a;
            }
            S[(size_t)m * gpr + g] = kqref_f32_to_f16(a);
            sc[(size_t)m * gpr + g] = a > 0.0f ? a : 1.0f;
        }
#define PAIR(m, i, px, py)                                                 \
    do {                                                                   \
        const float s_ = sc[(size_t)(m) * gpr + (2u * (i)) / G];           \
        px = w_at(W, w_dtype, (size_t)(m) * K + 2u * (i)) / s_;            \
        py = w_at(W, w_dtype, (size_t)(m) * K + 2u * (i) + 1u) / s_;       \
    } while (0)
    for (uint32_t b = 0; b < nblk; ++b) {
        const uint32_t r0 = b * rows_per_cb;
        const uint32_t rows = M - r0 < rows_per_cb ? M - r0 : rows_per_cb;
        const uint32_t N = rows * half;
        const uint32_t ns = N <= sample ? N : sample;
        float* P = (float*)malloc(sizeof(float) * 2 * ns);
        for (uint32_t j = 0; j < ns; ++j) {
            const uint32_t p = N <= sample ? j : draw(seed, b, j, N);
            PAIR(r0 + p / half, p % half, P[2 * j], P[2 * j + 1]);
        }
        float C[2 * KQREF_CB];
        for (uint32_t c = 0; c < KQREF_CB; ++c) {
            const uint32_t j = draw(seed, b, 0x80000000u + c, ns);
            C[2 * c] = P[2 * j];
            C[2 * c + 1] = P[2 * j + 1];
        }
        int64_t sx[KQREF_CB], sy[KQREF_CB];
        uint64_t cnt[KQREF_CB];
        for (uint32_t it = 0; it < iters; ++it) {
            memset(sx, 0, sizeof sx);
            memset(sy, 0, sizeof sy);
            memset(cnt, 0, sizeof cnt);
            for (uint32_t j = 0; j < ns; ++j) {
                const uint32_t a = nearest(P[2 * j], P[2 * j + 1], C);
                sx[a] += kqref_vq_fix(P[2 * j]);
                sy[a] += kqref_vq_fix(P[2 * j + 1]);
                ++cnt[a];
            }
            for (uint32_t c = 0; c < KQREF_CB; ++c)
                if (cnt[c]) {
                    C[2 * c] = kqref_vq_mean(sx[c], cnt[c]);
                    C[2 * c + 1] = kqref_vq_mean(sy[c], cnt[c]);
                }
        }
        free(P);
        for (uint32_t c = 0; c < 2 * KQREF_CB; ++c) {
            Cb[(size_t)b * 2 * KQREF_CB + c] = kqref_f32_to_f16(C[c]);
            if (centroids_out) centroids_out[(size_t)b * 2 * KQREF_CB + c] = C[c];
        }
        for (uint32_t m = r0; m < r0 + rows; ++m)
            for (uint32_t i = 0; i < half; ++i) {
                float px, py;
                PAIR(m, i, px, py);
                IDX[(size_t)m * half + i] = (uint8_t)nearest(px, py, C);
            }
    }
#undef PAIR
    free(sc);
}
