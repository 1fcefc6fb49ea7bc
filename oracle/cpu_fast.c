/*
 * cpu_fast.c -- timed CPU baseline (TEST/BENCH INFRASTRUCTURE ONLY).
 *
 * x86 restatement of the reference's CPU int4 GEMV, cpu_gemv_neon
 * hetero-gemv/src/cpu_gemv.h:88-103 with its chunk unpack chunk32
 * (cpu_gemv.h:26-46): per 32-weight chunk (16 bytes; byte i holds weight 2i
 * in its low nibble and 2i+1 in its high nibble), unpack the nibbles in
 * weight order, multiply-add against fp32 x, reduce the chunk to one float d,
 * then fold the group metadata once per chunk: acc += s*d + b*xs[chunk].
 * NEON zip/convert/fma become SSE unpack, AVX2 widen/convert and FMA.
 * Rows are split into blocks over nthreads pthreads.
 */
#include "kqref.h"

#include <immintrin.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

int kqref_cpu_fast_supported(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
           __builtin_cpu_supports("f16c");
}

typedef struct {
    const uint8_t* W; const uint16_t* SB; const float* xf; const float* xs; float* y;
    uint32_t K, G, m0, m1;
} fast_job;

__attribute__((target("avx2,fma,f16c")))
static inline float hsum256(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

__attribute__((target("avx2,fma,f16c")))
static inline float h2f(uint16_t h) {
    return _mm_cvtss_f32(_mm_cvtph_ps(_mm_cvtsi32_si128(h)));
}

__attribute__((target("avx2,fma,f16c")))
static void* fast_rows(void* p) {
    const fast_job* j = (const fast_job*)p;
    const uint32_t chunks = j->K / 32, cpg = j->G / 32, groups = j->K / j->G;
    const __m128i mask = _mm_set1_epi8(0x0F);
    for (uint32_t m = j->m0; m < j->m1; ++m) {
        const uint8_t* wp = j->W + (size_t)m * (j->K / 2);
        const uint16_t* sb = j->SB + (size_t)m * groups * 2;
        float accf = 0.0f;
        for (uint32_t c = 0; c < chunks; ++c) {
            __m128i v = _mm_loadu_si128((const __m128i*)(wp + c * 16));
            __m128i lo = _mm_and_si128(v, mask);
            __m128i hi = _mm_and_si128(_mm_srli_epi16(v, 4), mask);
            __m128i z0 = _mm_unpacklo_epi8(lo, hi); /* weights 0..15 */
            __m128i z1 = _mm_unpackhi_epi8(lo, hi); /* weights 16..31 */
            const float* xp = j->xf + (size_t)c * 32;
            __m256 a0 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(z0)), _mm256_loadu_ps(xp));
            __m256 a1 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(z0, 8))),
                                      _mm256_loadu_ps(xp + 8));
            a0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(z1)), _mm256_loadu_ps(xp + 16), a0);
            a1 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(z1, 8))),
                                 _mm256_loadu_ps(xp + 24), a1);
            float d = hsum256(_mm256_add_ps(a0, a1));
            uint32_t g = c / cpg;
            accf += h2f(sb[2 * g]) * d + h2f(sb[2 * g + 1]) * j->xs[c];
        }
        j->y[m] = accf;
    }
    return NULL;
}

__attribute__((target("avx2,fma,f16c")))
void kqref_int4_gemv_cpu_fast(const uint32_t* W, const uint16_t* SB, const uint16_t* X,
                              float* Y, uint32_t M, uint32_t K, uint32_t G, int nthreads) {
    /* fp32 copy of x and its per-32 sums: the inputs cpu_gemv_neon takes
     * (hetero-gemv/src/cpu_gemv.h:88-90) */
    float* xf = (float*)malloc(sizeof(float) * K);
    float* xs = (float*)malloc(sizeof(float) * (K / 32));
    for (uint32_t k = 0; k < K; ++k) xf[k] = h2f(X[k]);
    for (uint32_t c = 0; c < K / 32; ++c) {
        float s = 0.0f;
        for (uint32_t i = 0; i < 32; ++i) s += xf[c * 32 + i];
        xs[c] = s;
    }
    int n = nthreads > 0 ? nthreads : (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    if (n > 256) n = 256;
    pthread_t th[256];
    fast_job jobs[256];
    uint32_t chunk = (M + (uint32_t)n - 1) / (uint32_t)n;
    int started = 0;
    for (int i = 0; i < n; ++i) {
        uint32_t a = (uint32_t)i * chunk, b = a + chunk < M ? a + chunk : M;
        if (a >= b) break;
        jobs[i] = (fast_job){(const uint8_t*)W, SB, xf, xs, Y, K, G, a, b};
        started = i + 1;
        if (n == 1 || pthread_create(&th[i], NULL, fast_rows, &jobs[i]) != 0) {
            fast_rows(&jobs[i]);
            jobs[i].W = NULL;
        }
    }
    for (int i = 0; i < started; ++i)
        if (jobs[i].W) pthread_join(th[i], NULL);
    free(xf);
    free(xs);
}
