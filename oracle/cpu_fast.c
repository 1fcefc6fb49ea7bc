/*
 * cpu_fast.c -- timed CPU baseline (TEST/BENCH INFRASTRUCTURE ONLY).
 *
 * x86 restatements of the reference's CPU int4 GEMV paths
 * (hetero-gemv/src/cpu_gemv.h), fastest first:
 *
 *  - neon16 (cpu_gemv.h:55-84), with AVX-512-FP16: per 32-weight chunk
 *    (16 bytes; byte i holds weight 2i in its low nibble and 2i+1 in its high
 *    nibble) the nibbles are unpacked in weight order, widened to uint16 and
 *    converted to fp16, and four 8-lane fp16 FMAs against fp16 x accumulate
 *    them (lane i takes weights i, 8+i, 16+i, 24+i, as the NEON loop does);
 *    the chunk's d is the fp32 sum of the low four lanes plus the fp32 sum of
 *    the high four; the group metadata folds in once per chunk,
 *    acc += s*d + b*xs[chunk], in fp32.
 *  - neon (cpu_gemv.h:88-103), fp32: the same chunk unpack, fp32 FMAs against
 *    fp32 x, one reduction per chunk; with AVX-512F (16 lanes) or AVX2+FMA
 *    (8 lanes).
 *
 * Rows are split into contiguous blocks over a pool of worker threads that
 * is created once and reused by every call (the reference's harness runs its
 * CPU rows on std::thread workers beside the GPU dispatch).
 */
#include "kqref.h"

#include <cpuid.h>
#include <immintrin.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ---------------------------------------------------------------- */
/* paths                                                             */
/* ---------------------------------------------------------------- */
enum { PATH_NONE = 0, PATH_AVX2 = 1, PATH_AVX512 = 2, PATH_FP16 = 3 };

/* the fp16 arithmetic intrinsics need clang or gcc >= 12 */
#if defined(__clang__) || (defined(__GNUC__) && __GNUC__ >= 12)
#define KQ_HAVE_FP16 1
#else
#define KQ_HAVE_FP16 0
#endif

static int best_path(void) {
    __builtin_cpu_init();
#if KQ_HAVE_FP16
    /* CPUID.(EAX=7,ECX=0):EDX bit 23 = AVX512-FP16 (read directly: the
     * runtime's feature table may predate it) */
    unsigned a, b, c, d;
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512vl") &&
        __builtin_cpu_supports("avx512bw") && __get_cpuid_count(7, 0, &a, &b, &c, &d) &&
        (d >> 23 & 1u))
        return PATH_FP16;
#endif
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
        __builtin_cpu_supports("f16c"))
        return PATH_AVX512;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
        __builtin_cpu_supports("f16c"))
        return PATH_AVX2;
    return PATH_NONE;
}

int kqref_cpu_fast_supported(void) { return best_path() != PATH_NONE; }

const char* kqref_cpu_fast_path_name(int path) {
    switch (path <= 0 ? best_path() : path) {
        case PATH_FP16: return "neon16 (fp16 FMA) on AVX-512-FP16";
        case PATH_AVX512: return "neon (fp32 FMA) on AVX-512F";
        case PATH_AVX2: return "neon (fp32 FMA) on AVX2+FMA";
        default: return "none";
    }
}

typedef struct {
    const uint8_t* W; const uint16_t* SB; const uint16_t* xh; const float* xf; const float* xs;
    float* y; uint32_t K, G, m0, m1; int path;
} fast_job;

__attribute__((target("avx2,fma,f16c")))
static inline float h2f(uint16_t h) {
    return _mm_cvtss_f32(_mm_cvtph_ps(_mm_cvtsi32_si128(h)));
}

__attribute__((target("avx2,fma,f16c")))
static inline float hsum256(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

/* the 32 nibbles of a chunk in weight order: weights 0..15 and 16..31 */
__attribute__((target("avx2,fma,f16c")))
static inline void unpack32(const uint8_t* p, __m128i* z0, __m128i* z1) {
    const __m128i mask = _mm_set1_epi8(0x0F);
    const __m128i v = _mm_loadu_si128((const __m128i*)p);
    const __m128i lo = _mm_and_si128(v, mask);
    const __m128i hi = _mm_and_si128(_mm_srli_epi16(v, 4), mask);
    *z0 = _mm_unpacklo_epi8(lo, hi);
    *z1 = _mm_unpackhi_epi8(lo, hi);
}

__attribute__((target("avx2,fma,f16c")))
static void rows_avx2(const fast_job* j) {
    const uint32_t chunks = j->K / 32, cpg = j->G / 32, groups = j->K / j->G;
    for (uint32_t m = j->m0; m < j->m1; ++m) {
        const uint8_t* wp = j->W + (size_t)m * (j->K / 2);
        const uint16_t* sb = j->SB + (size_t)m * groups * 2;
        float accf = 0.0f;
        for (uint32_t c = 0; c < chunks; ++c) {
            __m128i z0, z1;
            unpack32(wp + c * 16, &z0, &z1);
            const float* xp = j->xf + (size_t)c * 32;
            __m256 a0 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(z0)), _mm256_loadu_ps(xp));
            __m256 a1 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(z0, 8))),
                                      _mm256_loadu_ps(xp + 8));
            a0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(z1)), _mm256_loadu_ps(xp + 16), a0);
            a1 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(z1, 8))),
                                 _mm256_loadu_ps(xp + 24), a1);
            const float d = hsum256(_mm256_add_ps(a0, a1));
            const uint32_t g = c / cpg;
            accf += h2f(sb[2 * g]) * d + h2f(sb[2 * g + 1]) * j->xs[c];
        }
        j->y[m] = accf;
    }
}

__attribute__((target("avx512f,avx512bw,f16c,fma")))
static void rows_avx512(const fast_job* j) {
    const uint32_t chunks = j->K / 32, cpg = j->G / 32, groups = j->K / j->G;
    for (uint32_t m = j->m0; m < j->m1; ++m) {
        const uint8_t* wp = j->W + (size_t)m * (j->K / 2);
        const uint16_t* sb = j->SB + (size_t)m * groups * 2;
        float accf = 0.0f;
        for (uint32_t c = 0; c < chunks; ++c) {
            __m128i z0, z1;
            unpack32(wp + c * 16, &z0, &z1);
            const float* xp = j->xf + (size_t)c * 32;
            __m512 a = _mm512_mul_ps(_mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(z0)), _mm512_loadu_ps(xp));
            a = _mm512_fmadd_ps(_mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(z1)), _mm512_loadu_ps(xp + 16), a);
            const float d = _mm512_reduce_add_ps(a);
            const uint32_t g = c / cpg;
            accf += h2f(sb[2 * g]) * d + h2f(sb[2 * g + 1]) * j->xs[c];
        }
        j->y[m] = accf;
    }
}

#if KQ_HAVE_FP16
__attribute__((target("avx512fp16,avx512vl,avx512bw,avx512f,f16c,fma")))
static void rows_fp16(const fast_job* j) {
    const uint32_t chunks = j->K / 32, cpg = j->G / 32, groups = j->K / j->G;
    for (uint32_t m = j->m0; m < j->m1; ++m) {
        const uint8_t* wp = j->W + (size_t)m * (j->K / 2);
        const uint16_t* sb = j->SB + (size_t)m * groups * 2;
        float accf = 0.0f;
        for (uint32_t c = 0; c < chunks; ++c) {
            __m128i z[2];
            unpack32(wp + c * 16, &z[0], &z[1]);
            const uint16_t* xp = j->xh + (size_t)c * 32;
            __m128h acc = _mm_setzero_ph();
            for (int h = 0; h < 2; ++h) {
                const __m128h a = _mm_cvtepu16_ph(_mm_cvtepu8_epi16(z[h]));
                const __m128h b = _mm_cvtepu16_ph(_mm_cvtepu8_epi16(_mm_srli_si128(z[h], 8)));
                acc = _mm_fmadd_ph(a, _mm_castsi128_ph(_mm_loadu_si128((const __m128i*)(xp + h * 16))), acc);
                acc = _mm_fmadd_ph(b, _mm_castsi128_ph(_mm_loadu_si128((const __m128i*)(xp + h * 16 + 8))),
                                   acc);
            }
            /* (float) sum of lanes 0-3 + (float) sum of lanes 4-7 */
            const __m256 f = _mm256_cvtph_ps(_mm_castph_si128(acc));
            __m128 lo = _mm256_castps256_ps128(f), hi = _mm256_extractf128_ps(f, 1);
            lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
            lo = _mm_add_ss(lo, _mm_shuffle_ps(lo, lo, 1));
            hi = _mm_add_ps(hi, _mm_movehl_ps(hi, hi));
            hi = _mm_add_ss(hi, _mm_shuffle_ps(hi, hi, 1));
            const float d = _mm_cvtss_f32(lo) + _mm_cvtss_f32(hi);
            const uint32_t g = c / cpg;
            accf += h2f(sb[2 * g]) * d + h2f(sb[2 * g + 1]) * j->xs[c];
        }
        j->y[m] = accf;
    }
}
#endif

static void run_job(const fast_job* j) {
    if (j->m0 >= j->m1) return;
    switch (j->path) {
#if KQ_HAVE_FP16
        case PATH_FP16: rows_fp16(j); break;
#endif
        case PATH_AVX512: rows_avx512(j); break;
        default: rows_avx2(j); break;
    }
}

/* ---------------------------------------------------------------- */
/* persistent worker pool                                            */
/* ---------------------------------------------------------------- */
#define MAX_WORKERS 256
static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t g_go = PTHREAD_COND_INITIALIZER, g_done = PTHREAD_COND_INITIALIZER;
static pthread_t g_th[MAX_WORKERS];
static int g_nthreads = 0;        /* workers running (the caller is worker 0) */
static unsigned long g_gen = 0;   /* job generation */
static int g_pending = 0;         /* workers still running the current job */
static fast_job g_jobs[MAX_WORKERS];
static unsigned long g_start[MAX_WORKERS]; /* generation when worker i was created */
static pthread_mutex_t g_call = PTHREAD_MUTEX_INITIALIZER; /* one call at a time */

static void* worker(void* arg) {
    const int id = (int)(intptr_t)arg;
    pthread_mutex_lock(&g_mu);
    unsigned long seen = g_start[id];
    pthread_mutex_unlock(&g_mu);
    for (;;) {
        pthread_mutex_lock(&g_mu);
        while (g_gen == seen) pthread_cond_wait(&g_go, &g_mu);
        seen = g_gen;
        pthread_mutex_unlock(&g_mu);
        run_job(&g_jobs[id]);
        pthread_mutex_lock(&g_mu);
        if (--g_pending == 0) pthread_cond_signal(&g_done);
        pthread_mutex_unlock(&g_mu);
    }
    return NULL;
}

/* workers 1 .. n-1 exist (created on demand, kept until the process ends) */
static int ensure_workers(int n) {
    pthread_mutex_lock(&g_mu);
    while (g_nthreads < n - 1) {
        g_start[g_nthreads + 1] = g_gen;
        if (pthread_create(&g_th[g_nthreads + 1], NULL, worker, (void*)(intptr_t)(g_nthreads + 1)) != 0)
            break;
        pthread_detach(g_th[g_nthreads + 1]);
        ++g_nthreads;
    }
    const int have = g_nthreads + 1;
    pthread_mutex_unlock(&g_mu);
    return have < n ? have : n;
}

static void parallel_rows(const fast_job* proto, uint32_t M, int n) {
    pthread_mutex_lock(&g_call);
    n = ensure_workers(n);
    const uint32_t chunk = (M + (uint32_t)n - 1) / (uint32_t)n;
    pthread_mutex_lock(&g_mu);
    for (int i = 0; i < MAX_WORKERS; ++i) {
        g_jobs[i] = *proto;
        const uint32_t a = (uint32_t)i * chunk;
        g_jobs[i].m0 = i < n && a < M ? a : M;
        g_jobs[i].m1 = i < n && a + chunk < M ? a + chunk : M;
    }
    g_pending = g_nthreads;  /* every live worker runs (idle ones get empty ranges) */
    ++g_gen;
    pthread_cond_broadcast(&g_go);
    pthread_mutex_unlock(&g_mu);
    run_job(&g_jobs[0]);
    pthread_mutex_lock(&g_mu);
    while (g_pending > 0) pthread_cond_wait(&g_done, &g_mu);
    pthread_mutex_unlock(&g_mu);
    pthread_mutex_unlock(&g_call);
}

/* path <= 0: the fastest the host supports */
__attribute__((target("avx2,fma,f16c")))
void kqref_int4_gemv_cpu_fast_path(const uint32_t* W, const uint16_t* SB, const uint16_t* X,
                                   float* Y, uint32_t M, uint32_t K, uint32_t G, int nthreads,
                                   int path) {
    const int best = best_path();
    if (path <= 0 || path > best) path = best;
    /* the inputs the reference's CPU paths take (cpu_gemv.h:55-58,88-90):
     * x as fp16 (neon16) or fp32, and the fp32 per-32 sums xs */
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
    if (n > MAX_WORKERS) n = MAX_WORKERS;
    fast_job proto = {(const uint8_t*)W, SB, X, xf, xs, Y, K, G, 0, 0, path};
    parallel_rows(&proto, M, n);
    free(xf);
    free(xs);
}

void kqref_int4_gemv_cpu_fast(const uint32_t* W, const uint16_t* SB, const uint16_t* X, float* Y,
                              uint32_t M, uint32_t K, uint32_t G, int nthreads) {
    kqref_int4_gemv_cpu_fast_path(W, SB, X, Y, M, K, G, nthreads, 0);
}
