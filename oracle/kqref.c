/*
 * kqref.c -- CPU oracle for the decode hot path (TEST INFRASTRUCTURE ONLY).
 * See kqref.h: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this; libkq never does.
 *
 * Each function is a restatement, in plain C with fp64 accumulation, of the
 * reference CPU code cited beside it. Threading follows the reference's
 * row-block split over all hardware threads (int4-gemv/src/main.mm:81-92).
 */
#include "kqref.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ */
/* scalar conversions                                                  */
/* ------------------------------------------------------------------ */

/* IEEE binary16 decode (sign, 5-bit exponent, 10-bit mantissa, subnormals). */
double kqref_f16_to_f64(uint16_t h) {
    uint32_t s = h >> 15, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    double v;
    if (e == 0)
        v = ldexp((double)m, -24);
    else if (e == 31)
        v = m ? NAN : INFINITY;
    else
        v = ldexp((double)(m | 0x400), (int)e - 25);
    return s ? -v : v;
}

/* bf16 is the top half of an fp32 word (moe-fused/src/main.mm:43). */
double kqref_bf16_to_f64(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
}

uint16_t kqref_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000;
    uint32_t ex = (x >> 23) & 0xff;
    uint32_t man = x & 0x7fffff;
    if (ex == 0xff) return (uint16_t)(sign | 0x7c00 | (man ? 0x200 : 0));
    int e = (int)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000;
        int shift = 14 - e;  /* 24-bit significand -> subnormal field */
        uint32_t q = man >> shift, rem = man & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (uint32_t)(e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) ++q; /* carry may reach inf: correct */
    return (uint16_t)(sign | q);
}

static double g_f16tab[65536];
static pthread_once_t g_tab_once = PTHREAD_ONCE_INIT;
static void build_tab(void) {
    for (uint32_t i = 0; i < 65536; ++i) g_f16tab[i] = kqref_f16_to_f64((uint16_t)i);
}
static inline double H(uint16_t h) { return g_f16tab[h]; }
static inline double BF(uint16_t h) { return kqref_bf16_to_f64(h); }
static inline double META(uint16_t h, int dt) { return dt == KQREF_BF16 ? BF(h) : H(h); }

/* ------------------------------------------------------------------ */
/* row-block threading (restates the std::thread split of              */
/* int4-gemv/src/main.mm:81-92 / moe-fused/src/main.mm:63-72)          */
/* ------------------------------------------------------------------ */
typedef void (*rows_fn)(void* ctx, uint32_t m0, uint32_t m1);
typedef struct { rows_fn fn; void* ctx; uint32_t m0, m1; } rows_job;
static void* rows_tramp(void* p) {
    rows_job* j = (rows_job*)p;
    j->fn(j->ctx, j->m0, j->m1);
    return NULL;
}
static int ncores(int nthreads) {
    if (nthreads > 0) return nthreads;
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}
static void par_rows(uint32_t M, int nthreads, rows_fn fn, void* ctx) {
    int n = ncores(nthreads);
    if (n > 256) n = 256;
    if (n <= 1 || M < 64) { fn(ctx, 0, M); return; }
    uint32_t chunk = (M + (uint32_t)n - 1) / (uint32_t)n;
    pthread_t th[256];
    rows_job jobs[256];
    int started = 0;
    for (int i = 0; i < n; ++i) {
        uint32_t a = (uint32_t)i * chunk, b = a + chunk < M ? a + chunk : M;
        if (a >= b) break;
        jobs[i] = (rows_job){fn, ctx, a, b};
        if (pthread_create(&th[i], NULL, rows_tramp, &jobs[i]) != 0) {
            fn(ctx, a, b);
            jobs[i].fn = NULL;
        }
        started = i + 1;
    }
    for (int i = 0; i < started; ++i)
        if (jobs[i].fn) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------ */
/* int4 GEMV                                                           */
/* ------------------------------------------------------------------ */
typedef struct {
    const uint32_t* W; const uint16_t* S; const uint16_t* B;
    int inter, dt; const uint16_t* x; double* y;
    uint32_t M, K, G;
} int4_ctx;

/* cpuRefRows int4-gemv/src/main.mm:64-79: for every k in order,
 * acc += (S*q + B) * x in fp64, q = (word >> 4*(k&7)) & 0xF, g = k / G. */
static void int4_rows(void* p, uint32_t m0, uint32_t m1) {
    const int4_ctx* c = (const int4_ctx*)p;
    const uint32_t wpr = c->K / 8, gpr = c->K / c->G;
    for (uint32_t m = m0; m < m1; ++m) {
        const uint32_t* wr = c->W + (size_t)m * wpr;
        double acc = 0.0;
        for (uint32_t k = 0; k < c->K; ++k) {
            uint32_t word = wr[k >> 3];
            uint32_t q = (word >> (4 * (k & 7))) & 0xF;
            uint32_t g = k / c->G;
            double s, b;
            if (c->inter) {  /* int4RefRows vq-gemv/src/main.mm:71-76: sb[2g], sb[2g+1] */
                const uint16_t* sb = c->S + (size_t)m * gpr * 2;
                s = META(sb[2 * g], c->dt);
                b = META(sb[2 * g + 1], c->dt);
            } else {
                s = META(c->S[(size_t)m * gpr + g], c->dt);
                b = META(c->B[(size_t)m * gpr + g], c->dt);
            }
            acc += (s * (double)q + b) * H(c->x[k]);
        }
        c->y[m] = acc;
    }
}

void kqref_int4_gemv_f64(const uint32_t* W, const uint16_t* S, const uint16_t* B,
                         int sb_interleaved, int sb_dtype, const uint16_t* X, double* Y,
                         uint32_t M, uint32_t K, uint32_t G, uint32_t batch, int nthreads) {
    pthread_once(&g_tab_once, build_tab);
    for (uint32_t b = 0; b < batch; ++b) {
        int4_ctx c = {W, S, B, sb_interleaved, sb_dtype, X + (size_t)b * K, Y + (size_t)b * M, M, K, G};
        par_rows(M, nthreads, int4_rows, &c);
    }
}

/* xsum32 int4-gemv/src/kernels.metal:54-65: for i = 0..7 the kernel does
 * s += float(v.x) + float(v.y) + float(v.z) + float(v.w) on half4 v =
 * x[8j+i], i.e. s = s + (((a + b) + c) + d) in fp32. Restated in that order
 * (volatile keeps every partial sum a rounded fp32). */
void kqref_xsum32(const uint16_t* X, float* xs, uint32_t K, uint32_t batch) {
    pthread_once(&g_tab_once, build_tab);
    for (uint32_t b = 0; b < batch; ++b)
        for (uint32_t j = 0; j < K / 32; ++j) {
            volatile float s = 0.0f;
            const uint16_t* p = X + (size_t)b * K + 32 * j;
            for (uint32_t i = 0; i < 8; ++i) {
                volatile float t = (float)H(p[4 * i]) + (float)H(p[4 * i + 1]);
                t = t + (float)H(p[4 * i + 2]);
                t = t + (float)H(p[4 * i + 3]);
                s = s + t;
            }
            xs[(size_t)b * (K / 32) + j] = s;
        }
}

/* ------------------------------------------------------------------ */
/* VQ GEMV                                                             */
/* ------------------------------------------------------------------ */
typedef struct {
    const uint8_t* IDX; const uint16_t* C; const uint16_t* S; const uint16_t* x; double* y;
    uint32_t M, K, rpc, sg;
} vq_ctx;

/* vqRefRows vq-gemv/src/main.mm:51-66: acc += s * (C[2c]*x[2i] + C[2c+1]*x[2i+1]),
 * s = S[m, i/16] for scale group 32; generalised to S[m, 2i/sg] and codebook
 * block m / rows_per_cb. */
static void vq_rows(void* p, uint32_t m0, uint32_t m1) {
    const vq_ctx* c = (const vq_ctx*)p;
    const uint32_t spr = c->K / c->sg;
    for (uint32_t m = m0; m < m1; ++m) {
        const uint8_t* ir = c->IDX + (size_t)m * (c->K / 2);
        const uint16_t* sr = c->S + (size_t)m * spr;
        const uint16_t* cb = c->C + (size_t)(m / c->rpc) * 512;
        double acc = 0.0;
        for (uint32_t i = 0; i < c->K / 2; ++i) {
            uint32_t code = ir[i];
            double s = H(sr[(2 * i) / c->sg]);
            acc += s * (H(cb[2 * code]) * H(c->x[2 * i]) + H(cb[2 * code + 1]) * H(c->x[2 * i + 1]));
        }
        c->y[m] = acc;
    }
}

void kqref_vq_gemv_f64(const uint8_t* IDX, const uint16_t* C, const uint16_t* S,
                       const uint16_t* X, double* Y, uint32_t M, uint32_t K,
                       uint32_t rows_per_cb, uint32_t scale_group, uint32_t batch,
                       int nthreads) {
    pthread_once(&g_tab_once, build_tab);
    for (uint32_t b = 0; b < batch; ++b) {
        vq_ctx c = {IDX, C, S, X + (size_t)b * K, Y + (size_t)b * M, M, K, rows_per_cb, scale_group};
        par_rows(M, nthreads, vq_rows, &c);
    }
}

/* ------------------------------------------------------------------ */
/* MoE                                                                 */
/* ------------------------------------------------------------------ */
static double elem(const void* p, int dt, size_t i) {
    if (dt == KQREF_F32) return (double)((const float*)p)[i];
    if (dt == KQREF_BF16) return BF(((const uint16_t*)p)[i]);
    return H(((const uint16_t*)p)[i]);
}

void kqref_moe_router_f64(const void* R, int r_dtype, const void* X, int x_dtype,
                          uint32_t batch, const kqref_moe_desc* d,
                          uint32_t* idx, double* wgt, double* logits) {
    pthread_once(&g_tab_once, build_tab);
    const uint32_t NE = d->n_experts, HID = d->hidden, TK = d->top_k;
    double* lg = (double*)malloc(sizeof(double) * NE);
    double* lg2 = (double*)malloc(sizeof(double) * NE);
    for (uint32_t b = 0; b < batch; ++b) {
        /* logits in fp64 (moe-fused/src/main.mm:304-309) */
        for (uint32_t e = 0; e < NE; ++e) {
            double s = 0.0;
            for (uint32_t k = 0; k < HID; ++k)
                s += elem(R, r_dtype, (size_t)e * HID + k) * elem(X, x_dtype, (size_t)b * HID + k);
            lg[e] = s;
            lg2[e] = s;
            if (logits) logits[(size_t)b * NE + e] = s;
        }
        /* top-k by repeated strict-greater argmax (moe-fused/src/main.mm:310-315) */
        double sel[64];
        for (uint32_t j = 0; j < TK; ++j) {
            uint32_t bi = 0;
            double bv = -1e300;
            for (uint32_t e = 0; e < NE; ++e)
                if (lg2[e] > bv) { bv = lg2[e]; bi = e; }
            idx[(size_t)b * TK + j] = bi;
            sel[j] = bv;
            lg2[bi] = -1e300;
        }
        /* softmax over the chosen k (moe-fused/src/main.mm:316-319) */
        double mx = sel[0], sm = 0.0;
        for (uint32_t j = 1; j < TK; ++j) mx = sel[j] > mx ? sel[j] : mx;
        double w[64];
        for (uint32_t j = 0; j < TK; ++j) { w[j] = exp(sel[j] - mx); sm += w[j]; }
        for (uint32_t j = 0; j < TK; ++j) wgt[(size_t)b * TK + j] = w[j] / sm;
    }
    free(lg);
    free(lg2);
}

typedef struct {
    const uint8_t* blob; uint64_t proj; const kqref_moe_desc* d;
    const double* x; double* y; uint32_t K;
} proj_ctx;

/* refProj moe-fused/src/main.mm:46-62: group 64, bf16 S/B, output bias BI. */
static void proj_rows(void* p, uint32_t m0, uint32_t m1) {
    const proj_ctx* c = (const proj_ctx*)p;
    const uint8_t* base = c->blob + c->proj;
    const uint32_t* W = (const uint32_t*)(base + c->d->sub_w);
    const uint16_t* S = (const uint16_t*)(base + c->d->sub_s);
    const uint16_t* B = (const uint16_t*)(base + c->d->sub_b);
    const uint16_t* BI = (const uint16_t*)(base + c->d->sub_bi);
    const uint32_t wpr = c->K / 8, gpr = c->K / 64;
    for (uint32_t m = m0; m < m1; ++m) {
        double a = 0.0;
        for (uint32_t k = 0; k < c->K; ++k) {
            uint32_t q = (W[(size_t)m * wpr + (k >> 3)] >> (4 * (k & 7))) & 0xF;
            a += (BF(S[(size_t)m * gpr + k / 64]) * q + BF(B[(size_t)m * gpr + k / 64])) * c->x[k];
        }
        c->y[m] = a + BF(BI[m]);
    }
}

void kqref_moe_proj_f64(const uint8_t* blob, uint64_t proj, const kqref_moe_desc* d,
                        const double* x, double* y, uint32_t M, uint32_t K, int nthreads) {
    pthread_once(&g_tab_once, build_tab);
    proj_ctx c = {blob, proj, d, x, y, K};
    par_rows(M, nthreads, proj_rows, &c);
}

double kqref_swiglu_f64(double g, double u) {
    double gg = g < 7.0 ? g : 7.0;
    double ll = u > 7.0 ? 7.0 : (u < -7.0 ? -7.0 : u);
    return (gg / (1.0 + exp(-1.702 * gg))) * (ll + 1.0);
}

void kqref_moe_gate_up_f64(const uint8_t* pool, const kqref_moe_desc* d, const uint32_t* idx,
                           const void* X, int x_dtype, uint32_t batch, double* Hout, int nthreads) {
    pthread_once(&g_tab_once, build_tab);
    const uint32_t HID = d->hidden, IN = d->inter, TK = d->top_k;
    double* xd = (double*)malloc(sizeof(double) * HID);
    double* g = (double*)malloc(sizeof(double) * IN);
    double* u = (double*)malloc(sizeof(double) * IN);
    for (uint32_t b = 0; b < batch; ++b) {
        for (uint32_t k = 0; k < HID; ++k) xd[k] = elem(X, x_dtype, (size_t)b * HID + k);
        for (uint32_t j = 0; j < TK; ++j) {
            const uint8_t* bb = pool + (size_t)idx[(size_t)b * TK + j] * d->blob;
            kqref_moe_proj_f64(bb, d->off_gate, d, xd, g, IN, HID, nthreads);
            kqref_moe_proj_f64(bb, d->off_up, d, xd, u, IN, HID, nthreads);
            double* h = Hout + ((size_t)b * TK + j) * IN;
            for (uint32_t i = 0; i < IN; ++i) h[i] = kqref_swiglu_f64(g[i], u[i]);
        }
    }
    free(xd); free(g); free(u);
}

void kqref_moe_down_f64(const uint8_t* pool, const kqref_moe_desc* d, const uint32_t* idx,
                        const double* wgt, const void* Hin, int h_dtype, uint32_t batch,
                        double* Y, int nthreads) {
    pthread_once(&g_tab_once, build_tab);
    const uint32_t HID = d->hidden, IN = d->inter, TK = d->top_k;
    double* h = (double*)malloc(sizeof(double) * IN);
    double* yy = (double*)malloc(sizeof(double) * HID);
    for (uint32_t b = 0; b < batch; ++b) {
        double* y = Y + (size_t)b * HID;
        for (uint32_t i = 0; i < HID; ++i) y[i] = 0.0;
        for (uint32_t j = 0; j < TK; ++j) {
            size_t slot = (size_t)b * TK + j;
            for (uint32_t i = 0; i < IN; ++i)
                h[i] = h_dtype == KQREF_F16 ? H(((const uint16_t*)Hin)[slot * IN + i])
                                            : ((const double*)Hin)[slot * IN + i];
            const uint8_t* bb = pool + (size_t)idx[slot] * d->blob;
            kqref_moe_proj_f64(bb, d->off_down, d, h, yy, HID, IN, nthreads);
            for (uint32_t i = 0; i < HID; ++i) y[i] += wgt[slot] * yy[i];
        }
    }
    free(h); free(yy);
}

void kqref_moe_block_f64(const uint8_t* pool, const kqref_moe_desc* d, const void* R, int r_dtype,
                         const void* X, int x_dtype, uint32_t batch, uint32_t* idx, double* wgt,
                         double* Y, int nthreads) {
    const size_t nh = (size_t)batch * d->top_k * d->inter;
    double* Hd = (double*)malloc(sizeof(double) * (nh ? nh : 1));
    kqref_moe_router_f64(R, r_dtype, X, x_dtype, batch, d, idx, wgt, NULL);
    kqref_moe_gate_up_f64(pool, d, idx, X, x_dtype, batch, Hd, nthreads);
    kqref_moe_down_f64(pool, d, idx, wgt, Hd, KQREF_F32, batch, Y, nthreads);
    free(Hd);
}
