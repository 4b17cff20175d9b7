/*
 * jhq_oracle.c — CPU restatement of the lrlorry/JHQ_GPU JHQ IVF path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): see jhq_oracle.h
 * for who may load it and for the pinning status of each function.
 *
 * Built with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf() placed where the reference's own build contracts one.
 */
#include "jhq_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#ifndef M_PI
#define M_PI 3.14159265358979323846
#endif
#ifndef M_SQRT2
#define M_SQRT2 1.41421356237309504880
#endif

/* ------------------------------------------------------------------------ */
/* Row-parallel loops.  Every row (vector, query) is computed by one thread   */
/* exactly as in the serial loop, so results do not depend on the thread     */
/* count; o_set_threads(1) (the default) runs everything on the caller.       */
/* ------------------------------------------------------------------------ */
static int g_threads = 1;

void o_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 256 ? 256 : n); }
int o_get_threads(void) { return g_threads; }

typedef void (*o_range_fn)(void* ctx, int64_t lo, int64_t hi);
typedef struct { o_range_fn fn; void* ctx; int64_t lo, hi; } o_job;

static void* o_job_run(void* a) {
    o_job* j = (o_job*)a;
    j->fn(j->ctx, j->lo, j->hi);
    return NULL;
}

/* fn(ctx, lo, hi) over [0, n) split into at most g_threads contiguous ranges. */
static void o_parallel(int64_t n, o_range_fn fn, void* ctx) {
    int T = g_threads;
    if (T > n) T = (int)n;
    if (T <= 1) {
        if (n > 0) fn(ctx, 0, n);
        return;
    }
    o_job jobs[256];
    pthread_t th[256];
    int started[256];
    for (int t = 0; t < T; t++) {
        jobs[t].fn = fn;
        jobs[t].ctx = ctx;
        jobs[t].lo = n * t / T;
        jobs[t].hi = n * (t + 1) / T;
        started[t] = 0;
    }
    for (int t = 1; t < T; t++) started[t] = pthread_create(&th[t], NULL, o_job_run, &jobs[t]) == 0;
    o_job_run(&jobs[0]);
    for (int t = 1; t < T; t++) {
        if (started[t]) pthread_join(th[t], NULL);
        else o_job_run(&jobs[t]); /* thread creation failed: run it here */
    }
}

/* ------------------------------------------------------------------------ */
/* std::mt19937 (C++ [rand.eng.mers] parameters), as used by                 */
/* cpu/jl_transform.cpp:27 (std::mt19937 rng(seed)).                         */
/* ------------------------------------------------------------------------ */
void o_mt_seed(o_mt19937* g, uint32_t seed) {
    g->mt[0] = seed;
    for (int i = 1; i < 624; i++)
        g->mt[i] = 1812433253u * (g->mt[i - 1] ^ (g->mt[i - 1] >> 30)) + (uint32_t)i;
    g->idx = 624;
}

static void o_mt_twist(o_mt19937* g) {
    for (int i = 0; i < 624; i++) {
        uint32_t y = (g->mt[i] & 0x80000000u) | (g->mt[(i + 1) % 624] & 0x7fffffffu);
        uint32_t v = g->mt[(i + 397) % 624] ^ (y >> 1);
        if (y & 1u) v ^= 0x9908b0dfu;
        g->mt[i] = v;
    }
    g->idx = 0;
}

uint32_t o_mt_next(o_mt19937* g) {
    if (g->idx >= 624) o_mt_twist(g);
    uint32_t y = g->mt[g->idx++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

void o_mt_fill(uint32_t seed, uint32_t* out, int64_t n) {
    o_mt19937 g;
    o_mt_seed(&g, seed);
    for (int64_t i = 0; i < n; i++) out[i] = o_mt_next(&g);
}

/* libstdc++ generate_canonical<float, 24>(mt19937): one 32-bit draw,
 * float(u) / 2^32, clamped below 1.                                          */
static float o_canonical(o_mt19937* g) {
    float s = (float)o_mt_next(g);
    float r = s / 4294967296.0f;
    if (r >= 1.0f) r = nextafterf(1.0f, 0.0f);
    return r;
}

/* libstdc++ normal_distribution<float>::operator() (Marsaglia polar method,
 * returns y*mult first and caches x*mult), as drawn by
 * cpu/jl_transform.cpp:28-29.  The reference compiles cpu/ with
 * -O3 -march=native, which contracts x*x + y*y into fma(x, x, y*y).          */
void o_normal_fill(uint32_t seed, float* out, int64_t n) {
    o_mt19937 g;
    o_mt_seed(&g, seed);
    int64_t i = 0;
    while (i < n) {
        float x, y, r2;
        do {
            x = (float)((double)(2.0f * o_canonical(&g)) - 1.0);
            y = (float)((double)(2.0f * o_canonical(&g)) - 1.0);
            r2 = fmaf(x, x, y * y);
        } while ((double)r2 > 1.0 || (double)r2 == 0.0);
        const float mult = sqrtf(-2.0f * logf(r2) / r2);
        out[i++] = y * mult;
        if (i < n) out[i++] = x * mult;
    }
}

/* ------------------------------------------------------------------------ */
/* cpu/erfinv.h:7-27 — Winitzki approximation plus one Newton step.          */
/* The -march=native build contracts 1-a*a, k2Pi/kC + 0.5*ln1 and            */
/* t*t - ln1/kC.                                                             */
/* ------------------------------------------------------------------------ */
float o_erfinv_f(float x) {
    if (x >= 1.0f) return INFINITY;
    if (x <= -1.0f) return -INFINITY;
    if (x == 0.0f) return 0.0f;
    const float sign = (x > 0.0f) ? 1.0f : -1.0f;
    const float a = fabsf(x);
    const float kC = 0.147f;
    const float k2Pi = 2.0f / 3.14159265358979f;
    const float ln1 = logf(fmaf(-a, a, 1.0f));
    const float t = fmaf(0.5f, ln1, k2Pi / kC);
    float z = sign * sqrtf(sqrtf(fmaf(t, t, -(ln1 / kC))) - t);
    const float err = erff(z) - x;
    const float der = (2.0f / sqrtf((float)M_PI)) * expf(-z * z);
    z -= err / der;
    return z;
}

/* cpu/codebook.cpp:60-80 — analytic Lloyd-Max 1-D codewords. */
void o_lloyd_max_c1d(float sigma, int K1D, float* c1d) {
    for (int i = 0; i < K1D; i++) {
        const float q_i = ((float)i + 0.5f) / (float)K1D;
        c1d[i] = sigma * (float)M_SQRT2 * o_erfinv_f(fmaf(2.0f, q_i, -1.0f));
    }
}

/* cpu/jl_transform.cpp:73-83 — sigma from raw vectors, double accumulation. */
float o_estimate_sigma(const float* x, int64_t n, int d) {
    double sum2 = 0.0;
    for (int64_t i = 0; i < n * (int64_t)d; i++) sum2 += (double)x[i] * (double)x[i];
    return (float)sqrt(sum2 / ((double)n * d));
}

static int cmp_float(const void* a, const void* b) {
    const float fa = *(const float*)a, fb = *(const float*)b;
    return (fa > fb) - (fa < fb);
}

static int nearest_sorted(const float* arr, int n, float v) {
    /* jhq_v14_streaming_add/encode.cu:6-18, cpu/codebook.cpp:82-94 */
    if (n == 1) return 0;
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (v < 0.5f * (arr[mid] + arr[mid + 1])) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}

/* cpu/codebook.cpp:8-58 — 1-D Lloyd k-means, quantile init. */
int o_train_1d_kmeans(const float* vals, int64_t n, int Kr, int max_iter, float* out) {
    if (n <= 0 || Kr <= 0) return 0;
    if (n < Kr) Kr = (int)n;
    float* sorted = (float*)malloc((size_t)n * sizeof(float));
    memcpy(sorted, vals, (size_t)n * sizeof(float));
    qsort(sorted, (size_t)n, sizeof(float), cmp_float);
    float* c = (float*)malloc((size_t)Kr * sizeof(float));
    const float nf = (float)n;
    for (int i = 0; i < Kr; i++) {
        int64_t idx = (int64_t)(((float)i + 0.5f) / (float)Kr * nf);
        if (idx > n - 1) idx = n - 1;
        c[i] = sorted[idx];
    }
    double* sum = (double*)malloc((size_t)Kr * sizeof(double));
    int64_t* cnt = (int64_t*)malloc((size_t)Kr * sizeof(int64_t));
    for (int iter = 0; iter < max_iter; iter++) {
        memset(sum, 0, (size_t)Kr * sizeof(double));
        memset(cnt, 0, (size_t)Kr * sizeof(int64_t));
        for (int64_t i = 0; i < n; i++) {
            const float v = vals[i];
            const int lo = nearest_sorted(c, Kr, v);
            sum[lo] += v;
            cnt[lo]++;
        }
        int changed = 0;
        for (int i = 0; i < Kr; i++) {
            float new_c;
            if (cnt[i] == 0) {
                int64_t idx = (int64_t)(((float)i + 0.5f) / (float)Kr * nf);
                if (idx > n - 1) idx = n - 1;
                new_c = sorted[idx];
            } else {
                new_c = (float)(sum[i] / (double)cnt[i]);
            }
            if (new_c != c[i]) { c[i] = new_c; changed = 1; }
        }
        qsort(c, (size_t)Kr, sizeof(float), cmp_float);
        if (!changed) break;
    }
    memcpy(out, c, (size_t)Kr * sizeof(float));
    free(sorted); free(c); free(sum); free(cnt);
    return Kr;
}

/* ------------------------------------------------------------------------ */
/* Householder QR, LAPACK xGEQR2 + xORG2R conventions (the reference calls    */
/* sgeqrf_/sorgqr_ at cpu/jl_transform.cpp:35-53).  beta = -sign(alpha)*norm  */
/* fixes the column signs of Q.  Computed in double, stored as float.         */
/* ------------------------------------------------------------------------ */
int o_householder_qr(int d, float* A32) {
    const int64_t n = d;
    double* A = (double*)malloc((size_t)(n * n) * sizeof(double));
    double* tau = (double*)malloc((size_t)n * sizeof(double));
    for (int64_t i = 0; i < n * n; i++) A[i] = (double)A32[i];
    /* xGEQR2 */
    for (int64_t k = 0; k < n; k++) {
        double* colk = A + k * n;
        const double alpha = colk[k];
        double ss = 0.0;
        for (int64_t i = k + 1; i < n; i++) ss += colk[i] * colk[i];
        if (ss == 0.0) { tau[k] = 0.0; continue; }
        const double nrm = sqrt(alpha * alpha + ss);
        const double beta = (alpha >= 0.0) ? -nrm : nrm;
        tau[k] = (beta - alpha) / beta;
        const double scal = 1.0 / (alpha - beta);
        for (int64_t i = k + 1; i < n; i++) colk[i] *= scal;
        colk[k] = beta;
        /* apply H_k = I - tau v v^T (v[k] = 1) to columns k+1.. */
        for (int64_t j = k + 1; j < n; j++) {
            double* colj = A + j * n;
            double w = colj[k];
            for (int64_t i = k + 1; i < n; i++) w += colk[i] * colj[i];
            w *= tau[k];
            colj[k] -= w;
            for (int64_t i = k + 1; i < n; i++) colj[i] -= w * colk[i];
        }
    }
    /* xORG2R */
    for (int64_t i = n - 1; i >= 0; i--) {
        double* coli = A + i * n;
        if (i < n - 1) {
            coli[i] = 1.0;
            for (int64_t j = i + 1; j < n; j++) {
                double* colj = A + j * n;
                double w = 0.0;
                for (int64_t r = i; r < n; r++) w += coli[r] * colj[r];
                w *= tau[i];
                for (int64_t r = i; r < n; r++) colj[r] -= w * coli[r];
            }
            for (int64_t r = i + 1; r < n; r++) coli[r] *= -tau[i];
        }
        coli[i] = 1.0 - tau[i];
        for (int64_t r = 0; r < i; r++) coli[r] = 0.0;
    }
    for (int64_t i = 0; i < n * n; i++) A32[i] = (float)A[i];
    free(A); free(tau);
    return 0;
}

/* cpu/jl_transform.cpp:25-56 — Gaussian fill in storage order, then QR. */
void o_build_rotation(int d, int seed, float* Pi) {
    o_normal_fill((uint32_t)seed, Pi, (int64_t)d * d);
    o_householder_qr(d, Pi);
}

/* ------------------------------------------------------------------------ */
/* Rotation y = Pi x (jhq_v14_streaming_add/jhq_gpu_index.cu:444-448 and      */
/* search.cu:338-339 use cuBLAS; this build pins the order to an fmaf chain   */
/* over k ascending, the order the HIP rotation kernel uses).                */
/* ------------------------------------------------------------------------ */
typedef struct { const float *P, *x; int d; float* y; } o_rot_ctx;

static void o_rotate_rows(void* c, int64_t lo, int64_t hi) {
    const o_rot_ctx* a = (const o_rot_ctx*)c;
    const int d = a->d;
    for (int64_t i = lo; i < hi; i++) {
        const float* xi = a->x + i * d;
        for (int j = 0; j < d; j++) {
            const float* pj = a->P + (int64_t)j * d;
            float acc = 0.0f;
            for (int k = 0; k < d; k++) acc = fmaf(xi[k], pj[k], acc);
            a->y[i * d + j] = acc;
        }
    }
}

void o_rotate(const float* P, const float* x, int64_t n, int d, float* y) {
    o_rot_ctx a = {P, x, d, y};
    o_parallel(n, o_rotate_rows, &a);
}

static int bits_per_dim(int d, int M, int K1D) {
    (void)d; (void)M;
    int b = 0;
    while ((1 << b) < K1D) b++;
    return b;
}

/* encode.cu:20-41 (primary_encode_kernel) == cpu/codebook.cpp:96-110. */
typedef struct { const float* y; int d, M; const float* c1d; int K1D; uint8_t* codes; } o_penc_ctx;

static void o_primary_encode_rows(void* c, int64_t lo, int64_t hi) {
    const o_penc_ctx* a = (const o_penc_ctx*)c;
    const float* y = a->y;
    const float* c1d = a->c1d;
    uint8_t* codes = a->codes;
    const int d = a->d, M = a->M, K1D = a->K1D;
    const int Ds = d / M, bpd = bits_per_dim(d, M, K1D);
    for (int64_t i = lo; i < hi; i++) {
        const float* yi = y + i * d;
        for (int m = 0; m < M; m++) {
            uint8_t cm = 0;
            for (int k = 0; k < Ds; k++) {
                const int j = nearest_sorted(c1d, K1D, yi[m * Ds + k]);
                cm |= (uint8_t)(j << (k * bpd));
            }
            codes[i * M + m] = cm;
        }
    }
}

void o_primary_encode(const float* y, int64_t n, int d, int M, const float* c1d,
                      int K1D, uint8_t* codes) {
    o_penc_ctx a = {y, d, M, c1d, K1D, codes};
    o_parallel(n, o_primary_encode_rows, &a);
}

/* encode.cu:43-86 (residual_encode_kernel): nibble packing (even j low
 * nibble), corr = 2 * sum_j yhat_j * rhat_j with the product contracted.     */
void o_residual_encode(const float* y, const uint8_t* primary, int64_t n, int d,
                       int M, const float* c1d, int K1D, const float* res_c1d,
                       int Kr, int Br, uint8_t* res_codes, float* corr) {
    o_residual_encode_rc(y, primary, n, d, M, c1d, K1D, res_c1d, Kr, 1, Br, res_codes, corr);
}

/* RC residual codebooks of Kr words: RC = 1 (every dimension, the
 * reference), or RC = M (dimension j uses codebook j / Ds; an extension with
 * no reference counterpart). */
typedef struct {
    const float* y; const uint8_t* primary; int d, M; const float* c1d; int K1D;
    const float* res_c1d; int Kr, RC, Br; uint8_t* res_codes; float* corr;
} o_renc_ctx;

static void o_residual_encode_rows(void* c, int64_t lo, int64_t hi) {
    const o_renc_ctx* a = (const o_renc_ctx*)c;
    const float* y = a->y;
    const uint8_t* primary = a->primary;
    const float *c1d = a->c1d, *res_c1d = a->res_c1d;
    uint8_t* res_codes = a->res_codes;
    float* corr = a->corr;
    const int d = a->d, M = a->M, K1D = a->K1D, Kr = a->Kr, RC = a->RC, Br = a->Br;
    const int Ds = d / M, bpd = bits_per_dim(d, M, K1D);
    const int bpv = (d * Br + 7) / 8;
    const int kmask = K1D - 1;
    for (int64_t i = lo; i < hi; i++) {
        const float* yi = y + i * d;
        const uint8_t* pc = primary + i * M;
        uint8_t* rc = res_codes + i * bpv;
        memset(rc, 0, (size_t)bpv);
        float dot = 0.0f;
        for (int j = 0; j < d; j++) {
            const int m = j / Ds, k = j % Ds;
            const int pidx = (pc[m] >> (k * bpd)) & kmask;
            const float yhat = c1d[pidx];
            const float resid = yi[j] - yhat;
            const float* rcb = res_c1d + (RC == 1 ? 0 : (int64_t)m * Kr);
            const int ri = nearest_sorted(rcb, Kr, resid);
            const float rhat = rcb[ri];
            if (Br == 4) {
                if (j % 2 == 0) rc[j / 2] = (uint8_t)(ri & 0x0F);
                else rc[j / 2] |= (uint8_t)((ri & 0x0F) << 4);
            } else {
                rc[j] = (uint8_t)ri;
            }
            dot = fmaf(yhat, rhat, dot);
        }
        corr[i] = 2.0f * dot;
    }
}

void o_residual_encode_rc(const float* y, const uint8_t* primary, int64_t n, int d,
                          int M, const float* c1d, int K1D, const float* res_c1d,
                          int Kr, int RC, int Br, uint8_t* res_codes, float* corr) {
    o_renc_ctx a = {y, primary, d, M, c1d, K1D, res_c1d, Kr, RC, Br, res_codes, corr};
    o_parallel(n, o_residual_encode_rows, &a);
}

/* cpu/codebook.cpp:161-171 */
void o_reconstruct(const uint8_t* code, int d, int M, const float* c1d, int K1D,
                   float* out) {
    const int Ds = d / M, bpd = bits_per_dim(d, M, K1D), mask = K1D - 1;
    for (int m = 0; m < M; m++)
        for (int k = 0; k < Ds; k++)
            out[m * Ds + k] = c1d[(code[m] >> (k * bpd)) & mask];
}

/* search.cu:65-91 (build_byte_lut_kernel) == cpu/codebook.cpp:112-129:
 * lut[m][v] = sum_k (q[m*Ds+k] - c1d[digit_k(v)])^2, accumulated with fma.  */
void o_flat_lut(const float* q_rot, int d, int M, const float* c1d, int K1D,
                float* lut) {
    const int Ds = d / M, bpd = bits_per_dim(d, M, K1D), mask = K1D - 1;
    for (int m = 0; m < M; m++) {
        const float* qm = q_rot + m * Ds;
        for (int v = 0; v < 256; v++) {
            float s = 0.0f;
            for (int k = 0; k < Ds && k < 8; k++) {
                const int j = (v >> (k * bpd)) & mask;
                const float diff = qm[k] - c1d[j];
                s = fmaf(diff, diff, s);
            }
            lut[m * 256 + v] = s;
        }
    }
}

/* cpu/codebook.cpp:131-145 */
void o_factored_lut(const float* q_rot, int d, int M, const float* c1d, int K1D,
                    float* lut) {
    const int Ds = d / M;
    for (int m = 0; m < M; m++)
        for (int k = 0; k < Ds; k++)
            for (int i = 0; i < K1D; i++) {
                const float diff = q_rot[m * Ds + k] - c1d[i];
                lut[(m * Ds + k) * K1D + i] = diff * diff;
            }
}

/* search.cu:146-151: dist = sum_m lut[m][code_m], m ascending. */
float o_adc_flat(const uint8_t* code, int M, const float* lut) {
    float dist = 0.0f;
    for (int m = 0; m < M; m++) dist += lut[m * 256 + code[m]];
    return dist;
}

/* cpu/codebook.cpp:147-159 */
float o_adc_factored(const uint8_t* code, int d, int M, int K1D, const float* lut) {
    const int Ds = d / M, mask = K1D - 1;
    int bpd = 0;
    while ((1 << bpd) < K1D) bpd++;
    float dist = 0.0f;
    for (int m = 0; m < M; m++)
        for (int k = 0; k < Ds; k++)
            dist += lut[(m * Ds + k) * K1D + ((code[m] >> (k * bpd)) & mask)];
    return dist;
}

/* ------------------------------------------------------------------------ */
/* IVF                                                                       */
/* ------------------------------------------------------------------------ */
/* jhq_gpu_index.cu:243-249: ||c||^2 accumulated in double. */
void o_cent_norms(const float* cent, int nlist, int d, float* norms) {
    for (int c = 0; c < nlist; c++) {
        double s = 0.0;
        const float* cc = cent + (int64_t)c * d;
        for (int j = 0; j < d; j++) s += (double)cc[j] * (double)cc[j];
        norms[c] = (float)s;
    }
}

static float dot_fma(const float* a, const float* b, int d) {
    float acc = 0.0f;
    for (int k = 0; k < d; k++) acc = fmaf(a[k], b[k], acc);
    return acc;
}

/* jhq_gpu_index.cu:23-40 (assign_from_dots_kernel): argmin ||c||^2 - 2<c,y>,
 * strict < so ties keep the lowest c.  <c,y> is the fmaf chain. */
typedef struct { const float *y, *cent, *norms; int d, nlist; int32_t* out; } o_asg_ctx;

static void o_assign_rows(void* c, int64_t lo, int64_t hi) {
    const o_asg_ctx* a = (const o_asg_ctx*)c;
    const float *y = a->y, *cent = a->cent, *norms = a->norms;
    const int d = a->d, nlist = a->nlist;
    int32_t* out = a->out;
    for (int64_t i = lo; i < hi; i++) {
        const float* yi = y + i * d;
        float best = fmaf(-2.0f, dot_fma(yi, cent, d), norms[0]);
        int bi = 0;
        for (int c = 1; c < nlist; c++) {
            const float s = fmaf(-2.0f, dot_fma(yi, cent + (int64_t)c * d, d), norms[c]);
            if (s < best) { best = s; bi = c; }
        }
        out[i] = bi;
    }
}

void o_assign(const float* y, int64_t n, int d, const float* cent,
              const float* norms, int nlist, int32_t* out) {
    o_asg_ctx a = {y, cent, norms, d, nlist, out};
    o_parallel(n, o_assign_rows, &a);
}

/* jhq_gpu_index.cu:228-299 (train_ivf_centroids). */
int o_train_ivf(const float* y, int64_t n, int d, int nlist, int iters, float* cent) {
    if (n < nlist) return -1;
    for (int c = 0; c < nlist; c++) {
        const int64_t src = (int64_t)c * n / nlist;
        memcpy(cent + (int64_t)c * d, y + src * d, (size_t)d * sizeof(float));
    }
    float* norms = (float*)malloc((size_t)nlist * sizeof(float));
    int32_t* asg = (int32_t*)malloc((size_t)n * sizeof(int32_t));
    double* sums = (double*)malloc((size_t)nlist * d * sizeof(double));
    int64_t* counts = (int64_t*)malloc((size_t)nlist * sizeof(int64_t));
    for (int iter = 0; iter < iters; iter++) {
        o_cent_norms(cent, nlist, d, norms);
        o_assign(y, n, d, cent, norms, nlist, asg);
        memset(sums, 0, (size_t)nlist * d * sizeof(double));
        memset(counts, 0, (size_t)nlist * sizeof(int64_t));
        for (int64_t i = 0; i < n; i++) {
            const int c = asg[i];
            counts[c]++;
            double* sc = sums + (int64_t)c * d;
            const float* yi = y + i * d;
            for (int j = 0; j < d; j++) sc[j] += yi[j];
        }
        for (int c = 0; c < nlist; c++) {
            float* cc = cent + (int64_t)c * d;
            if (counts[c] == 0) {
                const int64_t src = ((int64_t)c * 1103515245 + (int64_t)iter * 12345) % n;
                memcpy(cc, y + src * d, (size_t)d * sizeof(float));
                continue;
            }
            const double inv = 1.0 / (double)counts[c];
            const double* sc = sums + (int64_t)c * d;
            for (int j = 0; j < d; j++) cc[j] = (float)(sc[j] * inv);
        }
    }
    free(norms); free(asg); free(sums); free(counts);
    return 0;
}

/* jhq_gpu_index.cu:468-486: stable sort by list, offsets by prefix sum. */
void o_build_lists(const int32_t* assign, int64_t n, int nlist,
                   int32_t* offsets, int32_t* order) {
    memset(offsets, 0, (size_t)(nlist + 1) * sizeof(int32_t));
    for (int64_t i = 0; i < n; i++) offsets[assign[i] + 1]++;
    for (int c = 0; c < nlist; c++) offsets[c + 1] += offsets[c];
    int32_t* fill = (int32_t*)malloc((size_t)nlist * sizeof(int32_t));
    memcpy(fill, offsets, (size_t)nlist * sizeof(int32_t));
    for (int64_t i = 0; i < n; i++) order[fill[assign[i]]++] = (int32_t)i;
    free(fill);
}

/* ------------------------------------------------------------------------ */
/* Exact selection: jhq_v3_ivf/search.cu:22-25 (better_pair), :189-225 and    */
/* :242-279 — order by (dist, tag).                                          */
/* ------------------------------------------------------------------------ */
typedef struct { float d; int32_t t; } o_pair;

static int cmp_pair(const void* a, const void* b) {
    const o_pair* x = (const o_pair*)a;
    const o_pair* y = (const o_pair*)b;
    if (x->d < y->d) return -1;
    if (x->d > y->d) return 1;
    return (x->t > y->t) - (x->t < y->t);
}

int o_select_topk_pairs(const float* dist, const int32_t* tag, int64_t n, int k,
                        float* out_dist, int32_t* out_tag) {
    o_pair* p = (o_pair*)malloc((size_t)(n > 0 ? n : 1) * sizeof(o_pair));
    int64_t m = 0;
    for (int64_t i = 0; i < n; i++) {
        if (!(dist[i] < INFINITY)) continue; /* +inf never beats an empty slot */
        p[m].d = dist[i];
        p[m].t = tag[i];
        m++;
    }
    qsort(p, (size_t)m, sizeof(o_pair), cmp_pair);
    int filled = 0;
    for (int i = 0; i < k; i++) {
        if (i < m) { out_dist[i] = p[i].d; out_tag[i] = p[i].t; filled++; }
        else { out_dist[i] = INFINITY; out_tag[i] = -1; }
    }
    free(p);
    return filled;
}

int o_ck(float alpha, int k) {
    const int c = (int)ceilf(alpha * (float)k);
    return c > k ? c : k;
}

/* ------------------------------------------------------------------------ */
/* The approximate top-ck of the reference's IVF scan                         */
/* (jhq_v14_streaming_add/search.cu:105-195, scan_ivf_coalesced_kernel, one   */
/* 256-thread block per query).  Thread t visits candidates t, t+256, ... of   */
/* the probed lists laid end to end in probe order and keeps its 4 smallest   */
/* distances (insert at the last slot if strictly smaller, bubble up while    */
/* strictly smaller: :153-161); the 4*256 survivors sit at s[t*4 + i]         */
/* (:163-168).  Then ck rounds: every thread takes the first strict minimum   */
/* over s[t], s[t+256], ... (:176-178), a tree reduction keeps the left entry */
/* unless the right one is strictly smaller (:179-185), and the winner is     */
/* emitted and set to +inf (:186-191); no winner -> (+inf, -1).               */
/* ------------------------------------------------------------------------ */
#define V14_BLOCK 256
#define V14_KLOCAL 4

/* v14 block argmin over vals[0..n) with the strided per-thread scan and the
 * keep-left tree reduction; returns the winning index or -1. */
static int v14_block_argmin(const float* vals, int n) {
    float rv[V14_BLOCK];
    int ri[V14_BLOCK];
    for (int t = 0; t < V14_BLOCK; t++) {
        float bv = INFINITY;
        int bi = -1;
        for (int c = t; c < n; c += V14_BLOCK)
            if (vals[c] < bv) { bv = vals[c]; bi = c; }
        rv[t] = bv;
        ri[t] = bi;
    }
    for (int stride = V14_BLOCK >> 1; stride > 0; stride >>= 1)
        for (int t = 0; t < stride; t++)
            if (rv[t + stride] < rv[t]) { rv[t] = rv[t + stride]; ri[t] = ri[t + stride]; }
    return ri[0];
}

/* dists/poss: the query's candidates in the order the scan visits them
 * (local index = position in the probe-ordered concatenation). */
static void v14_topck(const float* dists, const int32_t* poss, int64_t total, int ck,
                      float* out_d, int32_t* out_p) {
    float sd[V14_BLOCK * V14_KLOCAL];
    int32_t sp[V14_BLOCK * V14_KLOCAL];
    for (int t = 0; t < V14_BLOCK; t++) {
        float ld[V14_KLOCAL];
        int32_t lp[V14_KLOCAL];
        for (int i = 0; i < V14_KLOCAL; i++) { ld[i] = INFINITY; lp[i] = -1; }
        for (int64_t c = t; c < total; c += V14_BLOCK) {
            const float dist = dists[c];
            if (dist < ld[V14_KLOCAL - 1]) {
                ld[V14_KLOCAL - 1] = dist;
                lp[V14_KLOCAL - 1] = poss[c];
                for (int i = V14_KLOCAL - 1; i > 0 && ld[i] < ld[i - 1]; --i) {
                    const float td = ld[i - 1]; ld[i - 1] = ld[i]; ld[i] = td;
                    const int32_t tp = lp[i - 1]; lp[i - 1] = lp[i]; lp[i] = tp;
                }
            }
        }
        for (int i = 0; i < V14_KLOCAL; i++) {
            sd[t * V14_KLOCAL + i] = ld[i];
            sp[t * V14_KLOCAL + i] = lp[i];
        }
    }
    for (int c = 0; c < ck; c++) {
        const int w = v14_block_argmin(sd, V14_BLOCK * V14_KLOCAL);
        out_d[c] = w >= 0 ? sd[w] : INFINITY;
        out_p[c] = w >= 0 ? sp[w] : -1;
        if (w >= 0) sd[w] = INFINITY;
    }
}

/* batched_topk_final_kernel (jhq_v14_streaming_add/search.cu:244-291): k
 * rounds of the same block argmin over the ck composite distances; the id is
 * list_ids[pos] of the winning slot, no winner -> (+inf, -1). */
static void v14_final(float* comp, const int32_t* cid, int ck, int k, float* out_d,
                      int32_t* out_i) {
    for (int r = 0; r < k; r++) {
        const int w = v14_block_argmin(comp, ck);
        out_i[r] = (w >= 0) ? cid[w] : -1;
        out_d[r] = (w >= 0) ? comp[w] : INFINITY;
        if (w >= 0) comp[w] = INFINITY;
    }
}

/* ------------------------------------------------------------------------ */
/* Whole search, one query at a time (jhq_v14_streaming_add/search.cu:315-386 */
/* pipeline).  mode 0: exact selection (jhq_v3_ivf/search.cu:22-25,189-279),  */
/* mode 1: the reference's approximate selection above.                       */
/* ------------------------------------------------------------------------ */
int o_search(const o_index* ix, const float* q, int64_t nq, int k,
             float* out_dist, int32_t* out_ids,
             int32_t* dbg_probes, int32_t* dbg_topck_pos, float* dbg_topck_dist) {
    return o_search_ex(ix, q, NULL, NULL, nq, k, out_dist, out_ids, dbg_probes,
                       dbg_topck_pos, dbg_topck_dist);
}

int o_search_ex(const o_index* ix, const float* q, const float* q_rot_in,
                const int32_t* probes_in, int64_t nq, int k,
                float* out_dist, int32_t* out_ids,
                int32_t* dbg_probes, int32_t* dbg_topck_pos, float* dbg_topck_dist) {
    return o_search_mode(ix, q, q_rot_in, probes_in, nq, k, 0, out_dist, out_ids, dbg_probes,
                         dbg_topck_pos, dbg_topck_dist);
}

typedef struct {
    const o_index* ix;
    const float *q, *q_rot_in;
    const int32_t* probes_in;
    int k, mode;
    float* out_dist;
    int32_t* out_ids;
    int32_t *dbg_probes, *dbg_topck_pos;
    float* dbg_topck_dist;
} o_search_ctx;

static void o_search_rows(void* cv, int64_t q0, int64_t q1) {
    const o_search_ctx* a = (const o_search_ctx*)cv;
    const o_index* ix = a->ix;
    const int k = a->k, mode = a->mode;
    const int d = ix->d, M = ix->M, nlist = ix->nlist;
    const int nprobe = ix->nprobe < nlist ? ix->nprobe : nlist;
    const int ck = o_ck(ix->alpha, k);
    const int Kr = ix->Kr, Br = ix->Br, bpv = ix->bpv;
    float* q_rot = (float*)malloc((size_t)d * sizeof(float));
    float* scores = (float*)malloc((size_t)nlist * sizeof(float));
    int32_t* cids = (int32_t*)malloc((size_t)nlist * sizeof(int32_t));
    float* pd = (float*)malloc((size_t)nprobe * sizeof(float));
    int32_t* probes = (int32_t*)malloc((size_t)nprobe * sizeof(int32_t));
    float* lut = (float*)malloc((size_t)M * 256 * sizeof(float));
    float* cd = (float*)malloc((size_t)ck * sizeof(float));
    int32_t* cp = (int32_t*)malloc((size_t)ck * sizeof(int32_t));
    float* comp = (float*)malloc((size_t)ck * sizeof(float));
    int32_t* cid = (int32_t*)malloc((size_t)ck * sizeof(int32_t));
    for (int c = 0; c < nlist; c++) cids[c] = c;

    for (int64_t qi = q0; qi < q1; qi++) {
        if (a->q_rot_in) memcpy(q_rot, a->q_rot_in + qi * d, (size_t)d * sizeof(float));
        else {
            /* y = Pi q, the fmaf chain of o_rotate */
            const float* qq = a->q + qi * d;
            for (int j = 0; j < d; j++) {
                const float* pj = ix->P + (int64_t)j * d;
                float acc = 0.0f;
                for (int kk = 0; kk < d; kk++) acc = fmaf(qq[kk], pj[kk], acc);
                q_rot[j] = acc;
            }
        }
        if (a->probes_in) {
            memcpy(probes, a->probes_in + qi * nprobe, (size_t)nprobe * sizeof(int32_t));
        } else {
            /* centroid scores: ||c||^2 - 2<c,q> (search.cu:31-32) */
            for (int c = 0; c < nlist; c++)
                scores[c] = fmaf(-2.0f, dot_fma(q_rot, ix->cent + (int64_t)c * d, d),
                                 ix->cent_norms[c]);
            o_select_topk_pairs(scores, cids, nlist, nprobe, pd, probes);
        }
        if (a->dbg_probes)
            memcpy(a->dbg_probes + qi * nprobe, probes, (size_t)nprobe * sizeof(int32_t));

        int64_t total = 0;
        for (int p = 0; p < nprobe; p++)
            total += ix->list_offsets[probes[p] + 1] - ix->list_offsets[probes[p]];
        float* dists = (float*)malloc((size_t)(total > 0 ? total : 1) * sizeof(float));
        int32_t* poss = (int32_t*)malloc((size_t)(total > 0 ? total : 1) * sizeof(int32_t));
        o_flat_lut(q_rot, d, M, ix->c1d, ix->K1D, lut);
        int64_t t = 0;
        for (int p = 0; p < nprobe; p++) {
            const int l = probes[p];
            for (int32_t pos = ix->list_offsets[l]; pos < ix->list_offsets[l + 1]; pos++) {
                dists[t] = o_adc_flat(ix->list_codes + (int64_t)pos * M, M, lut);
                poss[t] = pos;
                t++;
            }
        }
        if (mode == 1) v14_topck(dists, poss, total, ck, cd, cp);
        else o_select_topk_pairs(dists, poss, total, ck, cd, cp);
        free(dists); free(poss);
        if (a->dbg_topck_pos) memcpy(a->dbg_topck_pos + qi * ck, cp, (size_t)ck * sizeof(int32_t));
        if (a->dbg_topck_dist) memcpy(a->dbg_topck_dist + qi * ck, cd, (size_t)ck * sizeof(float));

        /* residual refine: search.cu:198-242 */
        for (int c = 0; c < ck; c++) {
            const int32_t pos = cp[c];
            if (pos < 0) { comp[c] = INFINITY; cid[c] = -1; continue; }
            const uint8_t* rc = ix->list_res + (int64_t)pos * bpv;
            float d_res = 0.0f;
            for (int j = 0; j < d; j++) {
                const int ri = (Br == 4) ? ((j % 2 == 0) ? (rc[j / 2] & 0x0F) : (rc[j / 2] >> 4))
                                         : rc[j];
                const float diff = q_rot[j] - ix->res_c1d[(ix->RC == 1 ? 0 : (j / ix->Ds) * Kr) + ri];
                const float lr = diff * diff;
                d_res = d_res + lr;
            }
            comp[c] = (cd[c] + d_res) + ix->list_corr[pos];
            cid[c] = ix->list_ids[pos];
        }
        if (mode == 1) {
            v14_final(comp, cid, ck, k, a->out_dist + qi * k, a->out_ids + qi * k);
        } else {
            /* final top-k by (dist, id): jhq_v3_ivf/search.cu:242-279 */
            o_select_topk_pairs(comp, cid, ck, k, a->out_dist + qi * k, a->out_ids + qi * k);
        }
    }
    free(q_rot); free(scores); free(cids); free(pd); free(probes); free(lut);
    free(cd); free(cp); free(comp); free(cid);
}

int o_search_mode(const o_index* ix, const float* q, const float* q_rot_in,
                  const int32_t* probes_in, int64_t nq, int k, int mode,
                  float* out_dist, int32_t* out_ids,
                  int32_t* dbg_probes, int32_t* dbg_topck_pos, float* dbg_topck_dist) {
    if (mode != 0 && mode != 1) return -1;
    o_search_ctx a = {ix, q, q_rot_in, probes_in, k, mode, out_dist, out_ids,
                      dbg_probes, dbg_topck_pos, dbg_topck_dist};
    o_parallel(nq, o_search_rows, &a);
    return 0;
}
