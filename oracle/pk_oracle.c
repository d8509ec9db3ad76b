/* The oracle's restatement of libpktito's int8 product path. Test
 * infrastructure only: see pk_oracle.h for what may use it and how each
 * function is pinned. Built with -ffp-contract=off, as the reference is
 * (Makefile:129 there), so no multiply and add written apart are fused.
 */
#include "pk_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <string.h>

/* a * b + c with one rounding (core/vmath.h:61-91). C99's fmaf is
 * specified as exactly that; glibc computes it correctly rounded with or
 * without the FMA instruction. */
float pko_fmaf(float a, float b, float c) { return fmaf(a, b, c); }

/* backend/ref/kernels.c:24-58. Per column t and block b: a NaN anywhere in
 * the block, an infinite amax, or an amax below 2^-121 gives d = +0 and
 * q = 0; otherwise d = amax / 127 and q = rint(v * (127 / amax)), both
 * divisions single IEEE operations. */
void pko_quantize(pko_act *a, const float *x, size_t xs) {
    const uint32_t qb = a->qb, nb = a->n / qb;
    for (uint32_t t = 0; t < a->T; t++) {
        for (uint32_t b = 0; b < nb; b++) {
            const float *v = x + (size_t)t * xs + (size_t)b * qb;
            int8_t *q = a->q + (size_t)t * a->n + (size_t)b * qb;
            float *d = a->d + (size_t)t * nb + b;
            float amax = 0.0f;
            int nan = 0;
            for (uint32_t i = 0; i < qb && !nan; i++) {
                if (isnan(v[i]))
                    nan = 1;
                else
                    amax = fmaxf(amax, fabsf(v[i]));
            }
            if (nan || !isfinite(amax) || amax < 0x1p-121f) {
                *d = 0.0f;
                memset(q, 0, qb);
                continue;
            }
            *d = amax / 127.0f;
            const float id = 127.0f / amax;
            for (uint32_t i = 0; i < qb; i++)
                q[i] = (int8_t)rintf(v[i] * id);
        }
    }
}

size_t pko_q8_index(uint32_t n, uint32_t r, uint32_t k) {
    /* core/pkf.h:34: panels of 16 rows, groups of 4 inputs, 64 bytes a group */
    return ((size_t)(r >> 4) * (n >> 2) + (k >> 2)) * 64 + (size_t)(r & 15) * 4 + (k & 3);
}

void pko_pack_q8(int8_t *panels, const int8_t *rowmajor, uint32_t rows, uint32_t n) {
    for (uint32_t r = 0; r < rows; r++)
        for (uint32_t k = 0; k < n; k++)
            panels[pko_q8_index(n, r, k)] = rowmajor[(size_t)r * n + k];
}

void pko_unpack_q8(int8_t *rowmajor, const int8_t *panels, uint32_t rows, uint32_t n) {
    for (uint32_t r = 0; r < rows; r++)
        for (uint32_t k = 0; k < n; k++)
            rowmajor[(size_t)r * n + k] = panels[pko_q8_index(n, r, k)];
}

/* backend/ref/kernels.c:66-86. For each column t and row r: an exact int32
 * sum per block, chained through fmaf with the block's scale in block order,
 * then times ws[r], plus bias[r], plus the old output, each its own rounding. */
void pko_gemm_q8(float *out, size_t os, const int8_t *w, const float *ws, const float *bias,
                 uint32_t rows, const pko_act *a, int add) {
    const uint32_t n = a->n, qb = a->qb, nb = n / qb;
    for (uint32_t t = 0; t < a->T; t++) {
        const int8_t *q = a->q + (size_t)t * n;
        const float *d = a->d + (size_t)t * nb;
        for (uint32_t r = 0; r < rows; r++) {
            float acc = 0.0f;
            for (uint32_t b = 0; b < nb; b++) {
                int32_t s = 0;
                for (uint32_t k = b * qb; k < (b + 1) * qb; k++)
                    s += (int32_t)w[pko_q8_index(n, r, k)] * q[k];
                acc = pko_fmaf((float)s, d[b], acc);
            }
            float v = acc * ws[r];
            if (bias)
                v = v + bias[r];
            float *o = out + (size_t)t * os + r;
            if (add)
                *o = *o + v;
            else
                *o = v;
        }
    }
}

/* tests/kcheck.c:217-239: the sums in int64, which cannot overflow. */
void pko_definition(float *out, size_t os, const int8_t *w, const float *ws, const float *bias,
                    uint32_t rows, const pko_act *a) {
    const uint32_t n = a->n, qb = a->qb, nb = n / qb;
    for (uint32_t t = 0; t < a->T; t++)
        for (uint32_t r = 0; r < rows; r++) {
            float acc = 0.0f;
            for (uint32_t b = 0; b < nb; b++) {
                int64_t s = 0;
                for (uint32_t k = b * qb; k < (b + 1) * qb; k++)
                    s += (int64_t)w[pko_q8_index(n, r, k)] * a->q[(size_t)t * n + k];
                acc = pko_fmaf((float)s, a->d[(size_t)t * nb + b], acc);
            }
            float v = acc * ws[r];
            if (bias)
                v = v + bias[r];
            out[(size_t)t * os + r] = v;
        }
}

/* ------------------------------------------------------------ threads --- */

typedef struct {
    pko_gemm_fn fn;
    float *out;
    size_t os;
    const int8_t *w;
    const float *ws, *bias;
    uint32_t rows;
    const pko_act *a;
    int add;
    atomic_uint next;
} gemm_deal;

static void *gemm_worker(void *arg) {
    gemm_deal *j = arg;
    const uint32_t slices = (j->rows + 63) / 64;
    for (;;) {
        uint32_t i = atomic_fetch_add(&j->next, 1);
        if (i >= slices)
            return NULL;
        uint32_t r0 = i * 64, nr = j->rows - r0 < 64 ? j->rows - r0 : 64;
        j->fn(j->out + r0, j->os, j->w + (size_t)r0 * j->a->n, j->ws + r0,
              j->bias ? j->bias + r0 : NULL, nr, j->a, j->add);
    }
}

void pko_gemm_threads(pko_gemm_fn fn, int nthreads, float *out, size_t os, const int8_t *w,
                      const float *ws, const float *bias, uint32_t rows, const pko_act *a, int add) {
    gemm_deal j = { fn, out, os, w, ws, bias, rows, a, add, 0 };
    pthread_t th[256];
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    int started = 1;
    for (int i = 1; i < nthreads; i++)
        if (pthread_create(&th[started], NULL, gemm_worker, &j) == 0)
            started++;
    gemm_worker(&j);
    for (int i = 1; i < started; i++)
        pthread_join(th[i], NULL);
}

typedef struct {
    pko_quant_fn fn;
    pko_act *a;
    const float *x;
    size_t xs;
    atomic_uint next;
} quant_deal;

static void *quant_worker(void *arg) {
    quant_deal *j = arg;
    const uint32_t items = (j->a->T + 15) / 16;
    for (;;) {
        uint32_t i = atomic_fetch_add(&j->next, 1);
        if (i >= items)
            return NULL;
        uint32_t t0 = i * 16, nt = j->a->T - t0 < 16 ? j->a->T - t0 : 16;
        pko_act sub = *j->a;
        sub.q += (size_t)t0 * sub.n;
        sub.d += (size_t)t0 * (sub.n / sub.qb);
        sub.T = nt;
        j->fn(&sub, j->x + (size_t)t0 * j->xs, j->xs);
    }
}

void pko_quantize_threads(pko_quant_fn fn, int nthreads, pko_act *a, const float *x, size_t xs) {
    quant_deal j = { fn, a, x, xs, 0 };
    pthread_t th[256];
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    int started = 1;
    for (int i = 1; i < nthreads; i++)
        if (pthread_create(&th[started], NULL, quant_worker, &j) == 0)
            started++;
    quant_worker(&j);
    for (int i = 1; i < started; i++)
        pthread_join(th[i], NULL);
}

/* ---------------------------------------------------------- generator --- */

/* xorshift64* (tests/kcheck.c:42-47), the high 32 bits of the product */
uint32_t pko_rnd(uint64_t *s) {
    uint64_t v = *s;
    v ^= v >> 12;
    v ^= v << 25;
    v ^= v >> 27;
    *s = v;
    return (uint32_t)((v * 0x2545F4914F6CDD1Dull) >> 32);
}

float pko_frand(uint64_t *s) { return (float)(pko_rnd(s) >> 8) / 8388608.0f - 1.0f; }

/* tests/kcheck.c:51-60: one draw in 24 each a +0, a -0, a subnormal, an
 * outlier thirty times the scale, and a half that lands on a tie once
 * scaled to 127; the rest uniform in [-scale, scale) */
float pko_awkward(uint64_t *s, float scale) {
    switch (pko_rnd(s) % 24) {
    case 0: return 0.0f;
    case 1: return -0.0f;
    case 2: return 1e-40f;
    case 3: return -scale * 30.0f;
    case 4: return scale * 0.5f;
    default: return scale * pko_frand(s);
    }
}

void pko_fill_awkward(uint64_t *s, float *x, size_t n, float scale) {
    for (size_t i = 0; i < n; i++)
        x[i] = pko_awkward(s, scale);
}
