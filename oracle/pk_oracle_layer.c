/* The oracle's restatement of the float kernels around the int8 products and
 * of one FastConformer encoder layer built from them, the reference's
 * device-resident dataflow. Test infrastructure only: see pk_oracle.h for
 * what may use it and how each function is pinned. Built with
 * -ffp-contract=off, as the reference is, so that no multiply and add
 * written apart are fused.
 */
#include "pk_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------ exp, sigmoid --- */

/* 2^n for n in [-126, 127], as the float whose exponent field is n + 127
 * (core/vmath.h:126-132) */
static float pow2i(int32_t n) {
    const uint32_t u = (uint32_t)(n + 127) << 23;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* core/vmath.h:134-147, with its constants (core/vmath.h:92-125): the
 * argument clamped to [-87, 88] (a NaN to -87), n = rint(x log2e), the
 * remainder r = x - n ln2 in two fmaf steps with ln2 split high and low, a
 * degree-6 polynomial in r by Horner's rule in fmaf, times 2^n. */
float pko_expf(float x) {
    x = fminf(fmaxf(x, -87.0f), 88.0f);
    const float n = rintf(x * 0x1.715476p+0f);
    float r = pko_fmaf(n, -0x1.62e430p-1f, x);
    r = pko_fmaf(n, 0x1.05c610p-29f, r);
    float p = 0x1.6ab980p-10f;
    p = pko_fmaf(p, r, 0x1.126d0cp-7f);
    p = pko_fmaf(p, r, 0x1.55589ap-5f);
    p = pko_fmaf(p, r, 0x1.55540ap-3f);
    p = pko_fmaf(p, r, 0x1.fffffap-2f);
    p = pko_fmaf(p, r, 1.0f);
    p = pko_fmaf(p, r, 1.0f);
    return p * pow2i((int32_t)n);
}

/* core/vmath.h:149-151 */
float pko_sigmoidf(float x) { return 1.0f / (1.0f + pko_expf(-x)); }

void pko_expf_n(float *y, const float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        y[i] = pko_expf(x[i]);
}

void pko_sigmoidf_n(float *y, const float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        y[i] = pko_sigmoidf(x[i]);
}

/* ------------------------------------------------------ float kernels --- */

/* backend/ref/kernels.c:90-105 and the contract at backend/kernels.h:85-103:
 * each output one fmaf chain over k in order from +0, W(k, r) at
 * w[((r / 16) ld + k) 16 + r % 16], then the bias and the optional ReLU. */
void pko_gemm_f32(float *out, size_t os, const float *w, uint32_t ld, uint32_t rows, uint32_t n,
                  const float *x, size_t xs, uint32_t T, const float *bias, size_t bs, int relu) {
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t r = 0; r < rows; r++) {
            const float *wp = w + (size_t)(r / 16) * ld * 16 + r % 16;
            float acc = 0.0f;
            for (uint32_t k = 0; k < n; k++)
                acc = pko_fmaf(wp[(size_t)16 * k], x[(size_t)t * xs + k], acc);
            const float v = acc + (bias ? bias[(size_t)t * bs + r] : 0.0f);
            out[(size_t)t * os + r] = relu ? (v > 0 ? v : 0) : v;
        }
}

/* The sum of a row in 16 lanes, element i into lane i % 16 in order, the
 * lanes combined as acc[i] += acc[i + h] for h = 8, 4, 2, 1
 * (backend/kernels.h:105-110, backend/ref/kernels.c:109-113). */
static float lanes_sum(float *acc) {
    for (int h = 8; h > 0; h /= 2)
        for (int i = 0; i < h; i++)
            acc[i] += acc[i + h];
    return acc[0];
}

/* backend/ref/kernels.c:115-132 (contract backend/kernels.h:112-122) */
void pko_layernorm(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t n,
                   const float *w, const float *b, float eps) {
    for (uint32_t t = 0; t < T; t++) {
        const float *v = x + (size_t)t * xs;
        float *o = out + (size_t)t * os;
        float acc[16] = { 0 };
        for (uint32_t i = 0; i < n; i++)
            acc[i % 16] += v[i];
        const float mean = lanes_sum(acc) / (float)n;
        memset(acc, 0, sizeof acc);
        for (uint32_t i = 0; i < n; i++) {
            const float c = v[i] - mean;
            acc[i % 16] += c * c;
        }
        const float var = lanes_sum(acc) / (float)n;
        const float r = 1.0f / sqrtf(var + eps);
        for (uint32_t i = 0; i < n; i++)
            o[i] = (v[i] - mean) * r * w[i] + b[i];
    }
}

/* backend/ref/kernels.c:134-147 (contract backend/kernels.h:124-130) */
void pko_softmax(float *x, uint32_t n, float scale) {
    float m = -INFINITY;
    for (uint32_t i = 0; i < n; i++) {
        x[i] = x[i] * scale;
        m = fmaxf(m, x[i]);
    }
    float acc[16] = { 0 };
    for (uint32_t i = 0; i < n; i++) {
        x[i] = pko_expf(x[i] - m);
        acc[i % 16] += x[i];
    }
    const float inv = 1.0f / lanes_sum(acc);
    for (uint32_t i = 0; i < n; i++)
        x[i] = x[i] * inv;
}

/* backend/ref/kernels.c:149-151 */
void pko_silu(float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        x[i] = x[i] * pko_sigmoidf(x[i]);
}

/* backend/ref/kernels.c:157-161 (contract backend/kernels.h:140-142) */
void pko_glu(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t n) {
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t i = 0; i < n; i++)
            out[(size_t)t * os + i] = x[(size_t)t * xs + i] * pko_sigmoidf(x[(size_t)t * xs + n + i]);
}

/* backend/ref/kernels.c:163-176 (contract backend/kernels.h:144-158) */
void pko_dwconv(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t C,
                const float *w, const float *b, uint32_t K) {
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t c = 0; c < C; c++) {
            float acc = 0.0f;
            for (uint32_t j = 0; j < K; j++) {
                const int64_t s = (int64_t)t + j - K / 2;
                if (s >= 0 && s < T)
                    acc = pko_fmaf(w[(size_t)c * K + j], x[(size_t)s * xs + c], acc);
            }
            const float v = acc + b[c];
            out[(size_t)t * os + c] = v * pko_sigmoidf(v);
        }
}

/* ------------------------------------------------------------ a layer --- */

/* The oracle's own kernels, as a table */
const pko_kernels pko_kernels_oracle = {
    pko_quantize, pko_gemm_q8, pko_gemm_f32, pko_layernorm, pko_softmax, pko_silu, pko_glu, pko_dwconv, pko_lstm,
};

static uint32_t up16(uint32_t x) { return (x + 15) & ~15u; }
static uint32_t min32(uint32_t a, uint32_t b) { return a < b ? a : b; }

/* items [0, n) over nthreads, dealt from an atomic counter as the
 * reference's pool deals them (core/pool.c); fn(arg, item, worker) */
typedef void (*par_fn)(void *arg, uint32_t item, int worker);

typedef struct {
    par_fn fn;
    void *arg;
    uint32_t n;
    atomic_uint next;
    int worker;
} par_job;

typedef struct {
    par_job *j;
    int worker;
} par_arg;

static void *par_worker(void *p) {
    par_arg *a = p;
    for (;;) {
        const uint32_t i = atomic_fetch_add(&a->j->next, 1);
        if (i >= a->j->n)
            return NULL;
        a->j->fn(a->j->arg, i, a->worker);
    }
}

static void par(int nthreads, uint32_t n, par_fn fn, void *arg) {
    par_job j = { fn, arg, n, 0, 0 };
    pthread_t th[256];
    par_arg args[256];
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    int started = 1;
    for (int i = 1; i < nthreads; i++) {
        args[started] = (par_arg){ &j, started };
        if (pthread_create(&th[started], NULL, par_worker, &args[started]) == 0)
            started++;
    }
    args[0] = (par_arg){ &j, 0 };
    par_worker(&args[0]);
    for (int i = 1; i < started; i++)
        pthread_join(th[i], NULL);
}

/* a worker's scratch: a row, and att_item's block buffers */
typedef struct {
    float *row, *sc, *bd, *qu, *qv;
} scratch;

typedef struct {
    const pko_kernels *k;
    const pko_layer *L;
    int nthreads;
    uint32_t T, qb, Tp, Pp;
    pko_act act, hid;
    float *u, *q, *kf, *pf, *o, *kp, *pp, *vp;
    scratch ws[256];
    /* the pass in flight */
    const float *px, *pw, *pb;
    uint32_t pn;
} lay;

/* a->act for T frames of n floats, blocks of qb (core/encoder.c:100-106) */
static pko_act *shape(pko_act *a, uint32_t T, uint32_t n, uint32_t qb) {
    a->n = n;
    a->qb = qb;
    a->T = T;
    return a;
}

/* The product of one uploaded matrix in 64-row slices over the threads
 * (core/encoder.c:64-76, pk_gemm; core/passes.c:60-109. The layer's
 * products have no bias.) */
static void gemm(lay *y, float *out, size_t os, const pko_q8 *w, const pko_act *a, int add) {
    pko_gemm_threads(y->k->gemm_q8, y->nthreads, out, os, w->q, w->s, NULL, w->rows, a, add);
}

/* Inputs [k0, k0 + n) of column t quantized alone (core/passes.c:111-118,
 * pk_quant_part): whole blocks, the bytes and scales of the whole column's */
static void quant_part(lay *y, pko_act *a, uint32_t t, uint32_t k0, uint32_t n, const float *x) {
    const size_t at = (size_t)t * a->n + k0;
    pko_act part = { a->q + at, a->d + at / a->qb, n, a->qb, 1 };
    y->k->quantize(&part, x, n);
}

/* normq (core/encoder.c:108-128): 16 frames an item, each layer-normed
 * through a row of scratch and quantized whole */
static void normq_item(void *arg, uint32_t i, int wk) {
    lay *y = arg;
    const uint32_t n = y->pn;
    float *row = y->ws[wk].row;
    for (uint32_t t = i * 16; t < min32(i * 16 + 16, y->T); t++) {
        y->k->layernorm(row, n, y->px + (size_t)t * n, n, 1, n, y->pw, y->pb, y->L->eps);
        quant_part(y, &y->act, t, 0, n, row);
    }
}

static void normq(lay *y, const float *x, uint32_t n, const float *w, const float *b) {
    shape(&y->act, y->T, n, y->qb);
    y->px = x, y->pw = w, y->pb = b, y->pn = n;
    par(y->nthreads, (y->T + 15) / 16, normq_item, y);
}

/* siluq (core/encoder.c:130-156): the hidden row SiLU'd through scratch and
 * quantized; the reference's slices are whole blocks, so a whole row's
 * quantize gives the same bytes and scales */
static void siluq_item(void *arg, uint32_t t, int wk) {
    lay *y = arg;
    const uint32_t F = y->L->F;
    float *row = y->ws[wk].row;
    memcpy(row, y->u + (size_t)t * F, F * sizeof(float));
    y->k->silu(row, F);
    quant_part(y, &y->hid, t, 0, F, row);
}

/* ff (core/encoder.c:321-327): x += down(siluq(up(normq(x)))) */
static void ff(lay *y, float *x, const float *nw, const float *nb, const pko_q8 *up, const pko_q8 *down) {
    const uint32_t D = y->L->D, F = y->L->F;
    normq(y, x, D, nw, nb);
    gemm(y, y->u, F, up, &y->act, 0);
    shape(&y->hid, y->T, F, y->qb);
    par(y->nthreads, y->T, siluq_item, y);
    gemm(y, x, D, down, &y->hid, 1);
}

/* K's and the positions' floats (src, n rows of D) as pk_k_gemm_f32's
 * panels (core/passes.c:207-236): (d, column j) of head h at
 * dst + h np dk + ((j / 16) dk + d) 16 + j % 16, columns n .. np zero. */
static void panels(float *dst, const float *src, uint32_t n, uint32_t np, uint32_t D, uint32_t dk) {
    for (uint32_t h = 0; h < D / dk; h++)
        for (uint32_t j = 0; j < np; j++)
            for (uint32_t d = 0; d < dk; d++)
                dst[(size_t)h * np * dk + ((size_t)(j / 16) * dk + d) * 16 + j % 16] =
                    j < n ? src[(size_t)j * D + h * dk + d] : 0.0f;
}

/* att_item (core/encoder.c:280-327): one head over 16 queries */
static void att_item(void *arg, uint32_t item, int wk) {
    lay *y = arg;
    const pko_layer *L = y->L;
    const pko_kernels *k = y->k;
    const uint32_t D = L->D, dk = D / L->H, T = y->T, Tp = y->Tp, Pp = y->Pp;
    const uint32_t nb = (T + 15) / 16, h = item / nb, i0 = (item % nb) * 16, i1 = min32(i0 + 16, T);
    const uint32_t nq = i1 - i0;
    const scratch *w = &y->ws[wk];
    const float *kp = y->kp + (size_t)h * Tp * dk, *pp = y->pp + (size_t)h * Pp * dk;
    const float *bu = L->bias_u + h * dk, *bv = L->bias_v + h * dk;
    for (uint32_t i = 0; i < nq; i++) {
        const float *q = y->q + (size_t)(i0 + i) * D + h * dk;
        for (uint32_t d = 0; d < dk; d++) {
            w->qu[i * dk + d] = q[d] + bu[d];
            w->qv[i * dk + d] = q[d] + bv[d];
        }
    }
    k->gemm_f32(w->sc, Tp, kp, dk, Tp, dk, w->qu, dk, nq, NULL, 0, 0);
    const uint32_t m_lo = T - i1, m_hi = 2 * T - 2 - i0, m_a = m_lo & ~15u;
    const uint32_t rows = up16(m_hi + 1 - m_a);
    k->gemm_f32(w->bd, rows, pp + (size_t)(m_a / 16) * dk * 16, dk, rows, dk, w->qv, dk, nq, NULL, 0, 0);
    const float scale = 1.0f / sqrtf((float)dk);
    for (uint32_t i = i0; i < i1; i++) {
        float *s = w->sc + (size_t)(i - i0) * Tp;
        const float *b = w->bd + (size_t)(i - i0) * rows + (T - 1 - i) - m_a;
        for (uint32_t j = 0; j < T; j++)
            s[j] = s[j] + b[j];
        k->softmax(s, T, scale);
    }
    k->gemm_f32(y->o + (size_t)i0 * D + h * dk, D, y->vp + (size_t)h * (dk / 16) * T * 16, T, dk, T, w->sc, Tp,
                nq, NULL, 0, 0);
}

/* glu_item and dw_item (core/encoder.c:158-176): GLU 16 frames an item;
 * then 64 channels an item over every frame, quantized there */
static void glu_item(void *arg, uint32_t i, int wk) {
    (void)wk;
    lay *y = arg;
    const uint32_t D = y->L->D, t0 = i * 16, nt = min32(16, y->T - t0);
    y->k->glu(y->q + (size_t)t0 * D, D, y->u + (size_t)t0 * 2 * D, 2 * D, nt, D);
}

static void dw_item(void *arg, uint32_t i, int wk) {
    (void)wk;
    lay *y = arg;
    const pko_layer *L = y->L;
    const uint32_t D = L->D, c0 = i * 64, nc = min32(64, D - c0);
    y->k->dwconv(y->o + c0, D, y->q + c0, D, y->T, nc, L->dw + (size_t)c0 * L->K, L->dw_b + c0, L->K);
    for (uint32_t t = 0; t < y->T; t++)
        quant_part(y, &y->act, t, c0, nc, y->o + (size_t)t * D + c0);
}

/* norm (core/encoder.c:86-99): 16 frames an item, in place */
static void norm_item(void *arg, uint32_t i, int wk) {
    (void)wk;
    lay *y = arg;
    const uint32_t D = y->L->D, t0 = i * 16, nt = min32(16, y->T - t0);
    float *x = (float *)y->px + (size_t)t0 * D;
    y->k->layernorm(x, D, x, D, nt, D, y->pw, y->pb, y->L->eps);
}

/* core/encoder.c:329-368, one layer in place on x [T][D] */
int pko_conformer_layer_with(const pko_kernels *k, const pko_layer *L, float *x, uint32_t T, const pko_act *ape,
                             uint32_t qb, int nthreads) {
    const uint32_t D = L->D, F = L->F, H = L->H, dk = D / L->H, R = 2 * T - 1;
    if (!k || T == 0 || D % 64 || F % 64 || D % H || dk % 16 || ape->T != R || ape->n != D || ape->qb != qb)
        return -1;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    lay *y = calloc(1, sizeof *y);
    if (!y)
        return -2;
    y->k = k, y->L = L, y->nthreads = nthreads, y->T = T, y->qb = qb, y->Tp = up16(T), y->Pp = up16(R) + 16;
    const uint32_t wide = F > 2 * D ? F : 2 * D;
    y->act.q = malloc((size_t)T * wide);
    y->act.d = malloc((size_t)T * (wide / qb) * sizeof(float));
    y->hid.q = malloc((size_t)T * F);
    y->hid.d = malloc((size_t)T * (F / qb) * sizeof(float));
    y->u = malloc((size_t)T * wide * sizeof(float));
    y->q = malloc((size_t)T * D * sizeof(float));
    y->kf = malloc((size_t)T * D * sizeof(float));
    y->pf = malloc((size_t)R * D * sizeof(float));
    y->o = malloc((size_t)T * D * sizeof(float));
    y->kp = malloc((size_t)H * y->Tp * dk * sizeof(float));
    y->pp = malloc((size_t)H * y->Pp * dk * sizeof(float));
    y->vp = malloc((size_t)T * D * sizeof(float));
    int ok = y->act.q && y->act.d && y->hid.q && y->hid.d && y->u && y->q && y->kf && y->pf && y->o && y->kp &&
             y->pp && y->vp;
    for (int i = 0; i < nthreads && ok; i++) {
        scratch *w = &y->ws[i];
        w->row = malloc((size_t)wide * sizeof(float));
        w->sc = malloc((size_t)16 * y->Tp * sizeof(float));
        w->bd = malloc((size_t)16 * (y->Pp + 32) * sizeof(float));
        w->qu = malloc((size_t)16 * dk * sizeof(float));
        w->qv = malloc((size_t)16 * dk * sizeof(float));
        ok = w->row && w->sc && w->bd && w->qu && w->qv;
    }
    if (ok) {
        ff(y, x, L->ff1_nw, L->ff1_nb, &L->ff1_up, &L->ff1_down);

        /* the attention (core/encoder.c:339-352) */
        normq(y, x, D, L->att_nw, L->att_nb);
        gemm(y, y->q, D, &L->q, &y->act, 0);
        gemm(y, y->kf, D, &L->k, &y->act, 0);
        panels(y->kp, y->kf, T, y->Tp, D, dk);
        /* V straight into the panels, one 16-row product a panel
         * (core/passes.c:164-182): (key j, dimension d) of head h at
         * vp + ((h dk + d) / 16) T 16 + j 16 + d % 16 */
        for (uint32_t r = 0; r < D; r += 16) {
            pko_q8 w16 = { L->v.q + (size_t)r * D, L->v.s + r, 16, D };
            gemm(y, y->vp + (size_t)(r / 16) * T * 16, 16, &w16, &y->act, 0);
        }
        gemm(y, y->pf, D, &L->pos, ape, 0);
        panels(y->pp, y->pf, R, y->Pp, D, dk);
        par(nthreads, H * ((T + 15) / 16), att_item, y);
        pko_quantize_threads(k->quantize, nthreads, shape(&y->act, T, D, qb), y->o, D);
        gemm(y, x, D, &L->o, &y->act, 1);

        /* the convolution module (core/encoder.c:354-362) */
        normq(y, x, D, L->conv_nw, L->conv_nb);
        gemm(y, y->u, 2 * D, &L->pw1, &y->act, 0);
        par(nthreads, (T + 15) / 16, glu_item, y);                 /* h, in q's room */
        shape(&y->act, T, D, qb);
        par(nthreads, (D + 63) / 64, dw_item, y);
        gemm(y, x, D, &L->pw2, &y->act, 1);

        ff(y, x, L->ff2_nw, L->ff2_nb, &L->ff2_up, &L->ff2_down);
        y->px = x, y->pw = L->out_nw, y->pb = L->out_nb;
        par(nthreads, (T + 15) / 16, norm_item, y);
    }
    free(y->act.q); free(y->act.d); free(y->hid.q); free(y->hid.d); free(y->u); free(y->q); free(y->kf);
    free(y->pf); free(y->o); free(y->kp); free(y->pp); free(y->vp);
    for (int i = 0; i < nthreads; i++) {
        scratch *w = &y->ws[i];
        free(w->row); free(w->sc); free(w->bd); free(w->qu); free(w->qv);
    }
    free(y);
    return ok ? 0 : -2;
}

int pko_conformer_layer(const pko_layer *L, float *x, uint32_t T, const pko_act *ape, uint32_t qb, int nthreads) {
    return pko_conformer_layer_with(&pko_kernels_oracle, L, x, T, ape, qb, nthreads);
}
