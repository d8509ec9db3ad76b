/* The oracle's restatement of the decoder's per-token work (core/decoder.c
 * in peterheb/libpktito): the prediction network's LSTM steps and the
 * joint, each of their products a quantize of one row and a T = 1 product.
 * Test infrastructure only: see pk_oracle.h for what may use it and how
 * each function is pinned. Built with -ffp-contract=off.
 */
#include "pk_oracle.h"

#include <math.h>
#include <string.h>

/* core/vmath.h:153-166 with its constants (core/vmath.h:104-116): below
 * |x| = 0.625, x + x^3 p(x^2) with p by Horner's rule in fmaf; above it
 * 1 - 2 / (e^2|x| + 1) with the sign of x. */
float pko_tanhf(float x) {
    const float a = fabsf(x);
    if (a < 0.625f) {
        const float x2 = x * x;
        float p = -0x1.75e1cep-8f;
        p = pko_fmaf(p, x2, 0x1.52269cp-6f);
        p = pko_fmaf(p, x2, -0x1.b83c5ap-5f);
        p = pko_fmaf(p, x2, 0x1.110726p-3f);
        p = pko_fmaf(p, x2, -0x1.555532p-2f);
        return pko_fmaf(x * x2, p, x);
    }
    const float e = pko_expf(2.0f * a);
    return copysignf(1.0f - 2.0f / (e + 1.0f), x);
}

void pko_tanhf_n(float *y, const float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        y[i] = pko_tanhf(x[i]);
}

/* backend/ref/kernels.c:203-213 (contract backend/kernels.h:180-187): the
 * gates i f g o of H units, then c = f c + i u and h = o tanh(c). */
void pko_lstm(float *h, float *c, const float *g, uint32_t H) {
    for (uint32_t j = 0; j < H; j++) {
        const float i = pko_sigmoidf(g[j]);
        const float f = pko_sigmoidf(g[H + j]);
        const float u = pko_tanhf(g[2 * H + j]);
        const float o = pko_sigmoidf(g[3 * H + j]);
        c[j] = f * c[j] + i * u;
        h[j] = o * pko_tanhf(c[j]);
    }
}

/* gemv (core/decoder.c:54-63): x quantized as one row of its matrix's cols
 * in one block, then the product with output stride 0 (the pool split of
 * large products computes the same bits). q holds cols bytes, d one float. */
static void gemv(const pko_kernels *k, int8_t *q, float *d, float *out, const pko_q8 *w, const float *bias,
                 const float *x, int add) {
    pko_act a = { q, d, w->cols, w->cols, 1 };
    k->quantize(&a, x, w->cols);
    k->gemm_q8(out, 0, w->q, w->s, bias, w->rows, &a, add);
}

void pko_gemv_with(const pko_kernels *k, int8_t *q, float *d, float *out, const pko_q8 *w, const float *bias,
                   const float *x, int add) {
    gemv(k, q, d, out, w, bias, x, add);
}

/* predict (core/decoder.c:65-79): the label's embedding up through the
 * LSTM layers, each layer's h and c (L x P) stepped in place, then the
 * joint's half of it into gp. q: max(P, J) bytes; gates: 4P floats. */
void pko_predict_with(const pko_kernels *k, const pko_decoder *m, uint32_t label, float *h, float *c,
                      float *gates, int8_t *q, float *gp) {
    const uint32_t P = m->P;
    float d;
    const float *x = m->embed + (size_t)label * P;
    for (uint32_t l = 0; l < m->L; l++) {
        float *hl = h + (size_t)l * P, *cl = c + (size_t)l * P;
        gemv(k, q, &d, gates, &m->lstm[l].wx, m->lstm[l].b, x, 0);
        gemv(k, q, &d, gates, &m->lstm[l].wh, NULL, hl, 1);
        k->lstm(hl, cl, gates, P);
        x = hl;
    }
    gemv(k, q, &d, gp, &m->jpred, m->jpred_b, x, 0);
}

/* joint (core/decoder.c:81-101): z = relu(f + gp), the logits, the first
 * best token of [0, V] and the first best duration of the n_dur after it.
 * z: J floats; logit: jout's rows. */
void pko_joint_with(const pko_kernels *k, const pko_decoder *m, const float *f, const float *gp, float *z,
                    int8_t *q, float *logit, uint32_t *tok, uint32_t *dur) {
    const uint32_t J = m->J, V = m->V;
    float d;
    for (uint32_t j = 0; j < J; j++) {
        const float v = f[j] + gp[j];
        z[j] = v > 0 ? v : 0;
    }
    gemv(k, q, &d, logit, &m->jout, m->jout_b, z, 0);
    uint32_t best = 0;
    for (uint32_t i = 1; i <= V; i++)
        if (logit[i] > logit[best])
            best = i;
    uint32_t bd = 0;
    for (uint32_t i = 1; i < m->n_dur; i++)
        if (logit[V + 1 + i] > logit[V + 1 + bd])
            bd = i;
    *tok = best;
    *dur = bd;
}

void pko_predict(const pko_decoder *m, uint32_t label, float *h, float *c, float *gates, int8_t *q, float *gp) {
    pko_predict_with(&pko_kernels_oracle, m, label, h, c, gates, q, gp);
}

void pko_joint(const pko_decoder *m, const float *f, const float *gp, float *z, int8_t *q, float *logit,
               uint32_t *tok, uint32_t *dur) {
    pko_joint_with(&pko_kernels_oracle, m, f, gp, z, q, logit, tok, dur);
}
