/* The model-load step of backend/hip: every int8 matrix of a model uploaded
 * to the GPU once, repacked there (pk_hip_upload_q8), after core/model.c's
 * load_file has bound the matrices to the mapped file (core/model.c:345-363,
 * :783-811); and released with the model (core/model.c:868-883). Copied to
 * core/ of a libpktito checkout beside model.c, and called from there.
 *
 * The matrices are those the model binds as pk_q8 (core/model.h): the
 * encoder's subsampling and layers, the decoder's LSTMs and joint, or a
 * diarizer's. A slim file (an NPU's encoder) has no encoder matrices.
 */
#include "model.h"
#include "pk_hip.h"

#include <stdio.h>

typedef int (*q8_fn)(const pk_q8 *q, void *ctx);

/* f over every pk_q8 the model binds, in a fixed order; stops at the first
 * nonzero result */
static int each_q8(const pk_model *m, q8_fn f, void *ctx) {
#define PK_EACH(x)                       \
    do {                                 \
        const int r_ = f(&(x), ctx);     \
        if (r_)                          \
            return r_;                   \
    } while (0)
    if (m->diar) {
        PK_EACH(m->dw.stack_w);
        for (uint32_t i = 0; m->dw.layers && i < m->n_layers; i++) {
            const pk_tlayer *L = &m->dw.layers[i];
            PK_EACH(L->q); PK_EACH(L->k); PK_EACH(L->v); PK_EACH(L->o);
            PK_EACH(L->up); PK_EACH(L->down);
        }
        PK_EACH(m->dw.proj); PK_EACH(m->dw.up); PK_EACH(m->dw.head_hidden); PK_EACH(m->dw.head_out);
        return 0;
    }
    if (!m->encoder_coreml) {
        PK_EACH(m->sub_pw1); PK_EACH(m->sub_pw2); PK_EACH(m->sub_out);
        for (uint32_t i = 0; m->layers && i < m->n_layers; i++) {
            const pk_layer *L = &m->layers[i];
            PK_EACH(L->ff1_up); PK_EACH(L->ff1_down); PK_EACH(L->ff2_up); PK_EACH(L->ff2_down);
            PK_EACH(L->q); PK_EACH(L->k); PK_EACH(L->v); PK_EACH(L->pos); PK_EACH(L->o);
            PK_EACH(L->pw1); PK_EACH(L->pw2);
        }
    }
    for (uint32_t i = 0; m->lstm && i < m->pred_layers; i++) {
        PK_EACH(m->lstm[i].wx);
        PK_EACH(m->lstm[i].wh);
    }
    PK_EACH(m->jenc); PK_EACH(m->jpred); PK_EACH(m->jout);
    return 0;
#undef PK_EACH
}

typedef struct {
    char *err;
    size_t errlen;
} up_ctx;

static int up_one(const pk_q8 *q, void *ctx) {
    if (!q->q)
        return 0;                           /* a matrix this file does not have */
    const int e = pk_hip_upload_q8(q->q, q->s, q->rows, q->cols);
    if (e) {
        up_ctx *c = ctx;
        snprintf(c->err, c->errlen, "uploading a %ux%u int8 matrix to the GPU: %s (%s)", (unsigned)q->rows,
                 (unsigned)q->cols, pk_hip_strerror(e), pk_hip_last_error());
        return -1;
    }
    return 0;
}

static int release_one(const pk_q8 *q, void *ctx) {
    (void)ctx;
    if (q->q && pk_hip_q8_find(q->q))
        pk_hip_release_q8(q->q);
    return 0;
}

/* 0, or -1 with why: every matrix of m in HBM. On failure the ones already
 * uploaded are released. */
int pk_hip_upload_model(const pk_model *m, char *err, size_t errlen) {
    up_ctx c = { err, errlen };
    if (each_q8(m, up_one, &c)) {
        each_q8(m, release_one, NULL);
        return -1;
    }
    return 0;
}

void pk_hip_release_model(const pk_model *m) { each_q8(m, release_one, NULL); }
