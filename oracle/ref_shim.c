/* A handle on the reference's own compiled backends, for the parity tests
 * and the CPU baseline. Test infrastructure only (see pk_oracle.h).
 *
 * oracle/Makefile compiles this file together with the reference's
 * backend/ref/kernels.c and its x86 backends, in place under the reference
 * checkout, into oracle/_ref/libpkref.so. It exposes each backend's table
 * (backend/kernels.h:242-278) by index, with a CPU-feature check standing in
 * for the reference's pk_os_cpu_lacks (core/os.c:840-911), so a caller can
 * run exactly the reference's quantize and gemm_q8.
 */
#include "kernels.h"
#include "pk_oracle.h"
#include "vmath.h"

#include <string.h>

extern const pk_kernels pk_kernels_ref, pk_kernels_avx2, pk_kernels_avx2_vnni,
    pk_kernels_avx512_vnni;

static const pk_kernels *const tables[] = {
    &pk_kernels_ref, &pk_kernels_avx512_vnni, &pk_kernels_avx2_vnni, &pk_kernels_avx2,
};

int pkref_count(void) { return (int)(sizeof tables / sizeof tables[0]); }

const char *pkref_id(int i) { return i >= 0 && i < pkref_count() ? tables[i]->id : NULL; }

const char *pkref_name(int i) { return i >= 0 && i < pkref_count() ? tables[i]->name : NULL; }

/* 1 when this CPU has every feature the backend's needs list names */
int pkref_usable(int i) {
    if (i < 0 || i >= pkref_count())
        return 0;
    __builtin_cpu_init();
    for (const char *const *n = tables[i]->needs; *n; n++) {
        int ok;
        if (!strcmp(*n, "avx2")) ok = __builtin_cpu_supports("avx2");
        else if (!strcmp(*n, "fma")) ok = __builtin_cpu_supports("fma");
        else if (!strcmp(*n, "avx512f")) ok = __builtin_cpu_supports("avx512f");
        else if (!strcmp(*n, "avx512vl")) ok = __builtin_cpu_supports("avx512vl");
        else if (!strcmp(*n, "avx512vnni")) ok = __builtin_cpu_supports("avx512vnni");
        else if (!strcmp(*n, "avxvnni")) ok = __builtin_cpu_supports("avxvnni");
        else ok = 0;
        if (!ok)
            return 0;
    }
    return 1;
}

void pkref_quantize(int i, pk_act *a, const float *x, size_t xs) { tables[i]->quantize(a, x, xs); }

void pkref_gemm_q8(int i, float *out, size_t os, const int8_t *w, const float *ws,
                   const float *bias, uint32_t rows, const pk_act *a, int add) {
    tables[i]->gemm_q8(out, os, w, ws, bias, rows, a, add);
}

/* The product over nthreads, 64-row slices from an atomic counter, as the
 * reference's tests/gemmbench.c:77-94 deals them. pk_act and pko_act have
 * one layout. */
void pkref_gemm_threads(int i, int nthreads, float *out, size_t os, const int8_t *w,
                        const float *ws, const float *bias, uint32_t rows, const pk_act *a,
                        int add) {
    pko_gemm_threads((pko_gemm_fn)tables[i]->gemm_q8, nthreads, out, os, w, ws, bias, rows,
                     (const pko_act *)a, add);
}

void pkref_quantize_threads(int i, int nthreads, pk_act *a, const float *x, size_t xs) {
    pko_quantize_threads((pko_quant_fn)tables[i]->quantize, nthreads, (pko_act *)a, x, xs);
}

/* The reference's float kernels and its inline exp and sigmoid
 * (core/vmath.h:134-151), for pinning the oracle's restatements. */
float pkref_expf(float x) { return pk_expf(x); }

float pkref_sigmoidf(float x) { return pk_sigmoidf(x); }

void pkref_expf_n(float *y, const float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        y[i] = pk_expf(x[i]);
}

void pkref_sigmoidf_n(float *y, const float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        y[i] = pk_sigmoidf(x[i]);
}

void pkref_gemm_f32(int i, float *out, size_t os, const float *w, uint32_t ld, uint32_t rows, uint32_t n,
                    const float *x, size_t xs, uint32_t T, const float *bias, size_t bs, int relu) {
    tables[i]->gemm_f32(out, os, w, ld, rows, n, x, xs, T, bias, bs, relu);
}

void pkref_layernorm(int i, float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t n,
                     const float *w, const float *b, float eps) {
    tables[i]->layernorm(out, os, x, xs, T, n, w, b, eps);
}

void pkref_softmax(int i, float *x, uint32_t n, float scale) { tables[i]->softmax(x, n, scale); }

void pkref_silu(int i, float *x, size_t n) { tables[i]->silu(x, n); }

void pkref_glu(int i, float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t n) {
    tables[i]->glu(out, os, x, xs, T, n);
}

void pkref_dwconv(int i, float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t C,
                  const float *w, const float *b, uint32_t K) {
    tables[i]->dwconv(out, os, x, xs, T, C, w, b, K);
}

/* Backend i's kernels as the oracle's table, for composing the layer from
 * the reference's own kernels (pk_act and pko_act share one layout). */
void pkref_kernels(int i, pko_kernels *k) {
    const pk_kernels *t = tables[i];
    k->quantize = (void (*)(pko_act *, const float *, size_t))t->quantize;
    k->gemm_q8 = (void (*)(float *, size_t, const int8_t *, const float *, const float *, uint32_t,
                           const pko_act *, int))t->gemm_q8;
    k->gemm_f32 = t->gemm_f32;
    k->layernorm = t->layernorm;
    k->softmax = t->softmax;
    k->silu = t->silu;
    k->glu = t->glu;
    k->dwconv = t->dwconv;
    k->lstm = t->lstm;
}

/* The reference's inline tanh (core/vmath.h:153-166) over an array */
void pkref_tanhf_n(float *y, const float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        y[i] = pk_tanhf(x[i]);
}

void pkref_lstm(int i, float *h, float *c, const float *g, uint32_t H) { tables[i]->lstm(h, c, g, H); }
