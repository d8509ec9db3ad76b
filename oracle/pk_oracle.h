/* The oracle: a CPU restatement of libpktito's int8 product path, for
 * checking the HIP path and for timing a CPU baseline beside it.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libpktito_amd/) links,
 * loads or calls this code; only tests/, the smoke check of
 * __graft_entry__.py and bench.py's cpu_baseline leg do, and only as the
 * checker or as the baseline being timed, never as the thing measured.
 *
 * What each function restates (file:line in peterheb/libpktito 0.9.8):
 *
 *   pko_quantize   backend/ref/kernels.c:24-58, the contract at
 *                  backend/kernels.h:47-58
 *   pko_gemm_q8    backend/ref/kernels.c:66-86, the contract at
 *                  backend/kernels.h:60-78; the PK_Q8 index of
 *                  backend/ref/kernels.c:61-64 and core/pkf.h:28-41
 *   pko_fmaf       core/vmath.h:61-91 (pk_fmaf: a*b+c rounded once)
 *   pko_definition tests/kcheck.c:217-239 (the int64 definition of a sum)
 *   pko_*_threads  the dealing of tests/gemmbench.c:77-94 (64-row slices
 *                  from an atomic counter) and core/passes.c:28-46
 *                  (16 columns an item)
 *   pko_rnd ...    tests/kcheck.c:40-60 (xorshift64*, frand, awkward)
 *
 * How each is pinned, beyond restating the formula:
 *   - against the reference's own compiled ref backend (oracle/_ref, built
 *     from the reference's sources by oracle/Makefile) on seeded cases;
 *   - against golden fixtures cut from that build (tests/golden/);
 *   - the int32 sums against an int64 brute force and closed forms
 *     (extreme rows of -128 / 127 against +-127, exact cancellation);
 *   - the epilogue against the d = 0, s < 0 case where fmaf(s, d, +0) is +0
 *     and a bare product -0, and against directed rounding modes;
 *   - the quantizer against its invariants (q in [-127, 127], zero block
 *     exactly when NaN, inf or amax < 2^-121, d = amax / 127 rounded once).
 * Every function here is pinned by at least one of these (tests/test_oracle.py).
 */
#ifndef PK_ORACLE_H
#define PK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

/* The layout of backend/kernels.h:41-45's pk_act. */
typedef struct {
    int8_t   *q;            /* [T][n] */
    float    *d;            /* [T][n / qb] */
    uint32_t  n, qb, T;
} pko_act;

typedef void (*pko_gemm_fn)(float *out, size_t os, const int8_t *w, const float *ws,
                            const float *bias, uint32_t rows, const pko_act *a, int add);
typedef void (*pko_quant_fn)(pko_act *a, const float *x, size_t xs);

float pko_fmaf(float a, float b, float c);
void  pko_quantize(pko_act *a, const float *x, size_t xs);
void  pko_gemm_q8(float *out, size_t os, const int8_t *w, const float *ws, const float *bias,
                  uint32_t rows, const pko_act *a, int add);

/* The byte index of q(r, k) in a PK_Q8 matrix of n inputs (core/pkf.h:34). */
size_t pko_q8_index(uint32_t n, uint32_t r, uint32_t k);
/* Row-major rows x n int8 into PK_Q8 panels, and back. */
void   pko_pack_q8(int8_t *panels, const int8_t *rowmajor, uint32_t rows, uint32_t n);
void   pko_unpack_q8(int8_t *rowmajor, const int8_t *panels, uint32_t rows, uint32_t n);

/* The definition, kcheck's way: every sum in int64, then pk_fmaf per block,
 * the scale, the bias. Writes T x rows floats at stride os; no add. */
void  pko_definition(float *out, size_t os, const int8_t *w, const float *ws, const float *bias,
                     uint32_t rows, const pko_act *a);

/* The whole product over nthreads pthreads, 64-row slices dealt from an
 * atomic counter, each slice one call of fn over every column. */
void  pko_gemm_threads(pko_gemm_fn fn, int nthreads, float *out, size_t os, const int8_t *w,
                       const float *ws, const float *bias, uint32_t rows, const pko_act *a, int add);
/* The quantizer over nthreads, 16 columns an item. */
void  pko_quantize_threads(pko_quant_fn fn, int nthreads, pko_act *a, const float *x, size_t xs);

/* kcheck's generator: xorshift64*, state kept by the caller. */
uint32_t pko_rnd(uint64_t *s);
float    pko_frand(uint64_t *s);                 /* [-1, 1) */
float    pko_awkward(uint64_t *s, float scale);  /* zeros, a subnormal, outliers, ties */
void     pko_fill_awkward(uint64_t *s, float *x, size_t n, float scale);

#endif
