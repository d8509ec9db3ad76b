/* The oracle: a CPU restatement of libpktito's int8 product path, for
 * checking the HIP path and for timing a CPU baseline beside it.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libpktito_amd/) links,
 * loads or calls this code; only tests/, the smoke check of
 * __graft_entry__.py and bench.py's cpu_baseline leg do, and only as what
 * the results are compared with or as the baseline being timed, never as the
 * thing measured.
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
 * and in pk_oracle_layer.c, the float kernels around the products and the
 * encoder layer they make (the device-resident layer's definition):
 *
 *   pko_expf, pko_sigmoidf    core/vmath.h:126-151 (the reference's own
 *                             exp polynomial, not libm's)
 *   pko_gemm_f32              backend/ref/kernels.c:90-105
 *   pko_layernorm             backend/ref/kernels.c:109-132 (16-lane sums)
 *   pko_softmax, pko_silu,    backend/ref/kernels.c:134-176
 *   pko_glu, pko_dwconv
 *   pko_conformer_layer       core/encoder.c:108-128 (normq), 147-156
 *                             (siluq_tile), 170-176 (dw_item), 280-327
 *                             (att_item), 321-368 (ff, layer);
 *                             core/passes.c:164-236 (the attention's panels)
 *
 * and in pk_oracle_dec.c, the decoder's per-token work:
 *
 *   pko_tanhf                 core/vmath.h:153-166
 *   pko_lstm                  backend/ref/kernels.c:203-213
 *   pko_gemv_with, pko_predict_with, pko_joint_with
 *                             core/decoder.c:54-101
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
 *     exactly when NaN, inf or amax < 2^-121, d = amax / 127 rounded once);
 *   - the float kernels against the reference's compiled ref table and its
 *     inline pk_expf / pk_sigmoidf (oracle/_ref) on seeded rows with NaNs,
 *     infinities, ties and the clamp's ends, pko_expf also against exp in
 *     double (within 1 ulp on [-87, 88]) and pko_layernorm against a
 *     float64 layer norm; the layer is these kernels and the int8 path
 *     composed in core/encoder.c's order, pinned through each of them and
 *     through invariants of the whole (a frame's outputs depend on other
 *     frames only through the attention and the convolution's K taps).
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

/* ------------------------------------------ float kernels and a layer --- */

float pko_expf(float x);
float pko_sigmoidf(float x);
void  pko_expf_n(float *y, const float *x, size_t n);       /* y[i] = pko_expf(x[i]) */
void  pko_sigmoidf_n(float *y, const float *x, size_t n);
void  pko_gemm_f32(float *out, size_t os, const float *w, uint32_t ld, uint32_t rows, uint32_t n,
                   const float *x, size_t xs, uint32_t T, const float *bias, size_t bs, int relu);
void  pko_layernorm(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t n,
                    const float *w, const float *b, float eps);
void  pko_softmax(float *x, uint32_t n, float scale);
void  pko_silu(float *x, size_t n);
void  pko_glu(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t n);
void  pko_dwconv(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t C,
                 const float *w, const float *b, uint32_t K);

/* A PK_Q8 matrix (core/model.h:39-43): panels, a scale a row. */
typedef struct {
    const int8_t *q;
    const float  *s;
    uint32_t      rows, cols;
} pko_q8;

/* One encoder layer's weights (core/model.h:45-53) and shapes: D = d_model,
 * H heads of D / H, F = ff_dim, K the depthwise taps. */
typedef struct {
    uint32_t D, H, F, K;
    float    eps;
    const float *ff1_nw, *ff1_nb, *att_nw, *att_nb, *conv_nw, *conv_nb;
    const float *ff2_nw, *ff2_nb, *out_nw, *out_nb;
    pko_q8 ff1_up, ff1_down, ff2_up, ff2_down;
    pko_q8 q, k, v, pos, o;
    const float *bias_u, *bias_v;
    pko_q8 pw1, pw2;
    const float *dw, *dw_b;
} pko_layer;

/* A kernel table of the calls the layer makes (backend/kernels.h:242-278's
 * entries), for composing the layer from the oracle's kernels or from a
 * backend of the reference's (oracle/ref_shim.c fills one). */
typedef struct {
    void (*quantize)(pko_act *a, const float *x, size_t xs);
    void (*gemm_q8)(float *out, size_t os, const int8_t *w, const float *ws, const float *bias, uint32_t rows,
                    const pko_act *a, int add);
    void (*gemm_f32)(float *out, size_t os, const float *w, uint32_t ld, uint32_t rows, uint32_t n,
                     const float *x, size_t xs, uint32_t T, const float *bias, size_t bs, int relu);
    void (*layernorm)(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t n,
                      const float *w, const float *b, float eps);
    void (*softmax)(float *x, uint32_t n, float scale);
    void (*silu)(float *x, size_t n);
    void (*glu)(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t n);
    void (*dwconv)(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t C,
                   const float *w, const float *b, uint32_t K);
    void (*lstm)(float *h, float *c, const float *g, uint32_t H);
} pko_kernels;

extern const pko_kernels pko_kernels_oracle;

/* One layer in place on x [T][D]: ape holds the positions' activations,
 * 2T - 1 frames of D quantized in blocks of qb (core/encoder.c:467-469), the
 * layer's blocks qb too. Every pass over nthreads, dealt in the reference's
 * items (16 frames, a head's 16 queries, 64 channels, 64-row slices). 0, or
 * -1 for shapes the layer does not take, -2 when out of memory. The _with
 * form takes the kernels from a table. */
int   pko_conformer_layer(const pko_layer *L, float *x, uint32_t T, const pko_act *ape, uint32_t qb,
                          int nthreads);
int   pko_conformer_layer_with(const pko_kernels *k, const pko_layer *L, float *x, uint32_t T,
                               const pko_act *ape, uint32_t qb, int nthreads);

/* ------------------------------------------------------- the decoder --- */

float pko_tanhf(float x);
void  pko_tanhf_n(float *y, const float *x, size_t n);
void  pko_lstm(float *h, float *c, const float *g, uint32_t H);

/* An LSTM layer (core/model.h:57-60): wx, wh [4P][P], b the biases summed. */
typedef struct {
    pko_q8 wx, wh;
    const float *b;
} pko_lstmw;

/* The prediction network and joint (core/model.h:124-131): P = pred_hidden,
 * L layers, J = joint_hidden, V = vocab (blank among [0, V]), n_dur
 * durations after the V + 1 token logits; jout has rows >= V + 1 + n_dur. */
typedef struct {
    uint32_t P, L, J, V, n_dur;
    const float *embed;            /* [V + 1][P] */
    const pko_lstmw *lstm;         /* [L] */
    pko_q8 jpred;
    const float *jpred_b;
    pko_q8 jout;
    const float *jout_b;
} pko_decoder;

/* core/decoder.c:54-101: gemv (one row quantized, a T = 1 product),
 * predict (the LSTM layers stepped in place, h and c L x P, then gp) and
 * joint (the logits and the first best token and duration). Scratch: q
 * max(P, J) bytes, gates 4P floats, z J floats, logit jout's rows. */
void  pko_gemv_with(const pko_kernels *k, int8_t *q, float *d, float *out, const pko_q8 *w, const float *bias,
                    const float *x, int add);
void  pko_predict_with(const pko_kernels *k, const pko_decoder *m, uint32_t label, float *h, float *c,
                       float *gates, int8_t *q, float *gp);
void  pko_joint_with(const pko_kernels *k, const pko_decoder *m, const float *f, const float *gp, float *z,
                     int8_t *q, float *logit, uint32_t *tok, uint32_t *dur);
void  pko_predict(const pko_decoder *m, uint32_t label, float *h, float *c, float *gates, int8_t *q, float *gp);
void  pko_joint(const pko_decoder *m, const float *f, const float *gp, float *z, int8_t *q, float *logit,
                uint32_t *tok, uint32_t *dur);

/* kcheck's generator: xorshift64*, state kept by the caller. */
uint32_t pko_rnd(uint64_t *s);
float    pko_frand(uint64_t *s);                 /* [-1, 1) */
float    pko_awkward(uint64_t *s, float scale);  /* zeros, a subnormal, outliers, ties */
void     pko_fill_awkward(uint64_t *s, float *x, size_t n, float scale);

#endif
