/* backend/hip: libpktito's int8 products on one MI355X (gfx950).
 *
 * This file is the drop-in: copied to backend/hip/kernels.c of a libpktito
 * checkout and built with -DPK_HAVE_hip (with small additions to the Makefile,
 * backend/kernels.c, core/os.c and core/model.c that list it, answer its
 * needs and upload a model's matrices at load), it exports the table
 * pk_kernels_hip beside the CPU backends'
 * (backend/kernels.h:242-278). The table's quantize and gemm_q8 are the
 * GPU's, through libpkhip.so's C ABI (include/pk_hip.h); they compute ref's
 * bits, as every backend must (backend/kernels.h:9-14). Its other eleven
 * kernels, the float ones this path does not cover, are the CPU's: those
 * of the first other backend of the build that this CPU runs, the one
 * backend/kernels.c would have picked without the GPU.
 *
 * The table's functions return nothing (backend/kernels.h:256-258), so a
 * device that fails in the middle of a product has no way to say so; this
 * table then stops the program with the library's message rather than
 * hand back other bits. Whether a device is there at all is asked before
 * the table is ever chosen: its needs are "hip", which core/os.c answers by
 * opening the device (pk_hip_init), and core/model.c uploads every matrix
 * of a model at load, where a failure is the load's error.
 */
#include "kernels.h"
#include "os.h"
#include "pk_hip.h"

#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>

extern const pk_kernels pk_kernels_hip;

/* The CPU backend that takes the float kernels: the first of the build's
 * backends, other than this one, whose needs this CPU meets. ref needs
 * nothing, so there always is one. */
static const pk_kernels *cpu(void) {
    static _Atomic(const pk_kernels *) kept;
    const pk_kernels *t = atomic_load_explicit(&kept, memory_order_acquire);
    if (t)
        return t;
    for (const pk_kernels *const *k = pk_kernels_built; *k && !t; k++)
        if (*k != &pk_kernels_hip && !pk_os_cpu_lacks((*k)->needs))
            t = *k;
    if (!t)
        t = &pk_kernels_ref;
    atomic_store_explicit(&kept, t, memory_order_release);
    return t;
}

static void failed(const char *what, int err) {
    fprintf(stderr, "pktito: backend hip: %s: %s: %s\n", what, pk_hip_strerror(err), pk_hip_last_error());
    abort();
}

static void k_quantize(pk_act *a, const float *x, size_t xs) {
    const int e = pk_hip_quantize((pk_hip_act *)a, x, xs);
    if (e)
        failed("quantize", e);
}

static void k_gemm_q8(float *out, size_t os, const int8_t *w, const float *ws, const float *bias,
                      uint32_t rows, const pk_act *a, int add) {
    const int e = pk_hip_gemm_q8(out, os, w, ws, bias, rows, (const pk_hip_act *)a, add);
    if (e)
        failed("gemm_q8", e);
}

/* the float kernels: the CPU's */

static void k_gemm_f32(float *out, size_t os, const float *w, uint32_t ld, uint32_t rows, uint32_t n,
                       const float *x, size_t xs, uint32_t T, const float *bias, size_t bs, int relu) {
    cpu()->gemm_f32(out, os, w, ld, rows, n, x, xs, T, bias, bs, relu);
}

static void k_layernorm(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t n,
                        const float *w, const float *b, float eps) {
    cpu()->layernorm(out, os, x, xs, T, n, w, b, eps);
}

static void k_softmax(float *x, uint32_t n, float scale) { cpu()->softmax(x, n, scale); }

static void k_silu(float *x, size_t n) { cpu()->silu(x, n); }

static void k_gelu(float *x, size_t n) { cpu()->gelu(x, n); }

static void k_glu(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t n) {
    cpu()->glu(out, os, x, xs, T, n);
}

static void k_dwconv(float *out, size_t os, const float *x, size_t xs, uint32_t T, uint32_t C,
                     const float *w, const float *b, uint32_t K) {
    cpu()->dwconv(out, os, x, xs, T, C, w, b, K);
}

static void k_conv3x3s2(float *out, const float *in, uint32_t r0, uint32_t Ti, uint32_t Fi, uint32_t C,
                        int depthwise, const float *w, const float *b, int relu, uint32_t t0, uint32_t t1) {
    cpu()->conv3x3s2(out, in, r0, Ti, Fi, C, depthwise, w, b, relu, t0, t1);
}

static void k_lstm(float *h, float *c, const float *g, uint32_t H) { cpu()->lstm(h, c, g, H); }

static void k_stft(float *out, size_t os, const float *const *x, uint32_t count, const pk_fft *f,
                   float *scratch) {
    cpu()->stft(out, os, x, count, f, scratch);
}

static void k_resample(float *y, const float *x, uint32_t nb, uint32_t orig, uint32_t nw, const float *k,
                       const size_t *at, const uint32_t *first, const uint32_t *len) {
    cpu()->resample(y, x, nb, orig, nw, k, at, first, len);
}

static const char *const needs[] = { "hip", NULL };

const pk_kernels pk_kernels_hip = {
    .id = "hip",
    .name = "hip (MI355X gfx950: int8 on MFMA, exact int32, the CPU's float kernels)",
    .needs = needs,
    .competes = 0,
    .quantize = k_quantize,
    .gemm_q8 = k_gemm_q8,
    .gemm_f32 = k_gemm_f32,
    .layernorm = k_layernorm,
    .softmax = k_softmax,
    .silu = k_silu,
    .gelu = k_gelu,
    .glu = k_glu,
    .dwconv = k_dwconv,
    .conv3x3s2 = k_conv3x3s2,
    .lstm = k_lstm,
    .stft = k_stft,
    .resample = k_resample,
};
