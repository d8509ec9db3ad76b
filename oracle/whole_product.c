/* Test infrastructure: the core/passes.c change a checkout with the hip
 * backend makes (one pk_k_gemm_q8 and one pk_k_quantize a product when the
 * hip table is in use), applied at link time to the reference's
 * passes.c compiled unedited where it lies. The link of _ref/dropin_cli_whole
 * renames every call of pk_gemm_on and pk_quantize_on from the library's
 * other files (encoder, decoder, diarizer) to these wrappers
 * (-Wl,--wrap=pk_gemm_on, --wrap=pk_quantize_on), and these do what the
 * change adds at the top of each function (core/passes.c:38 and :80): with
 * the hip table in use, the whole product in one pk_k_gemm_q8 call when no
 * tile callback follows it, and the whole quantize in one pk_k_quantize
 * call, instead of the pool's 64-row slices and 16-frame items. Everything
 * else goes on to the reference's own functions (__real_*). Each output is
 * still one call's whole, so the bits are the same (core/passes.c:1-6).
 * Calls between passes.c's own functions are not renamed (a source change
 * would cover them too); the encoder's, decoder's and diarizer's are. */
#include "kernels.h"
#include "model.h"
#include "passes.h"
#include "pool.h"

extern const pk_kernels pk_kernels_hip;

void __real_pk_gemm_on(pk_pool *p, float *out, size_t os, const pk_q8 *w, const float *bias,
                       const pk_act *act, int add, pk_tile_fn then, void *then_arg);
void __real_pk_quantize_on(pk_pool *p, pk_act *act, const float *x, size_t xs, uint32_t T, uint32_t n,
                           uint32_t qb);
void __wrap_pk_gemm_on(pk_pool *p, float *out, size_t os, const pk_q8 *w, const float *bias,
                       const pk_act *act, int add, pk_tile_fn then, void *then_arg);
void __wrap_pk_quantize_on(pk_pool *p, pk_act *act, const float *x, size_t xs, uint32_t T, uint32_t n,
                           uint32_t qb);

static int hip_in_use(void) { return pk_kernels_pick(NULL, 0) == &pk_kernels_hip; }

void __wrap_pk_gemm_on(pk_pool *p, float *out, size_t os, const pk_q8 *w, const float *bias,
                       const pk_act *act, int add, pk_tile_fn then, void *then_arg) {
    if (!then && hip_in_use()) {
        pk_k_gemm_q8(out, os, w->q, w->s, bias, w->rows, act, add);
        return;
    }
    __real_pk_gemm_on(p, out, os, w, bias, act, add, then, then_arg);
}

void __wrap_pk_quantize_on(pk_pool *p, pk_act *act, const float *x, size_t xs, uint32_t T, uint32_t n,
                           uint32_t qb) {
    if (hip_in_use()) {
        act->n = n;
        act->qb = qb;
        act->T = T;
        pk_k_quantize(act, x, xs);
        return;
    }
    __real_pk_quantize_on(p, act, x, xs, T, n, qb);
}
