/* Device helpers of the int8 path shared by its kernel files: the
 * quantizer's block rule on magnitude bits, the wave and lane-group maxima,
 * the per-wave scales of a column, the packed units' layout, and the
 * reference's own exp and sigmoid.
 *
 * The quantizer is backend/ref/kernels.c:24-58 (peterheb/libpktito), per
 * column t and block b of qb inputs:
 *   a NaN in the block, an infinite amax, or amax < 2^-121  ->  d = +0, q = 0
 *   otherwise d = amax / 127, id = 127 / amax, q = rint(x * id)
 * amax is a max, the same in any order. Both divisions are IEEE divisions
 * (hipcc's default correctly rounded fp32 divide), rint is v_rndne_f32.
 * Files including this are built with -ffp-contract=off.
 */
#ifndef PK_Q8_DEVICE_H
#define PK_Q8_DEVICE_H

#include "q8_internal.h"

#include <hip/hip_runtime.h>

#pragma clang fp contract(off)

namespace pkq8 {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int q1(float v, float id) { return (int)__builtin_rintf(v * id); }

__device__ __forceinline__ int pack4(float4 v, float id) {
    return (q1(v.x, id) & 0xff) | (q1(v.y, id) & 0xff) << 8 | (q1(v.z, id) & 0xff) << 16 |
           (q1(v.w, id) & 0xff) << 24;
}

/* The quantizer under a directed rounding mode rm (1 upward, 2 downward, 3
 * toward zero), as the reference's ref computes it when the host has set one
 * (its divisions, product and rintf all follow the mode). A division is
 * taken from its round-to-nearest quotient r and the sign of its remainder
 * a - r b, exact as one fmaf (also where r is subnormal: amax >= 2^-121 is a
 * multiple of 2^-144 and r b one of 2^-149), so the directed quotient is r
 * or its neighbour toward the true value; the product and rintf run with
 * the hardware's rounding mode set (ref_rintf). */
__device__ __forceinline__ float next_up(float x) {
    /* x finite; the neighbour toward +inf (the smallest subnormal after a zero) */
    const int b = __float_as_int(x);
    if ((b & 0x7fffffff) == 0)
        return __int_as_float(1);
    return __int_as_float(x > 0.0f ? b + 1 : b - 1);
}

__device__ __forceinline__ float next_down(float x) { return -next_up(-x); }

__device__ __forceinline__ float round_dir(float r, bool above, bool below, int rm) {
    if (rm == 1)
        return above ? next_up(r) : r;
    if (rm == 2)
        return below ? next_down(r) : r;
    return r > 0.0f && below ? next_down(r) : r < 0.0f && above ? next_up(r) : r;
}

/* a / b, b > 0 */
__device__ __forceinline__ float div_dir(float a, float b, int rm) {
    const float r = a / b;
    const float rem = __builtin_fmaf(-r, b, a);
    return round_dir(r, rem > 0.0f, rem < 0.0f, rm);
}

/* rintf as the reference's ref computes it on x86: built at -O3 without
 * SSE4.1, gcc inlines rintf(x) as copysign((|x| + 2^23) - 2^23, x) for |x| <
 * 2^23 (x itself otherwise), both operations in the current mode. To nearest
 * that is rint; under a directed mode it rounds |x|, so upward -43.18 gives
 * -44. The caller has set MODE.FP_ROUND to the mode. */
__device__ __forceinline__ float ref_rintf(float x) {
    const float a = __builtin_fabsf(x);
    if (!(a < 8388608.0f))
        return x;
    return __builtin_copysignf((a + 8388608.0f) - 8388608.0f, x);
}

/* The same block rule on magnitude bits: m = the largest (bits & 0x7fffffff)
 * of the block. Non-negative floats order as their bit patterns do, NaN above
 * infinity above every finite value, so the block holds a NaN or an infinity
 * exactly when m >= 0x7f800000, and otherwise m is the bits of amax; 2^-121
 * is 0x03000000. */
__device__ __forceinline__ bool zero_bits(uint32_t m) { return m >= 0x7f800000u || m < 0x03000000u; }

__device__ __forceinline__ int mag_bits(float v) { return (int)(__float_as_uint(v) & 0x7fffffffu); }

/* The maximum over the wave of a non-negative int, in every lane: DPP within
 * rows of 16 lanes (quad swaps, half mirror, mirror), the row broadcasts
 * across rows, then lane 63's value. All 64 lanes must be active. */
__device__ __forceinline__ int wave_max_nonneg(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));    /* quad_perm 1,0,3,2 */
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));    /* quad_perm 2,3,0,1 */
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));   /* row_half_mirror */
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false));   /* row_mirror */
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false));   /* row_bcast15: rows 1, 3 */
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false));   /* row_bcast31: rows 2, 3 */
    return __builtin_amdgcn_readlane(v, 63);
}

/* max of a non-negative int over aligned groups of W lanes (W = 8 or 16), in
 * every lane of the group: DPP quad swaps, half mirror, and mirror for 16 */
template <int W>
__device__ __forceinline__ int group_max_nonneg(int v) {
    static_assert(W == 8 || W == 16, "groups of 8 or 16 lanes");
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));
    if constexpr (W == 16)
        v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false));
    return v;
}

__device__ __forceinline__ int mag4(float4 f) {
    return max(max(mag_bits(f.x), mag_bits(f.y)), max(mag_bits(f.z), mag_bits(f.w)));
}

/* A block's scales from the largest magnitude's bits mb (backend/ref/kernels.c:
 * 24-58): zero (a NaN or an infinity, or an amax below 2^-121), else d =
 * amax / 127 and the multiplier 127 / amax. */
__device__ __forceinline__ void block_scales(uint32_t mb, bool &zero, float &dv, float &id) {
    zero = zero_bits(mb);
    dv = 0.0f;
    id = 0.0f;
    if (!zero) {
        const float amax = __uint_as_float(mb);
        dv = amax / 127.0f;
        id = 127.0f / amax;
    }
}

/* The scales of a column of n <= 4096 inputs that one wave holds, each lane
 * CH float4 chunks of it (chunk c of lane l is float4 l + 64 c, zeros past
 * the column). QB == 0: the column is one block, reduced over the wave;
 * QB == 32 or 64: chunk c's block of QB inputs, reduced within the QB / 4
 * lanes holding it. All 64 lanes active. */
template <int CH, int QB>
struct WaveScales {
    static constexpr int NB = QB ? CH : 1;
    float dv[NB], id[NB];
    bool zero[NB];

    __device__ __forceinline__ void block(int b, uint32_t mb) { block_scales(mb, zero[b], dv[b], id[b]); }

    __device__ __forceinline__ explicit WaveScales(const float4 (&v)[CH]) {
        if constexpr (QB == 0) {
            int m = 0;
#pragma unroll
            for (int c = 0; c < CH; c++)
                m = max(m, mag4(v[c]));
            block(0, (uint32_t)wave_max_nonneg(m));
        } else {
#pragma unroll
            for (int c = 0; c < CH; c++)
                block(c, (uint32_t)group_max_nonneg<QB / 4>(mag4(v[c])));
        }
    }
};

/* Where inputs k..k+3 of frame r of a 16-frame group sit in the group's
 * unit k / 64: at 16 (16 kq + r) + k % 16, kq = (k % 64) / 16. Unit u of
 * group g is unit u G + g of the packed copy of G groups. */
__device__ __forceinline__ uint32_t in_unit(uint32_t k, uint32_t r) {
    return (((k >> 4) & 3) * 16 + r) * 16 + (k & 15);
}

/* ----------------------------------------------------- exp and sigmoid --
 *
 * core/vmath.h:92-151 (peterheb/libpktito): the reference's own exp, not a
 * library's, so that every backend's lanes compute the same bits. The
 * argument clamped to [-87, 88] (a NaN to -87: fmaxf returns the operand
 * that is a number), n = rint(x log2e), the remainder r = x - n ln2 in two
 * FMAs with ln2 split high and low, a degree-6 polynomial in r by Horner's
 * rule in FMAs, times 2^n built in the exponent field. The constants are
 * the reference's. */
__device__ __forceinline__ float pk_expf(float x) {
    x = __builtin_fminf(__builtin_fmaxf(x, -87.0f), 88.0f);
    const float n = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(n, -0x1.62e430p-1f, x);
    r = __builtin_fmaf(n, 0x1.05c610p-29f, r);
    float p = 0x1.6ab980p-10f;
    p = __builtin_fmaf(p, r, 0x1.126d0cp-7f);
    p = __builtin_fmaf(p, r, 0x1.55589ap-5f);
    p = __builtin_fmaf(p, r, 0x1.55540ap-3f);
    p = __builtin_fmaf(p, r, 0x1.fffffap-2f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return p * __uint_as_float((uint32_t)((int32_t)n + 127) << 23);
}

/* core/vmath.h:149-151 */
__device__ __forceinline__ float pk_sigmoidf(float x) { return 1.0f / (1.0f + pk_expf(-x)); }

/* x * sigmoid(x): SiLU (backend/ref/kernels.c:149-151) */
__device__ __forceinline__ float pk_silu(float x) { return x * pk_sigmoidf(x); }

/* core/vmath.h:153-166 with its constants (core/vmath.h:104-116): below
 * |x| = 0.625, x + x^3 p(x^2) with p by Horner's rule in FMAs; above it
 * 1 - 2 / (e^2|x| + 1) with the sign of x. */
__device__ __forceinline__ float pk_tanhf(float x) {
    const float a = __builtin_fabsf(x);
    if (a < 0.625f) {
        const float x2 = x * x;
        float p = -0x1.75e1cep-8f;
        p = __builtin_fmaf(p, x2, 0x1.52269cp-6f);
        p = __builtin_fmaf(p, x2, -0x1.b83c5ap-5f);
        p = __builtin_fmaf(p, x2, 0x1.110726p-3f);
        p = __builtin_fmaf(p, x2, -0x1.555532p-2f);
        return __builtin_fmaf(x * x2, p, x);
    }
    const float e = pk_expf(2.0f * a);
    return __builtin_copysignf(1.0f - 2.0f / (e + 1.0f), x);
}

}  // namespace pkq8

#endif
