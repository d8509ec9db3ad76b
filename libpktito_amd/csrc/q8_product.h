/* Device helpers of the int8 products shared by their kernel files
 * (q8_kernels.hip, the per-launch tiles; q8_stream.hip, the streamed tiles;
 * tests/test_lds_waits.py checks both files' assembly): non-temporal output stores, LDS DMA
 * address spaces, explicit vmcnt / lgkmcnt waits, LDS fragment reads issued
 * as inline asm, compile-time unrolling, and the XCD-aware tile order. */
#ifndef PK_Q8_PRODUCT_H
#define PK_Q8_PRODUCT_H

#include "q8_device.h"
#include "q8_internal.h"

#include <hip/hip_runtime.h>

#include <type_traits>

namespace pkq8 {

/* Output stores: non-temporal unless the launch sets plain (GemmArgs::plain,
 * uniform). Measured: a product of up to a few tens of MB of outputs drains
 * its stores 12-21% sooner non-temporal; one of ~120 MB (the feed-forward
 * up projection at ten minutes of audio) runs ~7% sooner with plain stores.
 * The bits are the same. */
typedef float nt_f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store_out4(float *o, float4 v, int plain) {
    const nt_f4 nv = { v.x, v.y, v.z, v.w };
    if (plain)
        *(nt_f4 *)o = nv;
    else
        __builtin_nontemporal_store(nv, (nt_f4 *)o);
}

__device__ __forceinline__ void store_out1(float *o, float v, int plain) {
    if (plain)
        *o = v;
    else
        __builtin_nontemporal_store(v, o);
}

#define PK_AS1(p) ((const void __attribute__((address_space(1))) *)(p))
#define PK_AS3(p) ((void __attribute__((address_space(3))) *)(p))

/* s_waitcnt vmcnt(N), expcnt and lgkmcnt left alone (gfx9 encoding) */
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

/* the LDS byte address of a __shared__ pointer */
__device__ __forceinline__ uint32_t lds_addr(const int8_t *p) {
    return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) int8_t *)p);
}

/* 16 bytes from LDS, issued as written; the caller waits on lgkmcnt. The
 * compiler takes the result as ready when the asm ends, so nothing may copy
 * or reuse the destination before that wait: a kernel whose registers run
 * out (two fragment sets beside 256 accumulators) gets such copies, and
 * tests/test_lds_waits.py checks every kernel's assembly for them. */
__device__ __forceinline__ v4i lds_read16(uint32_t addr) {
    v4i r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr) : "memory");
    return r;
}

typedef int v2i __attribute__((ext_vector_type(2)));

/* 8 bytes from LDS, as lds_read16 */
__device__ __forceinline__ v2i lds_read8(uint32_t addr) {
    v2i r;
    asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(addr) : "memory");
    return r;
}

/* f(integral_constant<int, I>) for I in [I0, N), unrolled at compile time */
template <int I, int N, typename F>
__device__ __forceinline__ void for_static(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        for_static<I + 1, N>(f);
    }
}

/* s_waitcnt lgkmcnt(N), the other counters untouched */
template <int N>
__device__ __forceinline__ void wait_lgkm() {
    static_assert(N >= 0 && N < 16, "lgkmcnt is four bits");
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}

/* 4 bytes from LDS, issued as written; the caller waits on lgkmcnt */
__device__ __forceinline__ float lds_read4(uint32_t addr) {
    float r;
    asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(addr) : "memory");
    return r;
}

/* The hardware deals workgroup b to XCD b % 8. Renumbered so that each XCD
 * takes a contiguous run of tiles, and the run ordered in groups of 8 frame
 * tiles by every channel tile, the workgroups one XCD runs at once share
 * their inputs and weights in its L2. */
__device__ __forceinline__ void xcd_tile(uint32_t b, uint32_t nwg, uint32_t tiles_n, uint32_t tiles_m,
                                         uint32_t &tn, uint32_t &tm) {
    const uint32_t per = nwg / 8, rem = nwg % 8, x = b % 8, i = b / 8;
    const uint32_t nb = x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
    constexpr uint32_t GM = 8;
    const uint32_t group = nb / (GM * tiles_n), idx = nb % (GM * tiles_n);
    const uint32_t first = group * GM;
    const uint32_t gm = tiles_m - first < GM ? tiles_m - first : GM;
    tm = first + idx % gm;
    tn = idx / gm;
}

}  // namespace pkq8

#endif
