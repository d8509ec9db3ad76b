/* The int8 product path on gfx950: the quantizer, the weight repack, and the
 * int8 product with its fp32 epilogue.
 *
 * Bits. Every result is the reference's ref backend's
 * (backend/ref/kernels.c:24-86 in peterheb/libpktito): integer sums are
 * exact in any order, so the MFMAs may take the inputs in whatever order
 * their lanes hold them, and the few float operations a block or an output
 * has are written out one by one in ref's order. The file is built with
 * -ffp-contract=off and the pragma below, so that no multiply and add the
 * code keeps apart is fused, and without any flag that flushes denormals
 * (a block's scale can be subnormal) or relaxes division.
 */
#include "q8_internal.h"

#include <cstring>
#include "q8_device.h"
#include "q8_product.h"

#include <float.h>
#include <stdio.h>

#include <type_traits>

#pragma clang fp contract(off)

namespace pkq8 {

/* ------------------------------------------------------------ quantize --
 *
 * backend/ref/kernels.c:24-58, per column t and block b of qb inputs:
 *   a NaN in the block, an infinite amax, or amax < 2^-121  ->  d = +0, q = 0
 *   otherwise d = amax / 127, id = 127 / amax, q = rint(x * id)
 * amax is a max, the same in any order. Both divisions are IEEE divisions
 * (hipcc's default correctly rounded fp32 divide), rint is v_rndne_f32. */

__device__ __forceinline__ void absmax4(float4 v, float &amax, int &nan) {
    nan |= (v.x != v.x) | (v.y != v.y) | (v.z != v.z) | (v.w != v.w);
    amax = fmaxf(amax, fabsf(v.x));
    amax = fmaxf(amax, fabsf(v.y));
    amax = fmaxf(amax, fabsf(v.z));
    amax = fmaxf(amax, fabsf(v.w));
}

__device__ __forceinline__ bool zero_block(float amax, int nan) {
    return nan || !__builtin_isfinite(amax) || amax < 0x1p-121f;
}

/* A whole column is one block (qb == n, "per-row" quantization): one
 * workgroup of W waves a column, each thread up to CH chunks of 16 inputs,
 * held in registers between the max and the rounding. */
template <int W, int CH>
__global__ __launch_bounds__(64 * W) void quant_col_kernel(int8_t *__restrict__ q, float *__restrict__ d,
                                                           const float *__restrict__ x, size_t xs,
                                                           uint32_t n) {
    const uint32_t t = blockIdx.x, nch = n >> 4;
    const float *xr = x + (size_t)t * xs;
    float4 v[CH][4];
    float amax = 0.0f;
    int nan = 0;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t ch = threadIdx.x + c * 64 * W;
        if (ch < nch) {
            const float4 *p = (const float4 *)(xr + (size_t)ch * 16);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v[c][e] = p[e];
                absmax4(v[c][e], amax, nan);
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, off, 64));
        nan |= __shfl_xor(nan, off, 64);
    }
    if (W > 1) {
        __shared__ float sm[W];
        __shared__ int sn[W];
        if ((threadIdx.x & 63) == 0) {
            sm[threadIdx.x >> 6] = amax;
            sn[threadIdx.x >> 6] = nan;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < W; i++) {
            amax = fmaxf(amax, sm[i]);
            nan |= sn[i];
        }
    }
    const bool zero = zero_block(amax, nan);
    float dv = 0.0f, id = 0.0f;
    if (!zero) {
        dv = amax / 127.0f;
        id = 127.0f / amax;
    }
    int8_t *qr = q + (size_t)t * n;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t ch = threadIdx.x + c * 64 * W;
        if (ch < nch) {
            v4i o = {0, 0, 0, 0};
            if (!zero)
                o = v4i{pack4(v[c][0], id), pack4(v[c][1], id), pack4(v[c][2], id),
                        pack4(v[c][3], id)};
            *(v4i *)(qr + (size_t)ch * 16) = o;
        }
    }
    if (threadIdx.x == 0)
        d[t] = dv;
}

/* Blocks of qb = 16 * G inputs, G a power of two up to 64: one thread a
 * chunk of 16, a block's G threads adjacent lanes of one wave. */
template <int G>
__global__ __launch_bounds__(256) void quant_blk_kernel(int8_t *__restrict__ q, float *__restrict__ d,
                                                        const float *__restrict__ x, size_t xs,
                                                        uint32_t n, uint32_t T) {
    const uint32_t nch = n >> 4, nb = nch / G;
    const uint64_t total = (uint64_t)T * nch;
    uint64_t c = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const bool live = c < total;
    if (!live)
        c = total - 1;      /* a whole group is past the end or none of it is */
    const uint32_t t = (uint32_t)(c / nch), ch = (uint32_t)(c % nch);
    const float4 *p = (const float4 *)(x + (size_t)t * xs + (size_t)ch * 16);
    float4 v[4];
    float amax = 0.0f;
    int nan = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        v[e] = p[e];
        absmax4(v[e], amax, nan);
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, off, 64));
        nan |= __shfl_xor(nan, off, 64);
    }
    if (!live)
        return;
    const bool zero = zero_block(amax, nan);
    float dv = 0.0f, id = 0.0f;
    if (!zero) {
        dv = amax / 127.0f;
        id = 127.0f / amax;
    }
    v4i o = {0, 0, 0, 0};
    if (!zero)
        o = v4i{pack4(v[0], id), pack4(v[1], id), pack4(v[2], id), pack4(v[3], id)};
    *(v4i *)(q + (size_t)t * n + (size_t)ch * 16) = o;
    if (ch % G == 0)
        d[(size_t)t * nb + ch / G] = dv;
}

/* Any other qb (a multiple of 32 that is neither the whole column nor
 * 16 times a power of two): one thread a block, the reference's loop. */
__global__ __launch_bounds__(256) void quant_any_kernel(int8_t *__restrict__ q, float *__restrict__ d,
                                                        const float *__restrict__ x, size_t xs,
                                                        uint32_t n, uint32_t qb, uint32_t T) {
    const uint32_t nb = n / qb;
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)T * nb)
        return;
    const uint32_t t = (uint32_t)(i / nb), b = (uint32_t)(i % nb);
    const float *v = x + (size_t)t * xs + (size_t)b * qb;
    int8_t *qq = q + (size_t)t * n + (size_t)b * qb;
    float amax = 0.0f;
    int nan = 0;
    for (uint32_t k = 0; k < qb; k++) {
        nan |= v[k] != v[k];
        amax = fmaxf(amax, fabsf(v[k]));
    }
    const bool zero = zero_block(amax, nan);
    float dv = 0.0f, id = 0.0f;
    if (!zero) {
        dv = amax / 127.0f;
        id = 127.0f / amax;
    }
    for (uint32_t k = 0; k < qb; k++)
        qq[k] = zero ? 0 : (int8_t)q1(v[k], id);
    d[i] = dv;
}

/* The quantizer under a directed rounding mode (rm 1 upward, 2 downward, 3
 * toward zero): one thread a block, the reference's loop; the divisions
 * from their nearest quotients (div_dir), the product and ref's rintf in
 * the hardware's mode. The host entry launches it when the calling
 * thread's mode is not to nearest. */
__global__ __launch_bounds__(256) void quant_directed_kernel(int8_t *__restrict__ q, float *__restrict__ d,
                                                             const float *__restrict__ x, size_t xs, uint32_t n,
                                                             uint32_t qb, uint32_t T, int rm) {
    const uint32_t nb = n / qb;
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)T * nb)
        return;
    const uint32_t t = (uint32_t)(i / nb), b = (uint32_t)(i % nb);
    const float *v = x + (size_t)t * xs + (size_t)b * qb;
    int8_t *qq = q + (size_t)t * n + (size_t)b * qb;
    float amax = 0.0f;
    int nan = 0;
    for (uint32_t k = 0; k < qb; k++) {
        nan |= v[k] != v[k];
        amax = fmaxf(amax, fabsf(v[k]));
    }
    if (zero_block(amax, nan)) {
        for (uint32_t k = 0; k < qb; k++)
            qq[k] = 0;
        d[i] = 0.0f;
        return;
    }
    /* the divisions to nearest and corrected; then the mode for the rest */
    float id = div_dir(127.0f, amax, rm), dv = div_dir(amax, 127.0f, rm);
    asm volatile("" : "+v"(id), "+v"(dv));
    __builtin_amdgcn_s_setreg(2049, __builtin_amdgcn_readfirstlane(rm));    /* MODE.FP_ROUND, single */
    asm volatile("" : "+v"(id));
    for (uint32_t k = 0; k < qb; k++)
        qq[k] = (int8_t)((int)ref_rintf(v[k] * id) & 0xff);
    d[i] = dv;
}

int launch_quantize_directed(int8_t *q, float *d, const float *x, size_t xs, uint32_t n, uint32_t qb, uint32_t T,
                             int rm, hipStream_t s, const char **name) {
    if (T == 0)
        return 0;
    if (rm < 1 || rm > 3 || qb == 0 || n % qb)
        return -2;
    const uint64_t blocks = (uint64_t)T * (n / qb);
    quant_directed_kernel<<<(uint32_t)((blocks + 255) / 256), 256, 0, s>>>(q, d, x, xs, n, qb, T, rm);
    *name = "quant_directed";
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

/* One wave a column of n <= 4096 inputs, four columns a workgroup (the
 * quantizes of up to 5-9M inputs, where the kernel is one memory round
 * trip and wants its loads spread over the most CUs). */
/* What a quantize does to its inputs first: nothing, or SiLU (the feed-
 * forward's hidden activations, core/encoder.c:147-156). */
/* A quantize reads each input once: non-temporal loads keep them from
 * pushing the products' weights and activations out of the caches (the
 * 24-layer chain at 7500 frames: 11.43 -> 11.09 ms). */
typedef float v4f_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ntload4(const float4 *p) {
    const v4f_nt t = __builtin_nontemporal_load((const v4f_nt *)p);
    return make_float4(t.x, t.y, t.z, t.w);
}

template <int OP>
__device__ __forceinline__ float4 quant_in(float4 v) {
    if constexpr (OP == kOpSilu)
        return make_float4(pk_silu(v.x), pk_silu(v.y), pk_silu(v.z), pk_silu(v.w));
    else
        return v;
}

template <int CH, bool PACK, int QB, int OP = kOpPlain>
__global__ __launch_bounds__(256) void quant_wave_kernel(int8_t *__restrict__ q, int8_t *__restrict__ qp,
                                                         float *__restrict__ d, const float *__restrict__ x,
                                                         size_t xs, uint32_t n, uint32_t T) {
    const int lane = threadIdx.x & 63;
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T)
        return;
    const uint32_t n4 = n >> 2;
    const float4 *xr = (const float4 *)(x + (size_t)t * xs);
    float4 v[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        v[c] = i < n4 ? quant_in<OP>(ntload4(xr + i)) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const WaveScales<CH, QB> sc(v);
    int *qr = (int *)(q + (size_t)t * n);
    const uint32_t G = (T + 15) / 16, g = t >> 4, r = t & 15;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        const int cb = QB ? c : 0;
        if (i < n4) {
            const int v4 = sc.zero[cb] ? 0 : pack4(v[c], sc.id[cb]);
            if (!PACK || q)
                qr[i] = v4;
            if (PACK) {
                const uint32_t k = 4 * i;
                *(int *)(qp + ((size_t)(k >> 6) * G + g) * kUnitBytes + in_unit(k, r)) = v4;
            }
            if (QB && (i & (QB / 4 - 1)) == 0)
                d[(size_t)t * (n / QB) + (4 * i) / QB] = sc.dv[cb];
        }
    }
    if (QB == 0 && lane == 0)
        d[t] = sc.dv[0];
}

/* Blocks of QB inputs over wide columns (n > 1024): a wave a 1024-input
 * chunk of a column (S chunks a column), so a product's worth of columns
 * spreads over S times the waves; a block never straddles chunks, so each
 * wave's scales are its own. Writes the packed copy (and q when set) and d
 * as quant_wave_kernel does. */
template <int QB, int OP>
__global__ __launch_bounds__(256) void quant_chunk_kernel(int8_t *__restrict__ q, int8_t *__restrict__ qp,
                                                          float *__restrict__ d, const float *__restrict__ x,
                                                          size_t xs, uint32_t n, uint32_t T, uint32_t S) {
    static_assert(QB == 32 || QB == 64, "blocks within a chunk");
    const int lane = threadIdx.x & 63;
    const uint32_t w = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t t = w / S, i0 = (w % S) * 256;
    if (t >= T)
        return;
    const uint32_t n4 = n >> 2;
    const float4 *xr = (const float4 *)(x + (size_t)t * xs);
    float4 v[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t i = i0 + lane + 64 * c;
        v[c] = i < n4 ? quant_in<OP>(ntload4(xr + i)) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const WaveScales<4, QB> sc(v);
    int *qr = (int *)(q + (size_t)t * n);
    const uint32_t G = (T + 15) / 16, g = t >> 4, r = t & 15;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t i = i0 + lane + 64 * c;
        if (i < n4) {
            const int v4 = sc.zero[c] ? 0 : pack4(v[c], sc.id[c]);
            if (q)
                qr[i] = v4;
            const uint32_t k = 4 * i;
            *(int *)(qp + ((size_t)(k >> 6) * G + g) * kUnitBytes + in_unit(k, r)) = v4;
            if ((i & (QB / 4 - 1)) == 0)
                d[(size_t)t * (n / QB) + (4 * i) / QB] = sc.dv[c];
        }
    }
}

/* The packed copy of 5-9M inputs and more: half a 16-column group a
 * workgroup, 8 columns, a wave each quantizing its column as
 * quant_wave_kernel does (512 threads, so two workgroups fit a CU and one's
 * loads run under the other's stores). Workgroup b takes group b / 2,
 * columns 8 (b % 2) .. + 7; their bytes meet in LDS, and each quarter of
 * each unit holds the 8 columns' 16-byte pieces side by side, so the
 * workgroup writes whole 128-byte lines with 16-byte stores (7500 x 4096:
 * a whole group a 1024-thread workgroup 32.2 us, this 27.7 us, a quarter
 * group of half lines 30.9 us; 4-byte stores, quant_wave_kernel's, are
 * slower still at these sizes, which are bound by HBM). The stores are
 * ordinary ones: the product that reads the copy next finds it in the
 * memory-side cache (a layer of ten minutes of audio took 2% longer with
 * non-temporal stores). Columns past T are written as zero rows. */
template <int CH, int QB, int OP = kOpPlain>
__global__ __launch_bounds__(512) void quant_group_kernel(int8_t *__restrict__ q, int8_t *__restrict__ qp,
                                                          float *__restrict__ d, const float *__restrict__ x,
                                                          size_t xs, uint32_t n, uint32_t T) {
    __shared__ __attribute__((aligned(16))) int8_t units[CH * 4 * kUnitBytes / 2];
    const int lane = threadIdx.x & 63, rr = threadIdx.x >> 6;
    const uint32_t g = blockIdx.x >> 1, h = blockIdx.x & 1, G = (T + 15) / 16, t = 16 * g + 8 * h + rr;
    const uint32_t n4 = n >> 2, nw = 16 * ((n + 63) / 64);     /* 4-byte words a frame's units hold */
    const bool live = t < T;
    const float4 *xr = (const float4 *)(x + (size_t)(live ? t : 0) * xs);
    float4 v[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        v[c] = live && i < n4 ? quant_in<OP>(ntload4(xr + i)) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const WaveScales<CH, QB> sc(v);
    int *qr = (int *)(q + (size_t)t * n);
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        const int cb = QB ? c : 0;
        if (i < nw) {
            const bool in = live && i < n4;
            const int v4 = !in || sc.zero[cb] ? 0 : pack4(v[c], sc.id[cb]);
            /* piece (unit k / 64, quarter (k / 16) % 4, column rr) */
            const uint32_t k = 4 * i;
            *(int *)(units + (((k >> 6) * 4 + ((k >> 4) & 3)) * 8 + rr) * 16 + (k & 15)) = v4;
            if (in && q)
                qr[i] = v4;
            if (QB && in && (i & (QB / 4 - 1)) == 0)
                d[(size_t)t * (n / QB) + (4 * i) / QB] = sc.dv[cb];
        }
    }
    if (QB == 0 && live && lane == 0)
        d[t] = sc.dv[0];
    __syncthreads();
    /* 32 pieces a unit: quarter w / 8, column 8 h + w % 8 of the group */
    for (uint32_t j = threadIdx.x; j < 2 * nw; j += 512) {
        const uint32_t u = j >> 5, w = j & 31;
        const v4i val = *(const v4i *)(units + 16 * j);
        *(v4i *)(qp + ((size_t)u * G + g) * kUnitBytes + ((w >> 3) * 16 + 8 * h + (w & 7)) * 16) = val;
    }
}

/* The packed quantize's kernel by size: one wave a column below a number of
 * inputs, one workgroup a half group from there. The crossover, measured on
 * inputs the caches no longer hold, falls with the width: 1024 wide, 4.4M
 * inputs are sooner the first way and 5.9M the second; 4096 wide, 7.8M the
 * first and 11.7M the second. */
inline bool group_quantize(uint32_t n, uint32_t T) {
    return (uint64_t)T * n >= (n > 1024 ? 9ull << 20 : 5ull << 20);
}
static int g_quant_kernel = -1;

int set_quant_kernel(int kind) {
    const int was = g_quant_kernel;
    g_quant_kernel = kind < 0 || kind > 2 ? -1 : kind;
    return was;
}

template <int OP>
static int launch_quantize_packed_op(int8_t *q, int8_t *qp, float *d, const float *x, size_t xs, uint32_t n,
                                     uint32_t qb, uint32_t T, hipStream_t s, const char **name) {
    const uint32_t n4 = n / 4;
    const bool small = n4 <= 256;
    const bool group = g_quant_kernel < 0 ? group_quantize(n, T) : g_quant_kernel == 1;
    /* 2: one wave a whole column also where the column is wide and in blocks */
    const bool wide = !small && !group && g_quant_kernel != 2;
#define PK_QP(CH, QB, NAME)                                                                       \
    do {                                                                                          \
        if (group) {                                                                              \
            quant_group_kernel<CH, QB, OP><<<2 * ((T + 15) / 16), 512, 0, s>>>(q, qp, d, x, xs, n, T);   \
            *name = OP ? "quant_group_packed_silu" NAME : "quant_group_packed" NAME;                                                    \
        } else {                                                                                  \
            quant_wave_kernel<CH, true, QB, OP><<<(T + 3) / 4, 256, 0, s>>>(q, qp, d, x, xs, n, T);  \
            *name = OP ? "quant_wave_packed_silu" NAME : "quant_wave_packed" NAME;                                                     \
        }                                                                                         \
    } while (0)
    if (qb == n) {
        if (small) PK_QP(4, 0, "<4>"); else PK_QP(16, 0, "<16>");
    } else if (wide) {
        /* wide columns in blocks: a wave a 1024-input chunk */
        const uint32_t S = (n4 + 255) / 256;
        const uint32_t grid = (uint32_t)(((uint64_t)T * S + 3) / 4);
        if (qb == 32)
            quant_chunk_kernel<32, OP><<<grid, 256, 0, s>>>(q, qp, d, x, xs, n, T, S);
        else
            quant_chunk_kernel<64, OP><<<grid, 256, 0, s>>>(q, qp, d, x, xs, n, T, S);
        *name = OP ? (qb == 32 ? "quant_chunk_packed_silu<qb32>" : "quant_chunk_packed_silu<qb64>")
                   : (qb == 32 ? "quant_chunk_packed<qb32>" : "quant_chunk_packed<qb64>");
    } else if (qb == 32) {
        if (small) PK_QP(4, 32, "<4,qb32>"); else PK_QP(16, 32, "<16,qb32>");
    } else {
        if (small) PK_QP(4, 64, "<4,qb64>"); else PK_QP(16, 64, "<16,qb64>");
    }
#undef PK_QP
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

int launch_quantize_packed(int8_t *q, int8_t *qp, float *d, const float *x, size_t xs, uint32_t n,
                           uint32_t qb, uint32_t T, hipStream_t s, const char **name, int op) {
    if (T == 0)
        return 0;
    const uint32_t n4 = n / 4;
    if (n4 > 1024 || !(qb == n || qb == 32 || qb == 64) || (op != kOpPlain && op != kOpSilu))
        return -2;
    if (op == kOpSilu)
        return launch_quantize_packed_op<kOpSilu>(q, qp, d, x, xs, n, qb, T, s, name);
    return launch_quantize_packed_op<kOpPlain>(q, qp, d, x, xs, n, qb, T, s, name);
}

int launch_quantize(int8_t *q, float *d, const float *x, size_t xs, uint32_t n, uint32_t qb,
                    uint32_t T, hipStream_t s, const char **name) {
    if (T == 0)
        return 0;
    const uint32_t nch = n / 16, n4 = n / 4, grid4 = (T + 3) / 4;
    if (qb == n && n4 <= 256) {
        quant_wave_kernel<4, false, 0><<<grid4, 256, 0, s>>>(q, nullptr, d, x, xs, n, T);
        *name = "quant_wave<4>";
    } else if (qb == n && n4 <= 1024) {
        quant_wave_kernel<16, false, 0><<<grid4, 256, 0, s>>>(q, nullptr, d, x, xs, n, T);
        *name = "quant_wave<16>";
    } else if ((qb == 32 || qb == 64) && n4 <= 1024) {
        if (qb == 32) {
            if (n4 <= 256) quant_wave_kernel<4, false, 32><<<grid4, 256, 0, s>>>(q, nullptr, d, x, xs, n, T);
            else quant_wave_kernel<16, false, 32><<<grid4, 256, 0, s>>>(q, nullptr, d, x, xs, n, T);
            *name = "quant_wave<qb32>";
        } else {
            if (n4 <= 256) quant_wave_kernel<4, false, 64><<<grid4, 256, 0, s>>>(q, nullptr, d, x, xs, n, T);
            else quant_wave_kernel<16, false, 64><<<grid4, 256, 0, s>>>(q, nullptr, d, x, xs, n, T);
            *name = "quant_wave<qb64>";
        }
    } else if (qb == n && nch <= 1024) {
        quant_col_kernel<4, 4><<<T, 256, 0, s>>>(q, d, x, xs, n);
        *name = "quant_col<4,4>";
    } else {
        const uint32_t g = qb / 16;
        const uint64_t total = (uint64_t)T * nch;
        const uint32_t grid = (uint32_t)((total + 255) / 256);
        switch (g) {
#define PK_G(G)                                                                    \
    case G:                                                                        \
        quant_blk_kernel<G><<<grid, 256, 0, s>>>(q, d, x, xs, n, T);               \
        *name = "quant_blk<" #G ">";                                               \
        break;
            PK_G(2) PK_G(4) PK_G(8) PK_G(16) PK_G(32) PK_G(64)
#undef PK_G
        default: {
            const uint64_t blocks = (uint64_t)T * (n / qb);
            quant_any_kernel<<<(uint32_t)((blocks + 255) / 256), 256, 0, s>>>(q, d, x, xs, n, qb, T);
            *name = "quant_any";
        }
        }
    }
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

/* -------------------------------------------------------------- repack --
 *
 * PK_Q8 (core/pkf.h:28-41: q(r, k) at ((r/16)(cols/4) + k/4) 64 + (r%16) 4 +
 * k%4) into units (q8_internal.h), stage-major: unit (p, u) of panel p and
 * inputs [64 u, 64 u + 64) at byte 1024 (u panels + p). One thread a 16-byte
 * lane slot. */
__global__ __launch_bounds__(256) void repack_kernel(int8_t *__restrict__ dst,
                                                     const int8_t *__restrict__ src,
                                                     uint32_t panels, uint32_t cols, uint32_t ku) {
    const uint64_t slot = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (slot >= (uint64_t)panels * ku * 64)
        return;
    const uint32_t lane = (uint32_t)(slot & 63);
    const uint64_t unit = slot >> 6;                 /* u * panels + p */
    const uint32_t u = (uint32_t)(unit / panels), p = (uint32_t)(unit % panels);
    const uint32_t r = lane & 15, kq = lane >> 4;
    const uint32_t k0 = u * 64 + kq * 16;
    int o[4];
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const uint32_t k = k0 + 4 * g;
        o[g] = k < cols ? *(const int *)(src + ((size_t)p * (cols / 4) + k / 4) * 64 + r * 4) : 0;
    }
    *(v4i *)(dst + slot * 16) = v4i{o[0], o[1], o[2], o[3]};
}

int launch_repack(int8_t *dst, const int8_t *src, uint32_t rows, uint32_t cols, hipStream_t s) {
    const uint32_t panels = rows / 16, ku = units_per_panel(cols);
    const uint64_t slots = (uint64_t)panels * ku * 64;
    if (slots == 0)
        return 0;
    repack_kernel<<<(uint32_t)((slots + 255) / 256), 256, 0, s>>>(dst, src, panels, cols, ku);
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

/* ------------------------------------------------------------- product --
 *
 * out[t * os + r] (backend/kernels.h:60-78):
 *   acc = 0; per block b in order: s = exact int32 sum, acc = fmaf((float)s, d[t][b], acc)
 *   v = acc * ws[r]; if bias: v = v + bias[r]; out = add ? out + v : v
 *
 * The MFMA is v_mfma_i32_16x16x64_i8 with the weights as its A operand and
 * the activations as its B: a 16x16 tile's lane l holds output row (frame)
 * t = l % 16 and the four consecutive channels r = 4 (l / 16) + i, so the
 * epilogue reads one scale d[t] a tile and writes a float4 a lane. Both
 * operands come from LDS in the unit layout, one ds_read_b128 a lane a
 * 16x64 fragment, lanes in address order.
 *
 * A workgroup is WN x WM waves; each wave TN x TM tiles of 16x16: the
 * workgroup's tile is 16 TN WN channels by 16 TM WM frames. Inputs move in
 * stages of 64, double-buffered through LDS: each thread loads its share of
 * the next stage into registers with 128-bit global loads while the MFMAs
 * run on this one, then stores it to the other buffer.
 *
 * MODE 0: one block a column (qb == n): the int32 sums run over the whole
 *         input, and the epilogue's first operation is fmaf(s, d, +0).
 * MODE 1: blocks of a multiple of 64: each block's sums are turned into the
 *         float chain at the stage that ends it.
 * MODE 2: blocks of an odd multiple of 32: the 16x16x32 MFMA on each half
 *         stage, the chain updated at every block's end.
 *
 * Rows past the matrix and frames past T are clamped to the last one when
 * loaded (and never stored); inputs past n read a column's first inputs,
 * which meet the repacked matrix's zero padding, so every load is in bounds
 * and adds nothing. */

template <int WN, int WM, int TN, int TM, int MODE>
__device__ __forceinline__ void gemm_tile(const GemmArgs &g, const Seg &sg, uint32_t tn, uint32_t tm) {
    constexpr int NW = WN * WM;
    constexpr int BN = 16 * TN * WN, BM = 16 * TM * WM;
    constexpr int UB = BN / 16, UA = BM / 16, UNITS = UA + UB;
    static_assert(UNITS % NW == 0, "each wave loads whole units");
    constexpr int LPW = UNITS / NW;
    constexpr int FN = MODE == 0 ? 1 : TN, FM = MODE == 0 ? 1 : TM;
    __shared__ __attribute__((aligned(16))) int8_t lds[2][UNITS * kUnitBytes];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wn = wave % WN, wm = wave / WN;
    const uint32_t T = sg.T;
    const uint32_t n0 = tn * BN, m0 = tm * BM;
    const uint32_t npan = g.rows >> 4;
    const uint32_t n = g.n, ku = g.ku, kr = g.kr;

    if (g.rmode)
        __builtin_amdgcn_s_setreg(2049, g.rmode);    /* MODE.FP_ROUND, single precision */

    /* this thread's load slots: units [wave * LPW, wave * LPW + LPW) of a stage,
     * the weight units first */
    const int8_t *src[LPW];
    bool isw[LPW];
#pragma unroll
    for (int s = 0; s < LPW; s++) {
        const int u = wave * LPW + s;
        if (u < UB) {
            uint32_t p = n0 / 16 + u;
            p = p < npan ? p : npan - 1;
            src[s] = g.w + (size_t)p * kUnitBytes + lane * 16;
            isw[s] = true;
        } else {
            uint32_t row = m0 + (u - UB) * 16 + (lane & 15);
            row = row < T ? row : T - 1;
            src[s] = sg.q + (size_t)row * n;
            isw[s] = false;
        }
    }

    v4i stage[LPW];
    auto gload = [&](uint32_t kt) {
#pragma unroll
        for (int s = 0; s < LPW; s++) {
            if (isw[s]) {
                stage[s] = *(const v4i *)(src[s] + (size_t)kt * g.wstride);
            } else {
                /* inputs past n: the row's first 16, against zero weights */
                const uint32_t k = kt * 64 + (lane >> 4) * 16;
                stage[s] = *(const v4i *)(src[s] + (k < n ? k : 0));
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int s = 0; s < LPW; s++)
            *(v4i *)(&lds[buf][(wave * LPW + s) * kUnitBytes + lane * 16]) = stage[s];
    };

    v4i acc[TN][TM];
    float accf[FN][FM][4];
#pragma unroll
    for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++)
            acc[i][j] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
        for (int j = 0; j < FM; j++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                accf[i][j][r] = 0.0f;

    /* this lane's frame in each tile column j, clamped for the loads */
    uint32_t tj[TM];
#pragma unroll
    for (int j = 0; j < TM; j++) {
        const uint32_t t = m0 + (wm * TM + j) * 16 + (lane & 15);
        tj[j] = t < T ? t : T - 1;
    }

    /* block b's sums into the float chain (ref's acc = fmaf((float)s, d, acc)),
     * and the sums back to zero */
    auto chain = [&](uint32_t b) {
        if (MODE != 0) {
#pragma unroll
            for (int j = 0; j < TM; j++) {
                const float dt = sg.d[(size_t)tj[j] * g.nb + b];
#pragma unroll
                for (int i = 0; i < TN; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        float &f = accf[MODE == 0 ? 0 : i][MODE == 0 ? 0 : j][r];
                        f = __builtin_fmaf((float)acc[i][j][r], dt, f);
                        acc[i][j][r] = 0;
                    }
            }
        }
    };

    gload(0);
    lstore(0);
    __syncthreads();
    for (uint32_t kt = 0; kt < kr; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < kr)
            gload(kt + 1);
        const int8_t *lb = &lds[cur][0];
        if (MODE != 2) {
            v4i wf[TN], af[TM];
#pragma unroll
            for (int i = 0; i < TN; i++)
                wf[i] = *(const v4i *)(lb + (wn * TN + i) * kUnitBytes + lane * 16);
#pragma unroll
            for (int j = 0; j < TM; j++)
                af[j] = *(const v4i *)(lb + (UB + wm * TM + j) * kUnitBytes + lane * 16);
#pragma unroll
            for (int i = 0; i < TN; i++)
#pragma unroll
                for (int j = 0; j < TM; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[i], af[j], acc[i][j], 0, 0, 0);
            if (MODE == 1) {
                const uint32_t kend = (kt + 1) * 64;
                if (kend <= n && kend % g.qb == 0)
                    chain(kend / g.qb - 1);
            }
        } else {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                /* half h of the stage: 32 inputs, 8 bytes a lane, the same
                 * bytes of both operands */
                const int off = ((2 * h + (lane >> 5)) * 16 + (lane & 15)) * 16 + ((lane >> 4) & 1) * 8;
                long wf[TN], af[TM];
#pragma unroll
                for (int i = 0; i < TN; i++)
                    wf[i] = *(const long *)(lb + (wn * TN + i) * kUnitBytes + off);
#pragma unroll
                for (int j = 0; j < TM; j++)
                    af[j] = *(const long *)(lb + (UB + wm * TM + j) * kUnitBytes + off);
#pragma unroll
                for (int i = 0; i < TN; i++)
#pragma unroll
                    for (int j = 0; j < TM; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wf[i], af[j], acc[i][j], 0, 0, 0);
                const uint32_t kend = kt * 64 + 32 * (h + 1);
                if (kend <= n && kend % g.qb == 0)
                    chain(kend / g.qb - 1);
            }
        }
        if (kt + 1 < kr)
            lstore(cur ^ 1);
        __syncthreads();
    }

    /* the epilogue: ref's operations in ref's order, four channels a lane */
    const bool vec = ((sg.os & 3) == 0) && ((((uintptr_t)sg.out) & 15) == 0);
#pragma unroll
    for (int j = 0; j < TM; j++) {
        const uint32_t t = m0 + (wm * TM + j) * 16 + (lane & 15);
        if (t >= T)
            continue;
        const float dt = MODE == 0 ? sg.d[t] : 0.0f;
#pragma unroll
        for (int i = 0; i < TN; i++) {
            const uint32_t c = n0 + (wn * TN + i) * 16 + (lane >> 4) * 4;
            if (c >= g.rows)
                continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float a = MODE == 0 ? __builtin_fmaf((float)acc[i][j][r], dt, 0.0f)
                                          : accf[MODE == 0 ? 0 : i][MODE == 0 ? 0 : j][r];
                v[r] = a * g.ws[c + r];
                if (g.bias)
                    v[r] = v[r] + g.bias[c + r];
            }
            float *o = sg.out + (size_t)t * sg.os + c;
            if (vec) {
                float4 ov = make_float4(v[0], v[1], v[2], v[3]);
                if (g.add) {
                    const float4 old = *(const float4 *)o;
                    ov.x = old.x + ov.x;
                    ov.y = old.y + ov.y;
                    ov.z = old.z + ov.z;
                    ov.w = old.w + ov.w;
                }
                store_out4(o, ov, g.plain);
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    store_out1(o + r, g.add ? o[r] + v[r] : v[r], g.plain);
            }
        }
    }
}

/* One product: tiles with channels fastest, so neighbouring workgroups share
 * their frames' inputs. */
template <int WN, int WM, int TN, int TM, int MODE>
__global__ __launch_bounds__(64 * WN * WM) void gemm_q8_kernel(GemmArgs g, Seg sg, uint32_t tiles_n) {
    gemm_tile<WN, WM, TN, TM, MODE>(g, sg, blockIdx.x % tiles_n, blockIdx.x / tiles_n);
}

/* A grouped product: the segments' frame tiles one after another, each
 * workgroup finding its segment in the table. */
template <int WN, int WM, int TN, int TM, int MODE>
__global__ __launch_bounds__(64 * WN * WM) void gemm_q8_grouped_kernel(GemmArgs g, SegTable tab,
                                                                       uint32_t tiles_n) {
    const uint32_t tm = blockIdx.x / tiles_n;
    uint32_t i = 0;
    while (i + 1 < tab.nseg && tab.s[i + 1].tile0 <= tm)
        i++;
    gemm_tile<WN, WM, TN, TM, MODE>(g, tab.s[i], blockIdx.x % tiles_n, tm - tab.s[i].tile0);
}

/* The skinny product, a few frames (T <= 16): bound by streaming the weights
 * once. A workgroup takes one 16-row panel; its KW waves split the panel's
 * units between them, each reading its weight units straight from HBM (1 KB
 * contiguous a wave a unit) and the frames' inputs from L2, and their int32
 * sums meet in LDS. Per-row blocks only (MODE 0).
 *
 * SPLIT: S workgroups share a panel, each taking a run of its units (so a
 * product of few panels still spreads its weights over many CUs). Each writes
 * its exact int32 sums to the workspace's partials (agent-scope stores) and,
 * once they are written, counts itself in at the panel's counter; the last
 * one in reads the S partials back (agent-scope loads), adds them (integer
 * sums: the same bits in any order), zeroes the counter for the next call,
 * and runs ref's epilogue once. Workgroup b takes panel b % P8 (P8 the panels
 * rounded up to 8) and split b / P8, so a panel's splits share an XCD (the
 * hardware deals workgroup b to XCD b % 8) and meet in its L2. */
template <int KW, bool PACKED, bool SPLIT>
__global__ __launch_bounds__(64 * KW) void gemm_q8_skinny_kernel(GemmArgs g, Seg sg, uint32_t S, uint32_t P8,
                                                                 int32_t *part, uint32_t *cnt) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t p = SPLIT ? blockIdx.x % P8 : blockIdx.x, si = SPLIT ? blockIdx.x / P8 : 0;
    const uint32_t n = g.n, kr = g.kr, T = sg.T;
    if (SPLIT && p >= g.rows / 16)
        return;                                 /* padding up to a multiple of 8 panels */
    const uint32_t ulo = SPLIT ? si * kr / S : 0, uhi = SPLIT ? (si + 1) * kr / S : kr;
    if (g.rmode)
        __builtin_amdgcn_s_setreg(2049, g.rmode);
    const int8_t *wp = g.w + (size_t)p * kUnitBytes + lane * 16;
    const size_t ws_ = g.wstride;
    uint32_t row = lane & 15;
    row = row < T ? row : T - 1;
    /* packed: the frames are one group, unit u at qstride u, lane-ordered */
    const int8_t *ap = PACKED ? sg.q + lane * 16 : sg.q + (size_t)row * n;
    /* the epilogue's operands (wave 0's lanes of frames < T), loaded first
     * so that they arrive with the units */
    const uint32_t t = lane & 15, c = p * 16 + (lane >> 4) * 4;
    float *o = sg.out + (size_t)t * sg.os + c;
    float dt = 0.0f, wsr[4] = { 0, 0, 0, 0 }, br[4] = { 0, 0, 0, 0 }, old[4] = { 0, 0, 0, 0 };
    if (wave == 0 && t < T) {
        dt = sg.d[t];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            wsr[r] = g.ws[c + r];
            if (g.bias)
                br[r] = g.bias[c + r];
            if (g.add)
                old[r] = o[r];
        }
    }
    /* the wave's units u = ulo + wave + KW i, CU of them loaded at once
     * (every load of a batch issued before its first MFMA: one memory round
     * trip a batch, one batch for K <= 64 CU KW inputs); two accumulators so
     * that consecutive MFMAs do not wait on each other (exact int32 sums).
     * The weights, read once a call, load non-temporally: 8-11% sooner from
     * HBM (weights rotated over > 512 MB), the same when they are cached. */
    constexpr int CU = 8;
    v4i acc[2] = { { 0, 0, 0, 0 }, { 0, 0, 0, 0 } };
    for (uint32_t u0 = ulo + wave; u0 < uhi; u0 += CU * KW) {
        v4i wv[CU], av[CU];
#pragma unroll
        for (int i = 0; i < CU; i++) {
            const uint32_t u = u0 + i * KW;
            if (u < uhi) {
                const uint32_t k = u * 64 + (lane >> 4) * 16;
                wv[i] = __builtin_nontemporal_load((const v4i *)(wp + (size_t)u * ws_));
                av[i] = *(const v4i *)(ap + (PACKED ? (size_t)u * sg.qstride : (k < n ? k : 0)));
            }
        }
#pragma unroll
        for (int i = 0; i < CU; i++)
            if (u0 + i * KW < uhi)
                acc[i & 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv[i], av[i], acc[i & 1], 0, 0, 0);
    }
    __shared__ v4i red[KW][64];
    red[wave][lane] = acc[0] + acc[1];
    __syncthreads();
    if (wave != 0)
        return;
    v4i s = red[0][lane];
#pragma unroll
    for (int w = 1; w < KW; w++)
        s += red[w][lane];
    if constexpr (SPLIT) {
        int32_t *mine = part + ((size_t)p * kMaxSplit + si) * 256 + lane * 4;
#pragma unroll
        for (int r = 0; r < 4; r++)
            __hip_atomic_store(mine + r, s[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        /* the partial has reached the coherence point before the count */
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        uint32_t before = 0;
        if (lane == 0)
            before = __hip_atomic_fetch_add(cnt + p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        before = __builtin_amdgcn_readfirstlane(before);
        if (before != S - 1)
            return;
        asm volatile("" ::: "memory");
        const int32_t *all = part + (size_t)p * kMaxSplit * 256 + lane * 4;
        v4i tot = { 0, 0, 0, 0 };
        for (uint32_t k = 0; k < S; k++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                tot[r] += __hip_atomic_load(all + k * 256 + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0)
            __hip_atomic_store(cnt + p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s = tot;
    }
    if (t >= T)
        return;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float v = __builtin_fmaf((float)s[r], dt, 0.0f) * wsr[r];
        if (g.bias)
            v = v + br[r];
        store_out1(o + r, g.add ? old[r] + v : v, g.plain);
    }
}

static int g_forced_split = -1;

int set_skinny_split(int s) {
    const int was = g_forced_split;
    g_forced_split = s >= 1 && s <= (int)kMaxSplit ? s : -1;
    return was;
}

size_t skinny_workspace_bytes(uint32_t rows) {
    const size_t panels = rows / 16;
    return ((panels * 4 + 255) & ~(size_t)255) + panels * kMaxSplit * 1024;
}

/* How many workgroups share a panel. The hand-off through the workspace
 * (agent-scope stores, the counter, the last one's loads) costs ~1.5-2 us, so
 * a split pays only where one CU would stream a lot: measured (weights from
 * HBM, each launch alone), 16 frames: K = 4096 5.2 us whole against 5.7 at
 * two splits (1024 rows), K = 8192 8.2 against 6.3 at four (512 rows), K =
 * 16384 14.2-14.8 against 7.6-8.9 at four; one frame: K = 4096 3.8 against
 * 5.1 / 6.0 / 8.2 at two / four / eight, K = 16384 7.6-8.3 against 6.2-8.0 at
 * four. So: the bytes a panel's workgroup streams (its weight units, and its
 * frames' inputs from L2) at 192 KB or more take four splits, fewer take
 * none (forced: any count up to one a unit). */
static uint32_t skinny_splits(uint32_t panels, uint32_t kr, uint32_t T) {
    uint32_t s;
    if (g_forced_split > 0) {
        s = (uint32_t)g_forced_split;
    } else {
        const uint64_t per = (uint64_t)kr * 1024 * (16 + (T < 16 ? T : 16)) / 16;
        s = per >= (192u << 10) && panels * 4 <= 512 ? 4 : 1;
        if (s > kr / 2)
            s = 1;
    }
    if (s > kr)
        s = kr;
    if (s > kMaxSplit)
        s = kMaxSplit;
    return s < 1 ? 1 : s;
}

/* ----------------------------------------------- the pipelined product --
 *
 * MODE 0 (a block a column) with its loads in flight several stages ahead:
 * each stage's units go straight from global memory into LDS
 * (global_load_lds_dwordx4: a wave's 64 lanes write 1 KB, lane l at byte
 * 16 l, which is the unit layout), into a ring of four slots. At stage kt
 * a thread waits until its own loads of stage kt have landed (vmcnt counts
 * its later stages still in flight), the workgroup meets at a barrier, the
 * loads of stage kt + 3 go into the slot stage kt - 1 used, and the MFMAs
 * run on slot kt. Three stages are in flight while one is multiplied. The
 * slots are four distinct LDS arrays and the loop is unrolled by four, so
 * the compiler sees which slot each read and each load touches. */

/* A stage is UPS units of inputs (64 UPS of K) for the tile's UB weight
 * panels and UA frame groups: slot layout [kk < UPS][unit < UA + UB], 1 KB a
 * unit. Within a stage the fragments of sub-step kk + 1 are read while the
 * MFMAs of sub-step kk run (two register sets). */
template <int WN, int WM, int TN, int TM, int UPS, bool PACKED>
__device__ __forceinline__ void ring_tile(const GemmArgs &g, const Seg &sg, uint32_t tn, uint32_t tm) {
    constexpr int NW = WN * WM;
    constexpr int BN = 16 * TN * WN, BM = 16 * TM * WM;
    constexpr int UB = BN / 16, UA = BM / 16, UNITS = UA + UB;
    constexpr int SLOTU = UNITS * UPS;
    static_assert(SLOTU % NW == 0, "each wave loads whole units");
    constexpr int L = SLOTU / NW;
    static_assert(2 * L < 64, "the stages in flight fit vmcnt");
    constexpr int SLOT = SLOTU * kUnitBytes;
    static_assert(4 * SLOT <= 160 * 1024, "four slots fit a CU's LDS");
    constexpr int R = TN + TM;
    __shared__ __attribute__((aligned(1024))) int8_t s0[SLOT], s1[SLOT], s2[SLOT], s3[SLOT];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   /* uniform: scalar */
    const int wn = wave % WN, wm = wave / WN;
    const uint32_t T = sg.T;
    const uint32_t n0 = tn * BN, m0 = tm * BM;
    const uint32_t npan = g.rows >> 4;
    const uint32_t n = g.n, ku = g.ku, ns = g.ku / UPS;

    if (g.rmode)
        __builtin_amdgcn_s_setreg(2049, g.rmode);    /* MODE.FP_ROUND, single precision */

    /* this thread's lane of slot units [wave L, wave L + L): sub-step kk,
     * unit u (weights first) */
    const int8_t *src[L];
    bool isw[L];
    uint32_t sub[L];
#pragma unroll
    for (int s = 0; s < L; s++) {
        const int idx = wave * L + s, kk = idx / UNITS, u = idx % UNITS;
        sub[s] = kk;
        if (u < UB) {
            uint32_t p = n0 / 16 + u;
            p = p < npan ? p : npan - 1;
            src[s] = g.w + (size_t)p * kUnitBytes + lane * 16;
            isw[s] = true;
        } else if (PACKED) {
            const uint32_t ng = (T + 15) / 16;
            uint32_t gi = m0 / 16 + (u - UB);
            gi = gi < ng ? gi : ng - 1;
            src[s] = sg.q + (size_t)gi * kUnitBytes + lane * 16;
            isw[s] = false;
        } else {
            uint32_t row = m0 + (u - UB) * 16 + (lane & 15);
            row = row < T ? row : T - 1;
            src[s] = sg.q + (size_t)row * n;
            isw[s] = false;
        }
    }
    auto issue = [&](uint32_t j, int8_t *slot) {
#pragma unroll
        for (int s = 0; s < L; s++) {
            const uint32_t unit = j * UPS + sub[s];
            const int8_t *gp;
            if (isw[s]) {
                gp = src[s] + (size_t)unit * g.wstride;
            } else if (PACKED) {
                gp = src[s] + (size_t)unit * sg.qstride;
            } else {
                /* inputs past n: the row's first 16, against zero weights */
                const uint32_t k = unit * 64 + (lane >> 4) * 16;
                gp = src[s] + (k < n ? k : 0);
            }
            __builtin_amdgcn_global_load_lds(PK_AS1(gp), PK_AS3(slot + (wave * L + s) * kUnitBytes), 16, 0, 0);
        }
    };

    v4i acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++)
            acc[i][j] = v4i{0, 0, 0, 0};

    /* The fragments are read with ds_read_b128 written out, and waited for
     * with lgkmcnt before the MFMAs take them: the compiler, which cannot
     * tell the ring's slots apart across the loop's back edge, would
     * otherwise wait for every load in flight before the first read of each
     * pass. The barrier in landed() orders these reads after the loads. */
    const uint32_t wbase = lds_addr(s0) + (wn * TN) * kUnitBytes + lane * 16;
    const uint32_t abase = lds_addr(s0) + (UB + wm * TM) * kUnitBytes + lane * 16;
    /* A sub-step's fragments are read activations first, then the weight
     * fragments in order, and the MFMAs of weight fragment i start once it
     * has landed (lgkmcnt counts the reads after it), so the LDS reads of a
     * sub-step overlap its own MFMAs. */
    v4i f[R];
    auto sub_step = [&](uint32_t at) {
#pragma unroll
        for (int j = 0; j < TM; j++)
            f[TN + j] = lds_read16(abase + at + j * kUnitBytes);
#pragma unroll
        for (int i = 0; i < TN; i++)
            f[i] = lds_read16(wbase + at + i * kUnitBytes);
        for_static<0, TN>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            wait_lgkm<(TN - 1 - i < 15 ? TN - 1 - i : 15)>();
            asm volatile("" : "+v"(f[i]));
            if (i == 0) {
#pragma unroll
                for (int j = 0; j < TM; j++)
                    asm volatile("" : "+v"(f[TN + j]));
            }
#pragma unroll
            for (int j = 0; j < TM; j++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f[i], f[TN + j], acc[i][j], 0, 0, 0);
        });
    };
    auto compute = [&](const int8_t *lb) {
        const uint32_t at = lds_addr(lb) - lds_addr(s0);
#pragma unroll
        for (int kk = 0; kk < UPS; kk++)
            sub_step(at + kk * UNITS * kUnitBytes);
    };
    /* stage kt landed in every wave: at most min(2, ns - 1 - kt) later
     * stages of this thread's loads still in flight, then the barrier */
    auto landed = [&](uint32_t kt) {
        const uint32_t later = ns - 1 - kt;
        if (later >= 2)
            wait_vm<2 * L>();
        else if (later == 1)
            wait_vm<L>();
        else
            wait_vm<0>();
        __builtin_amdgcn_s_barrier();
    };

    /* ns is a multiple of four: every pass of the loop is four whole stages */
    issue(0, s0);
    issue(1, s1);
    issue(2, s2);
    for (uint32_t kt = 0; kt < ns; kt += 4) {
        landed(kt);
        if (kt + 3 < ns)
            issue(kt + 3, s3);
        compute(s0);
        landed(kt + 1);
        if (kt + 4 < ns)
            issue(kt + 4, s0);
        compute(s1);
        landed(kt + 2);
        if (kt + 5 < ns)
            issue(kt + 5, s1);
        compute(s2);
        landed(kt + 3);
        if (kt + 6 < ns)
            issue(kt + 6, s2);
        compute(s3);
    }
    wait_vm<0>();

    /* the epilogue: ref's operations in ref's order, four channels a lane */
    const bool vec = ((sg.os & 3) == 0) && ((((uintptr_t)sg.out) & 15) == 0);
#pragma unroll
    for (int j = 0; j < TM; j++) {
        const uint32_t t = m0 + (wm * TM + j) * 16 + (lane & 15);
        if (t >= T)
            continue;
        const float dt = sg.d[t];
#pragma unroll
        for (int i = 0; i < TN; i++) {
            const uint32_t c = n0 + (wn * TN + i) * 16 + (lane >> 4) * 4;
            if (c >= g.rows)
                continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                v[r] = __builtin_fmaf((float)acc[i][j][r], dt, 0.0f) * g.ws[c + r];
                if (g.bias)
                    v[r] = v[r] + g.bias[c + r];
            }
            float *o = sg.out + (size_t)t * sg.os + c;
            if (vec) {
                float4 ov = make_float4(v[0], v[1], v[2], v[3]);
                if (g.add) {
                    const float4 old = *(const float4 *)o;
                    ov.x = old.x + ov.x;
                    ov.y = old.y + ov.y;
                    ov.z = old.z + ov.z;
                    ov.w = old.w + ov.w;
                }
                store_out4(o, ov, g.plain);
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    store_out1(o + r, g.add ? o[r] + v[r] : v[r], g.plain);
            }
        }
    }
}

/* ------------------------------------------ the software-pipelined product --
 *
 * The same stages and the same LDS DMA as ring_tile, with the fragment reads
 * moved off the MFMAs' critical path. Every wave holds two fragment sets: the
 * MFMAs of sub-step g run on one while the ds_reads of sub-step g + 1 fill the
 * other, so LDS latency and LDS read time hide under the matrix pipe's work.
 * The barrier that lets a stage's slot be read moves to the start of the
 * previous stage's last sub-step: by then every wave has read that last
 * sub-step's fragments (a sub-step ahead), so the slot of stage s is free at
 * that barrier and takes stage s + NS at once; NS - 1 stages are in flight
 * while one is multiplied. */


/* BLK: 0, a block a column (qb == n); 1, blocks of one unit (qb == 64);
 * 2, blocks of half a unit (qb == 32). With blocks, each block's exact int32
 * sum comes from MFMAs of its own (with blocks of 32, a 16x16x32 MFMA on each
 * half of the unit, its 8 bytes a lane read from LDS where the unit holds
 * them), and enters ref's chain
 * acc = fmaf((float)s, d, acc) in block order; blocks past n (padding units)
 * are skipped. The stage's block scales ride with its units: each slot ends
 * with BM frames x the stage's blocks of d, frame-contiguous, loaded by DMA
 * with the units and read a sub-step ahead with the fragments. */
template <int WN, int WM, int TN, int TM, int UPS, int NS, int KG, bool PACKED, int BLK>
__device__ __forceinline__ void pipe_tile(const GemmArgs &g, const Seg &sg, uint32_t tn, uint32_t tm) {
    constexpr int NW = WN * WM;             /* waves of one K group */
    constexpr int BN = 16 * TN * WN, BM = 16 * TM * WM;
    constexpr int UB = BN / 16, UA = BM / 16, UNITS = UA + UB;
    constexpr int SLOTU = UNITS * UPS;
    static_assert(SLOTU % NW == 0, "each wave loads whole units");
    constexpr int L = SLOTU / NW;
    constexpr int BPU = BLK == 2 ? 2 : 1, BPS = BLK ? BPU * UPS : 0;     /* blocks a unit, a stage */
    static_assert(BLK == 0 || (KG == 1 && BM % 64 == 0), "blocks: one K group, whole 64-frame chunks");
    constexpr int DCH = BLK ? BM * BPS / 64 : 0;                          /* 64-float chunks of d a stage */
    constexpr int LD = (DCH + NW - 1) / NW, LT = L + LD;                  /* loads a wave issues a stage */
    static_assert(NS >= 2 && NS <= 8, "two to eight slots");
    static_assert((NS - 1) * LT < 64, "the stages in flight fit vmcnt");
    constexpr int DB = BLK ? (BM * BPS * 4 + kUnitBytes - 1) / kUnitBytes * kUnitBytes : 0;
    constexpr int SLOT = SLOTU * kUnitBytes + DB;
    static_assert(KG * NS * SLOT <= 160 * 1024, "the slots fit a CU's LDS");
    static_assert(KG == 1 || (KG - 1) * NW * TN * TM * kUnitBytes <= KG * NS * SLOT, "the partial sums fit the rings");
    static_assert((UPS & (UPS - 1)) == 0, "a power of two units a stage");
    static_assert(NS * UPS % 2 == 0, "the steady state is whole pairs of sub-steps");
    constexpr int R = TN + TM;
    __shared__ __attribute__((aligned(1024))) int8_t rings[KG * NS * SLOT];

    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    /* K group kg takes units [kg ku / KG, (kg + 1) ku / KG) with a ring of its
     * own; its NW waves tile the workgroup's outputs as a whole group would */
    const int kg = wv / NW, wave = wv % NW;
    const int wn = wave % WN, wm = wave / WN;
    int8_t *const ring = rings + kg * NS * SLOT;
    const uint32_t T = sg.T;
    const uint32_t n0 = tn * BN, m0 = tm * BM;
    const uint32_t npan = g.rows >> 4;
    const uint32_t n = g.n, kug = g.ku / KG, u0 = kg * kug, ns = kug / UPS, nb = g.nb;

    if (g.rmode)
        __builtin_amdgcn_s_setreg(2049, g.rmode);    /* MODE.FP_ROUND, single precision */

    const int8_t *src[L];
    bool isw[L];
    uint32_t sub[L];
#pragma unroll
    for (int s = 0; s < L; s++) {
        const int idx = wave * L + s, kk = idx / UNITS, u = idx % UNITS;
        sub[s] = kk;
        if (u < UB) {
            uint32_t p = n0 / 16 + u;
            p = p < npan ? p : npan - 1;
            src[s] = g.w + (size_t)p * kUnitBytes + lane * 16;
            isw[s] = true;
        } else if (PACKED) {
            const uint32_t ng = (T + 15) / 16;
            uint32_t gi = m0 / 16 + (u - UB);
            gi = gi < ng ? gi : ng - 1;
            src[s] = sg.q + (size_t)gi * kUnitBytes + lane * 16;
            isw[s] = false;
        } else {
            uint32_t row = m0 + (u - UB) * 16 + (lane & 15);
            row = row < T ? row : T - 1;
            src[s] = sg.q + (size_t)row * n;
            isw[s] = false;
        }
    }
    auto issue = [&](uint32_t j) {
        int8_t *slot = ring + (j % NS) * SLOT;
#pragma unroll
        for (int s = 0; s < L; s++) {
            const uint32_t unit = u0 + j * UPS + sub[s];
            const int8_t *gp;
            if (isw[s]) {
                gp = src[s] + (size_t)unit * g.wstride;
            } else if (PACKED) {
                gp = src[s] + (size_t)unit * sg.qstride;
            } else {
                const uint32_t k = unit * 64 + (lane >> 4) * 16;
                gp = src[s] + (k < n ? k : 0);
            }
            __builtin_amdgcn_global_load_lds(PK_AS1(gp), PK_AS3(slot + (wave * L + s) * kUnitBytes), 16, 0, 0);
        }
        if constexpr (BLK != 0) {
            /* chunk c: block c / (BM / 64) of the stage, frames (c % (BM / 64)) * 64 + lane;
             * a wave past the last chunk loads the last one again (the same bytes) */
#pragma unroll
            for (int i = 0; i < LD; i++) {
                const int c = wave + NW * i < DCH ? wave + NW * i : DCH - 1;
                const int blk = c / (BM / 64), fc = c % (BM / 64);
                uint32_t f = m0 + fc * 64 + lane;
                f = f < T ? f : T - 1;
                uint32_t bi = (u0 + j * UPS) * BPU + blk;
                bi = bi < nb ? bi : nb - 1;
                __builtin_amdgcn_global_load_lds(PK_AS1(sg.d + (size_t)f * nb + bi),
                                                 PK_AS3(slot + SLOTU * kUnitBytes + (blk * BM + fc * 64) * 4), 4, 0, 0);
            }
        }
    };

    v4i acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++)
            acc[i][j] = v4i{0, 0, 0, 0};
    float4 accf[BLK ? TN : 1][BLK ? TM : 1];
#pragma unroll
    for (int i = 0; i < (BLK ? TN : 1); i++)
#pragma unroll
        for (int j = 0; j < (BLK ? TM : 1); j++)
            accf[i][j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    /* With blocks of 32 (BLK 2) a lane reads, for each half h of a unit (one
     * block), the 8 bytes the 16x16x32 MFMA takes from it: row lane % 16,
     * inputs 32 h + 8 (lane / 16) .. + 7, which the unit holds at
     * ((2 h + lane / 32) 16 + lane % 16) 16 + 8 ((lane / 16) % 2); the bytes
     * of half h are 512 h further on. Otherwise a lane's 16-byte slot. */
    const uint32_t lofs = BLK == 2 ? ((lane >> 5) * 16 + (lane & 15)) * 16 + ((lane >> 4) & 1) * 8 : lane * 16;
    const uint32_t wbase = lds_addr(ring) + (wn * TN) * kUnitBytes + lofs;
    const uint32_t abase = lds_addr(ring) + (UB + wm * TM) * kUnitBytes + lofs;
    /* this lane's frame within the tile for frame tile j: (wm TM + j) 16 + lane % 16 */
    const uint32_t dbase = lds_addr(ring) + SLOTU * kUnitBytes + ((wm * TM) * 16 + (lane & 15)) * 4;
    /* LDS offset of sub-step gi's fragments */
    auto at_of = [&](uint32_t gi) {
        const uint32_t s = gi / UPS, kk = gi % UPS;
        return (s % NS) * SLOT + kk * UNITS * kUnitBytes;
    };
    struct Set {
        v4i f[R];
        float dv[BLK ? TM * BPU : 1];
    };
    auto read_set = [&](Set &st, uint32_t gi) {
        const uint32_t at = at_of(gi);
        if constexpr (BLK == 2) {
            /* f = { block 0's 8 bytes, block 1's 8 bytes } */
#pragma unroll
            for (int i = 0; i < TN; i++) {
                const v2i lo = lds_read8(wbase + at + i * kUnitBytes), hi = lds_read8(wbase + at + i * kUnitBytes + 512);
                st.f[i] = v4i{ lo.x, lo.y, hi.x, hi.y };
            }
#pragma unroll
            for (int j = 0; j < TM; j++) {
                const v2i lo = lds_read8(abase + at + j * kUnitBytes), hi = lds_read8(abase + at + j * kUnitBytes + 512);
                st.f[TN + j] = v4i{ lo.x, lo.y, hi.x, hi.y };
            }
        } else {
#pragma unroll
            for (int i = 0; i < TN; i++)
                st.f[i] = lds_read16(wbase + at + i * kUnitBytes);
#pragma unroll
            for (int j = 0; j < TM; j++)
                st.f[TN + j] = lds_read16(abase + at + j * kUnitBytes);
        }
        if constexpr (BLK != 0) {
            const uint32_t s = gi / UPS, kk = gi % UPS;
#pragma unroll
            for (int h = 0; h < BPU; h++)
#pragma unroll
                for (int j = 0; j < TM; j++)
                    st.dv[h * TM + j] = lds_read4(dbase + (s % NS) * SLOT + ((kk * BPU + h) * BM + j * 16) * 4);
        }
    };
    /* Sub-step gi multiplies the fragments read a sub-step ago (cur) and
     * reads gi + 1's (nxt). At the last sub-step of stage s < ns - 1 the
     * workgroup first waits for stage s + 1 (LATER stages of this thread's
     * loads may stay in flight) and meets, and with ISSUE refills stage s's
     * slot with stage s + NS. Every choice is a template argument, so the
     * loop below has no branch but its own and the accumulators stay put. */
    auto step = [&](uint32_t gi, auto barrier, auto later, auto refill, auto more, Set &cur, Set &nxt) {
        wait_lgkm<0>();
#pragma unroll
        for (int r = 0; r < R; r++)
            asm volatile("" : "+v"(cur.f[r]));
        if constexpr (BLK != 0) {
#pragma unroll
            for (int r = 0; r < TM * BPU; r++)
                asm volatile("" : "+v"(cur.dv[r]));
        }
        if constexpr (decltype(barrier)::value) {
            wait_vm<decltype(later)::value * LT>();
            __builtin_amdgcn_s_barrier();
            if constexpr (decltype(refill)::value)
                issue(gi / UPS + NS);
        }
        if constexpr (decltype(more)::value)
            read_set(nxt, gi + 1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (BLK == 0) {
#pragma unroll
            for (int i = 0; i < TN; i++)
#pragma unroll
                for (int j = 0; j < TM; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur.f[i], cur.f[TN + j], acc[i][j], 0, 0, 0);
        } else {
            const uint32_t u = u0 + gi;             /* the unit: uniform */
#pragma unroll
            for (int h = 0; h < BPU; h++) {
#pragma unroll
                for (int i = 0; i < TN; i++)
#pragma unroll
                    for (int j = 0; j < TM; j++) {
                        if constexpr (BLK == 2) {
                            /* block h alone: its 32 inputs, 8 bytes a lane */
                            const long wh = __builtin_bit_cast(long, v2i{ cur.f[i][2 * h], cur.f[i][2 * h + 1] });
                            const long ah = __builtin_bit_cast(long, v2i{ cur.f[TN + j][2 * h], cur.f[TN + j][2 * h + 1] });
                            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wh, ah, v4i{0, 0, 0, 0}, 0, 0, 0);
                        } else {
                            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur.f[i], cur.f[TN + j],
                                                                              v4i{0, 0, 0, 0}, 0, 0, 0);
                        }
                    }
                if (u * BPU + h < nb) {
#pragma unroll
                    for (int i = 0; i < TN; i++)
#pragma unroll
                        for (int j = 0; j < TM; j++) {
                            const float dvj = cur.dv[h * TM + j];
                            accf[i][j].x = __builtin_fmaf((float)acc[i][j][0], dvj, accf[i][j].x);
                            accf[i][j].y = __builtin_fmaf((float)acc[i][j][1], dvj, accf[i][j].y);
                            accf[i][j].z = __builtin_fmaf((float)acc[i][j][2], dvj, accf[i][j].z);
                            accf[i][j].w = __builtin_fmaf((float)acc[i][j][3], dvj, accf[i][j].w);
                        }
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    using yes = std::true_type;
    using no = std::false_type;
    Set f0, f1;
    auto setpair = [&](auto k) -> Set & {
        if constexpr (decltype(k)::value % 2 == 0) return f0; else return f1;
    };

    /* The epilogue's per-frame scales and per-channel scales and biases,
     * staged into LDS ahead of stage 0: the oldest loads of each wave, so
     * the wait for stage 0 covers them, and the epilogue finds them in LDS
     * instead of waiting a memory round trip after the last MFMA. Each
     * segment is whole 64-float chunks; indexes past the tile's frames or
     * channels read the last one (their results are never stored). With
     * blocks the frame scales are not used (the chain took them). */
    constexpr int ED = (BM + 63) / 64, EW = (BN + 63) / 64, ECH = ED + 2 * EW;
    __shared__ __attribute__((aligned(256))) float epi[ECH * 64];
    if (kg == 0) {
        const int nch = g.bias ? ECH : ED + EW;
        for (int c = BLK ? ED + wave : wave; c < nch; c += NW) {
            const float *a;
            if (c < ED) {
                const uint32_t t = m0 + c * 64 + lane;
                a = sg.d + (t < T ? t : T - 1);
            } else {
                const uint32_t r = n0 + ((c - ED) % EW) * 64 + lane;
                a = (c < ED + EW ? g.ws : g.bias) + (r < g.rows ? r : g.rows - 1);
            }
            __builtin_amdgcn_global_load_lds(PK_AS1(a), PK_AS3(epi + c * 64), 4, 0, 0);
        }
    }

    /* the caller guarantees ns >= NS */
#pragma unroll
    for (int j = 0; j < NS; j++)
        issue(j);
    wait_vm<(NS - 1) * LT>();
    __builtin_amdgcn_s_barrier();
    read_set(f0, 0);
    /* the first set lands before the loop: where the loop's entry copies
     * registers, it then copies the fragments, not what preceded them */
    wait_lgkm<0>();
#pragma unroll
    for (int r = 0; r < R; r++)
        asm volatile("" : "+v"(f0.f[r]));
    if constexpr (BLK != 0) {
#pragma unroll
        for (int r = 0; r < TM * BPU; r++)
            asm volatile("" : "+v"(f0.dv[r]));
    }

    /* steady state: stages [0, ns - NS), each refilling its slot; SPI
     * sub-steps a pass, an even number, so f0 and f1 alternate statically */
    constexpr int SPI = UPS > 2 ? UPS : 2;
    const uint32_t steady = (ns - NS) * UPS;
    for (uint32_t gi = 0; gi < steady; gi += SPI) {
        for_static<0, SPI>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            constexpr bool bar = k % UPS == UPS - 1;
            step(gi + k, std::integral_constant<bool, bar>{}, std::integral_constant<int, NS - 2>{},
                 std::integral_constant<bool, bar>{}, yes{}, setpair(std::integral_constant<int, k>{}),
                 setpair(std::integral_constant<int, k + 1>{}));
        });
    }
    /* drain: stages ns - NS .. ns - 2, loading nothing more; then the last */
    for_static<0, NS * UPS>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        constexpr int b = k / UPS;                        /* stage ns - NS + b */
        constexpr bool bar = k % UPS == UPS - 1 && b < NS - 1;
        constexpr int later = NS - 2 - b < 0 ? 0 : NS - 2 - b;
        constexpr bool more = k + 1 < NS * UPS;
        step(steady + k, std::integral_constant<bool, bar>{}, std::integral_constant<int, later>{}, no{},
             std::integral_constant<bool, more>{}, setpair(std::integral_constant<int, k>{}),
             setpair(std::integral_constant<int, k + 1>{}));
    });
    wait_vm<0>();

    if constexpr (KG > 1) {
        /* every wave is done reading its ring: the other groups hand their
         * int32 sums to group 0 through LDS (exact in any order) */
        __builtin_amdgcn_s_barrier();
        v4i *xch = (v4i *)rings;
        if (kg > 0) {
#pragma unroll
            for (int i = 0; i < TN; i++)
#pragma unroll
                for (int j = 0; j < TM; j++)
                    xch[(((kg - 1) * NW + wave) * TN * TM + i * TM + j) * 64 + lane] = acc[i][j];
        }
        __syncthreads();
        if (kg > 0)
            return;
#pragma unroll
        for (int h = 1; h < KG; h++)
#pragma unroll
            for (int i = 0; i < TN; i++)
#pragma unroll
                for (int j = 0; j < TM; j++)
                    acc[i][j] += xch[(((h - 1) * NW + wave) * TN * TM + i * TM + j) * 64 + lane];
    }

    if constexpr (BLK != 0 && WN == 2 && TN == 2) {
        if (g.oqp) {
            /* The outputs SiLU'd and quantized in blocks of oqb channels
             * (core/encoder.c:130-156) straight into the next product's
             * packed activations: the values are those the store below would
             * write, and pk_silu, the block's largest magnitude, its scales
             * and the rounding are the quantizer's own, so the bytes and
             * scales are a SiLU quantize's of the stored outputs. A wave
             * holds 32 channels of a frame in 4 lanes (l % 16 the frame) x 8
             * values: a block of 32 is one wave's, a block of 64 the two
             * channel waves', met in LDS. */
            __shared__ int bmax[BM][2];
            const uint32_t G = (T + 15) / 16;
            float sv[TM][TN][4];
            int mx[TM];
#pragma unroll
            for (int j = 0; j < TM; j++) {
                int m = 0;
#pragma unroll
                for (int i = 0; i < TN; i++) {
                    const uint32_t cl = (wn * TN + i) * 16 + (lane >> 4) * 4;
                    const float4 wsv = *(const float4 *)&epi[ED * 64 + cl];
                    const float wsr[4] = { wsv.x, wsv.y, wsv.z, wsv.w };
                    float bsr[4] = { 0, 0, 0, 0 };
                    if (g.bias) {
                        const float4 bv = *(const float4 *)&epi[(ED + EW) * 64 + cl];
                        bsr[0] = bv.x; bsr[1] = bv.y; bsr[2] = bv.z; bsr[3] = bv.w;
                    }
                    const float4 af = accf[i][j];
                    const float a4[4] = { af.x, af.y, af.z, af.w };
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        float v = a4[r] * wsr[r];
                        if (g.bias)
                            v = v + bsr[r];
                        sv[j][i][r] = pk_silu(v);
                        m = max(m, mag_bits(sv[j][i][r]));
                    }
                }
                m = max(m, __shfl_xor(m, 16));
                mx[j] = max(m, __shfl_xor(m, 32));
            }
            if (g.oqb == 64) {
#pragma unroll
                for (int j = 0; j < TM; j++)
                    if (lane < 16)
                        bmax[(wm * TM + j) * 16 + lane][wn] = mx[j];
                __syncthreads();
#pragma unroll
                for (int j = 0; j < TM; j++) {
                    const int fl = (wm * TM + j) * 16 + (lane & 15);
                    mx[j] = max(bmax[fl][0], bmax[fl][1]);
                }
            }
#pragma unroll
            for (int j = 0; j < TM; j++) {
                const uint32_t t = m0 + (wm * TM + j) * 16 + (lane & 15);
                if (t >= T)
                    continue;
                bool zero;
                float dv, id;
                block_scales((uint32_t)mx[j], zero, dv, id);
#pragma unroll
                for (int i = 0; i < TN; i++) {
                    const uint32_t c = n0 + (wn * TN + i) * 16 + (lane >> 4) * 4;
                    const int v4 = zero ? 0 : pack4(make_float4(sv[j][i][0], sv[j][i][1], sv[j][i][2], sv[j][i][3]), id);
                    *(int *)(g.oqp + ((size_t)(c >> 6) * G + (t >> 4)) * kUnitBytes + in_unit(c, t & 15)) = v4;
                }
                const uint32_t cb = n0 + wn * 32;       /* the wave's first channel */
                if ((lane >> 4) == 0 && cb % g.oqb == 0)
                    g.od[(size_t)t * (g.rows / g.oqb) + cb / g.oqb] = dv;
            }
            return;
        }
    }

    const bool vec = ((sg.os & 3) == 0) && ((((uintptr_t)sg.out) & 15) == 0);
    if constexpr (BLK == 0 && TN % 2 == 0 && BN * BM >= 128 * 128) {
        if (vec) {
            /* Vector stores of whole 128-byte lines, each from 8 consecutive
             * lanes in address order, where a block's own layout stores 64
             * bytes of 16 frames, one frame a lane: on tiles of 128 x 128 and
             * more, where the stores weigh most (measured at ten minutes of
             * audio: o 19.7-20.3 -> 19.3 us, the sweep 1.2% faster; on the
             * 64 x 64 tiles of one minute the moves cost more than they save,
             * ff down 9.7 -> 10.1 us, so those keep the loop below). Every
             * lane computes its block's values as below (ref's operations in
             * ref's order); then channel blocks 2k and 2k + 1 pair up and
             * swap the block for the lane's bit 3 (lanes l and l ^ 8 exchange
             * through DPP row_ror:8, a rotation by 8 inside each row of 16
             * lanes), so that each register of a pair holds 8 frames x 32
             * channels, lane (r, b, f) channel 16 b + 4 r of frame f; one
             * ds_bpermute a value moves that to lane 8 f + 4 b + r, whose 16
             * bytes are chunk 4 b + r of frame f's line. The moves copy bits,
             * and the residual (ref's last operation) is added where the
             * value lands. */
            const uint32_t hi = (lane >> 3) & 1;
            const int src = (int)((((lane & 3) << 4) | (((lane >> 2) & 1) << 3) | (lane >> 3)) * 4);
            /* with add, a frame block's residuals load at the start of the
             * block, before any of its stores (a load after a store would
             * wait for it: vmcnt counts both), from addresses clamped to the
             * call's last frame and channel group; only the stores are
             * predicated (measured at ten minutes of audio: o and pw2 18.6 ->
             * 17.9-18.6 us, the sweep 1.4% faster; a wave's residuals all at
             * once measured 19.4-19.7 us, loaded beside each store 18.8-19.0) */
            float4 old[TN];
            auto load_old = [&](int j, float4 *o4) {
#pragma unroll
                for (int k = 0; k < TN / 2; k++)
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const uint32_t t = m0 + (wm * TM + j) * 16 + h * 8 + (lane >> 3);
                        const uint32_t c = n0 + (wn * TN + 2 * k) * 16 + (lane & 7) * 4;
                        o4[2 * k + h] = *(const float4 *)(sg.out + (size_t)(t < T ? t : T - 1) * sg.os +
                                                          (c < g.rows ? c : g.rows - 4));
                    }
            };
#pragma unroll
            for (int j = 0; j < TM; j++) {
                if (g.add)
                    load_old(j, old);
                const uint32_t tl = (wm * TM + j) * 16;     /* the block's first frame in the tile */
                const float dt = epi[tl + (lane & 15)];
#pragma unroll
                for (int k = 0; k < TN / 2; k++) {
                    float v[2][4];
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        const uint32_t cl = (wn * TN + 2 * k + q) * 16 + (lane >> 4) * 4;
                        const float4 wsv = *(const float4 *)&epi[ED * 64 + cl];
                        const float wsr[4] = { wsv.x, wsv.y, wsv.z, wsv.w };
                        float bsr[4] = { 0, 0, 0, 0 };
                        if (g.bias) {
                            const float4 bv = *(const float4 *)&epi[(ED + EW) * 64 + cl];
                            bsr[0] = bv.x; bsr[1] = bv.y; bsr[2] = bv.z; bsr[3] = bv.w;
                        }
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            v[q][r] = __builtin_fmaf((float)acc[2 * k + q][j][r], dt, 0.0f) * wsr[r];
                            if (g.bias)
                                v[q][r] = v[q][r] + bsr[r];
                        }
                    }
                    float x[2][4];
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int a = __float_as_int(v[0][r]), bq = __float_as_int(v[1][r]);
                        const int ar = __builtin_amdgcn_update_dpp(0, a, 0x128, 0xF, 0xF, false);
                        const int br = __builtin_amdgcn_update_dpp(0, bq, 0x128, 0xF, 0xF, false);
                        x[0][r] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, hi ? br : a));     /* frames 0-7 */
                        x[1][r] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, hi ? bq : ar));    /* frames 8-15 */
                    }
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const uint32_t t = m0 + tl + h * 8 + (lane >> 3);
                        const uint32_t c = n0 + (wn * TN + 2 * k) * 16 + (lane & 7) * 4;
                        float4 ov = make_float4(x[h][0], x[h][1], x[h][2], x[h][3]);
                        if (g.add) {
                            const float4 o4 = old[2 * k + h];
                            ov.x = o4.x + ov.x;
                            ov.y = o4.y + ov.y;
                            ov.z = o4.z + ov.z;
                            ov.w = o4.w + ov.w;
                        }
                        if (t < T && c < g.rows)
                            store_out4(sg.out + (size_t)t * sg.os + c, ov, g.plain);
                    }
                }
            }
            return;
        }
    }
    /* The per-lane loop, in two compiled forms: PRE (vector stores with
     * add) loads the residuals before any store (a load after a store would
     * wait for it: vmcnt counts both), all of a wave's at once where they fit
     * in 32 registers, else a frame block's first, from addresses clamped to
     * the call's last frame and channel group (measured: ff down at one
     * minute of audio 9.8-9.9 -> 9.5-9.7 us); the other form is the plain
     * loop as it was, each residual loaded beside its store where there is
     * one (one form for both measured up to 3% slower on products without
     * add). */
    auto rows_loop = [&](auto prec) {
        constexpr bool PRE = decltype(prec)::value;
        constexpr bool ALL = TN * TM <= 8;
        float4 oldv[PRE && ALL ? TM : 1][TN];
        auto load_old = [&](int j, float4 *o4) {
#pragma unroll
            for (int i = 0; i < TN; i++) {
                const uint32_t t = m0 + (wm * TM + j) * 16 + (lane & 15);
                const uint32_t c = n0 + (wn * TN + i) * 16 + (lane >> 4) * 4;
                o4[i] = *(const float4 *)(sg.out + (size_t)(t < T ? t : T - 1) * sg.os + (c < g.rows ? c : g.rows - 4));
            }
        };
        if constexpr (PRE && ALL) {
#pragma unroll
            for (int j = 0; j < TM; j++)
                load_old(j, oldv[j]);
        }
#pragma unroll
        for (int j = 0; j < TM; j++) {
            if constexpr (PRE && !ALL)
                load_old(j, oldv[0]);
            const uint32_t t = m0 + (wm * TM + j) * 16 + (lane & 15);
            if (t >= T)
                continue;
            const float dt = BLK ? 0.0f : epi[t - m0];
#pragma unroll
            for (int i = 0; i < TN; i++) {
                const uint32_t c = n0 + (wn * TN + i) * 16 + (lane >> 4) * 4;
                if (c >= g.rows)
                    continue;
                const float4 wsv = *(const float4 *)&epi[ED * 64 + (c - n0)];
                const float wsr[4] = { wsv.x, wsv.y, wsv.z, wsv.w };
                float bsr[4] = { 0, 0, 0, 0 };
                if (g.bias) {
                    const float4 bv = *(const float4 *)&epi[(ED + EW) * 64 + (c - n0)];
                    bsr[0] = bv.x; bsr[1] = bv.y; bsr[2] = bv.z; bsr[3] = bv.w;
                }
                float v[4];
                if constexpr (BLK != 0) {
                    const float4 af = accf[i][j];
                    const float a4[4] = { af.x, af.y, af.z, af.w };
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        v[r] = a4[r] * wsr[r];
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        v[r] = __builtin_fmaf((float)acc[i][j][r], dt, 0.0f) * wsr[r];
                }
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (g.bias)
                        v[r] = v[r] + bsr[r];
                float *o = sg.out + (size_t)t * sg.os + c;
                if (vec) {
                    float4 ov = make_float4(v[0], v[1], v[2], v[3]);
                    if (g.add) {
                        float4 old;
                        if constexpr (PRE)
                            old = oldv[ALL ? j : 0][i];
                        else
                            old = *(const float4 *)o;
                        ov.x = old.x + ov.x;
                        ov.y = old.y + ov.y;
                        ov.z = old.z + ov.z;
                        ov.w = old.w + ov.w;
                    }
                    store_out4(o, ov, g.plain);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        store_out1(o + r, g.add ? o[r] + v[r] : v[r], g.plain);
                }
            }
        }
    };
    if (vec && g.add)
        rows_loop(std::true_type{});
    else
        rows_loop(std::false_type{});
}


template <int WN, int WM, int TN, int TM, int UPS, bool PACKED>
__global__ __launch_bounds__(64 * WN * WM) void gemm_ring_kernel(GemmArgs g, Seg sg, uint32_t tiles_n,
                                                                 uint32_t tiles_m) {
    uint32_t tn, tm;
    xcd_tile(blockIdx.x, gridDim.x, tiles_n, tiles_m, tn, tm);
    ring_tile<WN, WM, TN, TM, UPS, PACKED>(g, sg, tn, tm);
}

template <int WN, int WM, int TN, int TM, int UPS, bool PACKED>
__global__ __launch_bounds__(64 * WN * WM) void gemm_ring_grouped_kernel(GemmArgs g, SegTable tab,
                                                                         uint32_t tiles_n) {
    const uint32_t tm = blockIdx.x / tiles_n;
    uint32_t i = 0;
    while (i + 1 < tab.nseg && tab.s[i + 1].tile0 <= tm)
        i++;
    ring_tile<WN, WM, TN, TM, UPS, PACKED>(g, tab.s[i], blockIdx.x % tiles_n, tm - tab.s[i].tile0);
}

template <int WN, int WM, int TN, int TM, int UPS, bool PACKED>
static void run_ring1(const GemmArgs &g, const SegTable &tab, hipStream_t s) {
    constexpr uint32_t BN = 16 * TN * WN, BM = 16 * TM * WM;
    const uint32_t tiles_n = (g.rows + BN - 1) / BN;
    if (tab.nseg == 1) {
        const uint32_t tiles_m = (tab.s[0].T + BM - 1) / BM;
        gemm_ring_kernel<WN, WM, TN, TM, UPS, PACKED><<<tiles_n * tiles_m, 64 * WN * WM, 0, s>>>(g, tab.s[0], tiles_n, tiles_m);
    } else {
        SegTable t = tab;
        uint32_t tiles = 0;
        for (uint32_t i = 0; i < t.nseg; i++) {
            t.s[i].tile0 = tiles;
            tiles += (t.s[i].T + BM - 1) / BM;
        }
        gemm_ring_grouped_kernel<WN, WM, TN, TM, UPS, PACKED><<<tiles_n * tiles, 64 * WN * WM, 0, s>>>(g, t, tiles_n);
    }
}

template <int WN, int WM, int TN, int TM, int UPS>
static void run_ring(const GemmArgs &g, const SegTable &tab, hipStream_t s) {
    if (tab.s[0].qstride)
        run_ring1<WN, WM, TN, TM, UPS, true>(g, tab, s);
    else
        run_ring1<WN, WM, TN, TM, UPS, false>(g, tab, s);
}

template <int WN, int WM, int TN, int TM, int UPS, int NS, int KG, bool PACKED, int BLK>
__global__ __launch_bounds__(64 * WN * WM * KG) void gemm_pipe_kernel(GemmArgs g, Seg sg, uint32_t tiles_n,
                                                                      uint32_t tiles_m) {
    uint32_t tn, tm;
    xcd_tile(blockIdx.x, gridDim.x, tiles_n, tiles_m, tn, tm);
    pipe_tile<WN, WM, TN, TM, UPS, NS, KG, PACKED, BLK>(g, sg, tn, tm);
}

template <int WN, int WM, int TN, int TM, int UPS, int NS, int KG, bool PACKED, int BLK>
__global__ __launch_bounds__(64 * WN * WM * KG) void gemm_pipe_grouped_kernel(GemmArgs g, SegTable tab,
                                                                              uint32_t tiles_n) {
    const uint32_t tm = blockIdx.x / tiles_n;
    uint32_t i = 0;
    while (i + 1 < tab.nseg && tab.s[i + 1].tile0 <= tm)
        i++;
    pipe_tile<WN, WM, TN, TM, UPS, NS, KG, PACKED, BLK>(g, tab.s[i], blockIdx.x % tiles_n, tm - tab.s[i].tile0);
}

template <int WN, int WM, int TN, int TM, int UPS, int NS, int KG, bool PACKED, int BLK>
static void run_pipe1(const GemmArgs &g, const SegTable &tab, hipStream_t s) {
    constexpr uint32_t BN = 16 * TN * WN, BM = 16 * TM * WM;
    constexpr uint32_t threads = 64 * WN * WM * KG;
    const uint32_t tiles_n = (g.rows + BN - 1) / BN;
    if (tab.nseg == 1) {
        const uint32_t tiles_m = (tab.s[0].T + BM - 1) / BM;
        gemm_pipe_kernel<WN, WM, TN, TM, UPS, NS, KG, PACKED, BLK><<<tiles_n * tiles_m, threads, 0, s>>>(g, tab.s[0], tiles_n, tiles_m);
    } else {
        SegTable t = tab;
        uint32_t tiles = 0;
        for (uint32_t i = 0; i < t.nseg; i++) {
            t.s[i].tile0 = tiles;
            tiles += (t.s[i].T + BM - 1) / BM;
        }
        gemm_pipe_grouped_kernel<WN, WM, TN, TM, UPS, NS, KG, PACKED, BLK><<<tiles_n * tiles, threads, 0, s>>>(g, t, tiles_n);
    }
}

template <int WN, int WM, int TN, int TM, int UPS, int NS, int KG, int BLK>
__global__ __launch_bounds__(64 * WN * WM * KG) void gemm_pipe_batch_kernel(JobTable tab) {
    uint32_t j = 0;
    while (j + 1 < tab.njobs && tab.wg0[j + 1] <= blockIdx.x)
        j++;
    const uint32_t b = blockIdx.x - tab.wg0[j];
    if (b >= tab.tiles[j])
        return;                                 /* padding up to the next job's multiple of 8 */
    const uint32_t tiles_n = tab.tiles_n[j];
    uint32_t tn, tm;
    xcd_tile(b, tab.tiles[j], tiles_n, tab.tiles[j] / tiles_n, tn, tm);
    pipe_tile<WN, WM, TN, TM, UPS, NS, KG, true, BLK>(tab.g[j], tab.s[j], tn, tm);
}

template <int WN, int WM, int TN, int TM, int UPS, int NS, int KG, int BLK = 0>
static void run_pipe_batch(const JobTable &jobs, hipStream_t s) {
    constexpr uint32_t BN = 16 * TN * WN, BM = 16 * TM * WM;
    JobTable t = jobs;
    uint32_t wg = 0;
    for (uint32_t j = 0; j < t.njobs; j++) {
        t.wg0[j] = wg;
        t.tiles_n[j] = (t.g[j].rows + BN - 1) / BN;
        t.tiles[j] = t.tiles_n[j] * ((t.s[j].T + BM - 1) / BM);
        wg += (t.tiles[j] + 7) / 8 * 8;
    }
    t.wg0[t.njobs] = wg;
    gemm_pipe_batch_kernel<WN, WM, TN, TM, UPS, NS, KG, BLK><<<wg, 64 * WN * WM * KG, 0, s>>>(t);
}

template <int WN, int WM, int TN, int TM, int UPS, int NS, int KG = 1, int BLK = 0>
static void run_pipe(const GemmArgs &g, const SegTable &tab, hipStream_t s) {
    if (tab.s[0].qstride)
        run_pipe1<WN, WM, TN, TM, UPS, NS, KG, true, BLK>(g, tab, s);
    else
        run_pipe1<WN, WM, TN, TM, UPS, NS, KG, false, BLK>(g, tab, s);
}

/* The pipelined product's tile shapes: channels x frames, and the units of
 * inputs a stage (ku must divide into four stages of them). */
struct RingCfg {
    const char *name;
    uint32_t bn, bm, ups;
    uint32_t slots;                 /* 0: ring_tile (four slots, four-stage passes) */
    uint32_t kg;                    /* K groups of pipe_tile */
    void (*run)(const GemmArgs &, const SegTable &, hipStream_t);
    void (*batch)(const JobTable &, hipStream_t);   /* pipe_tile only */
    void (*run64)(const GemmArgs &, const SegTable &, hipStream_t);   /* blocks of 64 inputs, or null */
    void (*run32)(const GemmArgs &, const SegTable &, hipStream_t);   /* blocks of 32 inputs, or null */
    void (*batch64)(const JobTable &, hipStream_t);                   /* batches in blocks of 64, or null */
    void (*batch32)(const JobTable &, hipStream_t);                   /* batches in blocks of 32, or null */
};
static const RingCfg kRing[] = {
    /* ring_tile: name <channels x frames, units a stage> */
    { "ring<128x128,1>", 128, 128, 1, 0, 1, run_ring<2, 2, 4, 4, 1>, nullptr, nullptr, nullptr },
    { "ring<64x64,1>", 64, 64, 1, 0, 1, run_ring<2, 2, 2, 2, 1>, nullptr, nullptr, nullptr },
    { "ring<64x64,2>", 64, 64, 2, 0, 1, run_ring<2, 2, 2, 2, 2>, nullptr, nullptr, nullptr },
    { "ring<64x64,4>", 64, 64, 4, 0, 1, run_ring<2, 2, 2, 2, 4>, nullptr, nullptr, nullptr },
    /* pipe_tile: name <channels x frames, units a stage, slots>; w8: eight
     * waves of 64 x 32 */
    { "pipe<128x128,1,4>", 128, 128, 1, 4, 1, run_pipe<2, 2, 4, 4, 1, 4, 1>, run_pipe_batch<2, 2, 4, 4, 1, 4, 1>, run_pipe<2, 2, 4, 4, 1, 4, 1, 1>, run_pipe<2, 2, 4, 4, 1, 4, 1, 2>, run_pipe_batch<2, 2, 4, 4, 1, 4, 1, 1>, run_pipe_batch<2, 2, 4, 4, 1, 4, 1, 2> },
    { "pipe<128x128w8,1,4>", 128, 128, 1, 4, 1, run_pipe<2, 4, 4, 2, 1, 4, 1>, run_pipe_batch<2, 4, 4, 2, 1, 4, 1>, run_pipe<2, 4, 4, 2, 1, 4, 1, 1>, run_pipe<2, 4, 4, 2, 1, 4, 1, 2>, run_pipe_batch<2, 4, 4, 2, 1, 4, 1, 1>, run_pipe_batch<2, 4, 4, 2, 1, 4, 1, 2> },
    { "pipe<64x64,2,4>", 64, 64, 2, 4, 1, run_pipe<2, 2, 2, 2, 2, 4, 1>, run_pipe_batch<2, 2, 2, 2, 2, 4, 1>, run_pipe<2, 2, 2, 2, 2, 4, 1, 1>, run_pipe<2, 2, 2, 2, 2, 4, 1, 2>, run_pipe_batch<2, 2, 2, 2, 2, 4, 1, 1>, run_pipe_batch<2, 2, 2, 2, 2, 4, 1, 2> },
    { "pipe<64x64,4,4>", 64, 64, 4, 4, 1, run_pipe<2, 2, 2, 2, 4, 4, 1>, run_pipe_batch<2, 2, 2, 2, 4, 4, 1>, nullptr, nullptr },
    /* eight waves of 64 x 64 */
    { "pipe<128x256w8,1,4>", 128, 256, 1, 4, 1, run_pipe<2, 4, 4, 4, 1, 4, 1>, run_pipe_batch<2, 4, 4, 4, 1, 4, 1>, nullptr, nullptr },
    { "pipe<128x256w8,1,6>", 128, 256, 1, 6, 1, run_pipe<2, 4, 4, 4, 1, 6, 1>, run_pipe_batch<2, 4, 4, 4, 1, 6, 1>, nullptr, nullptr },
    { "pipe<256x128w8,1,4>", 256, 128, 1, 4, 1, run_pipe<4, 2, 4, 4, 1, 4, 1>, run_pipe_batch<4, 2, 4, 4, 1, 4, 1>, nullptr, nullptr },
    /* eight waves of 128 x 64 */
    { "pipe<256x256w8,1,4>", 256, 256, 1, 4, 1, run_pipe<2, 4, 8, 4, 1, 4, 1>, run_pipe_batch<2, 4, 8, 4, 1, 4, 1>, nullptr, nullptr },
    /* two K groups of four waves of 32 x 32 */
    { "pipe<64x64,2,4,k2>", 64, 64, 2, 4, 2, run_pipe<2, 2, 2, 2, 2, 4, 2>, run_pipe_batch<2, 2, 2, 2, 2, 4, 2>, nullptr, nullptr },
    { "pipe<64x64,1,4,k2>", 64, 64, 1, 4, 2, run_pipe<2, 2, 2, 2, 1, 4, 2>, run_pipe_batch<2, 2, 2, 2, 1, 4, 2>, nullptr, nullptr },
    { "pipe<64x64,2,2,k2>", 64, 64, 2, 2, 2, run_pipe<2, 2, 2, 2, 2, 2, 2>, run_pipe_batch<2, 2, 2, 2, 2, 2, 2>, nullptr, nullptr },
    /* three slots: three workgroups a CU */
    { "pipe<64x64,2,3>", 64, 64, 2, 3, 1, run_pipe<2, 2, 2, 2, 2, 3, 1>, run_pipe_batch<2, 2, 2, 2, 2, 3, 1>, run_pipe<2, 2, 2, 2, 2, 3, 1, 1>, run_pipe<2, 2, 2, 2, 2, 3, 1, 2>, run_pipe_batch<2, 2, 2, 2, 2, 3, 1, 1>, run_pipe_batch<2, 2, 2, 2, 2, 3, 1, 2> },
    { "pipe<64x64,2,3,k2>", 64, 64, 2, 3, 2, run_pipe<2, 2, 2, 2, 2, 3, 2>, run_pipe_batch<2, 2, 2, 2, 2, 3, 2>, nullptr, nullptr },
    /* eight waves of 32 x 16: two a SIMD, so one wave's block chain runs
     * beside the other's MFMAs where a product has too few tiles for two
     * workgroups a CU */
    { "pipe<64x64w8,2,4>", 64, 64, 2, 4, 1, run_pipe<2, 4, 2, 1, 2, 4, 1>, run_pipe_batch<2, 4, 2, 1, 2, 4, 1>, run_pipe<2, 4, 2, 1, 2, 4, 1, 1>, run_pipe<2, 4, 2, 1, 2, 4, 1, 2>, run_pipe_batch<2, 4, 2, 1, 2, 4, 1, 1>, run_pipe_batch<2, 4, 2, 1, 2, 4, 1, 2> },
};
constexpr int kNRing = sizeof kRing / sizeof kRing[0];

/* A forced tiling for tests and tuning (set_ring), -1 for the heuristic. */
static int g_forced_ring = -1;

/* Tiling indexes: [0, kNRing) the per-launch tiles above, then
 * [kNRing, kNRing + stream_count()) the streamed product's (q8_stream.hip). */
int set_ring(int i) {
    const int was = g_forced_ring;
    g_forced_ring = i >= 0 && i < kNRing + stream_count() ? i : -1;
    return was;
}

int ring_count() { return kNRing + stream_count(); }

const char *ring_name(int i) {
    return i >= 0 && i < kNRing ? kRing[i].name : i >= kNRing && i < kNRing + stream_count() ? stream_cfg(i - kNRing)->name : "";
}

/* whether tiling i takes ku units a panel: ring_tile runs whole passes of
 * four stages; pipe_tile needs its slots' worth of stages to start, and its
 * steady state runs whole passes of max(2, UPS) sub-steps, so with one unit
 * a stage the stages past the slots' first fill must be even in number (a
 * pass past them would load a stage beyond the last) */
static bool fits(int i, uint32_t ku) {
    if (i < 0 || i >= kNRing)
        return false;
    const RingCfg &c = kRing[i];
    if (c.slots == 0)
        return ku % (4 * c.ups) == 0;
    if (ku % (c.kg * c.ups) != 0)
        return false;
    const uint32_t ns = ku / (c.kg * c.ups);
    return ns >= c.slots && (c.ups > 1 || (ns - c.slots) % 2 == 0);
}

static int ring_index(const char *name) {
    for (int i = 0; i < kNRing; i++)
        if (!strcmp(kRing[i].name, name))
            return i;
    return -1;
}

/* The tile for a product of `frames` frames into `rows` channels. */
static int pick_ring(uint32_t rows, uint64_t frames, uint32_t ku) {
    if (g_forced_ring >= 0 && fits(g_forced_ring, ku))
        return g_forced_ring;
    auto tiles = [&](int i) { return (uint64_t)((rows + kRing[i].bn - 1) / kRing[i].bn) * ((frames + kRing[i].bm - 1) / kRing[i].bm); };
    static const int w8 = ring_index("pipe<64x64w8,2,4>"), s3 = ring_index("pipe<64x64,2,3>");
    /* measured on the layer's shapes at 750 and 7500 frames (every tiling,
     * every product): a CU's worth of 128 x 128 tiles takes the eight-wave
     * pipelined tile; fewer take 64 x 64 pipelined tiles of two-unit stages:
     * split into two K groups where the inputs are deep; eight waves of
     * 32 x 16 (two a SIMD) where the tiles leave CUs idle; three slots
     * (three workgroups a CU) where there are two tiles a CU or more;
     * inputs too short for their slots take the ring, 64 x 64, with longer
     * stages the fewer the tiles */
    if (tiles(0) >= 256 && fits(5, ku))
        return 5;
    if (ku >= 32 && tiles(6) < 512 && fits(13, ku))
        return 13;          /* deep inputs, few tiles: two K groups a tile */
    const uint64_t t64 = tiles(1);
    if (t64 < 256 && w8 >= 0 && fits(w8, ku))
        return w8;
    if (t64 >= 512 && s3 >= 0 && fits(s3, ku))
        return s3;
    if (fits(6, ku))
        return 6;
    if (t64 >= 512)
        return 1;
    if (t64 >= 256 && ku % 8 == 0)
        return 2;
    return ku % 16 == 0 ? 3 : ku % 8 == 0 ? 2 : 1;
}

/* The tile for a blocked product: the per-column pick, but deep inputs with
 * few tiles take the eight-wave tile (the two-K-group tiles have no blocked
 * build; measured in blocks of 32 and 64 at 750 frames). */
static int pick_blocked(uint32_t rows, uint64_t frames, uint32_t ku) {
    static const int w8 = ring_index("pipe<64x64w8,2,4>");
    const int c = pick_ring(rows, frames, ku);
    if (g_forced_ring < 0 && c == 13 && w8 >= 0 && fits(w8, ku))
        return w8;
    return c;
}

/* whether streamed tiling i (an index of kStream) takes ku units a panel: a
 * tile's stages fill the ring, and its sub-steps are whole passes */
static bool stream_fits(int i, uint32_t ku) {
    const StreamCfg &c = *stream_cfg(i);
    const uint32_t spi = c.ups > 2 ? c.ups : 2;
    return ku % spi == 0 && ku / c.ups >= c.slots;
}

/* whether a call's weights and activations span less than 2 GiB from their
 * first bytes: the streamed product reads them through buffer resources with
 * 32-bit offsets */
static bool stream_spans_fit(const GemmArgs &g, const Seg &sg) {
    constexpr uint64_t lim = (uint64_t)1 << 31;
    const uint64_t wspan = (uint64_t)g.ku * g.wstride;
    const uint64_t aspan = sg.qstride ? (uint64_t)g.ku * sg.qstride : (uint64_t)sg.T * g.n;
    return wspan < lim && aspan < lim;
}

/* The streamed tiling (an index of stream_cfg) for a per-row product of one
 * segment, or -1 for the per-launch tiles: the forced one where it fits;
 * else 256 x 128 streamed tiles where there are at least 400 of them, or 200
 * with deep inputs (4096). Measured at 7500 frames (each product alone): ff
 * up 41-44 against 46-47 us, pw1 24.2 against 25.9, the positions' 14999
 * rows 26-30 against 28-34, ff down 32.7-34.3 against 34.2-36.1; the 236-tile
 * products with 1024 inputs (q, k, v, o, pw2) run faster on the per-launch
 * tiles (two workgroups a CU fill each other's barrier waits where one tile
 * a CU leaves nothing to stream: q 15.3 against 16.5 us, o 18.6 against
 * 19.6). A batch (its rows the largest job's, its frames all jobs') takes
 * 128 x 256 streamed tiles where there are at least 1024 of them: the
 * attention's q, k, v and positions at 7500 frames 58.2-58.7 us against
 * 64.8-65.7 on the per-launch tiles (61.1-61.4 on 256 x 128) with the batch
 * alone, 63.2 against 64.8 inside the 24-layer sweep (each layer's weights
 * cold). */
static int pick_stream(uint32_t rows, uint64_t frames, uint32_t ku, bool batch = false) {
    if (g_forced_ring >= kNRing) {
        const int i = g_forced_ring - kNRing;
        return stream_fits(i, ku) ? i : -1;
    }
    const int i = batch ? 1 : 0;
    if (g_forced_ring >= 0 || !stream_fits(i, ku))
        return -1;
    const StreamCfg &c = *stream_cfg(i);
    const uint64_t tiles = (uint64_t)((rows + c.bn - 1) / c.bn) * ((frames + c.bm - 1) / c.bm);
    if (batch)
        return tiles >= 1024 ? i : -1;
    return tiles >= 400 || (ku >= 64 && tiles >= 200) ? i : -1;
}

template <int WN, int WM, int TN, int TM, int MODE>
static void run_tiled(const GemmArgs &g, const SegTable &tab, hipStream_t s) {
    constexpr uint32_t BN = 16 * TN * WN, BM = 16 * TM * WM;
    const uint32_t tiles_n = (g.rows + BN - 1) / BN;
    if (tab.nseg == 1) {
        const uint32_t tiles_m = (tab.s[0].T + BM - 1) / BM;
        gemm_q8_kernel<WN, WM, TN, TM, MODE><<<tiles_n * tiles_m, 64 * WN * WM, 0, s>>>(g, tab.s[0], tiles_n);
    } else {
        SegTable t = tab;
        uint32_t tiles = 0;
        for (uint32_t i = 0; i < t.nseg; i++) {
            t.s[i].tile0 = tiles;
            tiles += (t.s[i].T + BM - 1) / BM;
        }
        gemm_q8_grouped_kernel<WN, WM, TN, TM, MODE><<<tiles_n * tiles, 64 * WN * WM, 0, s>>>(g, t, tiles_n);
    }
}

template <int WN, int WM, int TN, int TM>
static void run_mode(const GemmArgs &g, const SegTable &tab, hipStream_t s, int mode) {
    if (mode == 0)
        run_tiled<WN, WM, TN, TM, 0>(g, tab, s);
    else if (mode == 1)
        run_tiled<WN, WM, TN, TM, 1>(g, tab, s);
    else
        run_tiled<WN, WM, TN, TM, 2>(g, tab, s);
}

int launch_gemm(const GemmArgs &ga, const SegTable &tab, hipStream_t s, const char **name) {
    uint64_t frames = 0;
    uint32_t tmax = 0;
    for (uint32_t i = 0; i < tab.nseg; i++) {
        frames += tab.s[i].T;
        tmax = tab.s[i].T > tmax ? tab.s[i].T : tmax;
    }
    GemmArgs g = ga;
    g.plain = frames * ga.rows * 4 > kPlainStoreBytes;
    if (frames == 0 || g.rows == 0)
        return 0;
    const int mode = g.qb == g.n ? 0 : g.qb % 64 == 0 ? 1 : 2;
    static const char *const modes[] = { "per-column", "blocks of 64k", "blocks of 32k" };
    static thread_local char buf[96];
    if (g.oqp && (mode == 0 || g.rmode != 0 || tab.nseg != 1 || !(g.oqb == 32 || g.oqb == 64) || g.rows % 64))
        return -3;                                  /* no fused SiLU quantize here */
    if (mode == 0 && tab.nseg == 1 && tmax <= 16) {
        const uint32_t panels = g.rows / 16;
        const bool packed = tab.s[0].qstride != 0;
        const uint32_t S = g.skw ? skinny_splits(panels, g.kr, tmax) : 1;
        if (S > 1) {
            /* the counters, then the partials (skinny_workspace_bytes) */
            uint32_t *cnt = (uint32_t *)g.skw;
            int32_t *part = (int32_t *)((char *)g.skw + (((size_t)panels * 4 + 255) & ~(size_t)255));
            const uint32_t P8 = (panels + 7) / 8 * 8;
            if (g.ku >= 32) {
                if (packed)
                    gemm_q8_skinny_kernel<8, true, true><<<P8 * S, 512, 0, s>>>(g, tab.s[0], S, P8, part, cnt);
                else
                    gemm_q8_skinny_kernel<8, false, true><<<P8 * S, 512, 0, s>>>(g, tab.s[0], S, P8, part, cnt);
            } else {
                if (packed)
                    gemm_q8_skinny_kernel<4, true, true><<<P8 * S, 256, 0, s>>>(g, tab.s[0], S, P8, part, cnt);
                else
                    gemm_q8_skinny_kernel<4, false, true><<<P8 * S, 256, 0, s>>>(g, tab.s[0], S, P8, part, cnt);
            }
            snprintf(buf, sizeof buf, "%s<%d> split %u", packed ? "skinny_packed" : "skinny", g.ku >= 32 ? 8 : 4, S);
            *name = buf;
            return hipPeekAtLastError() == hipSuccess ? 0 : -1;
        }
        if (g.ku >= 32) {
            if (packed)
                gemm_q8_skinny_kernel<8, true, false><<<panels, 512, 0, s>>>(g, tab.s[0], 1, 0, nullptr, nullptr);
            else
                gemm_q8_skinny_kernel<8, false, false><<<panels, 512, 0, s>>>(g, tab.s[0], 1, 0, nullptr, nullptr);
            *name = packed ? "skinny_packed<8>" : "skinny<8>";
        } else {
            if (packed)
                gemm_q8_skinny_kernel<4, true, false><<<panels, 256, 0, s>>>(g, tab.s[0], 1, 0, nullptr, nullptr);
            else
                gemm_q8_skinny_kernel<4, false, false><<<panels, 256, 0, s>>>(g, tab.s[0], 1, 0, nullptr, nullptr);
            *name = packed ? "skinny_packed<4>" : "skinny<4>";
        }
        return hipPeekAtLastError() == hipSuccess ? 0 : -1;
    }
    if (mode == 0 && tab.nseg == 1 && stream_spans_fit(g, tab.s[0])) {
        const int c = pick_stream(g.rows, frames, g.ku);
        if (c >= 0) {
            stream_cfg(c)->run(g, tab, s);
            *name = stream_cfg(c)->name;
            return hipPeekAtLastError() == hipSuccess ? 0 : -1;
        }
    }
    if (mode == 0) {
        const int c = pick_ring(g.rows, frames, g.ku);
        kRing[c].run(g, tab, s);
        *name = kRing[c].name;
        return hipPeekAtLastError() == hipSuccess ? 0 : -1;
    }
    /* blocks of 64 or 32 inputs (the encoder's modes): the pipelined tile
     * the heuristic picks for these frames, if it has a blocked variant */
    if ((mode == 1 && g.qb == 64) || (mode == 2 && g.qb == 32)) {
        int c = pick_blocked(g.rows, frames, g.ku);
        if (!(mode == 1 ? kRing[c].run64 : kRing[c].run32))
            c = fits(6, g.ku) ? 6 : 4;      /* 4 takes any ku: one unit a stage, four slots */
        if (g.oqp && (kRing[c].bn != 64 || kRing[c].bm != 64 || kRing[c].slots == 0 || kRing[c].kg != 1)) {
            /* the fused epilogue is the 64 x 64 pipelined tiles' (two channel
             * waves of 32) */
            if (!fits(6, g.ku))
                return -3;
            c = 6;
        }
        auto run = mode == 1 ? kRing[c].run64 : kRing[c].run32;
        if (run) {
            run(g, tab, s);
            snprintf(buf, sizeof buf, "%s %s%s", kRing[c].name, modes[mode], g.oqp ? " silu-quantized" : "");
            *name = buf;
            return hipPeekAtLastError() == hipSuccess ? 0 : -1;
        }
    }
    if (g.oqp)
        return -3;
    /* 128 x 128 tiles where they fill the chip, 64 x 64 where they do not */
    const uint64_t big = (uint64_t)((g.rows + 127) / 128) * ((frames + 127) / 128);
    if (big >= 256) {
        run_mode<2, 2, 4, 4>(g, tab, s, mode);
        snprintf(buf, sizeof buf, "tiled<128x128> %s", modes[mode]);
    } else {
        run_mode<2, 2, 2, 2>(g, tab, s, mode);
        snprintf(buf, sizeof buf, "tiled<64x64> %s", modes[mode]);
    }
    *name = buf;
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

int launch_gemm_batch(const JobTable &jobs_in, hipStream_t s, const char **name) {
    uint32_t rows = 0;
    uint64_t frames = 0, outs = 0;
    for (uint32_t j = 0; j < jobs_in.njobs; j++) {
        rows = jobs_in.g[j].rows > rows ? jobs_in.g[j].rows : rows;
        frames += jobs_in.s[j].T;
        outs += (uint64_t)jobs_in.s[j].T * jobs_in.g[j].rows * 4;
    }
    JobTable jobs = jobs_in;
    for (uint32_t j = 0; j < jobs.njobs; j++)
        jobs.g[j].plain = outs > kPlainStoreBytes;
    if (jobs.njobs == 0 || frames == 0)
        return 0;
    /* the tiling the jobs would take as one product of their frames; every
     * job shares the blocks (the caller checks) */
    const GemmArgs &g0 = jobs.g[0];
    const int mode = g0.qb == g0.n ? 0 : g0.qb == 64 ? 1 : g0.qb == 32 ? 2 : -1;
    bool spans = true;
    for (uint32_t j = 0; j < jobs.njobs; j++)
        spans = spans && stream_spans_fit(jobs.g[j], jobs.s[j]);
    if (mode == 0 && spans) {
        const int sc = pick_stream(rows, frames, g0.ku, true);
        if (sc >= 0) {
            stream_cfg(sc)->batch(jobs, s);
            *name = stream_cfg(sc)->name;
            return hipPeekAtLastError() == hipSuccess ? 0 : -1;
        }
    }
    const int c = mode == 0 ? pick_ring(rows, frames, g0.ku) : pick_blocked(rows, frames, g0.ku);
    auto batch = mode == 0 ? kRing[c].batch : mode == 1 ? kRing[c].batch64 : mode == 2 ? kRing[c].batch32 : nullptr;
    if (batch) {
        batch(jobs, s);
        static thread_local char buf[96];
        static const char *const modes[] = { "", " blocks of 64k", " blocks of 32k" };
        snprintf(buf, sizeof buf, "%s%s", kRing[c].name, modes[mode]);
        *name = buf;
        return hipPeekAtLastError() == hipSuccess ? 0 : -1;
    }
    /* inputs too short for the pipelined tile: one launch a job */
    for (uint32_t j = 0; j < jobs.njobs; j++) {
        if (jobs.s[j].T == 0)
            continue;
        SegTable t;
        t.nseg = 1;
        t.s[0] = jobs.s[j];
        if (const int r = launch_gemm(jobs.g[j], t, s, name))
            return r;
    }
    return 0;
}

}  // namespace pkq8
