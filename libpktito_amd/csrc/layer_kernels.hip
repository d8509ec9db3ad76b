/* The float kernels of the device-resident encoder layer: the producers that
 * make the int8 products' activations in place of the reference's fused CPU
 * passes (core/encoder.c:108-176 in peterheb/libpktito: normq, siluq_tile,
 * dw_item) and the attention's float products (core/encoder.c:280-327,
 * att_item), so that a layer's activations never leave HBM.
 *
 * Bits. Each output is the reference's ref backend's (backend/ref/
 * kernels.c:90-176): every sum the reference chains in order is one chain in
 * one lane here, in the same order (a row's 16 lane sums and their tree, a
 * float product's fmaf chain over its inputs, the depthwise taps); what is
 * order-free (a max, an elementwise function) is computed in whatever order
 * the lanes hold it. exp and sigmoid are the reference's own (q8_device.h).
 * Built with -ffp-contract=off; divisions and square roots are IEEE.
 */
#include "q8_device.h"
#include "q8_internal.h"

#include <math.h>
#include <mutex>

#pragma clang fp contract(off)

namespace pkq8 {

/* ---------------------------------------------------------- row sums --
 *
 * backend/kernels.h:105-110: a row's sum in 16 lanes, element i into lane
 * i % 16 in order, the lanes combined as acc[i] += acc[i + h] for h = 8, 4,
 * 2, 1. Here lane l of each 16-lane group holds acc[l]; the tree is the same
 * additions (a + b is b + a in IEEE arithmetic), the sum lands in the
 * group's lane 0 and is broadcast to the group. */
__device__ __forceinline__ float lanes16_sum(float v) {
    v = v + __shfl_down(v, 8, 16);
    v = v + __shfl_down(v, 4, 16);
    v = v + __shfl_down(v, 2, 16);
    v = v + __shfl_down(v, 1, 16);
    return __shfl(v, 0, 16);
}

/* The mean and 1 / sqrt(var + eps) of the row x[0, n) (n a multiple of 16)
 * as backend/ref/kernels.c:115-129 computes them, in every lane of a 16-lane
 * group whose lane l is l. x is the row staged in LDS: the chains read it
 * strided, and every read can be in flight before the first add. */
__device__ __forceinline__ void row_stats(const float *x, uint32_t n, float eps, uint32_t l, float &mean,
                                          float &r) {
    float acc = 0.0f;
#pragma unroll 16
    for (uint32_t j = l; j < n; j += 16)
        acc += x[j];
    mean = lanes16_sum(acc) / (float)n;
    acc = 0.0f;
#pragma unroll 16
    for (uint32_t j = l; j < n; j += 16) {
        const float c = x[j] - mean;
        acc += c * c;
    }
    const float var = lanes16_sum(acc) / (float)n;
    r = 1.0f / sqrtf(var + eps);
}

/* (v - mean) * r * w + b, left to right (backend/ref/kernels.c:130) */
__device__ __forceinline__ float4 normed(float4 v, float mean, float r, float4 w, float4 b) {
    return make_float4((v.x - mean) * r * w.x + b.x, (v.y - mean) * r * w.y + b.y, (v.z - mean) * r * w.z + b.z,
                       (v.w - mean) * r * w.w + b.w);
}

/* A wave's frame of n <= 256 CH floats: loaded once as float4 chunks
 * i + 64 c into registers and into the wave's LDS row, then its mean and
 * 1 / sqrt(var + eps) from the row. The same chunks of the norm's weights
 * and biases are loaded into wc and bc behind the frame's, so they arrive
 * while the sums run. */
template <int CH>
__device__ __forceinline__ void frame_stats(const float *__restrict__ xr, float *row, uint32_t n, float eps,
                                            int lane, float4 (&v)[CH], float &mean, float &r,
                                            const float *__restrict__ w, const float *__restrict__ b,
                                            float4 (&wc)[CH], float4 (&bc)[CH]) {
    const uint32_t n4 = n >> 2;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        if (i < n4)
            v[c] = ((const float4 *)xr)[i];
    }
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        wc[c] = bc[c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < n4) {
            wc[c] = ((const float4 *)w)[i];
            bc[c] = ((const float4 *)b)[i];
        }
    }
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        if (i < n4)
            ((float4 *)row)[i] = v[c];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    row_stats(row, n, eps, lane & 15, mean, r);
}

/* ------------------------------------------------------------- normq --
 *
 * core/encoder.c:108-128: each frame layer-normed and quantized whole, in
 * blocks of QB (0: the whole row), into the packed copy and d. One wave a
 * frame, four frames a workgroup. The row's sums take 16 lanes (their
 * chains are the reference's and cannot be split); the wave's other lanes
 * compute the same chains, which costs nothing on the critical path. Then
 * each lane normalizes its float4 chunks i + 64 c, as the quantizer holds
 * them. */
template <int CH, int QB>
__global__ __launch_bounds__(256) void normq_kernel(int8_t *__restrict__ qp, float *__restrict__ d,
                                                    const float *__restrict__ x, uint32_t n, uint32_t T,
                                                    const float *__restrict__ w, const float *__restrict__ b,
                                                    float eps) {
    __shared__ __attribute__((aligned(16))) float rows[4][256 * CH];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x * 4 + wv;
    if (t >= T)
        return;
    float4 v[CH], wc[CH], bc[CH];
    float mean, r;
    frame_stats<CH>(x + (size_t)t * n, rows[wv], n, eps, lane, v, mean, r, w, b, wc, bc);
    const uint32_t n4 = n >> 2;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        v[c] = i < n4 ? normed(v[c], mean, r, wc[c], bc[c]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const WaveScales<CH, QB> sc(v);
    const uint32_t G = (T + 15) / 16, g = t >> 4, fr = t & 15;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        const int cb = QB ? c : 0;
        if (i < n4) {
            const uint32_t k = 4 * i;
            *(int *)(qp + ((size_t)(k >> 6) * G + g) * kUnitBytes + in_unit(k, fr)) =
                sc.zero[cb] ? 0 : pack4(v[c], sc.id[cb]);
            if (QB && (i & (QB / 4 - 1)) == 0)
                d[(size_t)t * (n / QB) + k / QB] = sc.dv[cb];
        }
    }
    if (QB == 0 && lane == 0)
        d[t] = sc.dv[0];
}

/* core/encoder.c:86-99 (norm): the layer's last layer norm, in place. */
template <int CH>
__global__ __launch_bounds__(256) void norm_kernel(float *__restrict__ x, uint32_t n, uint32_t T,
                                                   const float *__restrict__ w, const float *__restrict__ b,
                                                   float eps) {
    __shared__ __attribute__((aligned(16))) float rows[4][256 * CH];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x * 4 + wv;
    if (t >= T)
        return;
    float *xr = x + (size_t)t * n;
    float4 v[CH], wc[CH], bc[CH];
    float mean, r;
    frame_stats<CH>(xr, rows[wv], n, eps, lane, v, mean, r, w, b, wc, bc);
    const uint32_t n4 = n >> 2;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        if (i < n4)
            ((float4 *)xr)[i] = normed(v[c], mean, r, wc[c], bc[c]);
    }
}

/* ---------------------------------------------------------- attention --
 *
 * core/encoder.c:280-327, per head h of dk dimensions, query i, key j:
 *   score(i, j) = chain_d fmaf(k_j[d], q_i[d] + u[d])
 *               + chain_d fmaf(p_{T-1-i+j}[d], q_i[d] + v[d])
 * each chain over d = 0 .. dk-1 in order from +0 (pk_k_gemm_f32), the two
 * added once; softmax over the T keys (pk_k_softmax: the scale, the max,
 * pk_expf, the 16-lane sum, one division, each e times 1 / sum); then
 *   o(i, d) = chain_j fmaf(v_j[d], P(i, j))  over j = 0 .. T-1 in order.
 * The reference lays K, P and V out as panels for its CPU kernel; the bits
 * depend only on each output's chain, so the products' row-major outputs
 * are read as they are. These are VALU kernels: an MFMA's sum of products
 * rounds differently from a chain of FMAs.
 *
 * Three kernels:
 *   scores   64 x 64 (query, key) tiles, each thread a 4 x 4 of them
 *            (queries ti + 16a, keys tj + 16b) and both chains of each; the
 *            head's dimensions staged 32 at a time through LDS (queries
 *            with each bias, keys, and the 127 position rows the tile's
 *            diagonals reach), read as float4 and prefetched a stage ahead;
 *   softmax  16 lanes a row: writes e and the row's 1 / sum;
 *   PV       32 queries x 32 dimensions a workgroup of 128, each thread 4
 *            consecutive queries x 2 dimensions (8 chains: the work is
 *            T^2 dk FMAs in only T dk chains, so the grid needs more,
 *            thinner threads than a product); keys 32 at a time through
 *            LDS with P = e * (1 / sum) formed as it is staged (the
 *            reference's x[i] * inv, one rounding) and kept key-major for
 *            one 16-byte read of a thread's 4 queries.
 * Measured at T = 750, 8 heads of 128 (MI355X): 51, 14 and 43 us. */
constexpr int kAT = 64;         /* queries and keys a score tile */
constexpr int kADC = 32;        /* dimensions a stage */
constexpr int kASD = kADC + 4;  /* an LDS row: 16-byte aligned, 4 banks apart */

__global__ __launch_bounds__(256) void att_scores_kernel(float *__restrict__ S, uint32_t Ts,
                                                         const float *__restrict__ qf,
                                                         const float *__restrict__ kf,
                                                         const float *__restrict__ pf,
                                                         const float *__restrict__ bu,
                                                         const float *__restrict__ bv, uint32_t T, uint32_t D,
                                                         uint32_t dk) {
    __shared__ __attribute__((aligned(16))) float squ[kAT][kASD], sqv[kAT][kASD], sk[kAT][kASD],
        sp[2 * kAT][kASD];
    const uint32_t j0 = blockIdx.x * kAT, i0 = blockIdx.y * kAT, h = blockIdx.z;
    const int tid = threadIdx.x, ti = tid >> 4, tj = tid & 15;
    const uint32_t R = 2 * T - 1;
    /* position row of local row 0: T - 1 - (i0 + 63) + j0 */
    const int64_t m0 = (int64_t)T - 1 - (int64_t)i0 - (kAT - 1) + (int64_t)j0;
    float sc[4][4], bd[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++)
            sc[a][b] = bd[a][b] = 0.0f;
    /* a stage in float4s: queries and keys 64 x 8 (2 a thread), positions
     * 128 x 8 (4 a thread, the last row zeros) */
    float4 rq[2], rk[2], rp[4];
    auto load = [&](uint32_t d0) {
        const uint32_t col = h * dk + d0;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int e = tid + 256 * k, r = e / 8, c4 = e % 8;
            const uint32_t i = i0 + r, j = j0 + r;
            rq[k] = i < T ? *(const float4 *)(qf + (size_t)i * D + col + 4 * c4) : make_float4(0, 0, 0, 0);
            rk[k] = j < T ? *(const float4 *)(kf + (size_t)j * D + col + 4 * c4) : make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int e = tid + 256 * k, r = e / 8, c4 = e % 8;
            const int64_t m = m0 + r;
            rp[k] = r < 2 * kAT - 1 && m >= 0 && m < (int64_t)R
                        ? *(const float4 *)(pf + (size_t)m * D + col + 4 * c4)
                        : make_float4(0, 0, 0, 0);
        }
    };
    auto store = [&](uint32_t d0) {
        const uint32_t col = h * dk + d0;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int e = tid + 256 * k, r = e / 8, c4 = e % 8;
            const float4 u4 = *(const float4 *)(bu + col + 4 * c4), v4 = *(const float4 *)(bv + col + 4 * c4);
            const float4 q = rq[k];
            *(float4 *)&squ[r][4 * c4] = make_float4(q.x + u4.x, q.y + u4.y, q.z + u4.z, q.w + u4.w);
            *(float4 *)&sqv[r][4 * c4] = make_float4(q.x + v4.x, q.y + v4.y, q.z + v4.z, q.w + v4.w);
            *(float4 *)&sk[r][4 * c4] = rk[k];
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int e = tid + 256 * k, r = e / 8, c4 = e % 8;
            *(float4 *)&sp[r][4 * c4] = rp[k];
        }
    };
    load(0);
    for (uint32_t d0 = 0; d0 < dk; d0 += kADC) {
        store(d0);
        __syncthreads();
        if (d0 + kADC < dk)
            load(d0 + kADC);
#pragma unroll
        for (int c = 0; c < kADC; c += 4) {
            float4 qu[4], qv[4], kk[4], pp[7];
#pragma unroll
            for (int a = 0; a < 4; a++) {
                qu[a] = *(const float4 *)&squ[ti + 16 * a][c];
                qv[a] = *(const float4 *)&sqv[ti + 16 * a][c];
                kk[a] = *(const float4 *)&sk[tj + 16 * a][c];
            }
            /* query ti + 16a against key tj + 16b reads local position row
             * 63 - ti + tj + 16 (b - a) */
#pragma unroll
            for (int e = 0; e < 7; e++)
                pp[e] = *(const float4 *)&sp[kAT - 1 - ti + tj + 16 * (e - 3)][c];
            /* the four dimensions in order, every chain one FMA each */
#define PK_ATT_DIM(F)                                                              \
    _Pragma("unroll") for (int a = 0; a < 4; a++)                                \
        _Pragma("unroll") for (int b = 0; b < 4; b++) {                          \
            sc[a][b] = __builtin_fmaf(kk[b].F, qu[a].F, sc[a][b]);               \
            bd[a][b] = __builtin_fmaf(pp[b - a + 3].F, qv[a].F, bd[a][b]);       \
        }
            PK_ATT_DIM(x) PK_ATT_DIM(y) PK_ATT_DIM(z) PK_ATT_DIM(w)
#undef PK_ATT_DIM
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t i = i0 + ti + 16 * a, j = j0 + tj + 16 * b;
            if (i < T && j < T)
                S[((size_t)h * T + i) * Ts + j] = sc[a][b] + bd[a][b];
        }
}

/* backend/ref/kernels.c:134-147 on rows of T scores, 16 lanes a row
 * (lane l takes keys l, l + 16, ... in order): each score becomes e, and
 * the row's 1 / sum goes to inv; the multiply is PV's. */
__global__ __launch_bounds__(256) void att_softmax_kernel(float *__restrict__ S, float *__restrict__ inv,
                                                          uint32_t Ts, uint32_t rows, uint32_t T, float scale) {
    const uint32_t row = blockIdx.x * 16 + (threadIdx.x >> 4), l = threadIdx.x & 15;
    if (row >= rows)
        return;
    float *x = S + (size_t)row * Ts;
    float m = -INFINITY;
#pragma unroll 8
    for (uint32_t j = l; j < T; j += 16)
        m = __builtin_fmaxf(m, x[j] * scale);
    m = __builtin_fmaxf(m, __shfl_xor(m, 8, 16));
    m = __builtin_fmaxf(m, __shfl_xor(m, 4, 16));
    m = __builtin_fmaxf(m, __shfl_xor(m, 2, 16));
    m = __builtin_fmaxf(m, __shfl_xor(m, 1, 16));
    float acc = 0.0f;
#pragma unroll 8
    for (uint32_t j = l; j < T; j += 16) {
        const float e = pk_expf(x[j] * scale - m);
        x[j] = e;
        acc += e;
    }
    const float r = 1.0f / lanes16_sum(acc);
    if (l == 0)
        inv[row] = r;
}

/* The same for rows of at most 16 REG keys: a lane's keys l, l + 16, ...
 * loaded at once into registers (one memory round trip a row instead of one
 * a few keys), the max, then e and the chain from registers in key order. */
template <int REG>
__global__ __launch_bounds__(256) void att_softmax_reg_kernel(float *__restrict__ S, float *__restrict__ inv,
                                                              uint32_t Ts, uint32_t rows, uint32_t T, float scale) {
    const uint32_t row = blockIdx.x * 16 + (threadIdx.x >> 4), l = threadIdx.x & 15;
    if (row >= rows)
        return;
    float *x = S + (size_t)row * Ts;
    float v[REG];
#pragma unroll
    for (int k = 0; k < REG; k++) {
        const uint32_t j = l + 16 * k;
        v[k] = j < T ? x[j] : 0.0f;
    }
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < REG; k++)
        if (l + 16 * k < T)
            m = __builtin_fmaxf(m, v[k] * scale);
    m = __builtin_fmaxf(m, __shfl_xor(m, 8, 16));
    m = __builtin_fmaxf(m, __shfl_xor(m, 4, 16));
    m = __builtin_fmaxf(m, __shfl_xor(m, 2, 16));
    m = __builtin_fmaxf(m, __shfl_xor(m, 1, 16));
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < REG; k++) {
        const uint32_t j = l + 16 * k;
        if (j < T) {
            const float e = pk_expf(v[k] * scale - m);
            x[j] = e;
            acc += e;
        }
    }
    const float r = 1.0f / lanes16_sum(acc);
    if (l == 0)
        inv[row] = r;
}

constexpr int kPI = 32, kPD = 32, kPJ = 32;    /* queries, dimensions, keys a stage of PV */

__global__ __launch_bounds__(128) void att_pv_kernel(float *__restrict__ of, const float *__restrict__ S,
                                                     const float *__restrict__ inv, uint32_t Ts,
                                                     const float *__restrict__ vf, uint32_t T, uint32_t D,
                                                     uint32_t dk) {
    constexpr int SPS = kPI + 4, SVS = kPD + 4;
    constexpr int NP = kPI * kPJ / 128, NV = kPJ * kPD / 128;
    __shared__ __attribute__((aligned(16))) float sPt[2][kPJ][SPS], sV[2][kPJ][SVS];
    const uint32_t d0 = blockIdx.x * kPD, i0 = blockIdx.y * kPI, h = blockIdx.z;
    const int tid = threadIdx.x, tq = tid >> 4, td = tid & 15;    /* queries 4 tq .. +3, dims 2 td, +1 */
    const float *Sh = S + (size_t)h * T * Ts;
    const uint32_t col = h * dk + d0;
    float acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; a++)
        acc[a][0] = acc[a][1] = 0.0f;
    /* the rows a thread stages stay the same: their 1 / sum */
    float rinv[NP], rp[NP], rv[NV];
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const uint32_t i = i0 + (tid + 128 * k) / kPJ;
        rinv[k] = i < T ? inv[(size_t)h * T + i] : 0.0f;
    }
    auto load = [&](uint32_t j0) {
#pragma unroll
        for (int k = 0; k < NP; k++) {
            const int e = tid + 128 * k, r = e / kPJ, c = e % kPJ;
            const uint32_t i = i0 + r, j = j0 + c;
            rp[k] = i < T && j < T ? Sh[(size_t)i * Ts + j] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int e = tid + 128 * k, r = e / kPD, c = e % kPD;
            const uint32_t j = j0 + r;
            rv[k] = j < T ? vf[(size_t)j * D + col + c] : 0.0f;
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int k = 0; k < NP; k++) {
            const int e = tid + 128 * k;
            sPt[buf][e % kPJ][e / kPJ] = rp[k] * rinv[k];
        }
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int e = tid + 128 * k;
            sV[buf][e / kPD][e % kPD] = rv[k];
        }
    };
    auto step = [&](int buf, int c) {
        const float4 p = *(const float4 *)&sPt[buf][c][4 * tq];
        const float2 v = *(const float2 *)&sV[buf][c][2 * td];
        acc[0][0] = __builtin_fmaf(v.x, p.x, acc[0][0]);
        acc[0][1] = __builtin_fmaf(v.y, p.x, acc[0][1]);
        acc[1][0] = __builtin_fmaf(v.x, p.y, acc[1][0]);
        acc[1][1] = __builtin_fmaf(v.y, p.y, acc[1][1]);
        acc[2][0] = __builtin_fmaf(v.x, p.z, acc[2][0]);
        acc[2][1] = __builtin_fmaf(v.y, p.z, acc[2][1]);
        acc[3][0] = __builtin_fmaf(v.x, p.w, acc[3][0]);
        acc[3][1] = __builtin_fmaf(v.y, p.w, acc[3][1]);
    };
    load(0);
    store(0);
    __syncthreads();
    int buf = 0;
    for (uint32_t j0 = 0; j0 < T; j0 += kPJ) {
        const bool more = j0 + kPJ < T;
        if (more)
            load(j0 + kPJ);
        if (T - j0 >= (uint32_t)kPJ) {
#pragma unroll
            for (int c = 0; c < kPJ; c++)
                step(buf, c);
        } else {
            /* exactly the T keys: a padding term would turn a -0 sum into +0 */
            const int jn = (int)(T - j0);
            for (int c = 0; c < jn; c++)
                step(buf, c);
        }
        if (more)
            store(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const uint32_t i = i0 + 4 * tq + a;
        if (i < T)
            *(float2 *)(of + (size_t)i * D + col + 2 * td) = make_float2(acc[a][0], acc[a][1]);
    }
}

/* ------------------------------------------------- attention on MFMA --
 *
 * The same chains on the matrix cores: v_mfma_f32_32x32x1_2b_f32 and
 * v_mfma_f32_16x16x1_4b_f32 have one input step (K = 1), so each output
 * takes exactly one product and one add a step, d = fma(a, b, d) with one
 * rounding (measured equal to v_fma_f32 on 1.2M outputs of every class of
 * input: subnormals, both zeros, infinities, NaN, exact cancellation; the
 * attention tests compare both paths with the oracle on such operands). A
 * chain of steps in the reference's order is then the reference's fmaf
 * chain, at the matrix cores' rate and with each operand one register a
 * lane for 2048 (or 1024) chains.
 *
 * 32x32x1_2b: two blocks of 32 x 32; lane l gives A[l / 32][l % 32] and
 * B[l / 32][l % 32]; output register r of lane l is block r / 16, row
 * 8 ((r % 16) / 4) + 4 (l / 32) + r % 4, column l % 32.
 * 16x16x1_4b: four blocks of 16 x 16; lane l gives A[l / 16][l % 16] and
 * B[l / 16][l % 16]; output register r of lane l is block r / 4, row
 * 4 (l / 16) + r % 4, column l % 16.
 *
 * The scores (content, then the position band added in) and PV, each
 * with its operands staged through LDS (below). */
typedef float v32f __attribute__((ext_vector_type(32)));
typedef float v16f __attribute__((ext_vector_type(16)));

/* The scores' chains over the head's dimensions, staged through LDS: a
 * workgroup 64 queries x 128 rows of y (keys; or, BAND, the position rows m
 * of the band its queries reach), wave (wq, wy) 32 queries x 64 rows on
 * 32x32x1_2b (its two blocks the two halves of its rows); dimensions in
 * stages of 16, double-buffered (30 KB: five workgroups a CU), each row's
 * 16 dimensions contiguous (rows padded to 20 floats: a wave's 16-byte
 * reads of 16 rows fall in distinct banks), a stage's operands read into
 * registers before its MFMAs: A = x + bias (one rounding, formed as staged), B = y. Content: S =
 * the chain. Band: S(i, j) = S(i, j) + the chain of (i, m) for m = T - 1 - i
 * + j, j a key (each (i, j) one lane's in the grid; the workgroup's rows
 * start at T - 1 - (i0 + 63), negative at the last query tiles, whose rows
 * there meet no key). */
constexpr int kSQ = 64, kSY = 128, kSD = 16, kSP = kSD + 4;

template <bool BAND>
__global__ __launch_bounds__(256) void att_dims_kernel(float *__restrict__ S, uint32_t Ts,
                                                       const float *__restrict__ xf, const float *__restrict__ yf,
                                                       const float *__restrict__ bias, uint32_t T, uint32_t D,
                                                       uint32_t dk) {
    __shared__ __attribute__((aligned(16))) float sa[2][kSQ][kSP], sb[2][kSY][kSP];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wq = w & 1, wy = w >> 1;
    const uint32_t h = blockIdx.z, i0 = blockIdx.y * kSQ;
    const uint32_t R = BAND ? 2 * T - 1 : T;
    const int64_t y0 = BAND ? (int64_t)T - 1 - (int64_t)(i0 + kSQ - 1) + (int64_t)blockIdx.x * kSY
                            : (int64_t)blockIdx.x * kSY;
    if (BAND && y0 > (int64_t)(2 * T - 2) - (int64_t)i0)
        return;                                         /* the whole workgroup: no row meets a key */
    const uint32_t col = h * dk;
    /* staging: x row tid % 64, dimensions 4 (tid / 64); y row tid % 128,
     * dimensions 4 (tid / 128 + 2 k), k < 2 */
    const int xrw = tid & 63, yrw = tid & 127;
    const uint32_t xi = min(i0 + xrw, T - 1);
    const int64_t yl = y0 + yrw;
    const uint32_t yi = (uint32_t)(yl < 0 ? 0 : yl >= (int64_t)R ? R - 1 : yl);
    const float *xr = xf + (size_t)xi * D + col, *yr = yf + (size_t)yi * D + col, *br = bias + col;
    /* a stage's loads, two sets in registers: stage s + 2 is loaded while
     * stage s is multiplied, so each load has two stages to land */
    struct Regs {
        float4 x, b, y[2];
    };
    const uint32_t ns = dk / kSD, last = (ns - 1) * kSD;
    auto load = [&](Regs &g, uint32_t d0) {
        d0 = d0 < last ? d0 : last;                 /* past the end: the last again, in bounds */
        g.x = *(const float4 *)(xr + d0 + 4 * (tid >> 6));
        g.b = *(const float4 *)(br + d0 + 4 * (tid >> 6));
#pragma unroll
        for (int k = 0; k < 2; k++)
            g.y[k] = *(const float4 *)(yr + d0 + 4 * ((tid >> 7) + 2 * k));
    };
    auto store = [&](const Regs &g, int b) {
        *(float4 *)&sa[b][xrw][4 * (tid >> 6)] = make_float4(g.x.x + g.b.x, g.x.y + g.b.y, g.x.z + g.b.z,
                                                             g.x.w + g.b.w);
#pragma unroll
        for (int k = 0; k < 2; k++)
            *(float4 *)&sb[b][yrw][4 * ((tid >> 7) + 2 * k)] = g.y[k];
    };
    v32f acc;
#pragma unroll
    for (int r = 0; r < 32; r++)
        acc[r] = 0.0f;
    const int ac = 32 * wq + (lane & 31), bc = 64 * wy + lane;
    auto mult = [&](int b) {
        float4 a4[kSD / 4], b4[kSD / 4];
#pragma unroll
        for (int k = 0; k < kSD / 4; k++) {
            a4[k] = *(const float4 *)&sa[b][ac][4 * k];
            b4[k] = *(const float4 *)&sb[b][bc][4 * k];
        }
#pragma unroll
        for (int k = 0; k < kSD / 4; k++) {
            acc = __builtin_amdgcn_mfma_f32_32x32x1f32(a4[k].x, b4[k].x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x1f32(a4[k].y, b4[k].y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x1f32(a4[k].z, b4[k].z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x1f32(a4[k].w, b4[k].w, acc, 0, 0, 0);
        }
    };
    /* ns is even (dk a multiple of 64): stages in pairs, the buffers and
     * register sets alternating statically. No load is issued for a stage
     * past the last: one still in flight at the end would hold every
     * output store behind a wait for it (its registers are reused), which
     * cost a workgroup ~5 us of its ~14. */
    Regs g0, g1;
    load(g0, 0);
    load(g1, kSD);
    store(g0, 0);
    __syncthreads();
    for (uint32_t st = 0; st < ns; st += 2) {
        const bool more = st + 2 < ns;
        if (more)
            load(g0, (st + 2) * kSD);
        mult(0);
        store(g1, 1);
        __syncthreads();
        if (more)
            load(g1, (st + 3) * kSD);
        mult(1);
        if (more)
            store(g0, 0);
        __syncthreads();
    }
    /* nothing is in flight here; saying so spares the stores below a wait
     * each for loads the compiler cannot rule out */
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));      /* vmcnt(0) */
    if (!BAND) {
#pragma unroll
        for (int r = 0; r < 32; r++) {
            const uint32_t rr = r & 15;
            const uint32_t qi = i0 + 32 * wq + 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);
            const int64_t kj = y0 + 64 * wy + 32 * (r >> 4) + (lane & 31);
            if (qi < T && kj < (int64_t)T)
                S[((size_t)h * T + qi) * Ts + (uint32_t)kj] = acc[r];
        }
    } else {
        /* all 32 old scores first, one wait, then their sums: no store
         * waits on another (no two registers hold the same (i, j); a load
         * issued after a store would wait for it, the counter being in
         * order); offsets from the head's scores fit 32 bits (the launcher
         * checks) */
        float *Sh = S + (size_t)h * T * Ts;
        uint32_t at[32];
        float old[32];
#pragma unroll
        for (int r = 0; r < 32; r++) {
            const int blk = r >> 4, rr = r & 15;
            const uint32_t qi = i0 + 32 * wq + 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);
            const int64_t kj = y0 + 64 * wy + 32 * blk + (lane & 31) - ((int64_t)T - 1 - (int64_t)qi);
            const bool in = qi < T && kj >= 0 && kj < (int64_t)T;
            at[r] = in ? qi * Ts + (uint32_t)kj : ~0u;
            old[r] = in ? Sh[at[r]] : 0.0f;
        }
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));      /* vmcnt(0) */
#pragma unroll
        for (int r = 0; r < 32; r++)
            if (at[r] != ~0u)
                Sh[at[r]] = old[r] + acc[r];
    }
}

/* PV: a workgroup 64 queries x 64 dimensions of a head, wave w the queries
 * i0 + 16 w .. + 15 (16x16x1_4b, its four blocks the 64 dimensions); keys
 * in stages of 64 through LDS, double-buffered (a stage's loads are in
 * flight for a stage's 64 MFMAs): the probabilities P = e * (1 / sum)
 * (formed as staged) query-major and the values dimension-major, each row
 * of keys contiguous and padded to 68 floats, so that a lane reads four
 * keys of its query (A) or of its dimension (B) with one 16-byte read, in
 * distinct banks across the wave; 32 keys' operands are read into
 * registers before their MFMAs. Exactly the T keys are multiplied. */
constexpr int kPVK = 64, kPVS = kPVK + 4;

__global__ __launch_bounds__(256) void att_pv_mfma_kernel(float *__restrict__ of, const float *__restrict__ S,
                                                          const float *__restrict__ inv, uint32_t Ts,
                                                          const float *__restrict__ vf, uint32_t T, uint32_t D,
                                                          uint32_t dk, int8_t *__restrict__ qp,
                                                          float *__restrict__ qd, uint32_t qb) {
    __shared__ __attribute__((aligned(16))) float sv[2][64][kPVS], sp[2][64][kPVS];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t h = blockIdx.z, d0 = blockIdx.y * 64, i0 = blockIdx.x * 64;
    const float *Sh = S + (size_t)h * T * Ts;
    const float *vh = vf + (size_t)h * dk + d0;
    /* staging: values key tid % 64, dimensions 4 (tid / 64 + 4 k); the
     * probabilities query tid / 16 + 16 k, keys 4 (tid % 16); k < 4 */
    const int vk = tid & 63, pr = tid >> 4, pc = 4 * (tid & 15);
    float rinv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t i = i0 + pr + 16 * k;
        rinv[k] = i < T ? inv[(size_t)h * T + i] : 0.0f;
    }
    float4 rv[4], rp[4];
    auto load = [&](uint32_t j0) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t j = j0 + vk;
            rv[k] = j < T ? *(const float4 *)(vh + (size_t)j * D + 4 * ((tid >> 6) + 4 * k))
                          : make_float4(0, 0, 0, 0);
            const uint32_t i = i0 + pr + 16 * k, jc = j0 + pc;
            rp[k] = i < T && jc < Ts ? *(const float4 *)(Sh + (size_t)i * Ts + jc) : make_float4(0, 0, 0, 0);
        }
    };
    auto store = [&](int b) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int d = 4 * ((tid >> 6) + 4 * k);
            sv[b][d][vk] = rv[k].x;
            sv[b][d + 1][vk] = rv[k].y;
            sv[b][d + 2][vk] = rv[k].z;
            sv[b][d + 3][vk] = rv[k].w;
            const float4 e = rp[k];
            const float r = rinv[k];
            *(float4 *)&sp[b][pr + 16 * k][pc] = make_float4(e.x * r, e.y * r, e.z * r, e.w * r);
        }
    };
    v16f acc;
#pragma unroll
    for (int r = 0; r < 16; r++)
        acc[r] = 0.0f;
    const int arow = 16 * w + (lane & 15);
    load(0);
    store(0);
    __syncthreads();
    const uint32_t ns = (T + kPVK - 1) / kPVK;
    for (uint32_t st = 0; st < ns; st++) {
        const int b = st & 1;
        const uint32_t j0 = st * kPVK;
        if (st + 1 < ns)
            load(j0 + kPVK);
        if (T - j0 >= (uint32_t)kPVK) {
#pragma unroll
            for (int half = 0; half < 2; half++) {
                float4 a4[8], b4[8];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    a4[k] = *(const float4 *)&sp[b][arow][32 * half + 4 * k];
                    b4[k] = *(const float4 *)&sv[b][lane][32 * half + 4 * k];
                }
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    acc = __builtin_amdgcn_mfma_f32_16x16x1f32(a4[k].x, b4[k].x, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x1f32(a4[k].y, b4[k].y, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x1f32(a4[k].z, b4[k].z, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x1f32(a4[k].w, b4[k].w, acc, 0, 0, 0);
                }
            }
        } else {
            /* exactly the T keys: a padding step would turn a -0 sum into +0 */
            const int nk = (int)(T - j0);
            for (int c = 0; c < nk; c++)
                acc = __builtin_amdgcn_mfma_f32_16x16x1f32(sp[b][arow][c], sv[b][lane][c], acc, 0, 0, 0);
        }
        if (st + 1 < ns)
            store(b ^ 1);
        __syncthreads();
    }
    if (!qp) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const uint32_t qi = i0 + 16 * w + 4 * (lane >> 4) + (r & 3);
            if (qi < T)
                of[(size_t)qi * D + h * dk + d0 + 16 * (r >> 2) + (lane & 15)] = acc[r];
        }
        return;
    }
    /* The outputs quantized in blocks of qb (32 or 64) channels of a frame,
     * as a quantize of them would (core/encoder.c:344-346), straight into
     * the output projection's packed activations and scales. Register r of
     * lane l is frame 4 (l / 16) + r % 4 of the wave's 16, channel 16 (r /
     * 4) + l % 16 of the tile's 64: a block is one or two register groups
     * r / 4 over the 16 lanes of a DPP row. The tile's four units (16
     * frames x 64 channels each) are put together in LDS and leave as
     * 16-byte stores. */
    const uint32_t c0 = h * dk + d0, G = (T + 15) / 16, NB = D / qb;
    int8_t *unit = (int8_t *)&sp[0][0][0];             /* 4 KB, free after the loop */
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++) {
        const uint32_t t = i0 + 16 * w + 4 * (lane >> 4) + s4;
#pragma unroll
        for (int bk = 0; bk < 2; bk++) {
            /* blocks of 64: one block of register groups 0..3 (bk 0 only);
             * blocks of 32: block bk of groups 2 bk, 2 bk + 1 */
            if (qb == 64 && bk == 1)
                continue;
            const int g0 = qb == 64 ? 0 : 2 * bk, ng = qb == 64 ? 4 : 2;
            int m = 0;
#pragma unroll
            for (int gi = 0; gi < 4; gi++)
                if (gi < ng)
                    m = max(m, mag_bits(acc[4 * (g0 + gi) + s4]));
            bool zero;
            float dv, id;
            block_scales((uint32_t)group_max_nonneg<16>(m), zero, dv, id);
#pragma unroll
            for (int gi = 0; gi < 4; gi++)
                if (gi < ng) {
                    const int gr = g0 + gi;
                    unit[(16 * w + 4 * (lane >> 4) + s4) / 16 * kUnitBytes +
                         in_unit(16 * gr + (lane & 15), (4 * (lane >> 4) + s4) & 15)] =
                        (int8_t)(zero ? 0 : q1(acc[4 * gr + s4], id));
                }
            if (t < T && (lane & 15) == 0)
                qd[(size_t)t * NB + (c0 + 16 * g0) / qb] = dv;
        }
    }
    __syncthreads();
    {
        const uint32_t gt = tid / 64, g = i0 / 16 + gt;   /* unit gt of the tile: frames 16 gt .. */
        if (g < G)
            *(v4i *)(qp + ((size_t)(c0 / 64) * G + g) * kUnitBytes + 16 * (tid & 63)) =
                *(const v4i *)(unit + gt * kUnitBytes + 16 * (tid & 63));
    }
}

/* --------------------------------------------------------------- dwq --
 *
 * core/encoder.c:158-176 (glu_item, dw_item): h = GLU(u) (backend/ref/
 * kernels.c:157-161), the depthwise convolution of K taps with its bias
 * and SiLU (backend/ref/kernels.c:163-176, the taps past the ends skipped),
 * and the blocks' quantize of each frame's 64 channels (whole blocks of 32
 * or 64). One workgroup a group of 16 frames and 64 channels, which is one
 * packed unit: h for the frames the taps reach goes through LDS, a lane
 * takes a channel, and the unit is put together in LDS and leaves as 1 KB. */
constexpr int kMaxTaps = 33;

__device__ __forceinline__ int half_max_nonneg(int v, int lane) {
    v = group_max_nonneg<16>(v);
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false));   /* row_bcast15: rows 1, 3 */
    const int lo = __builtin_amdgcn_readlane(v, 31), hi = __builtin_amdgcn_readlane(v, 63);
    return lane < 32 ? lo : hi;
}

template <int QB>
__global__ __launch_bounds__(256) void dwq_kernel(int8_t *__restrict__ qp, float *__restrict__ d,
                                                  const float *__restrict__ u, uint32_t T, uint32_t D,
                                                  const float *__restrict__ w, const float *__restrict__ b,
                                                  uint32_t K) {
    __shared__ float hs[16 + kMaxTaps - 1][64];
    __shared__ float wl[kMaxTaps][64];
    __shared__ __attribute__((aligned(16))) int8_t unit[kUnitBytes];
    const uint32_t g = blockIdx.x, G = gridDim.x, c0 = blockIdx.y * 64, t0 = 16 * g;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int64_t half = K / 2;
    const uint32_t rows = 16 + K - 1;
    /* GLU of the frames the taps reach: every load of a thread issued before
     * the first gate (one memory round trip), then h = a * sigmoid(g) */
    constexpr int kPT = (16 + kMaxTaps - 1) * 64 / 256;
    float ua[kPT], ug[kPT];
#pragma unroll
    for (int k = 0; k < kPT; k++) {
        const uint32_t e = tid + 256 * k, r = e / 64, c = e % 64;
        const int64_t s = (int64_t)t0 - half + r;
        const bool in = e < rows * 64 && s >= 0 && s < (int64_t)T;
        const float *us = u + (size_t)(in ? s : 0) * 2 * D + c0 + c;
        ua[k] = in ? us[0] : 0.0f;
        ug[k] = in ? us[D] : 0.0f;
    }
    /* the 64 channels' taps, tap-major */
    for (uint32_t e = tid; e < K * 64; e += 256)
        wl[e / 64][e % 64] = w[(size_t)(c0 + e % 64) * K + e / 64];
#pragma unroll
    for (int k = 0; k < kPT; k++) {
        const uint32_t e = tid + 256 * k, r = e / 64, c = e % 64;
        const int64_t s = (int64_t)t0 - half + r;
        if (e < rows * 64)
            hs[r][c] = s >= 0 && s < (int64_t)T ? ua[k] * pk_sigmoidf(ug[k]) : 0.0f;
    }
    __syncthreads();
    const uint32_t c = c0 + lane;
    const float bc = b[c];
    /* the wave's four frames side by side, each its own chain over the taps
     * in order (the taps past the ends skipped), so the four chains' steps
     * overlap */
    float acc[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
    for (uint32_t j = 0; j < K; j++) {
        const float wj = wl[j][lane];
#pragma unroll
        for (int f = 0; f < 4; f++) {
            const uint32_t r = 4 * wv + f;
            const int64_t s = (int64_t)t0 + r + j - half;
            if (s >= 0 && s < (int64_t)T)
                acc[f] = __builtin_fmaf(wj, hs[r + j][lane], acc[f]);
        }
    }
    /* the four frames' SiLU and block maxima, independent of each other */
    float y[4];
    uint32_t mbs[4];
#pragma unroll
    for (int f = 0; f < 4; f++) {
        y[f] = 0.0f;
        if (t0 + 4 * wv + f < T) {
            const float v = acc[f] + bc;
            y[f] = v * pk_sigmoidf(v);
        }
    }
#pragma unroll
    for (int f = 0; f < 4; f++)
        mbs[f] = (uint32_t)(QB == 64 ? wave_max_nonneg(mag_bits(y[f])) : half_max_nonneg(mag_bits(y[f]), lane));
#pragma unroll
    for (int f = 0; f < 4; f++) {
        const uint32_t r = 4 * wv + f, t = t0 + r;
        const uint32_t mb = mbs[f];
        const bool zero = zero_bits(mb);
        float dv = 0.0f, id = 0.0f;
        if (!zero) {
            const float amax = __uint_as_float(mb);
            dv = amax / 127.0f;
            id = 127.0f / amax;
        }
        unit[in_unit(lane, r)] = (int8_t)(zero ? 0 : q1(y[f], id));
        if (t < T && lane % QB == 0)
            d[(size_t)t * (D / QB) + c / QB] = dv;
    }
    __syncthreads();
    if (tid < 64)
        *(v4i *)(qp + ((size_t)(c0 / 64) * G + g) * kUnitBytes + 16 * tid) = *(const v4i *)(unit + 16 * tid);
}

/* ---------------------------------------------------------- launchers -- */

int launch_normq(int8_t *qp, float *d, const float *x, uint32_t n, uint32_t T, const float *w, const float *b,
                 float eps, uint32_t qb, hipStream_t s) {
    if (T == 0)
        return 0;
    if (n % 64 || n > 4096 || !(qb == n || qb == 32 || qb == 64))
        return -2;
    const uint32_t grid = (T + 3) / 4;
    const bool small = n <= 1024;
#define PK_NQ(CH, QB) normq_kernel<CH, QB><<<grid, 256, 0, s>>>(qp, d, x, n, T, w, b, eps)
    if (qb == n) {
        if (small) PK_NQ(4, 0); else PK_NQ(16, 0);
    } else if (qb == 32) {
        if (small) PK_NQ(4, 32); else PK_NQ(16, 32);
    } else {
        if (small) PK_NQ(4, 64); else PK_NQ(16, 64);
    }
#undef PK_NQ
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

int launch_norm(float *x, uint32_t n, uint32_t T, const float *w, const float *b, float eps, hipStream_t s) {
    if (T == 0)
        return 0;
    if (n % 64 || n > 4096)
        return -2;
    if (n <= 1024)
        norm_kernel<4><<<(T + 3) / 4, 256, 0, s>>>(x, n, T, w, b, eps);
    else
        norm_kernel<16><<<(T + 3) / 4, 256, 0, s>>>(x, n, T, w, b, eps);
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

/* Heads whose width is not a multiple of 64 (the tiled kernels' stage):
 * one thread an output, the same chains in the same order. A score is the
 * content chain fma(k, q + u) and the position chain fma(p_m, q + v) over
 * the head's dimensions in order from +0, m = T - 1 - i + j, then their sum;
 * an output is the chain fma(v_j, e_ij * (1 / sum_i)) over the T keys in
 * order from +0. Made for narrow heads at short lengths (the tiny models'
 * 16-wide heads): each thread walks its chains serially from global memory,
 * so the time grows as T^2 * D with no tiling at all; at thousands of frames
 * with 80- or 96-wide heads this is many times the tiled kernels' time for
 * 64-wide heads of the same model size. */
__global__ __launch_bounds__(256) void att_scores_small_kernel(float *__restrict__ S, uint32_t Ts,
                                                               const float *__restrict__ qf,
                                                               const float *__restrict__ kf,
                                                               const float *__restrict__ pf,
                                                               const float *__restrict__ bu,
                                                               const float *__restrict__ bv, uint32_t T,
                                                               uint32_t D, uint32_t dk) {
    const uint64_t id = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint32_t H = D / dk;
    if (id >= (uint64_t)H * T * T)
        return;
    const uint32_t j = (uint32_t)(id % T), i = (uint32_t)(id / T % T), h = (uint32_t)(id / ((uint64_t)T * T));
    const float *q = qf + (size_t)i * D + h * dk, *k = kf + (size_t)j * D + h * dk;
    const float *p = pf + (size_t)(T - 1 - i + j) * D + h * dk, *u = bu + h * dk, *v = bv + h * dk;
    float sc = 0.0f, bd = 0.0f;
    for (uint32_t d = 0; d < dk; d++) {
        sc = __builtin_fmaf(k[d], q[d] + u[d], sc);
        bd = __builtin_fmaf(p[d], q[d] + v[d], bd);
    }
    S[((size_t)h * T + i) * Ts + j] = sc + bd;
}

__global__ __launch_bounds__(256) void att_pv_small_kernel(float *__restrict__ of, const float *__restrict__ S,
                                                           const float *__restrict__ inv, uint32_t Ts,
                                                           const float *__restrict__ vf, uint32_t T, uint32_t D,
                                                           uint32_t dk) {
    const uint64_t id = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= (uint64_t)T * D)
        return;
    const uint32_t d = (uint32_t)(id % D), i = (uint32_t)(id / D), h = d / dk;
    const float *e = S + ((size_t)h * T + i) * Ts;
    const float r = inv[(size_t)h * T + i];
    float acc = 0.0f;
    for (uint32_t j = 0; j < T; j++)
        acc = __builtin_fmaf(vf[(size_t)j * D + d], e[j] * r, acc);
    of[(size_t)i * D + d] = acc;
}

/* The attention's kernels: 0 the matrix cores' (the default), 1 the VALU
 * chains; both compute the same bits. */
static int g_att_valu = 0;

int set_attention_kernels(int valu) {
    const int was = g_att_valu;
    g_att_valu = valu ? 1 : 0;
    return was;
}

uint32_t att_score_stride(uint32_t T) { return (T + 3) & ~3u; }

/* ---------------------------------------------------- static scratch --
 *
 * The attention's scores and row sums for callers that cannot allocate
 * (pk_hip_attention_noalloc_dev): a file-scope device array of
 * kStaticScratchBytes, which every GPU the library runs on holds from the
 * code object's load until the process ends. Host code never names the
 * array as memory: its address on a device is taken once, with that device
 * current (hipGetSymbolAddress), kept per device, and that address is what
 * the kernels are given. Every call on one GPU shares its array: calls that
 * overlap on one GPU race. */
static __device__ __align__(256) char scratch[kStaticScratchBytes];

static std::mutex g_scratch_mu;
static void *g_scratch_at[kMaxDevices];
static hipEvent_t g_scratch_ev[kMaxDevices];

void *static_scratch(int dev, int *err, hipEvent_t *last) {
    if (dev < 0 || dev >= kMaxDevices) {
        *err = (int)hipErrorInvalidDevice;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_at[dev]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev)
            e = hipErrorInvalidDevice;      /* the caller makes dev current first */
        void *p = nullptr;
        if (e == hipSuccess)
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        hipEvent_t ev = nullptr;
        if (e == hipSuccess && p)
            e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess || !p) {
            /* HIP keeps a failed call's error until it is read: read it
             * here, so that the next launch of any entry on this thread
             * does not report it as its own */
            (void)hipGetLastError();
            *err = (int)(e != hipSuccess ? e : hipErrorInvalidSymbol);
            return nullptr;
        }
        g_scratch_at[dev] = p;
        g_scratch_ev[dev] = ev;
    }
    *err = 0;
    if (last)
        *last = g_scratch_ev[dev];
    return g_scratch_at[dev];
}

size_t att_workspace_floats(uint32_t T, uint32_t H) {
    /* the scores, then each row's 1 / sum (16-byte aligned: the stride is
     * a multiple of 4 floats) */
    return (size_t)H * T * att_score_stride(T) + (size_t)H * T;
}

int launch_attention(float *of, float *ws, const float *qf, const float *kf, const float *vf, const float *pf,
                     const float *bu, const float *bv, uint32_t T, uint32_t D, uint32_t H, hipStream_t s,
                     int8_t *qp, float *qd, uint32_t qb) {
    if (T == 0)
        return 0;
    if (H == 0 || D % H || (D / H) % 16 || (uint64_t)T * att_score_stride(T) >= (1ull << 32) - 1)
        return -2;
    const bool small = (D / H) % 64 != 0;
    if (qp && (g_att_valu || small || !(qb == 32 || qb == 64)))
        return -2;                                  /* no quantizing epilogue there: nothing launched */
    const uint32_t dk = D / H, Ts = att_score_stride(T), tiles = (T + kAT - 1) / kAT, rows = H * T;
    float *S = ws, *inv = ws + (size_t)rows * Ts;
    if (small) {
        const uint64_t n = (uint64_t)H * T * T;
        att_scores_small_kernel<<<(uint32_t)((n + 255) / 256), 256, 0, s>>>(S, Ts, qf, kf, pf, bu, bv, T, D, dk);
    } else if (g_att_valu) {
        att_scores_kernel<<<dim3(tiles, tiles, H), 256, 0, s>>>(S, Ts, qf, kf, pf, bu, bv, T, D, dk);
    } else {
        const uint32_t qt = (T + kSQ - 1) / kSQ;
        att_dims_kernel<false><<<dim3((T + kSY - 1) / kSY, qt, H), 256, 0, s>>>(S, Ts, qf, kf, bu, T, D, dk);
        att_dims_kernel<true><<<dim3((T + kSQ - 1 + kSY - 1) / kSY, qt, H), 256, 0, s>>>(S, Ts, qf, pf, bv, T, D, dk);
    }
    const float scale = 1.0f / sqrtf((float)dk);
    if (T <= 16 * 16)
        att_softmax_reg_kernel<16><<<(rows + 15) / 16, 256, 0, s>>>(S, inv, Ts, rows, T, scale);
    else if (T <= 16 * 64)
        att_softmax_reg_kernel<64><<<(rows + 15) / 16, 256, 0, s>>>(S, inv, Ts, rows, T, scale);
    else
        att_softmax_kernel<<<(rows + 15) / 16, 256, 0, s>>>(S, inv, Ts, rows, T, scale);
    if (small)
        att_pv_small_kernel<<<(uint32_t)(((uint64_t)T * D + 255) / 256), 256, 0, s>>>(of, S, inv, Ts, vf, T, D, dk);
    else if (g_att_valu)
        att_pv_kernel<<<dim3(dk / kPD, (T + kPI - 1) / kPI, H), 128, 0, s>>>(of, S, inv, Ts, vf, T, D, dk);
    else
        att_pv_mfma_kernel<<<dim3((T + 63) / 64, dk / 64, H), 256, 0, s>>>(of, S, inv, Ts, vf, T, D, dk, qp, qd,
                                                                            qb);
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

int launch_dwq(int8_t *qp, float *d, const float *u, uint32_t T, uint32_t D, const float *w, const float *b,
               uint32_t K, uint32_t qb, hipStream_t s) {
    if (T == 0)
        return 0;
    if (D % 64 || K == 0 || K > (uint32_t)kMaxTaps || !(qb == 32 || qb == 64))
        return -2;
    const dim3 grid((T + 15) / 16, D / 64);
    if (qb == 32)
        dwq_kernel<32><<<grid, 256, 0, s>>>(qp, d, u, T, D, w, b, K);
    else
        dwq_kernel<64><<<grid, 256, 0, s>>>(qp, d, u, T, D, w, b, K);
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

}  // namespace pkq8
