/* The decoder's per-token work on the device (core/decoder.c:54-101 in
 * peterheb/libpktito): its products are T = 1 GEMVs, each a quantize of one
 * row and a product, latency-bound at a few microseconds of work. Each
 * launch here fuses what the reference runs as separate calls: the row's
 * quantize with its product (gemv), an LSTM layer's two products, their add
 * and its cell (lstm), and the joint's ReLU, quantize, product and argmax.
 *
 * Bits: the reference's ref backend's. The quantize is
 * backend/ref/kernels.c:24-58 with one block of the whole row; the sums are
 * exact int32 (v_dot4 over the repacked units, any order); the epilogue,
 * the cell (backend/ref/kernels.c:203-213) and the argmax (the first of
 * equal values) are the reference's operations in its order. Built with
 * -ffp-contract=off.
 */
#include "q8_device.h"
#include "q8_internal.h"

#pragma clang fp contract(off)

namespace pkq8 {

constexpr uint32_t kDecMaxCols = 4096;

/* Chunk i (elements 4i .. 4i + 3, 4i < n) of a row of n floats: one float4
 * load when the row is 16-byte aligned and n a multiple of 4 (AL), else
 * four loads with zeros past n. */
template <bool AL>
__device__ __forceinline__ float4 row4(const float *__restrict__ x, uint32_t i, uint32_t n) {
    if (AL)
        return ((const float4 *)x)[i];
    const uint32_t k = 4 * i;
    return make_float4(x[k], k + 1 < n ? x[k + 1] : 0.0f, k + 2 < n ? x[k + 2] : 0.0f, k + 3 < n ? x[k + 3] : 0.0f);
}

/* One row of n <= 256 CH values, quantized whole by one wave into q (LDS,
 * bytes, zero to 64 kr, kr <= 4 CH) in two steps. load_row: every lane
 * issues the loads of its chunks i + 64 c (value4(i) gives chunk i, zeros
 * past n), so the row costs one memory round trip, and the caller may
 * issue other loads behind them before it uses the row. */
template <int CH, typename F>
__device__ __forceinline__ void load_row(F value4, uint32_t n, int lane, float4 (&v)[CH]) {
    const uint32_t n4 = (n + 3) >> 2;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        v[c] = i < n4 ? value4(i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

/* quant_loaded: the loaded row quantized into q. Returns d (the block rule
 * on magnitude bits: a NaN or an infinity, or an amax below 2^-121, makes
 * the row zero). */
template <int CH>
__device__ __forceinline__ float quant_loaded(const float4 (&v)[CH], uint32_t n, uint32_t kr, int8_t *q, int lane) {
    const uint32_t n4 = (n + 3) >> 2;
    const WaveScales<CH, 0> sc(v);
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t i = lane + 64 * c;
        if (i < 16 * kr)
            ((int *)q)[i] = i < n4 && !sc.zero[0] ? pack4(v[c], sc.id[0]) : 0;
    }
    return sc.dv[0];
}

/* The exact int32 sums of the 16 rows of panel p over units [0, kr), kr <=
 * KU, in two steps. panel_load: lane l loads the unit's bytes 16 l .. 16 l
 * + 15 of each unit (the wave reads each 1 KB unit whole, every unit's load
 * issued before the first sum). panel_sum: lane l takes row l % 16 and
 * inputs 16 (l / 16) .. + 15 of each unit, and the four lanes of a row add
 * up by shuffles; every lane returns its row's sum. */
template <int KU>
__device__ __forceinline__ void panel_load(const int8_t *__restrict__ w, uint64_t wstride, uint32_t p, uint32_t kr,
                                           int lane, v4i (&wv)[KU]) {
    const int8_t *wp = w + (size_t)p * kUnitBytes + lane * 16;
#pragma unroll
    for (int u = 0; u < KU; u++)
        if (u < (int)kr)
            wv[u] = *(const v4i *)(wp + (size_t)u * wstride);
}

template <int KU>
__device__ __forceinline__ int panel_sum(const v4i (&wv)[KU], uint32_t kr, const int8_t *q, int lane) {
    const int8_t *qp = q + (lane >> 4) * 16;
    int s = 0;
#pragma unroll
    for (int u = 0; u < KU; u++)
        if (u < (int)kr) {
            const v4i av = *(const v4i *)(qp + 64 * u);
            s = __builtin_amdgcn_sdot4(wv[u][0], av[0], s, false);
            s = __builtin_amdgcn_sdot4(wv[u][1], av[1], s, false);
            s = __builtin_amdgcn_sdot4(wv[u][2], av[2], s, false);
            s = __builtin_amdgcn_sdot4(wv[u][3], av[3], s, false);
        }
    s += __shfl_xor(s, 16);
    s += __shfl_xor(s, 32);
    return s;
}

/* Whether a kernel of KU units a panel loads its panels behind its row,
 * before the quantize (one memory round trip instead of two): where the
 * panels fit the registers beside the row (the 64-unit kernels load them
 * after). */
template <int KU>
constexpr bool kEarly = KU <= 16;

template <int KU>
__device__ __forceinline__ int panel_dot(const int8_t *__restrict__ w, uint64_t wstride, uint32_t p, uint32_t kr,
                                         const int8_t *q, int lane) {
    v4i wv[KU];
    panel_load<KU>(w, wstride, p, kr, lane, wv);
    return panel_sum<KU>(wv, kr, q, lane);
}

/* gemm_q8's epilogue for one output of a one-block row
 * (backend/ref/kernels.c:75-84): fmaf((float)s, d, +0), times ws, plus the
 * bias br where there is a bias */
__device__ __forceinline__ float gemv_out(int s, float d, float ws, const float *bias, float br) {
    float v = __builtin_fmaf((float)s, d, 0.0f) * ws;
    if (bias)
        v = v + br;
    return v;
}

/* gemv: a wave a 16-row panel, the row quantized by every wave. CH float4
 * chunks a lane hold the row (n <= 256 CH), KU units the panel (kr <= KU);
 * AL as row4's. */
template <int CH, int KU, bool AL>
__global__ __launch_bounds__(64) void gemv_kernel(float *__restrict__ out, const int8_t *__restrict__ w,
                                                  uint64_t wstride, const float *__restrict__ ws,
                                                  const float *__restrict__ bias, const float *__restrict__ x,
                                                  uint32_t n, uint32_t kr, int add) {
    __shared__ __attribute__((aligned(16))) int8_t q[64 * KU];
    const int lane = threadIdx.x;
    const uint32_t p = blockIdx.x;
    float4 v[CH];
    load_row<CH>([&](uint32_t i) { return row4<AL>(x, i, n); }, n, lane, v);
    v4i wv[KU];
    if constexpr (kEarly<KU>)
        panel_load<KU>(w, wstride, p, kr, lane, wv);
    const uint32_t r = 16 * p + (lane & 15);
    const float wsr = ws[r], br = bias ? bias[r] : 0.0f, old = add ? out[r] : 0.0f;
    const float d = quant_loaded<CH>(v, n, kr, q, lane);
    __syncthreads();
    if constexpr (!kEarly<KU>)
        panel_load<KU>(w, wstride, p, kr, lane, wv);
    const int s = panel_sum<KU>(wv, kr, q, lane);
    if (lane < 16) {
        const float o = gemv_out(s, d, wsr, bias, br);
        out[r] = add ? old + o : o;
    }
}

/* An LSTM layer's step (core/decoder.c:68-75): a workgroup 16 units j0 ..
 * j0 + 15, wave w their gate w (rows w P + j), each gate wx x + b and then +
 * wh h as the reference's two calls make it, then the cell
 * (backend/ref/kernels.c:203-213). h_in is read, h_out written (other
 * workgroups still read h_in); c is stepped in place, each unit by one
 * thread. */
template <int CH, int KU, bool AL>
__global__ __launch_bounds__(256) void lstm_kernel(float *__restrict__ h_out, float *__restrict__ c,
                                                   const float *__restrict__ h_in, const float *__restrict__ x,
                                                   const int8_t *__restrict__ wx, const float *__restrict__ wxs,
                                                   const int8_t *__restrict__ wh, const float *__restrict__ whs,
                                                   uint64_t wstride, const float *__restrict__ b, uint32_t P,
                                                   uint32_t kr) {
    __shared__ __attribute__((aligned(16))) int8_t qx[64 * KU], qh[64 * KU];
    __shared__ float dq[2], gates[4][16];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t j0 = 16 * blockIdx.x;
    /* every load the step needs is issued before the first use: the row
     * (waves 0 and 1), the gate's two panels, the scales, the bias, c */
    float4 v[CH];
    if (wv == 0)
        load_row<CH>([&](uint32_t i) { return row4<AL>(x, i, P); }, P, lane, v);
    else if (wv == 1)
        load_row<CH>([&](uint32_t i) { return row4<AL>(h_in, i, P); }, P, lane, v);
    const uint32_t p = (wv * P + j0) / 16;
    constexpr int KE = kEarly<KU> ? KU : 1;       /* late: one panel's registers at a time */
    v4i wxv[KE], whv[KE];
    if constexpr (kEarly<KU>) {
        panel_load<KU>(wx, wstride, p, kr, lane, wxv);
        panel_load<KU>(wh, wstride, p, kr, lane, whv);
    }
    const uint32_t r = wv * P + j0 + (lane & 15);
    const float wxsr = wxs[r], whsr = whs[r], br = b ? b[r] : 0.0f;
    const float cold = threadIdx.x < 16 ? c[j0 + threadIdx.x] : 0.0f;
    if (wv == 0) {
        const float d = quant_loaded<CH>(v, P, kr, qx, lane);
        if (lane == 0)
            dq[0] = d;
    } else if (wv == 1) {
        const float d = quant_loaded<CH>(v, P, kr, qh, lane);
        if (lane == 0)
            dq[1] = d;
    }
    __syncthreads();
    int sx, sh;
    if constexpr (kEarly<KU>) {
        sx = panel_sum<KU>(wxv, kr, qx, lane);
        sh = panel_sum<KU>(whv, kr, qh, lane);
    } else {
        sx = panel_dot<KU>(wx, wstride, p, kr, qx, lane);
        sh = panel_dot<KU>(wh, wstride, p, kr, qh, lane);
    }
    if (lane < 16) {
        const float g = gemv_out(sx, dq[0], wxsr, b, br);
        gates[wv][lane] = g + gemv_out(sh, dq[1], whsr, nullptr, 0.0f);
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        const uint32_t t = threadIdx.x, j = j0 + t;
        const float i = pk_sigmoidf(gates[0][t]);
        const float f = pk_sigmoidf(gates[1][t]);
        const float u = pk_tanhf(gates[2][t]);
        const float o = pk_sigmoidf(gates[3][t]);
        const float cj = f * cold + i * u;
        c[j] = cj;
        h_out[j] = o * pk_tanhf(cj);
    }
}

/* The joint's logits (core/decoder.c:83-89): z = relu(f + gp) quantized by
 * every wave, a wave a 16-row panel of jout */
__device__ __forceinline__ float relu_sum(float a, float b) {
    const float v = a + b;
    return v > 0 ? v : 0.0f;
}

template <int CH, int KU, bool AL>
__global__ __launch_bounds__(64) void joint_kernel(float *__restrict__ logit, const int8_t *__restrict__ w,
                                                   uint64_t wstride, const float *__restrict__ ws,
                                                   const float *__restrict__ bias, const float *__restrict__ f,
                                                   const float *__restrict__ gp, uint32_t J, uint32_t kr) {
    __shared__ __attribute__((aligned(16))) int8_t q[64 * KU];
    const int lane = threadIdx.x;
    const uint32_t p = blockIdx.x;
    float4 vf[CH], vg[CH];
    load_row<CH>([&](uint32_t i) { return row4<AL>(f, i, J); }, J, lane, vf);
    load_row<CH>([&](uint32_t i) { return row4<AL>(gp, i, J); }, J, lane, vg);
    v4i wv[KU];
    if constexpr (kEarly<KU>)
        panel_load<KU>(w, wstride, p, kr, lane, wv);
    const uint32_t r = 16 * p + (lane & 15);
    const float wsr = ws[r], br = bias ? bias[r] : 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++)
        vf[c] = make_float4(relu_sum(vf[c].x, vg[c].x), relu_sum(vf[c].y, vg[c].y), relu_sum(vf[c].z, vg[c].z),
                            relu_sum(vf[c].w, vg[c].w));
    const float d = quant_loaded<CH>(vf, J, kr, q, lane);
    __syncthreads();
    if constexpr (!kEarly<KU>)
        panel_load<KU>(w, wstride, p, kr, lane, wv);
    const int s = panel_sum<KU>(wv, kr, q, lane);
    if (lane < 16)
        logit[r] = gemv_out(s, d, wsr, bias, br);
}

/* core/decoder.c:90-98: the first best token of [0, V] and the first best
 * duration of the n_dur after them. The scan's rule, best = i when
 * logit[i] > logit[best] from best = 0, picks the first index of the
 * maximum over the values that are not NaN, unless logit[0] is NaN (nothing
 * is greater than it). So a lane takes a contiguous run of at most RUN
 * (loaded at once) and keeps its first maximum over non-NaN values, the runs
 * meet in order (ties to the earlier run, +0 and -0 equal as the comparison
 * has them), and a NaN at 0 wins. The durations are few: lane 0 scans them. */
template <int RUN>
__global__ __launch_bounds__(64) void argmax_kernel(uint32_t *__restrict__ tok_dur, const float *__restrict__ logit,
                                                    uint32_t V, uint32_t n_dur) {
    const int lane = threadIdx.x;
    const uint32_t n = V + 1, run = (n + 63) / 64, a = lane * run;
    float lv[RUN];
#pragma unroll
    for (int k = 0; k < RUN; k++)
        lv[k] = k < (int)run && a + k < n ? logit[a + k] : 0.0f;
    /* the durations' logits, lane i the i-th (up to 64), loaded with the run */
    const float dv = lane < (int)n_dur ? logit[V + 1 + lane] : 0.0f;
    float bv = 0.0f;
    int bi = -1;
#pragma unroll
    for (int k = 0; k < RUN; k++) {
        const float v = lv[k];
        if (k < (int)run && a + k < n && v == v && (bi < 0 || v > bv)) {
            bv = v;
            bi = (int)(a + k);
        }
    }
    for (int off = 1; off < 64; off <<= 1) {
        const float ov = __shfl_down(bv, off);
        const int oi = __shfl_down(bi, off);
        if (lane + off < 64 && oi >= 0 && (bi < 0 || ov > bv)) {
            bv = ov;
            bi = oi;
        }
    }
    /* the scan over the durations, each compared with the best so far */
    uint32_t bd = 0;
    if (n_dur <= 64) {
        float bdv = __shfl(dv, 0);
        for (uint32_t i = 1; i < n_dur; i++) {
            const float x = __shfl(dv, (int)i);
            if (x > bdv) {
                bd = i;
                bdv = x;
            }
        }
    } else if (lane == 0) {
        for (uint32_t i = 1; i < n_dur; i++)
            if (logit[V + 1 + i] > logit[V + 1 + bd])
                bd = i;
    }
    if (lane == 0) {
        const float l0 = lv[0];                  /* lane 0's run starts at token 0 */
        const uint32_t best = l0 != l0 || bi < 0 ? 0u : (uint32_t)bi;
        tok_dur[0] = best;
        tok_dur[1] = bd;
    }
}

/* ---------------------------------------------------------- launchers -- */

static bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

/* The row's float4 chunks a lane and the panel's units a wave: up to 1024
 * inputs in 16 units, or 4096 in 64; float4 loads when the rows are 16-byte
 * aligned and n a multiple of 4 (al). */
#define PK_DEC_SIZE(n, kr, al, CALL)                        \
    do {                                                    \
        if ((n) <= 1024 && (kr) <= 16) {                    \
            constexpr int CH = 4, KU = 16;                  \
            if (al) {                                       \
                constexpr bool AL = true;                   \
                CALL;                                       \
            } else {                                        \
                constexpr bool AL = false;                  \
                CALL;                                       \
            }                                               \
        } else {                                            \
            constexpr int CH = 16, KU = 64;                 \
            if (al) {                                       \
                constexpr bool AL = true;                   \
                CALL;                                       \
            } else {                                        \
                constexpr bool AL = false;                  \
                CALL;                                       \
            }                                               \
        }                                                   \
    } while (0)

int launch_gemv(float *out, const int8_t *w, uint64_t wstride, const float *ws, const float *bias, const float *x,
                uint32_t rows, uint32_t n, uint32_t kr, int add, hipStream_t s) {
    if (n == 0 || n > kDecMaxCols || rows % 16 || 64 * kr > kDecMaxCols || 64 * kr < n)
        return -2;
    const bool al = n % 4 == 0 && al16(x);
    PK_DEC_SIZE(n, kr, al,
                (gemv_kernel<CH, KU, AL><<<rows / 16, 64, 0, s>>>(out, w, wstride, ws, bias, x, n, kr, add)));
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

int launch_lstm(float *h_out, float *c, const float *h_in, const float *x, const int8_t *wx, const float *wxs,
                const int8_t *wh, const float *whs, uint64_t wstride, const float *b, uint32_t P, uint32_t kr,
                hipStream_t s) {
    if (P == 0 || P % 16 || P > kDecMaxCols || 64 * kr > kDecMaxCols || 64 * kr < P)
        return -2;
    const bool al = al16(x) && al16(h_in);
    PK_DEC_SIZE(P, kr, al,
                (lstm_kernel<CH, KU, AL><<<P / 16, 256, 0, s>>>(h_out, c, h_in, x, wx, wxs, wh, whs, wstride, b, P,
                                                                kr)));
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

int launch_joint(float *logit, uint32_t *tok_dur, const int8_t *w, uint64_t wstride, const float *ws,
                 const float *bias, const float *f, const float *gp, uint32_t rows, uint32_t J, uint32_t kr,
                 uint32_t V, uint32_t n_dur, hipStream_t s) {
    if (J == 0 || J > kDecMaxCols || rows % 16 || 64 * kr > kDecMaxCols || 64 * kr < J || V + 1 + n_dur > rows ||
        n_dur == 0 || V + 1 > 64 * 64)
        return -2;
    const bool al = J % 4 == 0 && al16(f) && al16(gp);
    PK_DEC_SIZE(J, kr, al,
                (joint_kernel<CH, KU, AL><<<rows / 16, 64, 0, s>>>(logit, w, wstride, ws, bias, f, gp, J, kr)));
    if (V + 1 <= 64 * 32)
        argmax_kernel<32><<<1, 64, 0, s>>>(tok_dur, logit, V, n_dur);
    else
        argmax_kernel<64><<<1, 64, 0, s>>>(tok_dur, logit, V, n_dur);
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

}  // namespace pkq8
