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

/* panel_sum over a panel kept in LDS: unit u's bytes at wl + 1 KB u, in
 * the order panel_load reads them (lane l's 16 bytes at 16 l) */
template <int KU>
__device__ __forceinline__ int panel_sum_lds(const int8_t *wl, uint32_t kr, const int8_t *q, int lane) {
    v4i wv[KU];
#pragma unroll
    for (int u = 0; u < KU; u++)
        if (u < (int)kr)
            wv[u] = *(const v4i *)(wl + u * kUnitBytes + lane * 16);
    return panel_sum<KU>(wv, kr, q, lane);
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
template <int RUN, typename L>
__device__ __forceinline__ void argmax_wave(L logit_at, uint32_t V, uint32_t n_dur, int lane, uint32_t &tok,
                                            uint32_t &dur) {
    const uint32_t n = V + 1, run = (n + 63) / 64, a = lane * run;
    float lv[RUN];
#pragma unroll
    for (int k = 0; k < RUN; k++)
        lv[k] = k < (int)run && a + k < n ? logit_at(a + k) : 0.0f;
    /* the durations' logits, lane i the i-th (up to 64), loaded with the run */
    const float dv = lane < (int)n_dur ? logit_at(V + 1 + lane) : 0.0f;
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
    } else {
        if (lane == 0)
            for (uint32_t i = 1; i < n_dur; i++)
                if (logit_at(V + 1 + i) > logit_at(V + 1 + bd))
                    bd = i;
        bd = __shfl(bd, 0);
    }
    const float l0 = __shfl(lv[0], 0);          /* lane 0's run starts at token 0 */
    const int b0 = __shfl(bi, 0);
    tok = l0 != l0 || b0 < 0 ? 0u : (uint32_t)b0;
    dur = bd;
}

template <int RUN>
__global__ __launch_bounds__(64) void argmax_kernel(uint32_t *__restrict__ tok_dur, const float *__restrict__ logit,
                                                    uint32_t V, uint32_t n_dur) {
    uint32_t tok, dur;
    argmax_wave<RUN>([&](uint32_t i) { return logit[i]; }, V, n_dur, threadIdx.x, tok, dur);
    if (threadIdx.x == 0) {
        tok_dur[0] = tok;
        tok_dur[1] = dur;
    }
}

/* ------------------------------------------------------- the search -- *
 *
 * TDT's greedy search (core/decoder.c:121-147) over a segment's frames in one
 * launch: the prediction (the label's embedding through the LSTM layers and
 * jpred, :65-79), the joint and its argmax (:81-101), the duration step, the
 * max_symbols rule and the token list, with every state (h, c of each layer,
 * gp, the logits, the frame, the tokens) in HBM and registers, so the host
 * reads nothing between frames.
 *
 * Every workgroup runs the same control flow. A phase (an LSTM layer's step,
 * jpred, the joint's logits) splits its rows over the workgroups as the
 * one-launch kernels above split them, and ends at a grid barrier; after the
 * joint's barrier every workgroup reads all the logits and makes the same
 * argmax, so all of them take the same branch of the search and meet at the
 * same barriers. What one workgroup writes and another reads (h, gp, the
 * logits) goes through agent-scope atomic stores and loads, coherent across
 * the XCDs' L2s, and so does c, which the workgroup that steps it reads
 * back a token later. The launch is
 * cooperative (every workgroup resident at once), and every barrier's wait is
 * bounded: past its iteration limit a workgroup raises the error flag and
 * leaves, and the others see the flag in their waits and leave too, so a
 * launch always ends; the host reads the flag. The bits are the one-launch
 * kernels' (the same helpers in the same order), so the reference's. */

__device__ __forceinline__ float cload(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void cstore(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* chunk i of a row of n floats read coherently, zeros past n */
__device__ __forceinline__ float4 crow4(const float *x, uint32_t i, uint32_t n) {
    const uint32_t k = 4 * i;
    return make_float4(k < n ? cload(x + k) : 0.0f, k + 1 < n ? cload(x + k + 1) : 0.0f,
                       k + 2 < n ? cload(x + k + 2) : 0.0f, k + 3 < n ? cload(x + k + 3) : 0.0f);
}

template <int CH, int KU, bool RES>
__global__ __launch_bounds__(256) void search_kernel(SearchArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t q0[64 * KU], q1[64 * KU];
    __shared__ float dq[2], gates[4][16];
    __shared__ uint32_t shared_u[3];
    /* RES: the jpred panel wg (slot 0) and the jout panels wg and wg + G
     * (slots 1, 2) of this workgroup, loaded once */
    __shared__ __attribute__((aligned(16))) int8_t wres[RES ? 3 : 1][RES ? KU * kUnitBytes : 16];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t G = gridDim.x, wg = blockIdx.x;
    const uint32_t P = a.P, J = a.J;
    uint32_t nbar = 0;

    /* RES: each wave's gate panels of every LSTM layer (wx and wh, kResLayers
     * at most) held in registers for the whole segment, with their rows'
     * scales and biases; waves 1-3 the scale and bias of their jpred / jout
     * row */
    constexpr int RL = RES ? kResLayers : 1, RU = RES ? KU : 1;
    v4i rwx[RL][RU], rwh[RL][RU];
    float rxs[RL], rhs[RL], rb[RL], jsr = 0.0f, jbr = 0.0f;
    if constexpr (RES) {
        if (wg < P / 16) {
            const uint32_t j0 = 16 * wg, pn = (wv * P + j0) / 16, r = wv * P + j0 + (lane & 15);
#pragma unroll
            for (int l = 0; l < RL; l++)
                if (l < (int)a.L) {
                    panel_load<KU>(a.wx[l], a.lstm_stride, pn, a.kr_p, lane, rwx[l]);
                    panel_load<KU>(a.wh[l], a.lstm_stride, pn, a.kr_p, lane, rwh[l]);
                    rxs[l] = a.wxs[l][r];
                    rhs[l] = a.whs[l][r];
                    rb[l] = a.b[l] ? a.b[l][r] : 0.0f;
                }
        }
        if (wv >= 1) {
            const bool jp = wv == 1;
            const uint32_t pn = jp ? wg : wg + (wv - 2) * G, panels = jp ? J / 16 : a.rows_out / 16;
            if (pn < panels) {
                const uint32_t kr = jp ? a.kr_p : a.kr_j, r = 16 * pn + (lane & 15);
                v4i t[KU];
                panel_load<KU>(jp ? a.jpred : a.jout, jp ? a.jpred_stride : a.jout_stride, pn, kr, lane, t);
#pragma unroll
                for (int u = 0; u < KU; u++)
                    if (u < (int)kr)
                        *(v4i *)(wres[wv - 1] + u * kUnitBytes + lane * 16) = t[u];
                const float *bb = jp ? a.jpred_b : a.jout_b;
                jsr = (jp ? a.jpred_s : a.jout_s)[r];
                jbr = bb ? bb[r] : 0.0f;
            }
        }
        __syncthreads();
    }

    /* the grid barrier: this workgroup's stores have landed, then it counts
     * itself in and waits for the G arrivals of barrier nbar; false (leave)
     * on the error flag or past the iteration limit */
    auto barrier = [&]() -> bool {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        nbar++;
        if (wv == 0) {
            /* each workgroup stores the barrier's number to its own slot;
             * wave 0 reads every slot in one load (lane i slot i, G <= 64)
             * until all of them hold it: no two workgroups update one word */
            uint32_t *slot = a.sync + 64;
            if (lane == 0)
                __hip_atomic_store(slot + wg, nbar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            uint32_t it = 0, bad = 0;
            while (true) {
                const uint32_t v = lane < (int)G ? __hip_atomic_load(slot + lane, __ATOMIC_RELAXED,
                                                                     __HIP_MEMORY_SCOPE_AGENT) : nbar;
                if (__builtin_amdgcn_read_exec() == __ballot(v >= nbar))
                    break;
                if (++it >= a.spin || ((it & 15) == 0 &&
                                       __hip_atomic_load(a.sync + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
                    bad = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            if (bad && lane == 0)
                __hip_atomic_store(a.sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (lane == 0)
                shared_u[2] = bad;
        }
        __syncthreads();
        return shared_u[2] == 0;
    };

    /* one LSTM layer's step on units 16 wg .. + 15 (lstm_kernel's steps):
     * x, h_in and c read, c and h_out stored, all through the coherent
     * accessors (c is this workgroup's own, read back a token later) */
    auto lstm = [&](uint32_t l, const float *x, const float *h_in, float *h_out) {
        if (wg >= P / 16)
            return;
        float *c = a.c + (size_t)l * P;
        const uint32_t j0 = 16 * wg;
        float4 v[CH];
        if (wv == 0)
            load_row<CH>([&](uint32_t i) { return crow4(x, i, P); }, P, lane, v);
        else if (wv == 1)
            load_row<CH>([&](uint32_t i) { return crow4(h_in, i, P); }, P, lane, v);
        const uint32_t pn = (wv * P + j0) / 16;
        v4i wxv[RES ? 1 : KU], whv[RES ? 1 : KU];
        float wxsr = 0.0f, whsr = 0.0f, br = 0.0f;
        if constexpr (!RES) {
            panel_load<KU>(a.wx[l], a.lstm_stride, pn, a.kr_p, lane, wxv);
            panel_load<KU>(a.wh[l], a.lstm_stride, pn, a.kr_p, lane, whv);
            const uint32_t r = wv * P + j0 + (lane & 15);
            wxsr = a.wxs[l][r];
            whsr = a.whs[l][r];
            br = a.b[l] ? a.b[l][r] : 0.0f;
        }
        const float cold = threadIdx.x < 16 ? cload(c + j0 + threadIdx.x) : 0.0f;
        if (wv == 0) {
            const float d = quant_loaded<CH>(v, P, a.kr_p, q0, lane);
            if (lane == 0)
                dq[0] = d;
        } else if (wv == 1) {
            const float d = quant_loaded<CH>(v, P, a.kr_p, q1, lane);
            if (lane == 0)
                dq[1] = d;
        }
        __syncthreads();
        int sx = 0, sh = 0;
        if constexpr (RES) {
#pragma unroll
            for (int k = 0; k < RL; k++)
                if (k == (int)l) {
                    sx = panel_sum<KU>(rwx[k], a.kr_p, q0, lane);
                    sh = panel_sum<KU>(rwh[k], a.kr_p, q1, lane);
                    wxsr = rxs[k];
                    whsr = rhs[k];
                    br = rb[k];
                }
        } else {
            sx = panel_sum<KU>(wxv, a.kr_p, q0, lane);
            sh = panel_sum<KU>(whv, a.kr_p, q1, lane);
        }
        if (lane < 16) {
            const float g = gemv_out(sx, dq[0], wxsr, a.b[l], br);
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
            cstore(c + j, cj);
            cstore(h_out + j, o * pk_tanhf(cj));
        }
    };

    /* a row of n inputs (value4 gives its chunks) quantized once by wave 0,
     * then one 16-row panel of w a wave (panel 4 wg + wave, those below
     * panels): gemv_out into out, stored coherently */
    auto gemv = [&](auto value4, uint32_t n, uint32_t kr, const int8_t *w, uint64_t stride, const float *ws,
                    const float *bias, uint32_t panels, float *out) {
        const uint32_t pn = 4 * wg + wv;
        const bool mine = pn < panels;
        float4 v[CH];
        if (wv == 0)
            load_row<CH>(value4, n, lane, v);
        v4i wvv[KU];
        if (mine)
            panel_load<KU>(w, stride, pn, kr, lane, wvv);
        const uint32_t r = 16 * pn + (lane & 15);
        const float wsr = mine ? ws[r] : 0.0f, br = mine && bias ? bias[r] : 0.0f;
        if (wv == 0) {
            const float d = quant_loaded<CH>(v, n, kr, q0, lane);
            if (lane == 0)
                dq[0] = d;
        }
        __syncthreads();
        if (mine) {
            const int s = panel_sum<KU>(wvv, kr, q0, lane);
            if (lane < 16)
                cstore(out + r, gemv_out(s, dq[0], wsr, bias, br));
        }
    };

    /* RES: the row quantized by wave 0, then wave w1 sums the panel pn
     * kept in LDS slot w1 - 1 (jpred: wave 1, panel wg; jout: waves 2 and
     * 3, panels wg and wg + G) */
    auto gemv_res = [&](auto value4, uint32_t n, uint32_t kr, const float *bias, uint32_t panels, float *out,
                        bool joint) {
        float4 v[CH];
        if (wv == 0) {
            load_row<CH>(value4, n, lane, v);
            const float d = quant_loaded<CH>(v, n, kr, q0, lane);
            if (lane == 0)
                dq[0] = d;
        }
        __syncthreads();
        const bool mine = joint ? wv >= 2 : wv == 1;
        const uint32_t pn = joint ? wg + (wv - 2) * G : wg;
        if (mine && pn < panels) {
            const int s = panel_sum_lds<KU>(wres[wv - 1], kr, q0, lane);
            if (lane < 16)
                cstore(out + 16 * pn + lane, gemv_out(s, dq[0], jsr, bias, jbr));
        }
    };

    uint32_t cur = 0;                               /* bit l: which of layer l's two h buffers is current */
    auto predict = [&](uint32_t label) -> bool {
        const float *x = a.embed + (size_t)label * P;
        for (uint32_t l = 0; l < a.L; l++) {
            const uint32_t c0 = (cur >> l) & 1;
            const float *h_in = a.h + ((size_t)l * 2 + c0) * P;
            float *h_out = a.h + ((size_t)l * 2 + (c0 ^ 1)) * P;
            lstm(l, x, h_in, h_out);
            cur ^= 1u << l;
            if (!barrier())
                return false;
            x = h_out;
        }
        const float *hl = x;
        if constexpr (RES)
            gemv_res([&](uint32_t i) { return crow4(hl, i, P); }, P, a.kr_p, a.jpred_b, J / 16, a.gp, false);
        else
            gemv([&](uint32_t i) { return crow4(hl, i, P); }, P, a.kr_p, a.jpred, a.jpred_stride, a.jpred_s,
                 a.jpred_b, J / 16, a.gp);
        return barrier();
    };

    /* the joint at frame t: relu(f + gp) quantized, jout's panels, then every
     * workgroup's wave 0 takes the argmax of all the logits */
    auto joint = [&](uint32_t t, uint32_t &k, uint32_t &di) -> bool {
        const float *ft = a.f + (size_t)t * J;
        auto zrow = [&](uint32_t i) {
            const float4 fv = row4<false>(ft, i, J), gv = crow4(a.gp, i, J);
            return make_float4(relu_sum(fv.x, gv.x), relu_sum(fv.y, gv.y), relu_sum(fv.z, gv.z),
                               relu_sum(fv.w, gv.w));
        };
        if constexpr (RES)
            gemv_res(zrow, J, a.kr_j, a.jout_b, a.rows_out / 16, a.logit, true);
        else
            gemv(zrow, J, a.kr_j, a.jout, a.jout_stride, a.jout_s, a.jout_b, a.rows_out / 16, a.logit);
        if (!barrier())
            return false;
        if (wv == 0) {
            uint32_t tk, dd;
            argmax_wave<32>([&](uint32_t i) { return cload(a.logit + i); }, a.V, a.n_dur, lane, tk, dd);
            if (lane == 0) {
                shared_u[0] = tk;
                shared_u[1] = dd;
            }
        }
        __syncthreads();
        k = shared_u[0];
        di = shared_u[1];
        __syncthreads();
        return true;
    };

    const uint32_t T = a.T, blank = a.blank;
    uint32_t ntoks = 0, status = 0;
    if (!predict(blank))
        return;
    uint32_t t = 0, last = 0xffffffffu, lasts = 0;
    while (t < T) {
        uint32_t k, di, d, at;
        do {
            at = t;
            if (!joint(t, k, di))
                return;
            d = (uint32_t)a.dur[di];
            if (k == blank && d == 0)
                d = 1;
            t += d;
        } while (k == blank && t < T);
        if (k == blank)
            break;
        if (ntoks == a.cap) {
            status = 2;
            break;
        }
        if (wg == 0 && threadIdx.x == 0) {
            a.toks[3 * ntoks] = (int32_t)k;
            a.toks[3 * ntoks + 1] = (int32_t)at;
            a.toks[3 * ntoks + 2] = a.dur[di];
        }
        ntoks++;
        lasts = last == at ? lasts + 1 : 1;
        last = at;
        if (!predict(k))
            return;
        if (lasts >= a.max_symbols && last == t)
            t++;
    }
    if (wg == 0 && threadIdx.x == 0) {
        a.out[0] = ntoks;
        a.out[1] = status;
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

static bool g_search_resident = true;

bool set_search_resident(bool on) {
    const bool was = g_search_resident;
    g_search_resident = on;
    return was;
}

size_t search_workspace_bytes(uint32_t L, uint32_t P, uint32_t J, uint32_t rows_out, uint32_t cap) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    return up(512) + up((size_t)L * 2 * P * 4) + up((size_t)L * P * 4) + up((size_t)J * 4) + up((size_t)rows_out * 4) +
           up((size_t)cap * 12) + up(8);
}

int launch_search(SearchArgs &a, void *ws, hipStream_t s) {
    if (a.P == 0 || a.P % 16 || a.P > 1024 || a.J == 0 || a.J % 16 || a.J > 1024 || a.L == 0 ||
        a.L > (uint32_t)kMaxDecLayers || a.rows_out % 16 || a.V + 1 + a.n_dur > a.rows_out || a.n_dur == 0 ||
        a.n_dur > 64 || a.V + 1 > 64 * 32 || 64 * a.kr_p < a.P || a.kr_p > 16 || 64 * a.kr_j < a.J || a.kr_j > 16)
        return -2;
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    char *p = (char *)ws;
    a.sync = (uint32_t *)p;
    p += up(512);
    a.h = (float *)p;
    p += up((size_t)a.L * 2 * a.P * 4);
    a.c = (float *)p;
    p += up((size_t)a.L * a.P * 4);
    a.gp = (float *)p;
    p += up((size_t)a.J * 4);
    a.logit = (float *)p;
    p += up((size_t)a.rows_out * 4);
    a.toks = (int32_t *)p;
    p += up((size_t)a.cap * 12);
    a.out = (uint32_t *)p;
    /* the arrivals, the flag and the state start at zero (c and h: the
     * reference zeroes them a segment, core/decoder.c:158-165); the logits,
     * gp and the tokens are written before they are read */
    if (hipMemsetAsync(a.sync, 0, 512, s) != hipSuccess ||
        hipMemsetAsync(a.h, 0, up((size_t)a.L * 2 * a.P * 4) + up((size_t)a.L * a.P * 4), s) != hipSuccess ||
        hipMemsetAsync(a.out, 0, 8, s) != hipSuccess)
        return -1;
    /* resident: every panel's units and every layer's gate panels fit
     * (kr <= kResUnits, L <= kResLayers), one workgroup a jpred panel and
     * two a jout panel's pair; else the panels are loaded each token */
    uint32_t Gr = a.P / 16;
    Gr = Gr > a.J / 16 ? Gr : a.J / 16;
    Gr = Gr > (a.rows_out / 16 + 1) / 2 ? Gr : (a.rows_out / 16 + 1) / 2;
    const bool res = g_search_resident && a.L <= (uint32_t)kResLayers && a.kr_p <= (uint32_t)kResUnits &&
                     a.kr_j <= (uint32_t)kResUnits && Gr <= 64;
    uint32_t G = a.P / 16;
    G = G > (a.rows_out / 16 + 3) / 4 ? G : (a.rows_out / 16 + 3) / 4;
    G = G > (a.J / 16 + 3) / 4 ? G : (a.J / 16 + 3) / 4;
    if (res)
        G = Gr;
    if (G > 64)
        return -2;                              /* the barrier reads every workgroup's slot in one wave */
    void *args[] = { &a };
    const void *k = res ? (const void *)search_kernel<4, kResUnits, true> : (const void *)search_kernel<4, 16, false>;
    const hipError_t e = hipLaunchCooperativeKernel(k, dim3(G), dim3(256), args, 0, s);
    return e == hipSuccess ? 0 : -1;
}

}  // namespace pkq8
