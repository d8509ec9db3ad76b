/* The streamed product: int8 x int8 -> exact int32 -> the reference's fp32
 * epilogue (backend/ref/kernels.c:66-86, per-row blocks), for products with
 * many tiles a CU.
 *
 * Persistent workgroups: a grid of (CUs x workgroups a CU) walks the tile list,
 * workgroup b taking tiles b, b + G, b + 2G, ... in the XCD-aware order (the
 * tiles one XCD runs at once are one compact block of the output, so its L2
 * serves their shared weights and activations). Each workgroup has two kinds
 * of waves:
 *
 *   - NL loader waves issue every global -> LDS transfer: a continuous stream
 *     of K stages through an NS-slot ring that runs on across the workgroup's
 *     tiles (the next tile's first stages load under this tile's last ones),
 *     plus each tile's frame scales, channel scales and biases into one of two
 *     epilogue buffers. They alone wait on vmcnt.
 *   - WN x WM MFMA waves read fragments from the ring (two register sets, the
 *     next sub-step's reads issued before this one's MFMAs), multiply, and at
 *     a tile's end move their sums across lanes so that consecutive lanes hold
 *     consecutive bytes of each output line, run the epilogue from registers
 *     and store the outputs. They never wait on vmcnt in the K loop (the
 *     counter also counts stores on gfx950), so a tile's stores drain while
 *     the next tile's K loop runs; only a residual-adding epilogue waits, for
 *     its residuals.
 *
 * One s_barrier a stage meets both: the loaders arrive once the next stage has
 * landed, the MFMA waves once they hold the current stage's last fragments in
 * registers; after it the loaders refill the freed slot. Every wave of a
 * workgroup executes the same number of barriers (one before the first stage,
 * one after each stage but the workgroup's last). */
#include "q8_product.h"

#include <hip/hip_runtime.h>

namespace pkq8 {

/* s_waitcnt vmcnt(n * L) for a count n in [0, N) known only at run time */
template <int I, int N, int L>
__device__ __forceinline__ void wait_vm_n(uint32_t n) {
    if constexpr (I < N) {
        if (n == I) {
            wait_vm<I * L>();
            return;
        }
        wait_vm_n<I + 1, N, L>(n);
    } else {
        wait_vm<0>();
    }
}

/* Buffer resource word 3 for raw byte-addressed loads on gfx9 parts */
constexpr int kBufferFlags = 0x00020000;

/* 16 bytes from LDS at addr + OFF, issued as written (lds_read16 with the
 * instruction's immediate offset: one address register a fragment set) */
template <int OFF>
__device__ __forceinline__ v4i lds_read16_at(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offsets are 16 bits");
    v4i r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF) : "memory");
    return r;
}

/* The job and output tile of the workgroup-independent tile index v: the
 * jobs' tiles are numbered one after another; inside a job the XCD-aware
 * order of xcd_tile (v % 8 is the XCD a persistent workgroup of a grid that
 * is a multiple of 8 runs on, whatever the job's first index). */
__device__ __forceinline__ void stream_tile(const JobTable &tab, uint32_t v, uint32_t &j, uint32_t &tn,
                                            uint32_t &tm) {
    j = 0;
    while (j + 1 < tab.njobs && tab.wg0[j + 1] <= v)
        j++;
    const uint32_t tiles = tab.tiles[j], tiles_n = tab.tiles_n[j];
    xcd_tile(v - tab.wg0[j], tiles, tiles_n, tiles / tiles_n, tn, tm);
}

/* Loader wave WL of NL: the units [WL L, WL L + L) of every stage (index
 * idx: sub-step idx / UNITS, unit idx % UNITS, weight panels first, then
 * activation groups), all known at compile time; the tile's bases are
 * uniform. Stages run on across the workgroup's tiles: stage S is stage
 * S % ns of tile S / ns, in ring slot S % NS. */
template <int WL, int WN, int WM, int TN, int TM, int UPS, int NS, int NL, bool PACKED>
__device__ __forceinline__ void stream_loader(const JobTable &tab, int8_t *ring, float *epi,
                                              uint32_t b, uint32_t G, uint32_t total, uint32_t ns, int lane) {
    constexpr int BN = 16 * TN * WN, BM = 16 * TM * WM;
    constexpr int UB = BN / 16, UA = BM / 16, UNITS = UA + UB;
    constexpr int L = UNITS * UPS / NL;
    constexpr int SLOT = UNITS * UPS * kUnitBytes;
    constexpr int ED = BM / 64, EW = BN / 64, ECH = ED + 2 * EW;
    uint32_t rt = 0, rs = 0;            /* the next stage to issue: its tile, its stage in the tile */
    uint32_t j = 0, p0 = 0, g0 = 0;
    /* Buffer loads into LDS: the lane's 16 bytes at voffset, the unit's
     * uniform byte offset in soffset, so a load is one instruction on one
     * constant lane-offset register. The resources span the call's matrix
     * run and activations; a load past their records reads zeros. */
    __amdgpu_buffer_rsrc_t rw, ra;
    uint64_t wstride = 0, qstride = 0;
    uint32_t npan = 1, ng = 1;
    uint32_t aoff[UA];                  /* row-major activations: each unit's lane offset (its row) */
    const uint32_t loff = lane * 16;
    auto issue = [&](uint32_t slot) {
        if (rs == 0) {
            uint32_t tn, tm;
            stream_tile(tab, b + rt * G, j, tn, tm);
            const GemmArgs &g = tab.g[j];
            const Seg &sg = tab.s[j];
            const uint32_t n0 = tn * BN, m0 = tm * BM, T = sg.T;
            p0 = tn * (BN / 16);
            g0 = tm * (BM / 16);
            npan = g.rows >> 4;
            wstride = g.wstride;
            qstride = sg.qstride;
            ng = (T + 15) / 16;
            rw = __builtin_amdgcn_make_buffer_rsrc((void *)g.w, (short)0, (int)(g.ku * g.wstride), kBufferFlags);
            if constexpr (PACKED) {
                ra = __builtin_amdgcn_make_buffer_rsrc((void *)sg.q, (short)0, (int)(g.ku * sg.qstride), kBufferFlags);
            } else {
                ra = __builtin_amdgcn_make_buffer_rsrc((void *)sg.q, (short)0, (int)((uint64_t)T * g.n), kBufferFlags);
#pragma unroll
                for (int u = 0; u < UA; u++) {
                    uint32_t row = m0 + u * 16 + (lane & 15);
                    row = row < T ? row : T - 1;
                    aoff[u] = row * g.n + (lane >> 4) * 16;
                }
            }
            /* the tile's epilogue scales into epi[rt % 2]: the buffer tile
             * rt - 2 read, whose epilogue ended before the barrier at which
             * this stage is issued (a tile has ns >= NS stages) */
            const int nch = g.bias ? ECH : ED + EW;
            float *e = epi + (rt & 1) * ECH * 64;
            for (int c = WL; c < nch; c += NL) {
                const float *a;
                if (c < ED) {
                    const uint32_t t = m0 + c * 64 + lane;
                    a = sg.d + (t < T ? t : T - 1);
                } else {
                    const uint32_t r = n0 + ((c - ED) % EW) * 64 + lane;
                    a = (c < ED + EW ? g.ws : g.bias) + (r < g.rows ? r : g.rows - 1);
                }
                __builtin_amdgcn_global_load_lds(PK_AS1(a), PK_AS3(e + c * 64), 4, 0, 0);
            }
        }
        int8_t *sp = ring + slot * SLOT;
        for_static<0, L>([&](auto sc) {
            constexpr int s = decltype(sc)::value;
            constexpr int idx = WL * L + s, kk = idx / UNITS, u = idx % UNITS;
            const uint32_t unit = rs * UPS + kk;
            if constexpr (u < UB) {
                const uint32_t p = p0 + u < npan ? p0 + u : npan - 1;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, PK_AS3(sp + idx * kUnitBytes), 16, loff,
                                                         (uint32_t)(unit * wstride) + p * kUnitBytes, 0, 0);
            } else if constexpr (PACKED) {
                const uint32_t gi = g0 + (u - UB) < ng ? g0 + (u - UB) : ng - 1;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, PK_AS3(sp + idx * kUnitBytes), 16, loff,
                                                         (uint32_t)(unit * qstride) + gi * kUnitBytes, 0, 0);
            } else {
                /* inputs past n meet zero weights: what they read does not matter */
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, PK_AS3(sp + idx * kUnitBytes), 16, aoff[u - UB],
                                                         unit * 64, 0, 0);
            }
        });
        if (++rs == ns) {
            rs = 0;
            rt++;
        }
    };
    /* The wait for stage x counts only the unit loads issued after it; the
     * epilogue loads issued with a tile's first stage make the true count
     * larger, so the wait is for as much or more: never too little. */
    const uint32_t pro = total < (uint32_t)NS ? total : NS;
    for (uint32_t x = 0; x < pro; x++)
        issue(x);
    wait_vm_n<0, NS, L>(pro - 1);
    __builtin_amdgcn_s_barrier();
    uint32_t slot = 0;                  /* the slot of stage S */
    for (uint32_t S = 0; S + 1 < total; S++) {
        /* stage S + 1 must land; issued so far: stages up to min(S + NS - 1, total - 1) */
        const uint32_t hi = S + NS - 1 < total - 1 ? S + NS - 1 : total - 1;
        wait_vm_n<0, NS, L>(hi - (S + 1));
        __builtin_amdgcn_s_barrier();
        if (S + NS < total)
            issue(slot);                /* stage S + NS into stage S's slot */
        slot = slot + 1 == NS ? 0 : slot + 1;
    }
}

template <int WN, int WM, int TN, int TM, int UPS, int NS, int NL, bool PACKED>
__global__ __launch_bounds__(64 * (WN * WM + NL)) void gemm_stream_kernel(const JobTable tab, uint32_t ntiles) {
    constexpr int NW = WN * WM;
    constexpr int BN = 16 * TN * WN, BM = 16 * TM * WM;
    constexpr int UB = BN / 16, UA = BM / 16, UNITS = UA + UB;
    constexpr int SLOTU = UNITS * UPS;
    static_assert(SLOTU % NL == 0, "each loader loads whole units");
    constexpr int L = SLOTU / NL;
    constexpr int SLOT = SLOTU * kUnitBytes;
    static_assert(NS >= 2 && NS <= 8, "two to eight slots");
    static_assert((NS - 1) * L < 64, "the stages in flight fit vmcnt");
    static_assert(BM % 64 == 0 && BN % 64 == 0, "whole 64-float chunks of scales");
    constexpr int ED = BM / 64, EW = BN / 64, ECH = ED + 2 * EW;
    static_assert(UPS == 1 || UPS == 2 || UPS == 4, "one, two or four units a stage");
    constexpr int SPI = UPS > 2 ? UPS : 2;      /* sub-steps a pass: f0 and f1 alternate statically */
    constexpr int R = TN + TM;
    static_assert(NS * SLOT + 2 * ECH * 64 * 4 <= 160 * 1024, "the ring fits a CU's LDS");

    __shared__ __attribute__((aligned(1024))) int8_t ring[NS * SLOT];
    __shared__ __attribute__((aligned(256))) float epi[2][ECH * 64];

    const uint32_t G = gridDim.x, b = blockIdx.x;
    if (b >= ntiles)
        return;
    const uint32_t nr = (ntiles - b + G - 1) / G;       /* tiles of this workgroup */
    const uint32_t ku = tab.g[0].ku, ns = ku / UPS;      /* every job has ku units a panel */
    const uint32_t total = nr * ns;                      /* stages of this workgroup */
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    if (tab.g[0].rmode)
        __builtin_amdgcn_s_setreg(2049, tab.g[0].rmode);    /* MODE.FP_ROUND, single precision */

    if (wv >= NW) {
        /* ---------------------------------------------------------- loader */
        for_static<0, NL>([&](auto lc) {
            constexpr int WL = decltype(lc)::value;
            if (wv == NW + WL)
                stream_loader<WL, WN, WM, TN, TM, UPS, NS, NL, PACKED>(tab, ring, &epi[0][0], b, G, total, ns, lane);
        });
        return;
    }

    /* ------------------------------------------------------------ MFMA waves */
    const int wave = wv, wn = wave % WN, wm = wave / WN;
    const uint32_t lofs = lane * 16;
    const uint32_t wbase = lds_addr(ring) + (wn * TN) * kUnitBytes + lofs;
    const uint32_t abase = lds_addr(ring) + (UB + wm * TM) * kUnitBytes + lofs;
    struct Set {
        v4i f[R];
    };
    auto read_set = [&](Set &st, uint32_t slot, uint32_t kk) {
        const uint32_t at = slot * SLOT + kk * UNITS * kUnitBytes;
        const uint32_t wa = wbase + at, aa = abase + at;
        for_static<0, TN>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            st.f[i] = lds_read16_at<i * kUnitBytes>(wa);
        });
        for_static<0, TM>([&](auto jc) {
            constexpr int jj = decltype(jc)::value;
            st.f[TN + jj] = lds_read16_at<jj * kUnitBytes>(aa);
        });
    };
    v4i acc[TN][TM];
    uint32_t slot = 0;                  /* the slot of the current stage */
    /* sub-step k of a pass (static; a pass starts a stage): multiply cur,
     * read the next sub-step's fragments into nxt; at a stage's last sub-step
     * meet the loaders first (bar) and move to the next slot */
    auto step = [&](auto kc, bool bar, bool more, Set &cur, Set &nxt) {
        constexpr int k = decltype(kc)::value, kk = k % UPS;
        wait_lgkm<0>();
#pragma unroll
        for (int r = 0; r < R; r++)
            asm volatile("" : "+v"(cur.f[r]));
        if constexpr (kk == UPS - 1) {
            if (bar)
                __builtin_amdgcn_s_barrier();
            slot = slot + 1 == NS ? 0 : slot + 1;
        }
        if (more)
            read_set(nxt, slot, (kk + 1) % UPS);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < TN; i++)
#pragma unroll
            for (int jj = 0; jj < TM; jj++)
                acc[i][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur.f[i], cur.f[TN + jj], acc[i][jj], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    };
    Set f0, f1;
    auto setpair = [&](auto kc) -> Set & {
        if constexpr (decltype(kc)::value % 2 == 0) return f0; else return f1;
    };

    __builtin_amdgcn_s_barrier();
    read_set(f0, 0, 0);
    wait_lgkm<0>();
#pragma unroll
    for (int r = 0; r < R; r++)
        asm volatile("" : "+v"(f0.f[r]));

    for (uint32_t rt = 0; rt < nr; rt++) {
        const bool last = rt + 1 == nr;
        uint32_t j, tn, tm;
        stream_tile(tab, b + rt * G, j, tn, tm);
#pragma unroll
        for (int i = 0; i < TN; i++)
#pragma unroll
            for (int jj = 0; jj < TM; jj++)
                acc[i][jj] = v4i{0, 0, 0, 0};
        /* every pass but the last: a barrier at each stage's end */
        for (uint32_t gi = 0; gi + SPI < ku; gi += SPI) {
            for_static<0, SPI>([&](auto kc) {
                constexpr int k = decltype(kc)::value;
                step(kc, true, true, setpair(kc), setpair(std::integral_constant<int, k + 1>{}));
            });
        }
        /* the tile's last pass: its last sub-step meets the loaders unless
         * this is the last tile, and reads nothing: the next tile's first
         * fragments are read after the epilogue, which then has the
         * registers of both sets */
        for_static<0, SPI>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            constexpr bool end = k == SPI - 1;
            step(kc, !(end && last), !end, setpair(kc), setpair(std::integral_constant<int, k + 1>{}));
        });

        /* ------------------------------------------------------ epilogue */
        /* ref's order a value: fmaf((float)s, d, +0) * ws [+ bias] [+ out];
         * addresses past the tile's frames or channels are clamped to the
         * last ones for loads, and nothing is stored there */
        const GemmArgs &g = tab.g[j];
        const Seg &sg = tab.s[j];
        const uint32_t T = sg.T, n0 = tn * BN, m0 = tm * BM, rows = g.rows;
        const float *e = epi[rt & 1];
        /* the lane index through an empty asm, so that the offsets derived
         * from it are computed here rather than hoisted and held in
         * registers across the K loop */
        uint32_t ln = lane;
        asm volatile("" : "+v"(ln));
        const uint32_t cl = wn * TN * 16 + (ln >> 4) * 4;       /* the lane's first channel in the tile */
        auto frame = [&](int jj) { return m0 + (wm * TM + jj) * 16 + (ln & 15); };
        auto at = [&](int jj, int i) {
            const uint32_t t = frame(jj), c = n0 + cl + i * 16;
            return sg.out + (size_t)(t < T ? t : T - 1) * sg.os + (c < rows ? c : rows - 4);
        };
        /* the four outputs of sums s at channel c (tile-local) of one frame */
        auto value = [&](const v4i &s, uint32_t c, float dt) {
            const float4 wsv = *(const float4 *)&e[BM + c];
            float4 v;
            v.x = __builtin_fmaf((float)s[0], dt, 0.0f) * wsv.x;
            v.y = __builtin_fmaf((float)s[1], dt, 0.0f) * wsv.y;
            v.z = __builtin_fmaf((float)s[2], dt, 0.0f) * wsv.z;
            v.w = __builtin_fmaf((float)s[3], dt, 0.0f) * wsv.w;
            if (g.bias) {
                const float4 bv = *(const float4 *)&e[BM + BN + c];
                v.x = v.x + bv.x;
                v.y = v.y + bv.y;
                v.z = v.z + bv.z;
                v.w = v.w + bv.w;
            }
            return v;
        };
        /* The vector stores write whole 128-byte lines, each from 8
         * consecutive lanes in address order, where a block's own layout
         * stores 64 bytes of 16 frames, one frame a lane (measured: ff up at
         * ten minutes of audio 52.1-52.6 -> 49.6-50.4 us; the same store
         * pattern without the moves below 45.7-46.9 us, which is what they
         * cost). The sums move as integers before the epilogue, so
         * the bits are the same: channel blocks 2k and 2k + 1 pair up and
         * swap the block for the lane's bit 3 (lanes l and l ^ 8 exchange
         * through DPP row_ror:8, a rotation by 8 inside each row of 16
         * lanes), so that each register of a pair holds 8 frames x 32
         * channels, lane (r, b, f) channel 16 b + 4 r of frame f; then one
         * ds_bpermute a dword moves it to lane 8 f + 4 b + r, whose 16 bytes
         * are chunk 4 b + r of frame f's line. */
        static_assert(TN % 2 == 0, "channel blocks pair up");
        constexpr int NP = TN / 2;
        const uint32_t hi = (ln >> 3) & 1;
        /* the lane this one takes its sums from after the swap, in bytes */
        const int src = (int)((((ln & 3) << 4) | (((ln >> 2) & 1) << 3) | (ln >> 3)) * 4);
        const uint32_t cp = wn * TN * 16 + (ln & 7) * 4;                 /* the lane's first channel in pair 0 */
        auto frame2 = [&](int jj, int h) { return m0 + (wm * TM + jj) * 16 + h * 8 + (ln >> 3); };
        auto at2 = [&](int jj, int k, int h) {
            const uint32_t t = frame2(jj, h), c = n0 + cp + k * 32;
            return sg.out + (size_t)(t < T ? t : T - 1) * sg.os + (c < rows ? c : rows - 4);
        };
        /* one straight-line epilogue each for plain and residual-adding
         * vector stores (with add, frame block jj + 1's residuals load before
         * block jj's stores issue, so a block's wait, vmcnt counting stores
         * too, waits for the stores of two blocks back, never the last one's) */
        auto vec_rows = [&](auto addc) {
            constexpr bool ADD = decltype(addc)::value;
            float4 old[2][TN];
            auto load_old = [&](int jj, float4 *o) {
#pragma unroll
                for (int k = 0; k < NP; k++)
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        o[k * 2 + h] = *(const float4 *)at2(jj, k, h);
            };
            if constexpr (ADD)
                load_old(0, old[0]);
#pragma unroll
            for (int jj = 0; jj < TM; jj++) {
                if constexpr (ADD) {
                    if (jj + 1 < TM)
                        load_old(jj + 1, old[(jj + 1) & 1]);
                }
                float dt[2];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint32_t t = frame2(jj, h);
                    dt[h] = e[(t < T ? t : T - 1) - m0];
                }
#pragma unroll
                for (int k = 0; k < NP; k++) {
                    v4i x[2];
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        const int a = acc[2 * k][jj][d], bq = acc[2 * k + 1][jj][d];
                        const int ar = __builtin_amdgcn_update_dpp(0, a, 0x128, 0xF, 0xF, false);
                        const int br = __builtin_amdgcn_update_dpp(0, bq, 0x128, 0xF, 0xF, false);
                        x[0][d] = __builtin_amdgcn_ds_bpermute(src, hi ? br : a);     /* frames 0-7 of the block */
                        x[1][d] = __builtin_amdgcn_ds_bpermute(src, hi ? bq : ar);    /* frames 8-15 */
                    }
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const uint32_t t = frame2(jj, h);
                        float4 v = value(x[h], cp + k * 32, dt[h]);
                        if constexpr (ADD) {
                            const float4 o4 = old[jj & 1][k * 2 + h];
                            v.x = o4.x + v.x;
                            v.y = o4.y + v.y;
                            v.z = o4.z + v.z;
                            v.w = o4.w + v.w;
                            /* the sums happen on every lane, so every residual
                             * load is waited for here and none is left in
                             * flight into the next tile's loop (whose register
                             * writes would then wait on vmcnt, stores
                             * included) */
                            asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
                        }
                        if (t < T && n0 + cp + k * 32 < rows)
                            store_out4(at2(jj, k, h), v, g.plain);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);      /* one frame block's registers at a time */
            }
        };
        if (((sg.os & 3) == 0) && ((((uintptr_t)sg.out) & 15) == 0)) {
            if (g.add)
                vec_rows(std::true_type{});
            else
                vec_rows(std::false_type{});
        } else {
#pragma unroll
            for (int jj = 0; jj < TM; jj++) {
                const uint32_t t = frame(jj);
                const float dt = e[(t < T ? t : T - 1) - m0];
#pragma unroll
                for (int i = 0; i < TN; i++) {
                    const float4 v = value(acc[i][jj], cl + i * 16, dt);
                    if (t < T && n0 + cl + i * 16 < rows) {
                        float *o = at(jj, i);
                        store_out1(o, g.add ? o[0] + v.x : v.x, g.plain);
                        store_out1(o + 1, g.add ? o[1] + v.y : v.y, g.plain);
                        store_out1(o + 2, g.add ? o[2] + v.z : v.z, g.plain);
                        store_out1(o + 3, g.add ? o[3] + v.w : v.w, g.plain);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (!last) {
            read_set(f0, slot, 0);
            wait_lgkm<0>();
#pragma unroll
            for (int r = 0; r < R; r++)
                asm volatile("" : "+v"(f0.f[r]));
        }
    }
}

/* the CUs of the current device, taken once a device */
static uint32_t device_cus() {
    static uint32_t cus[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus[dev] = (uint32_t)n;
    }
    return cus[dev];
}

template <int WN, int WM, int TN, int TM, int UPS, int NS, int NL, int OCC>
static void run_stream_jobs(const JobTable &jobs, hipStream_t s, bool packed) {
    constexpr uint32_t BN = 16 * TN * WN, BM = 16 * TM * WM;
    constexpr uint32_t threads = 64 * (WN * WM + NL);
    JobTable t = jobs;
    uint32_t tiles = 0;
    for (uint32_t j = 0; j < t.njobs; j++) {
        t.wg0[j] = tiles;
        t.tiles_n[j] = (t.g[j].rows + BN - 1) / BN;
        t.tiles[j] = t.tiles_n[j] * ((t.s[j].T + BM - 1) / BM);
        tiles += t.tiles[j];
    }
    t.wg0[t.njobs] = tiles;
    if (tiles == 0)
        return;
    /* a multiple of 8 workgroups, so that workgroup b runs on XCD b % 8 in
     * every round of tiles */
    uint32_t grid = device_cus() * OCC;
    grid = grid / 8 * 8;
    if (tiles < grid)
        grid = tiles;
    if (packed)
        gemm_stream_kernel<WN, WM, TN, TM, UPS, NS, NL, true><<<grid, threads, 0, s>>>(t, tiles);
    else
        gemm_stream_kernel<WN, WM, TN, TM, UPS, NS, NL, false><<<grid, threads, 0, s>>>(t, tiles);
}

template <int WN, int WM, int TN, int TM, int UPS, int NS, int NL, int OCC>
static void run_stream(const GemmArgs &g, const SegTable &tab, hipStream_t s) {
    JobTable t;
    t.njobs = 1;
    t.g[0] = g;
    t.s[0] = tab.s[0];
    run_stream_jobs<WN, WM, TN, TM, UPS, NS, NL, OCC>(t, s, tab.s[0].qstride != 0);
}

template <int WN, int WM, int TN, int TM, int UPS, int NS, int NL, int OCC>
static void run_stream_batch(const JobTable &jobs, hipStream_t s) {
    run_stream_jobs<WN, WM, TN, TM, UPS, NS, NL, OCC>(jobs, s, true);
}



static const StreamCfg kStreamCfgs[] = {
    /* name <channels x frames, units a stage, slots, loader waves>: eight MFMA
     * waves of 64 x 64 and four loader waves, one workgroup a CU (the ring
     * and the loaders' share of the waves leave no room for a second) */
    { "stream<256x128,2,3,l4>", 256, 128, 2, 3, run_stream<4, 2, 4, 4, 2, 3, 4, 1>, run_stream_batch<4, 2, 4, 4, 2, 3, 4, 1> },
    { "stream<128x256,2,3,l4>", 128, 256, 2, 3, run_stream<2, 4, 4, 4, 2, 3, 4, 1>, run_stream_batch<2, 4, 4, 4, 2, 3, 4, 1> },
    { "stream<128x256,1,4,l4>", 128, 256, 1, 4, run_stream<2, 4, 4, 4, 1, 4, 4, 1>, run_stream_batch<2, 4, 4, 4, 1, 4, 4, 1> },
};

const StreamCfg *stream_cfg(int i) {
    return i >= 0 && i < stream_count() ? &kStreamCfgs[i] : nullptr;
}

int stream_count() { return (int)(sizeof kStreamCfgs / sizeof kStreamCfgs[0]); }

}  // namespace pkq8
