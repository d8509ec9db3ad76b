/* Internal interface between the HIP kernels (q8_kernels.hip) and the
 * runtime that exposes them through the C ABI (pk_hip.cpp). */
#ifndef PK_Q8_INTERNAL_H
#define PK_Q8_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace pkq8 {

/* A matrix in HBM, repacked from PK_Q8 (16-row panels, groups of 4 inputs)
 * into units of 16 rows by 64 inputs: a unit is 1 KB, the 16 rows' 64 bytes
 * in the order the 16x16x64 int8 MFMA takes an operand (byte 16 * (kq * 16 +
 * r) + kb holds row r, input 16 * kq + kb of the unit). Units are stored
 * stage-major: unit u of every panel, then unit u + 1 of every panel, so
 * unit (p, u) is at 1 KB * (u * panels + p) and the workgroups that load one
 * stage at once read one contiguous run of memory (a panel-major layout puts
 * a stage's units a panel's length apart, onto few HBM channels). Each panel
 * has ku units, ceil(cols / 64) rounded up to a multiple of 4 so that the
 * pipelined product's four-slot ring divides it, inputs past cols zero. A
 * run of panels starting at panel p0 is the matrix at byte 1 KB * p0 with the
 * same unit stride. */
constexpr uint32_t kUnitBytes = 1024;

inline uint32_t units_with_data(uint32_t cols) { return (cols + 63) / 64; }
inline uint32_t units_per_panel(uint32_t cols) { return (units_with_data(cols) + 3) & ~3u; }

/* One segment of activations and outputs. */
struct Seg {
    float *out;
    const int8_t *q;            /* row-major [T][n], or packed units when qstride != 0 */
    const float *d;
    uint64_t os;
    uint64_t qstride;           /* packed: bytes from a row group's unit u to its unit u + 1 */
    uint32_t T;
    uint32_t tile0;             /* the grouped launch's first M tile of this segment */
};

/* Packed activations: the frames in groups of 16, each group's inputs in
 * units of 64 like the weights (16 rows x 64 inputs, 1 KB, MFMA operand
 * order), stage-major: unit (g, u) at 1 KB * (u * G + g), G = ceil(T / 16),
 * ku units a group as for a matrix of n inputs. Rows past T and inputs past
 * n are left unwritten: rows past T are never stored, and inputs past n meet
 * zero weights. */
inline uint32_t packed_groups(uint32_t T) { return (T + 15) / 16; }
inline uint64_t packed_bytes(uint32_t n, uint32_t T) {
    return (uint64_t)packed_groups(T) * units_per_panel(n) * kUnitBytes;
}

constexpr int kMaxSegs = 64;

struct SegTable {
    Seg s[kMaxSegs];
    uint32_t nseg;
};

/* What every product launch shares. */
struct GemmArgs {
    const int8_t *w;            /* repacked weights: unit 0 of the call's first panel */
    uint64_t wstride;           /* bytes from a panel's unit u to its unit u + 1 */
    const float *ws, *bias;     /* at the first row of the call */
    uint32_t rows;              /* N, a multiple of 16 */
    uint32_t n;                 /* K, a multiple of 32 */
    uint32_t ku;                /* units a panel (the stride, a multiple of 4) */
    uint32_t kr;                /* units holding inputs: ceil(n / 64) */
    uint32_t qb, nb;            /* block inputs, blocks a column */
    int add;
    int rmode;                  /* 0 nearest, 1 upward, 2 downward, 3 toward zero */
    /* with oqp set (blocked products on 64 x 64 pipelined tiles, all rows of
     * the matrix, nearest rounding): the outputs are not stored but SiLU'd and
     * quantized in blocks of oqb into the packed copy oqp and the scales od,
     * the next product's activations, as a SiLU quantize of them would */
    int8_t *oqp = nullptr;
    float *od = nullptr;
    uint32_t oqb = 0;
    /* 1: plain output stores; 0: non-temporal (set by the launch from the
     * size of its outputs, kPlainStoreBytes) */
    int plain = 0;
    /* the skinny product's split-K workspace (skinny_workspace_bytes(rows),
     * zero before its first use; every call leaves its counters zero), or
     * null: no split */
    void *skw = nullptr;
};

/* The skinny product split over K: at most kMaxSplit workgroups a panel; the
 * workspace a product of rows channels needs (a counter a panel, then
 * kMaxSplit partials of 1 KB a panel); forcing a split (1..kMaxSplit, -1 the
 * heuristic; returns the one forced before). */
constexpr uint32_t kMaxSplit = 8;
size_t skinny_workspace_bytes(uint32_t rows);
int set_skinny_split(int s);

/* Outputs of a launch above this many bytes are stored plain. */
constexpr uint64_t kPlainStoreBytes = (uint64_t)64 << 20;

int launch_repack(int8_t *dst, const int8_t *src, uint32_t rows, uint32_t cols, hipStream_t s);

int launch_quantize(int8_t *q, float *d, const float *x, size_t xs, uint32_t n, uint32_t qb,
                    uint32_t T, hipStream_t s, const char **name);

/* The quantizer under a directed rounding mode (rm 1 upward, 2 downward, 3
 * toward zero), one thread a block: -2 for rm or qb it does not take. */
int launch_quantize_directed(int8_t *q, float *d, const float *x, size_t xs, uint32_t n, uint32_t qb, uint32_t T,
                             int rm, hipStream_t s, const char **name);

/* Quantize (n <= 4096; qb == n, 32 or 64) writing the packed copy qp, and
 * the row-major q too when q is not NULL. */
int launch_quantize_packed(int8_t *q, int8_t *qp, float *d, const float *x, size_t xs, uint32_t n,
                           uint32_t qb, uint32_t T, hipStream_t s, const char **name, int op = 0);

/* The pipelined product's tilings: how many, and forcing one (-1: the
 * heuristic); returns the one forced before. */
int ring_count();
const char *ring_name(int i);
int set_ring(int i);

/* The packed quantize's kernel: 0 one wave a column (a wave a 1024-input
 * chunk of a wide column in blocks), 1 one workgroup a half group, 2 one wave a
 * whole column, -1 by size; returns the one forced before. */
int set_quant_kernel(int kind);

/* The attention's score and PV kernels: 0 the matrix cores', 1 the VALU
 * chains; returns the one set before. */
int set_attention_kernels(int valu);

/* The quantize's op on its inputs (launch_quantize_packed's op). */
constexpr int kOpPlain = 0, kOpSilu = 1;

/* The device-resident layer's float kernels (layer_kernels.hip): 0, -2 for
 * shapes they do not take, -1 for a failed launch. */
int launch_normq(int8_t *qp, float *d, const float *x, uint32_t n, uint32_t T, const float *w, const float *b,
                 float eps, uint32_t qb, hipStream_t s);
int launch_norm(float *x, uint32_t n, uint32_t T, const float *w, const float *b, float eps, hipStream_t s);
/* The attention's workspace: H x T rows of att_score_stride(T) scores and
 * H x T row sums' inverses, att_workspace_floats(T, H) floats. */
uint32_t att_score_stride(uint32_t T);
size_t att_workspace_floats(uint32_t T, uint32_t H);
/* The attention's output into of, or with qp set (the matrix-core kernels
 * only; -2 else), quantized in blocks of qb = 32 or 64 channels into the
 * packed copy qp and the scales qd instead (of is not written). */
int launch_attention(float *of, float *ws, const float *qf, const float *kf, const float *vf, const float *pf,
                     const float *bu, const float *bv, uint32_t T, uint32_t D, uint32_t H, hipStream_t s,
                     int8_t *qp = nullptr, float *qd = nullptr, uint32_t qb = 0);
/* The attention's static scratch (layer_kernels.hip) for callers that
 * cannot allocate: its bytes, and its address on device dev, which must be
 * current (taken once a device; NULL with the HIP error in *err if it
 * cannot be had), with, in *last when last is set, an event of that device
 * created at the same time, which the entry records after each use so that
 * the next use waits for it. */
constexpr size_t kStaticScratchBytes = (size_t)24 << 20;
constexpr int kMaxDevices = 64;
void *static_scratch(int dev, int *err, hipEvent_t *last = nullptr);

int launch_dwq(int8_t *qp, float *d, const float *u, uint32_t T, uint32_t D, const float *w, const float *b,
               uint32_t K, uint32_t qb, hipStream_t s);

/* The decoder's fused per-token launches (dec_kernels.hip): w the device
 * units of a matrix (wstride its panels x 1 KB), kr its units with data. */
int launch_gemv(float *out, const int8_t *w, uint64_t wstride, const float *ws, const float *bias, const float *x,
                uint32_t rows, uint32_t n, uint32_t kr, int add, hipStream_t s);
int launch_lstm(float *h_out, float *c, const float *h_in, const float *x, const int8_t *wx, const float *wxs,
                const int8_t *wh, const float *whs, uint64_t wstride, const float *b, uint32_t P, uint32_t kr,
                hipStream_t s);
int launch_joint(float *logit, uint32_t *tok_dur, const int8_t *w, uint64_t wstride, const float *ws,
                 const float *bias, const float *f, const float *gp, uint32_t rows, uint32_t J, uint32_t kr,
                 uint32_t V, uint32_t n_dur, hipStream_t s);

/* The decoder's greedy search in one cooperative launch (dec_kernels.hip):
 * the launch's arguments, the caller filling everything above the
 * workspace's pieces; launch_search carves ws (search_workspace_bytes),
 * zeroes the arrivals, the flag and the state on s, and launches. 0, -2 for
 * shapes it does not take, -1 for a failed call. */
constexpr int kMaxDecLayers = 8;
/* the search keeps its panels resident (gate panels in registers, the
 * joint's in LDS) up to this many LSTM layers and units a panel row */
constexpr int kResLayers = 2, kResUnits = 10;

struct SearchArgs {
    const float *f;                                 /* [T][J], the joint's encoder half of each frame */
    const float *embed;                             /* [V + 1][P] */
    const int8_t *wx[kMaxDecLayers], *wh[kMaxDecLayers];
    const float *wxs[kMaxDecLayers], *whs[kMaxDecLayers], *b[kMaxDecLayers];
    const int8_t *jpred, *jout;
    const float *jpred_s, *jpred_b, *jout_s, *jout_b;
    uint64_t lstm_stride, jpred_stride, jout_stride; /* the matrices' unit strides */
    uint32_t P, L, J, V, n_dur, rows_out, blank, max_symbols, T, cap, kr_p, kr_j, spin;
    int32_t dur[64];
    uint32_t *sync;                                 /* [1] the error flag, [64 + b] workgroup b's last barrier: zero at launch */
    float *h;                                       /* [L][2][P], zero at launch */
    float *c;                                       /* [L][P], zero at launch */
    float *gp;                                      /* [J] */
    float *logit;                                   /* [rows_out] */
    int32_t *toks;                                  /* [cap][3]: token, frame, duration */
    uint32_t *out;                                  /* [0] tokens, [1] 0, or 2 when cap was reached */
};

size_t search_workspace_bytes(uint32_t L, uint32_t P, uint32_t J, uint32_t rows_out, uint32_t cap);
int launch_search(SearchArgs &a, void *ws, hipStream_t s);
/* tests: false makes the search load its panels each token where they
 * would fit resident; returns the previous setting */
bool set_search_resident(bool on);

/* Measurement aids (diag_kernels.hip): an empty launch; a streaming read of
 * bytes (a multiple of 16) at p, 16-byte aligned. */
int launch_empty(hipStream_t s);
int launch_stream_read(const void *p, uint64_t bytes, uint32_t *sink, hipStream_t s);
/* workgroups of four waves, each iters rounds of eight int8 16x16x64 MFMAs */
int launch_mfma_rate(uint32_t workgroups, uint32_t iters, uint32_t *sink, hipStream_t s);

/* One product; table->nseg == 1 for a plain call. With g.oqp set, -3 where
 * the fused SiLU quantize is not available (nothing launched). */
int launch_gemm(const GemmArgs &g, const SegTable &table, hipStream_t s, const char **name);

/* Independent products in one launch: job j is the product g[j] x s[j] (one
 * segment each). All share n, ku, per-row blocks, packed activations and the
 * rounding mode. Its workgroups start at wg0[j], a multiple of 8, so every
 * job's first tile runs on XCD 0 and the XCD-aware tile order holds inside
 * each job; the workgroups between one job's tiles and the next job's start
 * do nothing. */
constexpr int kMaxJobs = 8;

struct JobTable {
    GemmArgs g[kMaxJobs];
    Seg s[kMaxJobs];
    uint32_t wg0[kMaxJobs + 1];
    uint32_t tiles_n[kMaxJobs], tiles[kMaxJobs];
    uint32_t njobs;
};

int launch_gemm_batch(const JobTable &jobs, hipStream_t s, const char **name);

/* The streamed product's tilings (q8_stream.hip): persistent workgroups over
 * the tile list, loader waves apart from the MFMA waves; per-row blocks, one
 * segment or a batch of jobs sharing ku. */
struct StreamCfg {
    const char *name;
    uint32_t bn, bm, ups, slots;        /* channels x frames, units a stage, ring slots */
    void (*run)(const GemmArgs &, const SegTable &, hipStream_t);
    void (*batch)(const JobTable &, hipStream_t);
};
const StreamCfg *stream_cfg(int i);     /* nullptr past the last */
int stream_count();

}  // namespace pkq8

#endif
