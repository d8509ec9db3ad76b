/* pk_hip.h - the C ABI of libpkhip.so, libpktito's int8 product path on one
 * MI355X (gfx950).
 *
 * libpktito's backend seam is a table of function pointers (the reference's
 * backend/kernels.h:242-278, pk_kernels). The int8 path is two of them:
 *
 *   quantize   fp32 activations to int8, per column in blocks of qb, a scale
 *              a block                     (backend/kernels.h:47-58)
 *   gemm_q8    the int8 product with exact int32 sums and the fixed fp32
 *              epilogue                    (backend/kernels.h:60-78)
 *
 * This library computes both on the GPU with the reference's bits: the int8
 * activations, their scales and every fp32 output are those of the
 * reference's scalar ref backend (backend/ref/kernels.c:24-86) on the same
 * inputs. The entry points come in five groups:
 *
 *   1. the drop-in: pk_hip_quantize and pk_hip_gemm_q8 take host pointers and
 *      the arguments of the table's quantize and gemm_q8, and return with the
 *      results in host memory, as the table's functions do;
 *   2. the upload: the model-load step that repacks each PK_Q8 matrix once
 *      into HBM (the reference binds matrices at core/model.c:345-363);
 *   3. the device-resident path: the same two operations on device pointers,
 *      asynchronous on a caller's stream, for callers that keep activations
 *      in HBM;
 *   4. the device-resident encoder layer: the passes the reference runs
 *      between its products, fused with their quantizes, and a whole layer
 *      in one call (core/encoder.c:108-368);
 *   5. the decoder's token steps: its T = 1 products fused into one launch a
 *      step (core/decoder.c:54-101).
 *
 * Every function returns PK_HIP_OK or an error code (pk_hip_strerror names it,
 * pk_hip_last_error gives the calling thread's last message); nothing falls
 * back to the CPU. No function here prints.
 */
#ifndef PK_HIP_H
#define PK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The activations of one product: the reference's pk_act
 * (backend/kernels.h:41-45), field for field, so a pk_act * may be passed
 * wherever a pk_hip_act * is taken.
 *   q  [T][n] int8, column t at q + t * n
 *   d  [T][n / qb] fp32, each block's scale */
typedef struct {
    int8_t   *q;
    float    *d;
    uint32_t  n, qb, T;
} pk_hip_act;

enum {
    PK_HIP_OK = 0,
    PK_HIP_EINVAL = 1,      /* arguments outside the contract */
    PK_HIP_ENODEV = 2,      /* no usable gfx950 device */
    PK_HIP_ENOMEM = 3,      /* a device or pinned allocation failed */
    PK_HIP_EDEVICE = 4,     /* a HIP call or a kernel launch failed */
    PK_HIP_ENOTUP = 5,      /* gemm_q8's w is inside no uploaded matrix */
    PK_HIP_EROUND = 6,      /* the caller's rounding mode is one this entry does not take */
    PK_HIP_ETIMEOUT = 7,    /* a launch's bounded wait ran out (the launch ended, its results are not whole) */
};

/* The error code's name, and the calling thread's last error message. */
const char *pk_hip_strerror(int err);
const char *pk_hip_last_error(void);

/* Opens the device (the one current on the calling thread, else device 0)
 * once a process; later calls return the first call's result. Every other
 * function calls it. The environment's PKTITO_HIP_DISABLE=1 makes it fail
 * with PK_HIP_ENODEV, so a caller's no-device path can be tested anywhere. */
int pk_hip_init(void);

/* ------------------------------------------------------------ upload --- */

/* Repacks the PK_Q8 matrix q (rows x cols, the reference's core/pkf.h:28-41
 * layout) into HBM with its rows scales s, once, and records the host range
 * [q, q + rows * cols) so that gemm_q8 calls whose w points at any whole
 * panel inside it run on the device copy. rows % 16 == 0, cols % 32 == 0,
 * cols <= 16384 (core/model.c:354). Replaces nothing in the reference: it is
 * the step a GPU backend adds after core/model.c's load_file (:783-811). The
 * host bytes and scales must not change while the matrix is uploaded (a
 * model's are its mapped file's): gemm_q8 reads the device copies, the
 * scales too when its ws is the uploaded s at that panel. A range that
 * shares any byte with an uploaded matrix's is refused (PK_HIP_EINVAL),
 * also when two threads upload it at once: one of them is taken. */
int pk_hip_upload_q8(const int8_t *q, const float *s, uint32_t rows, uint32_t cols);

/* Frees the device copy of the matrix whose host bytes start at q
 * (core/model.c:868-883's pk_model_free gains this call); all of them.
 * These wait for host-pointer products (pk_hip_gemm_q8) in flight on other
 * threads; the device-resident entries below are asynchronous, so their
 * caller must not release a matrix while products on it are queued. */
int pk_hip_release_q8(const int8_t *q);
void pk_hip_release_all(void);

/* -------------------------------------------------------- the drop-in --- */

/* The table's quantize (backend/kernels.h:47-58, :256), on host pointers:
 * a->q, a->d and x are host memory; returns with q and d written. Follows
 * the calling thread's rounding mode as the reference's ref does (both
 * divisions, the product and rintf; backend/ref/kernels.c:24-58); the
 * device-pointer quantizes below round to nearest. */
int pk_hip_quantize(pk_hip_act *a, const float *x, size_t xs);

/* The table's gemm_q8 (backend/kernels.h:60-78, :257-258), on host pointers:
 * out[t * os + r] for r < rows, t < a->T, w the PK_Q8 panels of those rows
 * and ws, bias their scales and biases. Where w is a whole panel of an
 * uploaded matrix the device copy is used; any other w (a caller's own
 * buffer, as the reference's checkers pass) is copied to the device and
 * repacked for this call alone: slower, the same bits. The floats between
 * one column's outputs and the next are not touched. Any of the four IEEE
 * rounding modes the calling thread has set. A release of the matrix
 * waits until the call has returned. */
int pk_hip_gemm_q8(float *out, size_t os, const int8_t *w, const float *ws, const float *bias,
                   uint32_t rows, const pk_hip_act *a, int add);

/* ------------------------------------------- the device-resident path --- */

/* An uploaded matrix, found by its host bytes; NULL if none holds q. */
typedef struct pk_hip_q8 pk_hip_q8;
const pk_hip_q8 *pk_hip_q8_find(const int8_t *q);
/* Its device scales (rows floats), rows and cols. */
const float *pk_hip_q8_scales(const pk_hip_q8 *m);
uint32_t pk_hip_q8_rows(const pk_hip_q8 *m);
uint32_t pk_hip_q8_cols(const pk_hip_q8 *m);

/* quantize on device pointers (a->q, a->d, x), enqueued on stream (a
 * hipStream_t; NULL for the null stream). q and x 16-byte aligned, xs a
 * multiple of 4 floats. Round-to-nearest. */
int pk_hip_quantize_dev(pk_hip_act *a, const float *x, size_t xs, void *stream);

/* gemm_q8 on device pointers: out, ws, bias, a->q and a->d in device memory;
 * the weights are rows [r0, r0 + rows) of the uploaded matrix m (r0 and rows
 * multiples of 16). ws and bias point at row r0's scale and bias (ws may be
 * pk_hip_q8_scales(m) + r0). a->q 16-byte aligned. rmode is the IEEE
 * rounding of the epilogue: 0 to nearest, 1 upward, 2 downward, 3 toward
 * zero. Enqueued on stream; returns once launched. */
int pk_hip_gemm_q8_dev(float *out, size_t os, const pk_hip_q8 *m, uint32_t r0, uint32_t rows,
                       const float *ws, const float *bias, const pk_hip_act *a, int add,
                       int rmode, void *stream);

/* Packed activations, for callers whose quantized activations feed only
 * products: the frames in groups of 16 and each group's inputs in units of
 * 16 frames x 64 inputs laid out as the MFMA takes them, unit u of every
 * group before unit u + 1 (the repacked weights' layout), so that a
 * product's activation tiles are contiguous 1 KB reads. Same q bytes, same
 * d, same outputs as the row-major path. No counterpart in the reference,
 * whose pk_act is row-major (backend/kernels.h:41-45): an extension of the
 * device-resident path. */

/* Bytes a packed copy of T columns of n inputs takes. */
size_t pk_hip_packed_bytes(uint32_t n, uint32_t T);

/* quantize (blocks of the whole row, or of 32 or 64 inputs: the encoder's
 * modes; n <= 4096) writing d and the packed copy qp, and the row-major a->q
 * too unless it is NULL. Device pointers; qp 16-byte aligned and
 * pk_hip_packed_bytes(n, T) long. */
int pk_hip_quantize_packed_dev(pk_hip_act *a, int8_t *qp, const float *x, size_t xs, void *stream);

/* gemm_q8_dev with the activations read from the packed copy qp (a->q is
 * not read; a->d, n, qb and T are; qb the whole row, 32 or 64). */
int pk_hip_gemm_q8_packed_dev(float *out, size_t os, const pk_hip_q8 *m, uint32_t r0, uint32_t rows,
                              const float *ws, const float *bias, const pk_hip_act *a, const int8_t *qp,
                              int add, int rmode, void *stream);

/* The few-frame products (T <= 16, blocks of the whole row: the decoder's
 * per-row callers, core/decoder.c:53-63 and :83-101, and the skinny
 * configs) bound by streaming the weights once: with a workspace, the K
 * inputs of each 16-row panel are split over up to 8 workgroups, so a
 * matrix of few panels (1024 or 1040 rows: 64 or 65 panels) spreads its
 * weights over the chip's CUs instead of one CU a panel. The workgroups of
 * a panel hand their exact int32 sums over in the workspace and the last
 * one runs the epilogue once: the same bits as the entries above. No
 * counterpart in the reference (its CPU calls have no split to make).
 *
 * pk_hip_gemm_workspace(rows): the bytes of workspace a product of rows
 * channels takes. The workspace is device memory, 256-byte aligned and zero
 * before its first use: it starts with a counter a panel, which every call
 * leaves at zero again, then the partial sums, which a call writes before it
 * reads them. Calls that overlap in time (two streams) need workspaces of
 * their own. */
size_t pk_hip_gemm_workspace(uint32_t rows);

/* pk_hip_gemm_q8_dev and pk_hip_gemm_q8_packed_dev with that workspace
 * (work, work_bytes >= pk_hip_gemm_workspace(rows)); NULL: no split. Other
 * calls (T > 16, blocks of 32 or 64) run as the entries above and leave it
 * untouched. */
int pk_hip_gemm_q8_ws_dev(float *out, size_t os, const pk_hip_q8 *m, uint32_t r0, uint32_t rows,
                          const float *ws, const float *bias, const pk_hip_act *a, int add, int rmode,
                          void *work, size_t work_bytes, void *stream);
int pk_hip_gemm_q8_packed_ws_dev(float *out, size_t os, const pk_hip_q8 *m, uint32_t r0, uint32_t rows,
                                 const float *ws, const float *bias, const pk_hip_act *a, const int8_t *qp,
                                 int add, int rmode, void *work, size_t work_bytes, void *stream);

/* One segment of a grouped product: its own activations and outputs. */
typedef struct {
    float      *out;
    size_t      os;
    pk_hip_act  a;
} pk_hip_seg;

/* gemm_q8 of one matrix over nseg segments of activations in a single launch
 * (the ragged batch of segments of different lengths that the reference runs
 * as concurrent lanes, core/asr.c:346-570): each segment's outputs are the
 * bits pk_hip_gemm_q8_dev gives it alone. Device pointers throughout; the
 * segments share n and qb; nseg <= 64. */
int pk_hip_gemm_q8_grouped_dev(const pk_hip_q8 *m, uint32_t r0, uint32_t rows, const float *ws,
                               const float *bias, const pk_hip_seg *segs, uint32_t nseg, int add,
                               void *stream);

/* One product of a batch: an uploaded matrix's run of panels [r0, r0 + rows)
 * with its scales and bias at r0 (device), the packed activations qp of a
 * (a->q is not read), and the outputs out[t * os + r]. */
typedef struct {
    float             *out;
    size_t             os;
    const pk_hip_q8   *m;
    uint32_t           r0, rows;
    const float       *ws, *bias;
    pk_hip_act         a;
    const int8_t      *qp;
    int                add;
} pk_hip_job;

/* njobs <= 8 independent products in one launch, each job's outputs the bits
 * pk_hip_gemm_q8_packed_dev gives it alone. The reference runs such products
 * one after another (core/encoder.c:329-368: the attention's q, k and v of one
 * activation, and the positions' projection); a device-resident caller
 * launches them together. The jobs share n and qb (per-row, qb == n, or
 * blocks of 32 or 64); device pointers throughout. */
int pk_hip_gemm_q8_batch_dev(const pk_hip_job *jobs, uint32_t njobs, int rmode, void *stream);

/* ----------------------------------------- the device-resident layer --- */

/* The producers of the encoder's activations (core/encoder.c), each fused
 * with the quantize that follows it there and writing the packed copy qp
 * (pk_hip_packed_bytes(a->n, a->T) long) and a->d that the next product
 * reads; a->q is not written. Device pointers, 16-byte aligned; a->qb the
 * whole row, 32 or 64 (dwq: 32 or 64). Same bits as the reference's pass
 * followed by its quantize. No counterpart in the reference's kernel table:
 * these are its CPU passes between the products (core/encoder.c:108-176),
 * which a device-resident caller runs where the activations already are. */

/* normq (core/encoder.c:108-128): each of a->T frames of a->n floats at x
 * (frame t at x + t a->n) layer-normed by w, b, eps (backend/kernels.h:
 * 112-122) and quantized; a->n a multiple of 64 up to 4096. */
int pk_hip_normq_dev(pk_hip_act *a, int8_t *qp, const float *x, const float *w, const float *b, float eps,
                     void *stream);

/* siluq (core/encoder.c:130-156): SiLU of each frame (stride xs) then the
 * quantize; a->n a multiple of 32 up to 4096. */
int pk_hip_siluq_dev(pk_hip_act *a, int8_t *qp, const float *x, size_t xs, void *stream);

/* dw (core/encoder.c:158-176): GLU of u [T][2 a->n] (backend/kernels.h:
 * 140-142), the depthwise convolution of K <= 33 taps w [a->n][K] with bias
 * b and SiLU (backend/kernels.h:144-158), quantized; a->n a multiple of 64. */
int pk_hip_dwq_dev(pk_hip_act *a, int8_t *qp, const float *u, const float *w, const float *b, uint32_t K,
                   void *stream);

/* The layer norm in place over T rows of n floats (backend/kernels.h:
 * 112-122; core/encoder.c:86-99); n a multiple of 64 up to 4096. */
int pk_hip_layernorm_dev(float *x, uint32_t T, uint32_t n, const float *w, const float *b, float eps,
                         void *stream);

/* The attention's float part (core/encoder.c:280-327): H heads of D / H
 * dimensions (a multiple of 16; heads of a multiple of 64 run on the
 * tiled kernels, others on one thread an output: fine for the tiny models'
 * 16-wide heads, slow, with no tiling, for long inputs), o [T][D] from the
 * products' outputs q, k,
 * v [T][D] and the positions' p [2T - 1][D] with the biases u and v [D]:
 * Transformer-XL's scores, the softmax, the weighted values, each output
 * the chain pk_k_gemm_f32 and pk_k_softmax make. The scores live in ws,
 * pk_hip_attention_workspace(T, H) bytes. */
size_t pk_hip_attention_workspace(uint32_t T, uint32_t H);
int pk_hip_attention_dev(float *o, const float *q, const float *k, const float *v, const float *p,
                         const float *bias_u, const float *bias_v, uint32_t T, uint32_t D, uint32_t H, void *ws,
                         size_t ws_bytes, void *stream);

/* pk_hip_attention_dev with its scores and row sums in a static scratch
 * array of the library (24 MiB on each GPU it runs on, held until the
 * process ends) instead of a workspace: no allocation of any kind, for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * pk_hip_attention_workspace(T, H) must be at most 24 MiB (T up to 884 at 8
 * heads), else PK_HIP_EINVAL. Every call on one GPU shares the array; it
 * keeps the last call's contents, and each call rewrites every score it
 * reads. Outside stream capture a call's kernels wait for the previous
 * call's on that GPU (an event the library records after each call), so
 * calls on two streams or threads take turns. Under capture the call adds
 * no such wait: the caller orders a graph's replays against each other and
 * against other calls (replays of one graph on one stream are ordered). */
int pk_hip_attention_noalloc_dev(float *o, const float *q, const float *k, const float *v, const float *p,
                                 const float *bias_u, const float *bias_v, uint32_t T, uint32_t D, uint32_t H,
                                 void *stream);

/* One encoder layer's weights on the device (core/model.h:45-53): the
 * eleven matrices uploaded, the vectors as device pointers. D = d_model
 * (a multiple of 64 up to 4096), H heads of D / H (a multiple of 16),
 * F = ff_dim (a multiple of 64 up to 4096), K depthwise taps (<= 33). */
typedef struct {
    uint32_t D, H, F, K;
    float    eps;
    const float *ff1_nw, *ff1_nb, *att_nw, *att_nb, *conv_nw, *conv_nb;
    const float *ff2_nw, *ff2_nb, *out_nw, *out_nb;
    const pk_hip_q8 *ff1_up, *ff1_down, *ff2_up, *ff2_down;
    const pk_hip_q8 *q, *k, *v, *pos, *o;
    const float *bias_u, *bias_v;
    const pk_hip_q8 *pw1, *pw2;
    const float *dw, *dw_b;
} pk_hip_layer;

/* Bytes of device workspace pk_hip_layer_dev needs at T frames. */
size_t pk_hip_layer_workspace(const pk_hip_layer *L, uint32_t T, uint32_t qb);

/* One layer (core/encoder.c:321-368) in place on x [T][D] in HBM: the
 * positions' activations ape_qp / ape_d are 2T - 1 frames of D quantized in
 * blocks of qb (pk_hip_quantize_packed_dev once an encode, core/encoder.c:
 * 467-469); the layer's activations are quantized in blocks of qb (32 or
 * 64, the encoder's modes, core/encoder.c:50-56). Every kernel on stream,
 * nothing allocated: ws is ws_bytes >= pk_hip_layer_workspace(L, T, qb) of
 * device memory. The same bits as the reference's layer() over its ref
 * kernels. Calls that overlap on one workspace race. */
int pk_hip_layer_dev(const pk_hip_layer *L, float *x, uint32_t T, const int8_t *ape_qp, const float *ape_d,
                     uint32_t qb, void *ws, size_t ws_bytes, void *stream);

/* ------------------------------------------ the decoder's token steps --- */

/* The decoder's per-token products (core/decoder.c:54-101), each a quantize
 * of one row (one block) and a T = 1 product, latency-bound: each entry is
 * one launch (the joint two) that fuses what the reference runs as separate
 * calls. Device pointers; the matrices uploaded, cols <= 4096. Same bits as
 * the reference's calls over its ref kernels. No counterpart in the kernel
 * table: these are core/decoder.c's steps, for a caller whose prediction
 * state lives in HBM. */

/* gemv (core/decoder.c:54-63): x (m's cols floats) quantized whole and
 * multiplied: out[r] for every row r of m, plus bias[r] if bias, added to
 * out[r] if add. */
int pk_hip_gemv_dev(float *out, const pk_hip_q8 *m, const float *bias, const float *x, int add, void *stream);

/* One LSTM layer's step (core/decoder.c:68-75): gates = wx x + b, then
 * + wh h_in (the reference's two calls), then the cell (backend/kernels.h:
 * 180-187): c stepped in place, the new h to h_out (which must not be h_in).
 * wx and wh are [4P][P], x, h_in, h_out and c P floats, b 4P. */
int pk_hip_lstm_step_dev(float *h_out, float *c, const float *h_in, const float *x, const pk_hip_q8 *wx,
                         const pk_hip_q8 *wh, const float *b, void *stream);

/* The joint (core/decoder.c:81-101): the logits of jout (its rows) from
 * relu(f + gp) (jout's cols floats each) plus jout_b, and tok_dur[0] = the
 * first best token of logits [0, V], tok_dur[1] = the first best duration
 * index among the n_dur logits after them. */
int pk_hip_joint_dev(float *logit, uint32_t *tok_dur, const pk_hip_q8 *jout, const float *jout_b, const float *f,
                     const float *gp, uint32_t V, uint32_t n_dur, void *stream);

/* The decoder's weights on the device, for the search below: shapes and
 * durations by value, the matrices uploaded, the vectors device pointers
 * (core/model.h's prediction network and joint). */
#define PK_HIP_DEC_MAX_LAYERS 8
typedef struct {
    uint32_t P, L, J, V, n_dur, blank, max_symbols;
    int32_t  dur[64];                               /* n_dur <= 64 */
    const float *embed;                             /* [V + 1][P] */
    const pk_hip_q8 *wx[PK_HIP_DEC_MAX_LAYERS], *wh[PK_HIP_DEC_MAX_LAYERS];   /* [4P][P] */
    const float *b[PK_HIP_DEC_MAX_LAYERS];          /* 4P each, or NULL */
    const pk_hip_q8 *jpred, *jout;                  /* [J][P]; [rows][J], rows >= V + 1 + n_dur */
    const float *jpred_b, *jout_b;
} pk_hip_decoder;

/* TDT's greedy search over a segment (core/decoder.c:121-147 and pk_decode,
 * :158-173: the state zeroed, the blank's prediction first) in one launch on
 * the device: the LSTM layers, jpred, the joint, its argmax, the duration
 * step and the max_symbols rule, with no host round trip between frames.
 * f: T frames of the joint's encoder half, device, [T][J] (pk_joint_frames'
 * output). Returns once the search has ended, with *ntoks tokens in toks
 * (host, 3 int32 a token: id, frame, duration, as pk_tok), the reference's
 * tokens. cap must be at least T * max_symbols (the most a search can emit).
 * ws: pk_hip_search_workspace(d, cap) bytes of device memory, 256-byte
 * aligned. P and J multiples of 16 up to 1024, V + 1 <= 2048, L <= 8.
 * spin_limit: the iterations a grid-wide wait may take before the launch
 * gives up (0: the default, about a second); a launch that gives up ends
 * and the call returns PK_HIP_ETIMEOUT. Not for stream capture (the launch
 * is cooperative and the call synchronizes). No counterpart in the kernel
 * table: core/decoder.c's loop, for a caller whose frames live in HBM. */
size_t pk_hip_search_workspace(const pk_hip_decoder *d, uint32_t cap);
int pk_hip_search_dev(const pk_hip_decoder *d, const float *f, uint32_t T, int32_t *toks, uint32_t cap,
                      uint32_t *ntoks, void *ws, size_t ws_bytes, uint32_t spin_limit, void *stream);

/* Measurement aids, with no counterpart in the reference: the floors a
 * small product's time is read against. pk_hip_empty_dev launches an empty
 * kernel; pk_hip_stream_read_dev reads the bytes at p (16-byte aligned,
 * bytes a multiple of 16) with non-temporal 16-byte loads, one a thread
 * over as many workgroups as they need (at most 32768, four loads a thread
 * in flight beyond that), and writes *sink only if the loads' fold meets a
 * fixed constant (so nothing is written in practice; sink is device
 * memory). */
int pk_hip_empty_dev(void *stream);
int pk_hip_stream_read_dev(const void *p, size_t bytes, uint32_t *sink, void *stream);
/* A measurement aid with no counterpart in the reference: the int8 matrix
 * cores' rate, for checking the published peak on the machine.
 * workgroups of four waves each run iters rounds of eight independent
 * v_mfma_i32_16x16x64_i8 (32768 ops each) on registers, nothing loaded;
 * *sink as for pk_hip_stream_read_dev. */
int pk_hip_mfma_rate_dev(uint32_t workgroups, uint32_t iters, uint32_t *sink, void *stream);

/* The kernel variant the calling thread launched last, for profiling and
 * tests. */
const char *pk_hip_last_kernel(void);

/* Tests and tuning: the number of tilings of the per-column product, each
 * one's name (the name pk_hip_last_kernel gives its launches; "" past the
 * last), and forcing one of them for every later launch in the process (-1
 * restores the automatic choice); returns the index forced before. Not
 * thread-safe against launches in flight on other threads. Every tiling
 * computes the same bits. */
int pk_hip_tilings(void);
const char *pk_hip_tiling_name(int index);
int pk_hip_force_tiling(int index);

/* Tests and tuning: how many workgroups share a panel in every later split
 * few-frame product (1..8; fewer where the panel has fewer units), -1 the
 * automatic choice; returns the one forced before. All compute the same
 * bits. */
int pk_hip_force_split(int splits);

/* Tests and tuning: 0 makes every later search load its LSTM, jpred and
 * jout panels from memory each token even where they fit resident (gate
 * panels in registers, the joint's panels in LDS, loaded once a launch:
 * P and J up to 640, at most 2 LSTM layers), 1 restores that; returns the
 * previous setting. Both compute the same tokens. */
int pk_hip_force_search_resident(int on);

/* Tests and tuning: forcing the packed quantize's kernel for every later
 * launch in the process: 0 one wave a column (or a wave a 1024-input chunk
 * of a column over 1024 inputs in blocks), 1 one workgroup a half
 * 16-column group, 2 one wave a whole column, -1 the automatic choice by size;
 * returns the one forced before. All compute the same bits. */
int pk_hip_force_quantize(int kind);

/* Tests and tuning: the attention's score and PV products for every later
 * launch in the process: 0 on the matrix cores (one-step fp32 MFMAs, the
 * default), 1 as VALU fma chains; returns the one set before. Both compute
 * the same bits. */
int pk_hip_force_attention(int valu);

#ifdef __cplusplus
}
#endif

#endif /* PK_HIP_H */
