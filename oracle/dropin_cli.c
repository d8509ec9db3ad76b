/* Test infrastructure: a transcription through the reference's own library
 * (core/model.c, core/asr.c, core/encoder.c, core/decoder.c, compiled where
 * they lie), on the kernel table PKTITO_KERNELS names (backend/kernels.c:
 * 291-312), printed token by token so that two runs compare with cmp as
 * tests/check-c.sh compares transcripts (:73-81).
 *
 *   dropin_cli MODEL.pkf SECONDS SEED FAST THREADS
 *
 * The audio is SECONDS of 16 kHz from SEED (xorshift64*: a few tones, their
 * loudness swelling and fading, and noise). Under PKTITO_KERNELS=hip every
 * int8 matrix of the model is uploaded after the load and released before
 * the free, as a checkout with the hip backend does in core/model.c's load
 * and free (:783-811, :868-883: pk_hip_upload_model after the matrices are
 * bound, pk_hip_release_model before they are unmapped). FAST 1 is the encoder's fast mode, blocks of 64 inputs
 * (pk_asr_set_fast_mode; blocks of 32 otherwise).
 *
 * A diarizer's model (pk_model_speakers > 0, core/pktito.h:117-119) is run
 * through the reference's diarizer instead (core/diar.c's pk_diar_run,
 * core/pktito.h:660-686: its products go to the same table in blocks of
 * 32), and every row of speaker probabilities is printed as exact hex
 * floats, "row i: p0 p1 ...", then "rows N S". FAST is then unused.
 *
 *   dropin_cli MODEL.pkf SECONDS SEED FAST THREADS --layers OUT
 *
 * also writes the reference's own encoder layers (core/encoder.c:338-368,
 * static, so reached through pk_encode, core/encoder.c:429-506, with the
 * model's n_layers set to 0, 1, ... in turn on the same features) to OUT:
 * each layer's input and output, the positions' quantized encodings and
 * every layer's weights, for the oracle's layer to be compared with. Layout
 * (little-endian): "PKLD", u32 Te, D, H, F, K, qb, L; f32 eps; f32 x[L + 1]
 * [Te][D]; i8 ape_q[2Te - 1][D]; f32 ape_d[2Te - 1][D / qb]; f32 pe[2Te - 1]
 * [D] (the encodings before their quantize); then a layer:
 * f32 ff1_nw, ff1_nb, att_nw, att_nb, conv_nw, conv_nb, ff2_nw, ff2_nb,
 * out_nw, out_nb, bias_u, bias_v [D]; f32 dw [D][K]; f32 dw_b [D]; and
 * ff1_up, ff1_down, ff2_up, ff2_down, q, k, v, pos, o, pw1, pw2 each as u32
 * rows, cols, i8 panels [rows * cols], f32 scales [rows].
 *
 *   dropin_cli MODEL.pkf SECONDS SEED FAST THREADS --decoder OUT
 *
 * writes the reference's decoder's input and output instead: the joint's
 * encoder half of every frame (pk_joint_frames, core/decoder.c:149-156),
 * the prediction network and joint, and the tokens its search emitted
 * (core/decoder.c:121-147). Layout: "PKDC", u32 Te, P, L, J, V, n_dur,
 * blank, max_symbols, dur[n_dur]; f32 f[Te][J]; f32 embed[V + 1][P]; per
 * LSTM layer wx, wh (u32 rows, cols, i8 panels, f32 scales) and f32 b[4P];
 * jpred, f32 jpred_b[J]; jout, f32 jout_b[its rows]; jenc, f32 jenc_b[J]
 * (the joint's encoder half, f's product); u32 ntoks; i32 (id, frame, dur)
 * a token.
 *
 *   dropin_cli --time-passes THREADS SECONDS [M K N]
 *
 * needs no model: times the reference's own pool entries on a synthetic
 * product (default M = 750 frames, K = 1024 inputs, N = 4096 rows, the
 * configs' first shape: int8 weights uniform in [-127, 127] in PK_Q8 panels,
 * scales uniform in [1e-3, 1e-2], frames N(0, 1) by Box-Muller from a fixed
 * xorshift64* seed), on the table PKTITO_KERNELS names: pk_quantize_on
 * (per-row blocks) then pk_gemm_on (no bias, no add, no callback) over a
 * pool of THREADS, repeated until SECONDS have gone by, as the encoder makes
 * them (core/encoder.c:63-77). Under PKTITO_KERNELS=hip the matrix is
 * uploaded first, as a model's load does. Prints one JSON line: the table,
 * the threads, the calls, and the quantize's, the product's and the pair's
 * mean milliseconds. Built twice: _ref/dropin_cli (the pool's own dealing)
 * and _ref/dropin_cli_whole (whole_product.c: one call a product under
 * hip), so the two dealings time side by side. */
#include "pktito.h"
#include "model.h"
#include "asr.h"
#include "mel.h"
#include "kernels.h"
#include "os.h"
#include "passes.h"
#include "pool.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void put(FILE *f, const void *p, size_t bytes) {
    if (bytes && fwrite(p, 1, bytes, f) != bytes) {
        fprintf(stderr, "write failed\n");
        exit(1);
    }
}

static void put_u32(FILE *f, uint32_t v) { put(f, &v, 4); }

static void put_q8(FILE *f, const pk_q8 *w) {
    put_u32(f, w->rows);
    put_u32(f, w->cols);
    put(f, w->q, (size_t)w->rows * w->cols);
    put(f, w->s, (size_t)w->rows * sizeof(float));
}

/* The encoder's layers one at a time (see the header): pk_asr_run has
 * sized every buffer for these samples; the features are made once. */
static int dump_layers(pk_model *m, pk_asr *a, const float *x, size_t n, const char *path) {
    const uint32_t L = m->n_layers, D = m->d_model;
    const size_t T0 = pk_mel_frames(m, n);
    pk_mel(a, x, n);
    FILE *f = fopen(path, "wb");
    if (!f)
        return -1;
    uint32_t Te = 0;
    for (uint32_t l = 0; l <= L; l++) {
        m->n_layers = l;
        Te = pk_encode(a, (uint32_t)T0);
        if (!Te || Te >= 100) {     /* a longer input races its layers' threads (core/encoder.c:403-427) */
            fclose(f);
            return -1;
        }
        if (l == 0) {
            put(f, "PKLD", 4);
            const uint32_t hdr[7] = { Te, D, m->n_heads, m->ff_dim, m->conv_kernel, a->ape.qb, L };
            put(f, hdr, sizeof hdr);
            put(f, &m->ln_eps, 4);
        }
        put(f, a->x, (size_t)Te * D * sizeof(float));
    }
    m->n_layers = L;
    const size_t R = 2 * (size_t)Te - 1;
    put(f, a->ape.q, R * D);
    put(f, a->ape.d, R * (D / a->ape.qb) * sizeof(float));
    put(f, a->pe, R * D * sizeof(float));
    for (uint32_t l = 0; l < L; l++) {
        const pk_layer *y = &m->layers[l];
        const float *vec[] = { y->ff1_nw, y->ff1_nb, y->att_nw, y->att_nb, y->conv_nw, y->conv_nb,
                               y->ff2_nw, y->ff2_nb, y->out_nw, y->out_nb, y->bias_u, y->bias_v };
        for (size_t i = 0; i < sizeof vec / sizeof vec[0]; i++)
            put(f, vec[i], (size_t)D * sizeof(float));
        put(f, y->dw, (size_t)D * m->conv_kernel * sizeof(float));
        put(f, y->dw_b, (size_t)D * sizeof(float));
        const pk_q8 *mats[] = { &y->ff1_up, &y->ff1_down, &y->ff2_up, &y->ff2_down, &y->q, &y->k, &y->v,
                                &y->pos, &y->o, &y->pw1, &y->pw2 };
        for (size_t i = 0; i < sizeof mats / sizeof mats[0]; i++)
            put_q8(f, mats[i]);
    }
    return fclose(f) ? -1 : 0;
}

/* The decoder's input, weights and tokens after pk_asr_run (see the
 * header): the run's one chunk left its joint frames in a->fproj[0]. */
static int dump_decoder(const pk_model *m, const pk_asr *a, uint32_t Te, const char *path) {
    FILE *f = fopen(path, "wb");
    if (!f)
        return -1;
    const uint32_t P = m->pred_hidden, J = m->joint_hidden;
    put(f, "PKDC", 4);
    const uint32_t hdr[8] = { Te, P, m->pred_layers, J, m->vocab, m->n_dur, m->blank, m->max_symbols };
    put(f, hdr, sizeof hdr);
    put(f, m->dur, (size_t)m->n_dur * 4);
    put(f, a->fproj[0], (size_t)Te * J * sizeof(float));
    put(f, m->embed, (size_t)(m->vocab + 1) * P * sizeof(float));
    for (uint32_t l = 0; l < m->pred_layers; l++) {
        put_q8(f, &m->lstm[l].wx);
        put_q8(f, &m->lstm[l].wh);
        put(f, m->lstm[l].b, (size_t)4 * P * sizeof(float));
    }
    put_q8(f, &m->jpred);
    put(f, m->jpred_b, (size_t)J * sizeof(float));
    put_q8(f, &m->jout);
    put(f, m->jout_b, (size_t)m->jout.rows * sizeof(float));
    put_q8(f, &m->jenc);
    put(f, m->jenc_b, (size_t)J * sizeof(float));
    put_u32(f, (uint32_t)a->ntoks);
    for (size_t i = 0; i < a->ntoks; i++) {
        const int32_t t3[3] = { a->toks[i].id, a->toks[i].frame, a->toks[i].dur };
        put(f, t3, sizeof t3);
    }
    return fclose(f) ? -1 : 0;
}

int pk_hip_upload_model(const pk_model *m, char *err, size_t errlen);
int pk_hip_upload_q8(const int8_t *q, const float *s, uint32_t rows, uint32_t cols);
int pk_hip_release_q8(const int8_t *q);


void pk_hip_release_model(const pk_model *m);

static uint64_t g_s;
static double unit(void) {
    g_s ^= g_s >> 12;
    g_s ^= g_s << 25;
    g_s ^= g_s >> 27;
    return (double)((g_s * 0x2545F4914F6CDD1Dull) >> 11) / 9007199254740992.0;
}

/* pk_diar_fn: a run of rows, printed and counted as they come */
static long g_rows;
static int print_rows(void *arg, int64_t row, size_t n, const float *p) {
    const int S = *(const int *)arg;
    g_rows += (long)n;
    for (size_t i = 0; i < n; i++) {
        printf("row %lld:", (long long)(row + (int64_t)i));
        for (int s = 0; s < S; s++)
            printf(" %a", p[i * S + s]);
        printf("\n");
    }
    return 0;
}

/* --time-passes (see the header) */
static int time_passes(int threads, double secs, uint32_t M, uint32_t K, uint32_t N) {
    if (threads < 1 || M == 0 || K % 32 || N % 16 || K > 16384)
        return 2;
    g_s = 0x9E3779B97F4A7C15ull * 7 + 1;
    int8_t *w = malloc((size_t)N * K);
    float *ws = malloc((size_t)N * sizeof *ws), *x = malloc((size_t)M * K * sizeof *x);
    float *out = malloc((size_t)M * N * sizeof *out), *d = malloc((size_t)M * sizeof *d);
    int8_t *q = malloc((size_t)M * K);
    if (!w || !ws || !x || !out || !d || !q)
        return 1;
    /* PK_Q8: panels of 16 rows, groups of 4 inputs (core/pkf.h:28-41) */
    for (uint32_t r = 0; r < N; r++)
        for (uint32_t k = 0; k < K; k++)
            w[((size_t)(r / 16) * (K / 4) + k / 4) * 64 + (r % 16) * 4 + k % 4] = (int8_t)(-127 + (int)(unit() * 255));
    for (uint32_t r = 0; r < N; r++)
        ws[r] = (float)(1e-3 + 9e-3 * unit());
    for (size_t i = 0; i < (size_t)M * K; i += 2) {
        const double u1 = unit() + 1e-300, u2 = unit(), rr = sqrt(-2 * log(u1));
        x[i] = (float)(rr * cos(6.283185307179586 * u2));
        if (i + 1 < (size_t)M * K)
            x[i + 1] = (float)(rr * sin(6.283185307179586 * u2));
    }
    const char *want = getenv("PKTITO_KERNELS");
    const int hip = want && !strcmp(want, "hip");
    if (hip && pk_hip_upload_q8(w, ws, N, K)) {
        fprintf(stderr, "upload failed\n");
        return 1;
    }
    pk_pool *p = pk_pool_new(threads);
    pk_q8 mat = { w, ws, N, K };
    pk_act act = { q, d, K, K, M };
    double tq = 0, tg = 0, t0 = pk_os_now();
    long calls = 0;
    /* one untimed pair first: the table's pick, the upload's first use */
    pk_quantize_on(p, &act, x, K, M, K, K);
    pk_gemm_on(p, out, N, &mat, NULL, &act, 0, NULL, NULL);
    t0 = pk_os_now();
    while (pk_os_now() - t0 < secs || calls < 3) {
        const double a = pk_os_now();
        pk_quantize_on(p, &act, x, K, M, K, K);
        const double b = pk_os_now();
        pk_gemm_on(p, out, N, &mat, NULL, &act, 0, NULL, NULL);
        const double c = pk_os_now();
        tq += b - a;
        tg += c - b;
        calls++;
    }
    double chk = 0;
    for (size_t i = 0; i < (size_t)M * N; i += 997)
        chk += out[i];
    printf("{\"table\": \"%s\", \"threads\": %d, \"M\": %u, \"K\": %u, \"N\": %u, \"calls\": %ld, "
           "\"quantize_ms\": %.4f, \"gemm_ms\": %.4f, \"pair_ms\": %.4f, \"tops\": %.4f, \"check\": %.6g}\n",
           pk_k_name(), threads, M, K, N, calls, 1e3 * tq / calls, 1e3 * tg / calls, 1e3 * (tq + tg) / calls,
           2.0 * M * K * N / (tg / calls) / 1e12, chk);
    pk_pool_free(p);
    if (hip)
        pk_hip_release_q8(w);
    free(w);
    free(ws);
    free(x);
    free(out);
    free(d);
    free(q);
    return 0;
}

int main(int argc, char **argv) {
    if (argc >= 4 && !strcmp(argv[1], "--time-passes"))
        return time_passes(atoi(argv[2]), atof(argv[3]), argc > 4 ? (uint32_t)atoi(argv[4]) : 750,
                           argc > 5 ? (uint32_t)atoi(argv[5]) : 1024, argc > 6 ? (uint32_t)atoi(argv[6]) : 4096);
    if (argc < 6) {
        fprintf(stderr, "usage: %s MODEL.pkf SECONDS SEED FAST THREADS\n", argv[0]);
        return 2;
    }
    const double secs = atof(argv[2]);
    g_s = strtoull(argv[3], NULL, 10) * 0x9E3779B97F4A7C15ull + 1;
    const int fast = atoi(argv[4]), threads = atoi(argv[5]);
    char err[512];
    pk_model *m = pk_model_load(argv[1], err, sizeof err);
    if (!m) {
        fprintf(stderr, "load: %s\n", err);
        return 1;
    }
    const char *want = getenv("PKTITO_KERNELS");
    const int hip = want && !strcmp(want, "hip");
    if (hip && pk_hip_upload_model(m, err, sizeof err)) {
        fprintf(stderr, "upload: %s\n", err);
        return 1;
    }
    const size_t n = (size_t)(secs * 16000);
    float *x = malloc(n * sizeof *x);
    double f[4], ph[4];
    for (int i = 0; i < 4; i++)
        f[i] = 80 + 900 * unit(), ph[i] = 6.283185307179586 * unit();
    for (size_t i = 0; i < n; i++) {
        const double t = i / 16000.0, env = 0.5 + 0.5 * sin(6.283185307179586 * t / 3.1);
        double v = 0.05 * (2 * unit() - 1);
        for (int k = 0; k < 4; k++)
            v += 0.12 * env * sin(6.283185307179586 * f[k] * t + ph[k]);
        x[i] = (float)v;
    }
    if (pk_model_speakers(m) > 0) {
        int S = pk_model_speakers(m);
        pk_diar *d = pk_diar_new(m, threads);
        if (!d) {
            fprintf(stderr, "pk_diar_new failed\n");
            return 1;
        }
        if (pk_diar_run(d, x, n, print_rows, &S)) {
            fprintf(stderr, "pk_diar_run failed\n");
            return 1;
        }
        printf("rows %ld %d\n", g_rows, S);
        fprintf(stderr, "backend: %s\n", pk_backend());
        pk_diar_free(d);
        if (hip)
            pk_hip_release_model(m);
        pk_model_free(m);
        free(x);
        return 0;
    }
    pk_asr *a = pk_asr_new(m, threads);
    if (!a) {
        fprintf(stderr, "pk_asr_new failed\n");
        return 1;
    }
    pk_asr_set_fast_mode(a, fast);
    const pk_tok *toks;
    const long c = pk_asr_run(a, x, n, &toks);
    if (c < 0) {
        fprintf(stderr, "pk_asr_run failed\n");
        return 1;
    }
    printf("tokens %ld\n", c);
    for (long i = 0; i < c; i++)
        printf("%d %d %d\n", toks[i].id, toks[i].frame, toks[i].dur);
    if (argc >= 8 && !strcmp(argv[6], "--decoder") &&
        dump_decoder(m, a, (uint32_t)pk_enc_frames((uint32_t)pk_mel_frames(m, n)), argv[7])) {
        fprintf(stderr, "decoder dump failed\n");
        return 1;
    }
    if (argc >= 8 && !strcmp(argv[6], "--layers") && dump_layers(m, a, x, n, argv[7])) {
        fprintf(stderr, "layer dump failed\n");
        return 1;
    }
    fprintf(stderr, "backend: %s\n", pk_backend());
    pk_asr_free(a);
    if (hip)
        pk_hip_release_model(m);
    pk_model_free(m);
    free(x);
    return 0;
}
