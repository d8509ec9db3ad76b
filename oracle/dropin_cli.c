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
 * the free: the steps INTEGRATION.md adds to core/model.c (:783-811,
 * :868-883). FAST 1 is the encoder's fast mode, blocks of 64 inputs
 * (pk_asr_set_fast_mode; blocks of 32 otherwise). */
#include "pktito.h"
#include "model.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int pk_hip_upload_model(const pk_model *m, char *err, size_t errlen);
void pk_hip_release_model(const pk_model *m);

static uint64_t g_s;
static double unit(void) {
    g_s ^= g_s >> 12;
    g_s ^= g_s << 25;
    g_s ^= g_s >> 27;
    return (double)((g_s * 0x2545F4914F6CDD1Dull) >> 11) / 9007199254740992.0;
}

int main(int argc, char **argv) {
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
    fprintf(stderr, "backend: %s\n", pk_backend());
    pk_asr_free(a);
    if (hip)
        pk_hip_release_model(m);
    pk_model_free(m);
    free(x);
    return 0;
}
