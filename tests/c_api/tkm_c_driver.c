/*
 * A C program that uses only the public API of tkm.h, compiled against the reference's own
 * include/tkm.h and linked with the reference's unchanged front end (src/tkm_core.c,
 * src/tkm_registry.c) and this build's libtkm_hip.so in place of src/tkm_gpu.cu.  It is the
 * drop-in check of the runtime: nothing here knows about HIP.  oracle/Makefile (target
 * `driver`) builds it into oracle/_ref/ in the build container; tests/test_c_driver_gpu.py runs
 * it on the GPU.
 *
 *   tkm_c_driver numcheck
 *       the GPU gradient check protocol of the reference's CLI (src/main.c:245-295): for each
 *       testable op, `input: 1x1x32 / test: <op> -> SoftmaxCE` at batch 2, labels {3, 7},
 *       inputs sin(0.4 i) * 1.5 + 0.2 (0.5 where |x| < 0.1), dL/dx[8] against the central
 *       difference (eps 1e-3) of tkm_eval_current_loss; relative error below 5e-3.  Exit code:
 *       the number of failing ops.
 *   tkm_c_driver train <model.tkm> <batch> <steps> <lr> <weights.bin>
 *       tkm_load_file, steps on one synthetic batch (the loss must fall), tkm_save_weights,
 *       then a second runtime that tkm_load_weights the file must reproduce the last loss.
 *   tkm_c_driver source <mode> <model.tkm> <batch>
 *       (no GPU) the front end's graph of the model through tkm_codegen_cuda_string, printed,
 *       with the pointwise ops' code chosen by tkm_hip_use_registry_code(mode).
 *   tkm_c_driver registry <model.tkm> <batch> <dir>
 *       one training step of the model with each code mode (0: this build's formulas, 1: the
 *       registry's code of every pointwise op, 2: every pointwise op as an op unknown to this
 *       build), from the same initial weights; modes 1 and 2 must agree bit for bit, modes 0
 *       and 1 within rounding (loss, input gradient, every updated weight).
 *
 *   tkm_c_driver dataset
 *       tkm_runtime_train_dataset and tkm_runtime_eval_dataset through a C loader callback
 *       (docs/C_API.md 6.5): training over the loader's full batches equals stepping the same
 *       batches by hand on a second runtime (mean loss and every weight bit for bit); evaluation
 *       with a short final batch counts what tkm_runtime_eval counts over all samples; a loader
 *       error, a short training batch and an overfull batch make the helpers fail.
 *   tkm_c_driver infer
 *       a tensor-output graph built with the front end's own calls: tkm_runtime_ignite_inference
 *       and tkm_runtime_ignite on it give bit-equal tkm_runtime_forward outputs, and
 *       tkm_runtime_forward refuses a short output buffer and a loss graph.
 *
 * `source` and `registry` use one function of this build's extensions (include/tkm_hip.h).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tkm.h"

static const char *const OPS[] = {
    "SiLU", "ReLU", "ReLU2", "LeakyReLU", "ELU", "GELU", "Mish", "HardSwish", "HardSigmoid", "Tanh", "Sigmoid",
    "SwishBeta", "Sin", "CosGate", "SoftCap", "Clamp", "Scale", "LayerScale", "DyT", "PReLU", "xATLU", "Softplus",
    "Snake(1.7)",
};

static int numcheck(void) {
    const int B = 2;
    const float eps = 1e-3f, tol = 5e-3f;
    float x[64];
    uint8_t y[2] = {3, 7};
    for (int i = 0; i < 64; ++i) {
        x[i] = sinf(0.4f * (float)i) * 1.5f + 0.2f;
        if (fabsf(x[i]) < 0.1f) x[i] = 0.5f;
    }
    int failed = 0;
    for (size_t k = 0; k < sizeof OPS / sizeof OPS[0]; ++k) {
        char dsl[128];
        snprintf(dsl, sizeof dsl, "input: 1x1x32\ntest: %s -> SoftmaxCE", OPS[k]);
        TkmRuntime *rt = tkm_load_string(dsl, B);
        if (!rt) {
            printf("  %-12s load failed\n", OPS[k]);
            ++failed;
            continue;
        }
        tkm_runtime_step(rt, x, y, 0.0f);
        const float ana = tkm_get_grad_sample(rt, 0, 8);
        x[8] += eps;
        tkm_runtime_step(rt, x, y, 0.0f);
        const float lp = tkm_eval_current_loss(rt);
        x[8] -= 2.0f * eps;
        tkm_runtime_step(rt, x, y, 0.0f);
        const float lm = tkm_eval_current_loss(rt);
        x[8] += eps;
        const float num = (lp - lm) / (2.0f * eps);
        const float rel = fabsf(ana - num) / fmaxf(1.0f, fmaxf(fabsf(ana), fabsf(num)));
        const int ok = isfinite(ana) && isfinite(num) && rel < tol;
        printf("  %-12s analytical %+9.5f numerical %+9.5f rel %.2e %s\n", OPS[k], ana, num, rel, ok ? "PASS" : "FAIL");
        failed += !ok;
        tkm_runtime_free(rt);
    }
    return failed;
}

static uint32_t lcg(uint32_t *s) { return *s = *s * 1664525u + 1013904223u; }

void tkm_hip_use_registry_code(int mode);   /* include/tkm_hip.h */

static char *read_text(const char *path) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    const long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    char *t = (char *)malloc((size_t)n + 1);
    if (t && fread(t, 1, (size_t)n, f) != (size_t)n) {
        free(t);
        t = NULL;
    }
    if (t) t[n] = '\0';
    fclose(f);
    return t;
}

static int source(int mode, const char *path, int batch) {
    char *text = read_text(path);
    TkmGraph *g = (TkmGraph *)calloc(1, sizeof(TkmGraph));
    if (!text || !g) return 1;
    tkm_parse_dsl(g, text, batch);
    tkm_optimize_and_bind(g);
    tkm_plan_memory(g);
    tkm_hip_use_registry_code(mode);
    char *src = tkm_codegen_cuda_string(g);
    if (src) fputs(src, stdout);
    free(src);
    free(g);
    free(text);
    return src ? 0 : 1;
}

/* The float arrays of a TKM1 weights file (count, sizes and values). */
static float *read_weights(const char *path, size_t *n_out) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    uint32_t hdr[2];
    float *all = NULL;
    size_t n = 0;
    if (fread(hdr, 4, 2, f) == 2 && hdr[0] == 0x544B4D31u) {
        for (uint32_t t = 0; t < hdr[1]; ++t) {
            uint32_t c;
            if (fread(&c, 4, 1, f) != 1) break;
            float *grown = (float *)realloc(all, (n + c) * sizeof(float));
            if (!grown) break;
            all = grown;
            if (fread(all + n, 4, c, f) != c) break;
            n += c;
        }
    }
    fclose(f);
    *n_out = n;
    return all;
}

static int registry(const char *path, int batch, const char *dir) {
    float loss[3], grad[3][64];
    float *w[3] = {NULL, NULL, NULL};
    size_t nw[3] = {0, 0, 0};
    for (int mode = 0; mode < 3; ++mode) {
        tkm_hip_use_registry_code(mode);
        TkmRuntime *rt = tkm_load_file(path, batch);
        if (!rt) return 1;
        const size_t n_in = tkm_runtime_input_elements(rt);
        float *x = (float *)malloc(n_in * sizeof(float));
        uint8_t *y = (uint8_t *)malloc((size_t)batch);
        uint32_t s = 777u;
        for (size_t i = 0; i < n_in; ++i) x[i] = ((float)(lcg(&s) >> 8) * (1.0f / 16777216.0f) - 0.5f) * 2.0f;
        for (int b = 0; b < batch; ++b) y[b] = (uint8_t)((lcg(&s) >> 24) % 10);
        loss[mode] = tkm_runtime_step(rt, x, y, 0.05f);
        for (int i = 0; i < 64; ++i) grad[mode][i] = tkm_get_grad_sample(rt, 0, i * 7);
        char wpath[512];
        snprintf(wpath, sizeof wpath, "%s/w%d.bin", dir, mode);
        if (!tkm_save_weights(rt, wpath)) return 1;
        w[mode] = read_weights(wpath, &nw[mode]);
        tkm_runtime_free(rt);
        free(x);
        free(y);
        printf("  mode %d: loss %.7f, %zu weights\n", mode, loss[mode], nw[mode]);
    }
    tkm_hip_use_registry_code(1);
    int rc = 0;
    if (!w[0] || nw[0] == 0 || nw[0] != nw[1] || nw[1] != nw[2]) rc = 1;
    /* 1 and 2: the same pasted code */
    if (!rc && (loss[1] != loss[2] || memcmp(grad[1], grad[2], sizeof grad[1]) || memcmp(w[1], w[2], nw[1] * 4))) {
        printf("  modes 1 and 2 differ\n");
        rc = 1;
    }
    /* 0 and 1: this build's formulas against the registry's code */
    double gmax = 0, gerr = 0, werr = 0;
    for (int i = 0; i < 64; ++i) {
        gmax = fmax(gmax, fabs(grad[0][i]));
        gerr = fmax(gerr, fabs(grad[0][i] - grad[1][i]));
    }
    for (size_t i = 0; !rc && i < nw[0]; ++i) werr = fmax(werr, fabs((double)w[0][i] - w[1][i]) / fmax(1.0, fabs(w[1][i])));
    printf("  formulas vs registry code: loss rel %.2e, input gradient %.2e of its max, weights %.2e\n",
           fabs(loss[0] - loss[1]) / fabs(loss[1]), gerr / (gmax > 0 ? gmax : 1), werr);
    if (!rc && (!(fabs(loss[0] - loss[1]) <= 1e-3 * fabs(loss[1])) || !(gerr <= 2e-2 * gmax) || !(werr <= 1e-4)))
        rc = 1;
    for (int m = 0; m < 3; ++m) free(w[m]);
    printf("registry %s: %s\n", path, rc ? "FAIL" : "PASS");
    return rc;
}

static int train(const char *path, int batch, int steps, float lr, const char *weights) {
    TkmRuntime *rt = tkm_load_file(path, batch);
    if (!rt) {
        printf("tkm_load_file(%s) failed\n", path);
        return 1;
    }
    const size_t n_in = tkm_runtime_input_elements(rt);
    float *x = (float *)malloc(n_in * sizeof(float));
    uint8_t *y = (uint8_t *)malloc((size_t)batch);
    uint32_t s = 12345u;
    for (size_t i = 0; i < n_in; ++i) x[i] = ((float)(lcg(&s) >> 8) * (1.0f / 16777216.0f) - 0.5f) * 3.0f;
    for (int b = 0; b < batch; ++b) y[b] = (uint8_t)(lcg(&s) >> 24);
    float first = NAN, last = NAN;
    for (int k = 0; k < steps; ++k) {
        last = tkm_runtime_step(rt, x, y, lr);
        if (k == 0) first = last;
        printf("  step %d loss %.6f\n", k, last);
    }
    int rc = !(isfinite(first) && isfinite(last) && last < first);
    if (!tkm_save_weights(rt, weights)) rc = 1;
    const float next = tkm_runtime_step(rt, x, y, 0.0f);
    TkmRuntime *rt2 = tkm_load_file(path, batch);
    if (!rt2 || !tkm_load_weights(rt2, weights)) {
        rc = 1;
    } else {
        const float again = tkm_runtime_step(rt2, x, y, 0.0f);
        printf("  reloaded weights: loss %.6f (saved runtime %.6f)\n", again, next);
        if (again != next) rc = 1;
    }
    if (rt2) tkm_runtime_free(rt2);
    tkm_runtime_free(rt);
    free(x);
    free(y);
    printf("train %s: %s\n", path, rc ? "FAIL" : "PASS");
    return rc;
}

/* ---- dataset helpers through a loader callback ----------------------------------------- */

typedef struct {
    const float *x;            /* n samples of `per` floats */
    const uint8_t *y;
    size_t n, per, pos;
    int fail_at;               /* >= 0: the call with this index returns -1 */
    int calls;
    int overfill;              /* report one sample more than the capacity */
} loader;

static int next_batch(void *user, float *h_input, uint8_t *h_labels, size_t capacity, size_t *out_count) {
    loader *L = (loader *)user;
    if (L->fail_at >= 0 && L->calls++ == L->fail_at) return -1;
    const size_t left = L->n - L->pos, k = left < capacity ? left : capacity;
    if (k == 0) return 0;
    memcpy(h_input, L->x + L->pos * L->per, k * L->per * sizeof(float));
    memcpy(h_labels, L->y + L->pos, k);
    L->pos += k;
    *out_count = k + (L->overfill ? capacity : 0);
    return 1;
}

static const char *const MLP = "input: 1x1x32\nmlp: FC(48) -> SiLU -> FC(10) -> SoftmaxCE\n";

static uint8_t *weights_of(TkmRuntime *rt, size_t *n) {
    *n = tkm_runtime_weight_bytes(rt);
    uint8_t *w = (uint8_t *)malloc(*n);
    if (w && !tkm_save_weights_buffer(rt, w, *n, NULL)) {
        free(w);
        w = NULL;
    }
    return w;
}

static int dataset(void) {
    const int B = 4;
    const size_t per = 32, full = 5, n = full * B + 3;   /* a short final batch of 3 */
    float *x = (float *)malloc(n * per * sizeof(float));
    uint8_t *y = (uint8_t *)malloc(n);
    uint32_t s = 777u;
    for (size_t i = 0; i < n * per; ++i) x[i] = ((float)(lcg(&s) >> 8) * (1.0f / 16777216.0f) - 0.5f) * 4.0f;
    for (size_t i = 0; i < n; ++i) y[i] = (uint8_t)((lcg(&s) >> 24) % 10);
    TkmRuntime *a = tkm_load_string(MLP, B), *b = tkm_load_string(MLP, B);
    int rc = !a || !b;
    if (!rc) {
        /* training: the loader's batches, the short last one an error, so train the full ones */
        loader L = {x, y, full * B, per, 0, -1, 0, 0};
        float avg = NAN;
        const int ok = tkm_runtime_train_dataset(a, next_batch, &L, 0, 0.05f, &avg);
        double sum = 0.0;
        for (size_t k = 0; k < full; ++k) sum += tkm_runtime_step(b, x + k * B * per, y + k * B, 0.05f);
        const float want = (float)(sum / (double)full);
        size_t na = 0, nb = 0;
        uint8_t *wa = weights_of(a, &na), *wb = weights_of(b, &nb);
        const int same = wa && wb && na == nb && !memcmp(wa, wb, na);
        printf("  train_dataset: ok %d, mean loss %.7f (by hand %.7f), weights %s\n", ok, avg, want,
               same ? "bit-equal" : "DIFFER");
        if (!ok || avg != want || !same) rc = 1;
        free(wa);
        free(wb);
        /* max_batches stops early; the loader's position shows it */
        loader M = {x, y, full * B, per, 0, -1, 0, 0};
        if (!tkm_runtime_train_dataset(a, next_batch, &M, 2, 0.0f, &avg) || M.pos != 2 * (size_t)B) rc = 1;
        /* evaluation over all samples, the last batch short */
        loader E = {x, y, n, per, 0, -1, 0, 0};
        int correct = -1;
        size_t samples = 0;
        const int eok = tkm_runtime_eval_dataset(a, next_batch, &E, 0, &correct, &samples);
        const int direct = tkm_runtime_eval(a, x, y, (int)n);
        printf("  eval_dataset: ok %d, %d correct of %zu (tkm_runtime_eval: %d of %zu)\n", eok, correct, samples,
               direct, n);
        if (!eok || samples != n || correct != direct) rc = 1;
        /* failures: a loader error, a short training batch, an overfull batch, no batch at all */
        loader F = {x, y, n, per, 0, 1, 0, 0}, G = {x, y, n, per, 0, -1, 0, 0}, H = {x, y, n, per, 0, -1, 0, 1},
               Z = {x, y, 0, per, 0, -1, 0, 0};
        const int f1 = tkm_runtime_train_dataset(a, next_batch, &F, 0, 0.0f, &avg);
        const int f2 = tkm_runtime_train_dataset(a, next_batch, &G, 0, 0.0f, &avg);   /* ends short */
        const int f3 = tkm_runtime_eval_dataset(a, next_batch, &H, 0, &correct, &samples);
        const int f4 = tkm_runtime_eval_dataset(a, next_batch, &Z, 0, &correct, &samples);
        printf("  refused: loader error %d, short training batch %d, overfull batch %d, empty %d\n", !f1, !f2,
               !f3, !f4);
        if (f1 || f2 || f3 || f4) rc = 1;
    }
    if (a) tkm_runtime_free(a);
    if (b) tkm_runtime_free(b);
    free(x);
    free(y);
    printf("dataset: %s\n", rc ? "FAIL" : "PASS");
    return rc;
}

/* ---- the inference runtime ----------------------------------------------------------------- */

static TkmGraph *front_end(const char *text, int batch) {
    TkmGraph *g = (TkmGraph *)calloc(1, sizeof(TkmGraph));
    if (!g) return NULL;
    tkm_parse_dsl(g, text, batch);
    tkm_optimize_and_bind(g);
    tkm_plan_memory(g);
    return g;
}

static int infer(void) {
    const int B = 3;
    TkmGraph *g = front_end("input: 1x4x32\nmlp: FC(48) -> SiLU -> FC(24) -> Tanh\n", B);
    char *src = g ? tkm_codegen_cuda_string(g) : NULL;
    TkmRuntime *inf = src ? tkm_runtime_ignite_inference(g, src) : NULL;
    TkmRuntime *trn = src ? tkm_runtime_ignite(g, src) : NULL;
    int rc = !inf || !trn;
    if (!rc) {
        const size_t nin = tkm_runtime_input_elements(inf), nout = tkm_runtime_output_elements(inf);
        float *x = (float *)malloc(nin * sizeof(float));
        float *oi = (float *)calloc(nout, sizeof(float)), *ot = (float *)calloc(nout, sizeof(float));
        uint32_t s = 99u;
        for (size_t i = 0; i < nin; ++i) x[i] = ((float)(lcg(&s) >> 8) * (1.0f / 16777216.0f) - 0.5f) * 2.0f;
        const size_t gi = tkm_runtime_forward(inf, x, oi, nout), gt = tkm_runtime_forward(trn, x, ot, nout);
        int finite = 1;
        for (size_t i = 0; i < nout; ++i) finite &= isfinite(oi[i]) && fabsf(oi[i]) <= 1.0f;
        const int same = gi == nout && gt == nout && !memcmp(oi, ot, nout * sizeof(float));
        /* a second call reuses the runtime's buffers and gives the same output */
        const size_t again = tkm_runtime_forward(inf, x, ot, nout);
        const int stable = again == nout && !memcmp(oi, ot, nout * sizeof(float));
        const size_t shortcap = tkm_runtime_forward(inf, x, ot, nout - 1);
        printf("  forward: %zu outputs (B %d x 4 rows x 24), inference vs training runtime %s, repeat %s, "
               "short buffer -> %zu\n", nout, B, same ? "bit-equal" : "DIFFER", stable ? "equal" : "DIFFERS",
               shortcap);
        if (nout != (size_t)B * 4 * 24 || !same || !finite || !stable || shortcap != 0 ||
            nin != (size_t)B * 4 * 32)
            rc = 1;
        free(x);
        free(oi);
        free(ot);
    }
    TkmRuntime *loss = tkm_load_string(MLP, 2);
    if (!loss) {
        rc = 1;
    } else {
        float xin[64] = {0}, out[64];
        const size_t got = tkm_runtime_forward(loss, xin, out, 64);
        printf("  loss graph: output elements %zu, forward -> %zu\n", tkm_runtime_output_elements(loss), got);
        if (got != 0 || tkm_runtime_output_elements(loss) != 0) rc = 1;
        tkm_runtime_free(loss);
    }
    if (inf) tkm_runtime_free(inf);
    if (trn) tkm_runtime_free(trn);
    free(src);
    free(g);
    printf("infer: %s\n", rc ? "FAIL" : "PASS");
    return rc;
}

int main(int argc, char **argv) {
    if (argc >= 2 && !strcmp(argv[1], "numcheck")) {
        const int failed = numcheck();
        printf("numcheck: %d failing\n", failed);
        return failed;
    }
    if (argc >= 7 && !strcmp(argv[1], "train"))
        return train(argv[2], atoi(argv[3]), atoi(argv[4]), (float)atof(argv[5]), argv[6]);
    if (argc >= 5 && !strcmp(argv[1], "source")) return source(atoi(argv[2]), argv[3], atoi(argv[4]));
    if (argc >= 5 && !strcmp(argv[1], "registry")) return registry(argv[2], atoi(argv[3]), argv[4]);
    if (argc >= 2 && !strcmp(argv[1], "dataset")) return dataset();
    if (argc >= 2 && !strcmp(argv[1], "infer")) return infer();
    fprintf(stderr, "usage: %s numcheck | train <model.tkm> <batch> <steps> <lr> <weights.bin> | "
                    "source <mode> <model.tkm> <batch> | registry <model.tkm> <batch> <dir> | dataset | infer\n",
            argv[0]);
    return 2;
}
