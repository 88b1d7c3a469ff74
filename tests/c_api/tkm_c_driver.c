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
 * The last two use one function of this build's extensions (include/tkm_hip.h).
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
    fprintf(stderr, "usage: %s numcheck | train <model.tkm> <batch> <steps> <lr> <weights.bin> | "
                    "source <mode> <model.tkm> <batch> | registry <model.tkm> <batch> <dir>\n", argv[0]);
    return 2;
}
