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
    fprintf(stderr, "usage: %s numcheck | train <model.tkm> <batch> <steps> <lr> <weights.bin>\n", argv[0]);
    return 2;
}
