/*
 * Run-time compilation, module loading and launching of generated kernels, and step-graph
 * capture (include/tkm_prep.h).
 *
 * Reference sequence being replaced (src/tkm_gpu.cu):
 *   1047-1078  NVRTC compile -> PTX -> cuModuleLoadDataEx -> cuModuleGetFunction per group
 *   1142-1174  kernel-argument resolution and cuLaunchKernel(grid_x, block_x, 0 LDS, stream)
 *   1498-1508  capture of the whole step into a CUDA graph, instantiated once, replayed per step
 * Here: hipRTC builds a gfx950 code object directly (no intermediate assembly), hipModuleLoadData
 * loads it on the current device, and hipModuleLaunchKernel launches with 2-D grids.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>
#include <hip/hiprtc.h>

#include "tkm_prep_internal.h"

struct tkm_prep {
    tkm_prep_desc desc;
    tkm_prep_geom geom;
    hipModule_t module;
    hipFunction_t fwd, bwd, reduce;
};

struct tkm_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

/* -packed-fp32-ops: the generated code uses no v_pk_{add,mul,fma}_f32 */
static const char *const RTC_OPTIONS[] = {
    "--offload-arch=gfx950", "-O3", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
};

static char *dup_string(const char *s, size_t n) {
    char *r = (char *)malloc(n + 1);
    if (r) {
        memcpy(r, s, n);
        r[n] = 0;
    }
    return r;
}

int tkm_rtc_compile(const char *src, const char *name, void **code, size_t *code_bytes, char **log) {
    if (code) *code = NULL;
    if (code_bytes) *code_bytes = 0;
    if (log) *log = NULL;
    if (!src || !code || !code_bytes) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_rtc_compile: NULL argument");
    hiprtcProgram prog;
    hiprtcResult r = hiprtcCreateProgram(&prog, src, name ? name : "tkm_generated.hip", 0, NULL, NULL);
    if (r != HIPRTC_SUCCESS)
        return tkm_set_error(TKM_ATTN_ECOMPILE, "hiprtcCreateProgram: %s", hiprtcGetErrorString(r));
    r = hiprtcCompileProgram(prog, (int)(sizeof RTC_OPTIONS / sizeof RTC_OPTIONS[0]), RTC_OPTIONS);
    size_t log_bytes = 0;
    char *text = NULL;
    if (hiprtcGetProgramLogSize(prog, &log_bytes) == HIPRTC_SUCCESS && log_bytes > 1) {
        text = (char *)malloc(log_bytes + 1);
        if (text && hiprtcGetProgramLog(prog, text) == HIPRTC_SUCCESS) text[log_bytes] = 0;
        else if (text) text[0] = 0;
    }
    int status = TKM_ATTN_OK;
    if (r != HIPRTC_SUCCESS) {
        status = tkm_set_error(TKM_ATTN_ECOMPILE, "hipRTC: %s: %.180s", hiprtcGetErrorString(r), text ? text : "");
    } else {
        size_t n = 0;
        if (hiprtcGetCodeSize(prog, &n) != HIPRTC_SUCCESS || n == 0) {
            status = tkm_set_error(TKM_ATTN_ECOMPILE, "hipRTC produced no code object");
        } else {
            char *buf = (char *)malloc(n);
            if (!buf) {
                status = tkm_set_error(TKM_ATTN_ECOMPILE, "out of host memory");
            } else if (hiprtcGetCode(prog, buf) != HIPRTC_SUCCESS) {
                free(buf);
                status = tkm_set_error(TKM_ATTN_ECOMPILE, "hiprtcGetCode failed");
            } else {
                *code = buf;
                *code_bytes = n;
            }
        }
    }
    hiprtcDestroyProgram(&prog);
    if (log && text && text[0]) *log = dup_string(text, strlen(text));
    free(text);
    return status;
}

static int hip_fail(const char *what, hipError_t e) {
    return tkm_set_error(TKM_ATTN_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

static int current_device_is_gfx950(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail("hipGetDevice", e);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return hip_fail("hipGetDeviceProperties", e);
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return tkm_set_error(TKM_ATTN_EDEVICE, "device %d is %s; the generated kernels target gfx950",
                             dev, prop.gcnArchName);
    return TKM_ATTN_OK;
}

int tkm_rtc_load(const char *src, const char *name, void **module) {
    *module = NULL;
    int rc = current_device_is_gfx950();
    if (rc) return rc;
    void *code = NULL;
    size_t code_bytes = 0;
    rc = tkm_rtc_compile(src, name, &code, &code_bytes, NULL);
    if (rc) return rc;
    hipModule_t m = NULL;
    hipError_t e = hipModuleLoadData(&m, code);
    free(code);
    if (e != hipSuccess) return hip_fail("hipModuleLoadData", e);
    *module = (void *)m;
    return TKM_ATTN_OK;
}

int tkm_rtc_function(void *module, const char *name, void **fn) {
    hipFunction_t f = NULL;
    hipError_t e = hipModuleGetFunction(&f, (hipModule_t)module, name);
    if (e != hipSuccess) return hip_fail(name, e);
    *fn = (void *)f;
    return TKM_ATTN_OK;
}

void tkm_rtc_unload(void *module) {
    if (module) hipModuleUnload((hipModule_t)module);
}

int tkm_rtc_launch(void *fn, unsigned gx, unsigned gy, unsigned block, void **args, void *stream, const char *what) {
    hipError_t e = hipModuleLaunchKernel((hipFunction_t)fn, gx, gy, 1, block, 1, 1, 0, (hipStream_t)stream, args, NULL);
    if (e != hipSuccess) return tkm_set_error(TKM_ATTN_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
    return TKM_ATTN_OK;
}

int tkm_prep_create(const tkm_prep_desc *d, tkm_prep **out) {
    if (!out) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_prep_create: out is NULL");
    *out = NULL;
    int rc = tkm_prep_check_desc(d);
    if (rc) return rc;
    char *src = tkm_prep_source(d);
    if (!src) return TKM_ATTN_EINVAL;
    void *module = NULL;
    rc = tkm_rtc_load(src, "tkm_qkv_prep.hip", &module);
    free(src);
    if (rc) return rc;
    tkm_prep *p = (tkm_prep *)calloc(1, sizeof *p);
    if (!p) {
        tkm_rtc_unload(module);
        return tkm_set_error(TKM_ATTN_EINVAL, "out of host memory");
    }
    p->desc = *d;
    tkm_prep_geometry(d, &p->geom);
    p->module = (hipModule_t)module;
    char name[96];
    hipFunction_t *fns[3] = {&p->fwd, &p->bwd, &p->reduce};
    const char *fmt[3] = {"tkm_plasma_fwd_g%d", "tkm_plasma_bwd_g%d", "tkm_plasma_bwd_g%d_reduce"};
    for (int i = 0; i < 3; ++i) {
        snprintf(name, sizeof name, fmt[i], d->group_id);
        rc = tkm_rtc_function(module, name, (void **)fns[i]);
        if (rc) {
            tkm_rtc_unload(module);
            free(p);
            return rc;
        }
    }
    *out = p;
    return TKM_ATTN_OK;
}

void tkm_prep_destroy(tkm_prep *p) {
    if (!p) return;
    hipModuleUnload(p->module);
    free(p);
}

static int aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

static int launch(hipFunction_t f, unsigned gx, unsigned gy, unsigned block, void **args, void *stream,
                  const char *what) {
    return tkm_rtc_launch((void *)f, gx, gy, block, args, stream, what);
}

static int check_rows(int rows) {
    if (rows < 0) return tkm_set_error(TKM_ATTN_EINVAL, "rows %d must be >= 0", rows);
    if (rows > (1 << 26)) return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "rows %d above 2^26", rows);
    return TKM_ATTN_OK;
}

int tkm_prep_fwd(const tkm_prep *p, const void *in, void *out, const float *bias, const float *gamma,
                 float *save_istd, void *save_xhat, int rows, void *stream) {
    if (!p) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_prep_fwd: NULL handle");
    int rc = check_rows(rows);
    if (rc) return rc;
    if (rows == 0) return TKM_ATTN_OK;             /* nothing to do; row tensors may be NULL */
    if (!in || !out || !bias) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_prep_fwd: in, out and bias are required");
    if (p->desc.has_qknorm && (!gamma || !save_istd || !save_xhat))
        return tkm_set_error(TKM_ATTN_EINVAL, "tkm_prep_fwd: QKNorm needs gamma, save_istd and save_xhat");
    if (!aligned16(in) || !aligned16(out) || !aligned16(bias) ||
        (p->desc.has_qknorm && (!aligned16(gamma) || !aligned16(save_xhat) || !aligned16(save_istd))))
        return tkm_set_error(TKM_ATTN_EALIGN, "tkm_prep_fwd: pointers must be 16-byte aligned");
    void *args[] = {(void *)&in, (void *)&out, (void *)&bias, (void *)&gamma, (void *)&save_istd,
                    (void *)&save_xhat, (void *)&rows};
    const int rpb = 4 * TKM_PREP_FWD_RPW;
    return launch(p->fwd, (unsigned)((p->geom.CH + 63) / 64), (unsigned)((rows + rpb - 1) / rpb), 256, args, stream,
                  "qkv-prep forward");
}

size_t tkm_prep_bwd_workspace_bytes(const tkm_prep *p, int rows) {
    if (!p || rows < 0) return 0;
    size_t b = (size_t)tkm_bwd_bands(rows, (p->geom.CH + 63) / 64) * (size_t)p->geom.part_width * sizeof(float);
    return (b + 255) & ~(size_t)255;
}

int tkm_prep_bwd(const tkm_prep *p, const void *dout, void *din, const void *save_xhat, const float *save_istd,
                 const float *gamma, float *dgamma, float *dbias, int rows, int accumulate, void *workspace,
                 size_t workspace_bytes, void *stream) {
    if (!p) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_prep_bwd: NULL handle");
    int rc = check_rows(rows);
    if (rc) return rc;
    if (accumulate != 0 && accumulate != 1) return tkm_set_error(TKM_ATTN_EINVAL, "accumulate must be 0 or 1");
    /* With rows == 0 the row tensors (dout, din, save_xhat, save_istd) may be NULL; dbias and
     * dgamma are still cleared (accumulate = 0) or kept (accumulate = 1). */
    if (!dbias) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_prep_bwd: dbias is required");
    if (rows > 0 && (!dout || !din)) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_prep_bwd: dout and din are required");
    if (rows > 0 && dout == din) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_prep_bwd: din must not alias dout");
    if (p->desc.has_qknorm && (!gamma || !dgamma || (rows > 0 && (!save_xhat || !save_istd))))
        return tkm_set_error(TKM_ATTN_EINVAL, "tkm_prep_bwd: QKNorm needs save_xhat, save_istd, gamma and dgamma");
    if (!aligned16(dout) || !aligned16(din) || !aligned16(dbias) || !aligned16(workspace) ||
        (p->desc.has_qknorm && (!aligned16(save_xhat) || !aligned16(save_istd) || !aligned16(gamma) ||
                                !aligned16(dgamma))))
        return tkm_set_error(TKM_ATTN_EALIGN, "tkm_prep_bwd: pointers must be 16-byte aligned");
    const size_t need = tkm_prep_bwd_workspace_bytes(p, rows);
    if (!workspace || workspace_bytes < need)
        return tkm_set_error(TKM_ATTN_EWORKSPACE, "tkm_prep_bwd: workspace of %zu bytes needed, %zu given", need,
                             workspace ? workspace_bytes : (size_t)0);
    int bands = tkm_bwd_bands(rows, (p->geom.CH + 63) / 64);
    int band = (rows + bands - 1) / bands;
    float *part = (float *)workspace;
    void *a1[] = {(void *)&dout, (void *)&din, (void *)&save_xhat, (void *)&save_istd, (void *)&gamma,
                  (void *)&part, (void *)&rows, (void *)&band, (void *)&accumulate};
    rc = launch(p->bwd, (unsigned)((p->geom.CH + 63) / 64), (unsigned)bands, 256, a1, stream, "qkv-prep backward");
    if (rc) return rc;
    void *a2[] = {(void *)&part, (void *)&dbias, (void *)&dgamma, (void *)&bands, (void *)&accumulate};
    return launch(p->reduce, (unsigned)((p->geom.part_width + 63) / 64), 1, 64 * TKM_REDUCE_WAVES, a2, stream,
                  "qkv-prep backward reduction");
}

int tkm_graph_begin(void *stream) {
    if (!stream) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_graph_begin: capture needs a created stream, not NULL");
    hipError_t e = hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeGlobal);
    return e == hipSuccess ? TKM_ATTN_OK : hip_fail("hipStreamBeginCapture", e);
}

int tkm_graph_end(void *stream, tkm_graph **out) {
    if (!out) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_graph_end: out is NULL");
    *out = NULL;
    if (!stream) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_graph_end: stream is NULL");
    hipGraph_t graph = NULL;
    hipError_t e = hipStreamEndCapture((hipStream_t)stream, &graph);
    if (e != hipSuccess) return hip_fail("hipStreamEndCapture", e);
    hipGraphExec_t exec = NULL;
    e = hipGraphInstantiate(&exec, graph, NULL, NULL, 0);
    if (e != hipSuccess) {
        hipGraphDestroy(graph);
        return hip_fail("hipGraphInstantiate", e);
    }
    tkm_graph *g = (tkm_graph *)calloc(1, sizeof *g);
    if (!g) {
        hipGraphExecDestroy(exec);
        hipGraphDestroy(graph);
        return tkm_set_error(TKM_ATTN_EINVAL, "out of host memory");
    }
    g->graph = graph;
    g->exec = exec;
    *out = g;
    return TKM_ATTN_OK;
}

int tkm_graph_launch(const tkm_graph *g, void *stream) {
    if (!g) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_graph_launch: NULL graph");
    hipError_t e = hipGraphLaunch(g->exec, (hipStream_t)stream);
    return e == hipSuccess ? TKM_ATTN_OK : hip_fail("hipGraphLaunch", e);
}

void tkm_graph_destroy(tkm_graph *g) {
    if (!g) return;
    hipGraphExecDestroy(g->exec);
    hipGraphDestroy(g->graph);
    free(g);
}
