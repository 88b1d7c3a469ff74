/*
 * Plasma epilogue runtime: create (emit + hipRTC + load), argument lists, launches
 * (include/tkm_plasma.h).  Replaces, for plasma groups, the reference's per-group function
 * lookup (src/tkm_gpu.cu:1074-1077) and launch_plasma_sig (src/tkm_gpu.cu:1166-1174).
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tkm_plasma_internal.h"

struct tkm_plasma {
    tkm_plasma_desc desc;
    tkm_plasma_geom geom;
    void *module;
    void *fwd, *bwd, *reduce;
};

int tkm_plasma_create(const tkm_plasma_desc *d, tkm_plasma **out) {
    if (!out) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_plasma_create: out is NULL");
    *out = NULL;
    int rc = tkm_plasma_check_desc(d);
    if (rc) return rc;
    tkm_plasma *p = (tkm_plasma *)calloc(1, sizeof *p);
    if (!p) return tkm_set_error(TKM_ATTN_EINVAL, "out of host memory");
    p->desc = *d;
    tkm_plasma_geometry(d, &p->geom);
    char *src = tkm_plasma_source(d);
    if (!src) {
        free(p);
        return TKM_ATTN_EINVAL;
    }
    rc = tkm_rtc_load(src, "tkm_plasma.hip", &p->module);
    free(src);
    if (rc) {
        free(p);
        return rc;
    }
    char name[96];
    snprintf(name, sizeof name, "tkm_plasma_fwd_g%d", d->group_id);
    rc = tkm_rtc_function(p->module, name, &p->fwd);
    if (!rc) {
        snprintf(name, sizeof name, "tkm_plasma_bwd_g%d", d->group_id);
        rc = tkm_rtc_function(p->module, name, &p->bwd);
    }
    if (!rc && p->geom.n_par > 0) {
        snprintf(name, sizeof name, "tkm_plasma_bwd_g%d_reduce", d->group_id);
        rc = tkm_rtc_function(p->module, name, &p->reduce);
    }
    if (rc) {
        tkm_rtc_unload(p->module);
        free(p);
        return rc;
    }
    *out = p;
    return TKM_ATTN_OK;
}

void tkm_plasma_destroy(tkm_plasma *p) {
    if (!p) return;
    tkm_rtc_unload(p->module);
    free(p);
}

int tkm_plasma_num_args(const tkm_plasma *p, int pass) {
    if (!p || (pass != 0 && pass != 1)) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_plasma_num_args: bad handle or pass");
    return pass == 0 ? p->geom.n_fwd : p->geom.n_bwd + p->geom.n_par;
}

int tkm_plasma_arg(const tkm_plasma *p, int pass, int i, int *kind, int *node) {
    const int n = tkm_plasma_num_args(p, pass);
    if (n < 0) return n;
    if (i < 0 || i >= n || !kind || !node) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_plasma_arg: index %d of %d", i, n);
    const tkm_plasma_argd *a = pass == 0 ? &p->geom.fwd[i]
                              : (i < p->geom.n_bwd ? &p->geom.bwd[i] : &p->geom.par[i - p->geom.n_bwd]);
    *kind = a->kind;
    *node = a->node;
    return TKM_ATTN_OK;
}

static int check_ptrs(void *const *args, const tkm_plasma_argd *a, int n, int rows, const char *fn) {
    for (int i = 0; i < n; ++i) {
        const int row_tensor = a[i].kind == TKM_ARG_IN || a[i].kind == TKM_ARG_OUT || a[i].kind == TKM_ARG_DOUT ||
                               a[i].kind == TKM_ARG_DIN || a[i].kind == TKM_ARG_SAVE_XHAT ||
                               a[i].kind == TKM_ARG_SAVE_ISTD || a[i].kind == TKM_ARG_BRANCH_IN ||
                               a[i].kind == TKM_ARG_DBRANCH;
        if (!args[i]) {
            if (row_tensor && rows == 0) continue;
            return tkm_set_error(TKM_ATTN_EINVAL, "%s: argument %d (kind %d, node %d) is NULL", fn, i, a[i].kind, a[i].node);
        }
        const uintptr_t align = a[i].kind == TKM_ARG_SAVE_ISTD ? 4u : 16u;
        if ((uintptr_t)args[i] % align)
            return tkm_set_error(TKM_ATTN_EALIGN, "%s: argument %d (kind %d) must be %u-byte aligned", fn, i, a[i].kind,
                                 (unsigned)align);
    }
    return TKM_ATTN_OK;
}

static int check_rows(int rows) {
    if (rows < 0) return tkm_set_error(TKM_ATTN_EINVAL, "rows %d must be >= 0", rows);
    if (rows > (1 << 26)) return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "rows %d above 2^26", rows);
    return TKM_ATTN_OK;
}

int tkm_plasma_fwd(const tkm_plasma *p, void *const *args, int rows, void *stream) {
    if (!p || !args) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_plasma_fwd: NULL handle or argument list");
    int rc = check_rows(rows);
    if (rc) return rc;
    if (rows == 0) return TKM_ATTN_OK;
    const tkm_plasma_geom *g = &p->geom;
    rc = check_ptrs(args, g->fwd, g->n_fwd, rows, "tkm_plasma_fwd");
    if (rc) return rc;
    void *kargs[TKM_PLASMA_MAX_ARGS + 1];
    for (int i = 0; i < g->n_fwd; ++i) kargs[i] = (void *)&args[i];
    kargs[g->n_fwd] = (void *)&rows;
    const int rpb = TKM_PLASMA_FWD_RPI * 4 * g->RW;
    return tkm_rtc_launch(p->fwd, (unsigned)g->XB, (unsigned)((rows + rpb - 1) / rpb), 256, kargs, stream,
                          "plasma forward");
}

size_t tkm_plasma_bwd_workspace_bytes(const tkm_plasma *p, int rows) {
    if (!p || rows < 0 || p->geom.n_par == 0) return 0;
    size_t b = (size_t)tkm_bwd_bands(rows, p->geom.XB) * (size_t)p->geom.part_width * sizeof(float);
    return (b + 255) & ~(size_t)255;
}

int tkm_plasma_bwd(const tkm_plasma *p, void *const *args, int rows, int acc_flags, void *workspace,
                   size_t workspace_bytes, void *stream) {
    if (!p || !args) return tkm_set_error(TKM_ATTN_EINVAL, "tkm_plasma_bwd: NULL handle or argument list");
    int rc = check_rows(rows);
    if (rc) return rc;
    if (acc_flags & ~(TKM_PLASMA_ACC_DIN | TKM_PLASMA_ACC_PARAMS | TKM_PLASMA_ACC_BRANCH))
        return tkm_set_error(TKM_ATTN_EINVAL, "tkm_plasma_bwd: unknown accumulation flags 0x%x", acc_flags);
    const tkm_plasma_geom *g = &p->geom;
    rc = check_ptrs(args, g->bwd, g->n_bwd, rows, "tkm_plasma_bwd");
    if (!rc) rc = check_ptrs(args + g->n_bwd, g->par, g->n_par, rows, "tkm_plasma_bwd");
    if (rc) return rc;
    for (int i = 0; i < g->n_bwd; ++i)
        if (rows > 0 && g->bwd[i].kind == TKM_ARG_DIN && args[i] == args[0])
            return tkm_set_error(TKM_ATTN_EINVAL, "tkm_plasma_bwd: din must not alias dout");
    const size_t need = tkm_plasma_bwd_workspace_bytes(p, rows);
    if (need && (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 15u)))
        return tkm_set_error(TKM_ATTN_EWORKSPACE, "tkm_plasma_bwd: a 16-byte aligned workspace of %zu bytes is needed",
                             need);
    const int bands = tkm_bwd_bands(rows, p->geom.XB);
    int band = (rows + bands - 1) / bands;
    float *part = (float *)workspace;
    if (rows > 0 || g->n_par > 0) {
        void *kargs[TKM_PLASMA_MAX_ARGS + 4];
        for (int i = 0; i < g->n_bwd; ++i) kargs[i] = (void *)&args[i];
        kargs[g->n_bwd] = (void *)&part;
        kargs[g->n_bwd + 1] = (void *)&rows;
        kargs[g->n_bwd + 2] = (void *)&band;
        kargs[g->n_bwd + 3] = (void *)&acc_flags;
        rc = tkm_rtc_launch(p->bwd, (unsigned)g->XB, (unsigned)bands, 256, kargs, stream, "plasma backward");
        if (rc) return rc;
    }
    if (g->n_par == 0) return TKM_ATTN_OK;
    int acc_params = (acc_flags & TKM_PLASMA_ACC_PARAMS) ? 1 : 0;
    void *rargs[TKM_PLASMA_MAX_ARGS + 3];
    rargs[0] = (void *)&part;
    rargs[1] = (void *)&bands;
    rargs[2] = (void *)&acc_params;
    for (int i = 0; i < g->n_par; ++i) rargs[3 + i] = (void *)&args[g->n_bwd + i];
    return tkm_rtc_launch(p->reduce, (unsigned)((g->part_width + 63) / 64), 1, 64 * TKM_REDUCE_WAVES, rargs, stream,
                          "plasma backward reduction");
}
