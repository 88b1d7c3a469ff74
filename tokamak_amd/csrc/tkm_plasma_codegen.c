/*
 * Plasma epilogue generator: HIP C for a chain of row-wise ops behind a GEMM
 * (include/tkm_plasma.h; reference src/tkm_codegen.c:297-625, registry src/tkm_registry.c).
 *
 * Lane layout (gfx950, 64-lane waves, 4 waves per block):
 *   - a lane owns one 8-channel chunk (16 bytes) of a row;
 *   - L = lanes per row = min(64, next power of two >= C/8); a wave covers 64/L rows at once,
 *     so narrow rows (C < 512) still fill the wave;
 *   - a norm group (64 channels, or the whole row when C <= 64) is min(8, L) aligned lanes:
 *     its sums are DPP adds inside the lane row; every lane runs the reductions (lanes past
 *     the row end hold zeros), only loads and stores are predicated;
 *   - forward: 4 rows per lane slot, loads first;
 *   - backward: rows in bands (about 2048 blocks in all, at least 16 rows per band);
 *     parameter-gradient sums stay in registers over the band, the block's lane slots combine
 *     through LDS in a fixed order into one partial row per band, and a reduce kernel (16
 *     waves per column group) adds the bands in order (no atomics).
 */
#include <ctype.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tkm_plasma.h"
#include "tkm_codegen_internal.h"
#include "tkm_plasma_internal.h"

typedef tkm_sbuf sbuf;
#define sb_add tkm_sb_add

/* Flags of an op. */
enum { F_W = 1, F_BETA = 2, F_BIAS = 4, F_NORM = 8, F_BRANCH = 16, F_MASK = 32, F_SEED = 64 };

typedef struct {
    const char *name;
    int flags;
    float fval;           /* registry default */
    const char *fwd;      /* on float x; may read fv, w, b */
    const char *bwd;      /* on float g (gradient) with input p; may read fv, w; may add to aw */
} op_info;

/* Element formulas of the registry's ops (src/tkm_registry.c:186-456), one element at a time. */
static const op_info OPS[TKM_OP_COUNT] = {
    [TKM_OP_BIAS] = {"Bias", F_BIAS, 0.0f, "x += b;", ""},
    [TKM_OP_RMSNORM] = {"RMSNorm", F_NORM | F_W, 1e-5f, NULL, NULL},
    [TKM_OP_LN] = {"LN", F_NORM | F_W | F_BETA, 1e-5f, NULL, NULL},
    [TKM_OP_BN] = {"BN", F_NORM | F_W | F_BETA, 1e-2f, NULL, NULL},
    [TKM_OP_L2NORM] = {"L2Norm", F_NORM, 1e-5f, NULL, NULL},
    [TKM_OP_SILU] = {"SiLU", 0, 0.0f, "x = x / (1.0f + __expf(-x));",
                     "{ const float s = 1.0f / (1.0f + __expf(-p)); g *= s * (1.0f + p * (1.0f - s)); }"},
    [TKM_OP_RELU] = {"ReLU", 0, 0.0f, "x = fmaxf(x, 0.0f);", "g *= p > 0.0f ? 1.0f : 0.0f;"},
    [TKM_OP_RELU2] = {"ReLU2", 0, 0.0f, "{ const float r = fmaxf(x, 0.0f); x = r * r; }",
                      "g *= p > 0.0f ? 2.0f * p : 0.0f;"},
    [TKM_OP_LEAKY_RELU] = {"LeakyReLU", 0, 0.01f, "x = x > 0.0f ? x : x * fv;", "g *= p > 0.0f ? 1.0f : fv;"},
    [TKM_OP_ELU] = {"ELU", 0, 1.0f, "x = x > 0.0f ? x : fv * (__expf(x) - 1.0f);",
                    "g *= p > 0.0f ? 1.0f : fv * __expf(p);"},
    [TKM_OP_GELU] = {"GELU", 0, 0.0f,
                     "x = 0.5f * x * (1.0f + tanhf(0.79788456f * (x + 0.044715f * x * x * x)));",
                     "{ const float t = tanhf(0.79788456f * (p + 0.044715f * p * p * p));"
                     " g *= 0.5f * (1.0f + t) + 0.5f * p * (1.0f - t * t) * 0.79788456f * (1.0f + 0.134145f * p * p); }"},
    [TKM_OP_MISH] = {"Mish", 0, 0.0f,
                     "{ const float sp = x > 20.0f ? x : __logf(1.0f + __expf(x)); x = x * tanhf(sp); }",
                     "{ const float sp = p > 20.0f ? p : __logf(1.0f + __expf(p)), t = tanhf(sp);"
                     " const float sg = 1.0f / (1.0f + __expf(-p)); g *= t + p * (1.0f - t * t) * sg; }"},
    [TKM_OP_HARDSWISH] = {"HardSwish", 0, 0.0f, "x = x * fminf(fmaxf(x + 3.0f, 0.0f), 6.0f) * 0.16666667f;",
                          "g *= p <= -3.0f ? 0.0f : (p >= 3.0f ? 1.0f : (2.0f * p + 3.0f) * 0.16666667f);"},
    [TKM_OP_HARDSIGMOID] = {"HardSigmoid", 0, 0.0f, "x = fminf(fmaxf((x + 3.0f) * 0.16666667f, 0.0f), 1.0f);",
                            "g *= (p > -3.0f && p < 3.0f) ? 0.16666667f : 0.0f;"},
    [TKM_OP_TANH] = {"Tanh", 0, 0.0f, "x = tanhf(x);", "{ const float t = tanhf(p); g *= 1.0f - t * t; }"},
    [TKM_OP_SIGMOID] = {"Sigmoid", 0, 0.0f, "x = 1.0f / (1.0f + __expf(-x));",
                        "{ const float s = 1.0f / (1.0f + __expf(-p)); g *= s * (1.0f - s); }"},
    [TKM_OP_SWISH_BETA] = {"SwishBeta", 0, 1.5f, "x = x / (1.0f + __expf(-fv * x));",
                           "{ const float s = 1.0f / (1.0f + __expf(-fv * p)); g *= s * (1.0f + fv * p * (1.0f - s)); }"},
    [TKM_OP_SIN] = {"Sin", 0, 1.0f, "x = __sinf(fv * x);", "g *= fv * __cosf(fv * p);"},
    [TKM_OP_COSGATE] = {"CosGate", 0, 0.0f, "x = x * __cosf(x);",
                        "{ float sn, cs; __sincosf(p, &sn, &cs); g *= cs - p * sn; }"},
    [TKM_OP_SOFTCAP] = {"SoftCap", 0, 30.0f, "x = fv * tanhf(x / fv);",
                        "{ const float t = tanhf(p / fv); g *= 1.0f - t * t; }"},
    [TKM_OP_CLAMP] = {"Clamp", 0, 6.0f, "x = fminf(fmaxf(x, -fv), fv);", "g *= (p > -fv && p < fv) ? 1.0f : 0.0f;"},
    [TKM_OP_SCALE] = {"Scale", 0, 1.0f, "x *= fv;", "g *= fv;"},
    [TKM_OP_LAYERSCALE] = {"LayerScale", F_W, 1e-4f, "x *= w;", "aw += g * p; g *= w;"},
    [TKM_OP_DYT] = {"DyT", F_W, 0.5f, "x = tanhf(fv * x) * w;",
                    "{ const float t = tanhf(fv * p); aw += g * t; g *= w * fv * (1.0f - t * t); }"},
    [TKM_OP_PRELU] = {"PReLU", F_W, 0.25f, "x = x > 0.0f ? x : x * w * fv;",
                      "if (p <= 0.0f) aw += g * p * fv; g *= p > 0.0f ? 1.0f : w * fv;"},
    [TKM_OP_XATLU] = {"xATLU", F_W, 0.5f,
                      "{ const float s = 1.0f / (1.0f + __expf(-x)); x = x * (w * s + (1.0f - w)); }",
                      "{ const float s = 1.0f / (1.0f + __expf(-p)); aw += g * p * (s - 1.0f);"
                      " g *= (1.0f - w) + w * s * (1.0f + p * (1.0f - s)); }"},
    [TKM_OP_SOFTPLUS] = {"Softplus", 0, 0.0f, "x = logf(1.0f + expf(x));", "g *= 1.0f / (1.0f + expf(-p));"},
    [TKM_OP_SNAKE] = {"Snake", 0, 1.0f, "{ const float sn = sinf(fv * x); x = x + sn * sn / fv; }",
                      "g *= 1.0f + sinf(2.0f * fv * p);"},
    [TKM_OP_ADD] = {"Add", F_BRANCH, 0.0f, NULL, NULL},
    [TKM_OP_DROP] = {"Drop", F_MASK | F_SEED, 0.1f, NULL, NULL},
    [TKM_OP_FORMULA] = {"Formula", 0, 0.0f, NULL, NULL},
    [TKM_OP_FORMULA_W] = {"FormulaW", F_W, 0.0f, NULL, NULL},
    [TKM_OP_FORMULA_B] = {"FormulaB", F_BIAS, 0.0f, NULL, NULL},
};

int tkm_plasma_op_pointwise(int op) {
    return op >= 0 && op < TKM_OP_COUNT && !(OPS[op].flags & (F_NORM | F_MASK | F_BRANCH | F_BETA));
}

static int is_formula_op(int op) { return op == TKM_OP_FORMULA || op == TKM_OP_FORMULA_W || op == TKM_OP_FORMULA_B; }

float tkm_plasma_default_fval(int op) { return (op >= 0 && op < TKM_OP_COUNT) ? OPS[op].fval : 0.0f; }

/* ---- geometry and argument lists ------------------------------------------------------- */

static int pow2ceil(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

static const tkm_plasma_node *node_at(const tkm_plasma_desc *d, int k) {
    if (d->twin) {
        if (k < d->n_left) return &d->left_ops[k];
        k -= d->n_left;
        if (k < d->n_right) return &d->right_ops[k];
        k -= d->n_right;
    }
    return &d->main_ops[k];
}

static int n_nodes(const tkm_plasma_desc *d) { return d->twin ? d->n_left + d->n_right + d->n_main : d->n_main; }

int tkm_plasma_check_desc(const tkm_plasma_desc *d) { return tkm_plasma_check_desc_f(d, NULL); }

int tkm_plasma_check_desc_f(const tkm_plasma_desc *d, const tkm_plasma_formula *formulas) {
    if (!d) return tkm_set_error(TKM_ATTN_EINVAL, "descriptor is NULL");
    if (d->channels <= 0 || d->channels % 2 != 0 || d->channels > (1 << 20))
        return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "channels %d: must be positive, even and at most 2^20",
                             d->channels);
    if (d->twin != 0 && d->twin != 1) return tkm_set_error(TKM_ATTN_EINVAL, "twin must be 0 or 1");
    if (d->group_id < 0) return tkm_set_error(TKM_ATTN_EINVAL, "group_id %d must be >= 0", d->group_id);
    if (d->dtype != TKM_ATTN_F16 && d->dtype != TKM_ATTN_BF16)
        return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "dtype %d", d->dtype);
    if (d->n_main < 0 || d->n_main > TKM_PLASMA_MAX_NODES || (d->twin && (d->n_left < 0 || d->n_right < 0 ||
        d->n_left > TKM_PLASMA_MAX_NODES || d->n_right > TKM_PLASMA_MAX_NODES)))
        return tkm_set_error(TKM_ATTN_EINVAL, "chain lengths must be in [0, %d]", TKM_PLASMA_MAX_NODES);
    for (int k = 0; k < n_nodes(d); ++k) {
        const tkm_plasma_node *n = node_at(d, k);
        if (n->op < 0 || n->op >= TKM_OP_COUNT) return tkm_set_error(TKM_ATTN_EINVAL, "node %d: unknown op %d", k, n->op);
        if (is_formula_op(n->op) && !(formulas && formulas[k].fwd && formulas[k].bwd))
            return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "node %d: %s needs the registry's code of its op (whole-graph "
                                 "generator with the front end linked)", k, OPS[n->op].name);
        if (formulas && formulas[k].fwd && !tkm_plasma_op_pointwise(n->op))
            return tkm_set_error(TKM_ATTN_EINVAL, "node %d: %s does not take registry code", k, OPS[n->op].name);
        if (!isfinite(n->fval)) return tkm_set_error(TKM_ATTN_EINVAL, "node %d: fval must be finite", k);
        const int f = OPS[n->op].flags;
        const int in_gate = d->twin && k < d->n_left + d->n_right;
        if (in_gate && (f & (F_NORM | F_BRANCH)))
            return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "node %d: %s inside a twin gate chain", k, OPS[n->op].name);
        if ((f & F_NORM) && d->channels % 8 != 0)
            return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "node %d: %s needs the channel count (%d) to be a multiple of 8",
                                 k, OPS[n->op].name, d->channels);
        if ((f & F_NORM) && !(n->fval > 0.0f))
            return tkm_set_error(TKM_ATTN_EINVAL, "node %d: %s epsilon must be > 0", k, OPS[n->op].name);
        if ((n->op == TKM_OP_SOFTCAP || n->op == TKM_OP_SNAKE) && n->fval == 0.0f)
            return tkm_set_error(TKM_ATTN_EINVAL, "node %d: %s needs fval != 0", k, OPS[n->op].name);
        if (n->op == TKM_OP_DROP && !(n->fval >= 0.0f && n->fval < 1.0f))
            return tkm_set_error(TKM_ATTN_EINVAL, "node %d: Drop needs 0 <= fval < 1", k);
        if (n->op == TKM_OP_DROP && (n->rng_type < 0 || n->rng_type > 4 || n->node_id < 0))
            return tkm_set_error(TKM_ATTN_EINVAL, "node %d: Drop needs rng_type in [0, 4] and node_id >= 0", k);
    }
    return TKM_ATTN_OK;
}

void tkm_plasma_geometry(const tkm_plasma_desc *d, tkm_plasma_geom *g) {
    memset(g, 0, sizeof *g);
    g->C = d->channels;
    g->CW = d->channels % 8 == 0 ? 8 : 2;
    g->CH = d->channels / g->CW;
    g->L = g->CH >= 64 ? 64 : pow2ceil(g->CH);
    g->RW = 64 / g->L;
    g->XB = (g->CH + g->L - 1) / g->L;
    g->NGL = g->L < 8 ? g->L : 8;
    g->NG = (d->channels + 63) / 64;
    g->n_nodes = n_nodes(d);
    /* argument lists */
    int nf = 0, nb = 0;
    g->fwd[nf].kind = TKM_ARG_IN;  g->fwd[nf++].node = -1;
    g->fwd[nf].kind = TKM_ARG_OUT; g->fwd[nf++].node = -1;
    g->bwd[nb].kind = TKM_ARG_DOUT; g->bwd[nb++].node = -1;
    g->bwd[nb].kind = TKM_ARG_IN;   g->bwd[nb++].node = -1;
    g->bwd[nb].kind = TKM_ARG_DIN;  g->bwd[nb++].node = -1;
    for (int k = 0; k < g->n_nodes; ++k) {
        const int f = OPS[node_at(d, k)->op].flags;
        const struct { int flag, kind; } fa[] = {{F_W, TKM_ARG_WEIGHT}, {F_BETA, TKM_ARG_BETA}, {F_BIAS, TKM_ARG_BIAS},
                                                {F_NORM, TKM_ARG_SAVE_XHAT}, {F_NORM, TKM_ARG_SAVE_ISTD},
                                                {F_BRANCH, TKM_ARG_BRANCH_IN}, {F_MASK, TKM_ARG_SAVE_MASK},
                                                {F_SEED, TKM_ARG_SEED}};
        for (size_t i = 0; i < sizeof fa / sizeof fa[0]; ++i)
            if (f & fa[i].flag) { g->fwd[nf].kind = fa[i].kind; g->fwd[nf++].node = k; }
        /* backward: what the replay and the gradient read, then what it writes */
        const struct { int flag, kind; } ba[] = {{F_W, TKM_ARG_WEIGHT}, {F_BETA, TKM_ARG_BETA}, {F_BIAS, TKM_ARG_BIAS},
                                                {F_NORM, TKM_ARG_SAVE_XHAT}, {F_NORM, TKM_ARG_SAVE_ISTD},
                                                {F_BRANCH, TKM_ARG_BRANCH_IN}, {F_BRANCH, TKM_ARG_DBRANCH},
                                                {F_MASK, TKM_ARG_SAVE_MASK}};
        for (size_t i = 0; i < sizeof ba / sizeof ba[0]; ++i)
            if (f & ba[i].flag) { g->bwd[nb].kind = ba[i].kind; g->bwd[nb++].node = k; }
        /* parameter gradients, in node order: one partial column block of C floats each */
        if (f & F_W) { g->par[g->n_par].kind = TKM_ARG_DWEIGHT; g->par[g->n_par++].node = k; }
        if (f & F_BETA) { g->par[g->n_par].kind = TKM_ARG_DBETA; g->par[g->n_par++].node = k; }
        if (f & F_BIAS) { g->par[g->n_par].kind = TKM_ARG_DBIAS; g->par[g->n_par++].node = k; }
    }
    g->n_fwd = nf;
    g->n_bwd = nb;
    g->part_width = g->n_par * g->C;
}

/* ---- emission -------------------------------------------------------------------------- */

/* Suffix of the prelude's pack / unpack helpers: 8-channel chunks (rows a multiple of 8 wide)
 * or 2-channel chunks. */
static const char *kind16(const tkm_plasma_desc *d) {
    const int narrow = d->channels % 8 != 0;
    return d->dtype == TKM_ATTN_BF16 ? (narrow ? "bf16_2" : "bf16") : (narrow ? "f16_2" : "f16");
}

static const char *arg_decl(int kind, int bwd) {
    switch (kind) {
        case TKM_ARG_SAVE_XHAT: return bwd ? "const TKM_VEC *__restrict__" : "TKM_VEC *__restrict__";
        case TKM_ARG_SAVE_ISTD: return bwd ? "const float *__restrict__" : "float *__restrict__";
        case TKM_ARG_IN: case TKM_ARG_DOUT: case TKM_ARG_BRANCH_IN:
            return "const TKM_VEC *__restrict__";
        case TKM_ARG_OUT: case TKM_ARG_DIN: case TKM_ARG_DBRANCH:
            return "TKM_VEC *__restrict__";
        case TKM_ARG_WEIGHT: case TKM_ARG_BETA: case TKM_ARG_BIAS:
            return "const TKM_PVEC *__restrict__";
        case TKM_ARG_SAVE_MASK: return bwd ? "const TKM_MVEC *__restrict__" : "TKM_MVEC *__restrict__";
        case TKM_ARG_SEED: return "const uint32_t *__restrict__";
        default: return "float *__restrict__";
    }
}

static const char *arg_prefix(int kind) {
    switch (kind) {
        case TKM_ARG_IN: return "in";
        case TKM_ARG_OUT: return "out";
        case TKM_ARG_DOUT: return "dout";
        case TKM_ARG_DIN: return "din";
        case TKM_ARG_WEIGHT: return "w";
        case TKM_ARG_BETA: return "beta";
        case TKM_ARG_BIAS: return "bias";
        case TKM_ARG_SAVE_XHAT: return "xhat";
        case TKM_ARG_SAVE_ISTD: return "istd";
        case TKM_ARG_BRANCH_IN: return "branch";
        case TKM_ARG_DBRANCH: return "dbranch";
        case TKM_ARG_DWEIGHT: return "dw";
        case TKM_ARG_DBETA: return "dbeta";
        case TKM_ARG_SAVE_MASK: return "mask";
        case TKM_ARG_SEED: return "seed";
        default: return "dbias";
    }
}

/* Internal argument list of pass 0 (forward) or 1 (backward): the geometry's pointer
 * arguments with their internal declarations and names, then the scalars. */
int tkm_plasma_need(const tkm_plasma_desc *d, int pass, tkm_kparam *out) {
    tkm_plasma_geom g;
    tkm_plasma_geometry(d, &g);
    const tkm_plasma_argd *a = pass ? g.bwd : g.fwd;
    const int na = pass ? g.n_bwd : g.n_fwd;
    int n = 0;
    for (int i = 0; i < na; ++i, ++n) {
        out[n].kind = a[i].kind;
        out[n].node = a[i].node;
        snprintf(out[n].decl, sizeof out[n].decl, "%s", arg_decl(a[i].kind, pass));
        if (a[i].node < 0) snprintf(out[n].name, sizeof out[n].name, "%s", arg_prefix(a[i].kind));
        else snprintf(out[n].name, sizeof out[n].name, "%s_%d", arg_prefix(a[i].kind), a[i].node);
    }
    const struct { int kind; const char *decl, *name; } sc[] = {
        {TKM_KP_PART, "float *__restrict__", "part"}, {TKM_KP_ROWS, "int", "rows"},
        {TKM_KP_BAND, "int", "band"}, {TKM_KP_ACC, "int", "acc_flags"}};
    for (int i = pass ? 0 : 1; i < (pass ? 4 : 2); ++i, ++n) {
        out[n].kind = sc[i].kind;
        out[n].node = -1;
        snprintf(out[n].decl, sizeof out[n].decl, "%s", sc[i].decl);
        snprintf(out[n].name, sizeof out[n].name, "%s", sc[i].name);
    }
    return n;
}

static void default_plan(const tkm_kparam *need, int n, tkm_kplan *pl) {
    pl->n = 0;
    for (int i = 0; i < n; ++i) tkm_kplan_add(pl, need[i].kind, need[i].node, need[i].decl, need[i].name);
}

/* Kernel header and parameter aliases for pass `pass` under `plan` (NULL: the internal list). */
static int emit_header(sbuf *s, const tkm_plasma_desc *d, int pass, const tkm_kplan *plan) {
    tkm_kparam need[TKM_KPLAN_MAX];
    const int n = tkm_plasma_need(d, pass, need);
    tkm_kplan def;
    if (!plan) {
        default_plan(need, n, &def);
        plan = &def;
    }
    sb_add(s, "extern \"C\" __global__ __launch_bounds__(256) void tkm_plasma_%s_g%d", pass ? "bwd" : "fwd",
           d->group_id);
    return tkm_emit_plan_params(s, plan, need, n);
}

/* Loads the lane's Drop keep bits of node k into `mm` (as a 64-bit word: pair p in bits
 * 16p..16p+15). */
static void emit_mask_load(sbuf *s, const tkm_plasma_geom *g, int k) {
    if (g->CW == 8)
        sb_add(s, "            const uint2 mw = live ? mask_%d[(size_t)r * TKM_CH + ch] : make_uint2(0u, 0u);\n"
                  "            const unsigned long long mm = (unsigned long long)mw.x | ((unsigned long long)mw.y << 32);\n",
               k);
    else
        sb_add(s, "            const unsigned long long mm = live ? (unsigned long long)mask_%d[(size_t)r * TKM_CH + ch] "
                  ": 0ull;\n", k);
}

static const char *rng_struct(int rng_type) {
    switch (rng_type) {
        case 1: return "RngXorshift32";
        case 3: return "RngPcg32";
        case 4: return "RngPhilox";
        default: return "RngWangXorshift32";
    }
}

/* lane slot, chunk and row mapping shared by the kernels */
static void emit_lane_map(sbuf *s) {
    sb_add(s, "    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;\n");
    sb_add(s, "    const int ch = blockIdx.x * TKM_L + (lane & (TKM_L - 1));   /* 8-channel chunk of the row */\n");
    sb_add(s, "    const int slot = wave * TKM_RW + lane / TKM_L;                /* row slot in the block */\n");
    sb_add(s, "    const bool ok = ch < TKM_CH;\n");
}

/* per-node parameter registers */
static void emit_param_loads(sbuf *s, const tkm_plasma_desc *d, const tkm_plasma_geom *g) {
    for (int k = 0; k < g->n_nodes; ++k) {
        const int f = OPS[node_at(d, k)->op].flags;
        const char *names[3] = {"w", "beta", "bias"};
        const int flags[3] = {F_W, F_BETA, F_BIAS};
        for (int i = 0; i < 3; ++i) {
            if (!(f & flags[i])) continue;
            sb_add(s, "    float %s%d[TKM_CW];\n", names[i], k);
            sb_add(s, "    tkm_ld_param(%s_%d, ch, ok, %s%d);\n", names[i], k, names[i], k);
        }
    }
}

/* ---- registry code of pointwise ops ---------------------------------------------------------
 * The reference's generator pastes a pointwise op's TkmOpSpec code into its per-channel-pair
 * kernels (src/tkm_codegen.c:296-357, 404-460).  Here each pair of a lane's chunk runs the same
 * code in a block of its own that declares what the code reads: v (forward) or dy and pre
 * (backward) as float2, fval, w_vec / b_vec with the pair at tid = 0, and acc_dw / acc_db for
 * the parameter gradients, which then join this kernel's band sums. */

/* A user formula in x and fval (TkmOpSpec fwd_expr / bwd_expr) with x replaced by `xname`,
 * pi by its value and the math functions by their float versions, as the reference's
 * generator translates them (src/tkm_codegen.c:72-103); everything else unchanged. */
static void emit_expr(sbuf *s, const char *expr, const char *xname) {
    static const char *const map[][2] = {{"exp", "expf"}, {"log", "logf"}, {"ln", "logf"}, {"sqrt", "sqrtf"},
                                         {"sin", "sinf"}, {"cos", "cosf"}, {"tanh", "tanhf"}, {"abs", "fabsf"},
                                         {"max", "fmaxf"}, {"min", "fminf"}, {"pow", "powf"}};
    for (const char *p = expr; *p;) {
        if (isalpha((unsigned char)*p) || *p == '_') {
            char name[32];
            int len = 0;
            while ((isalnum((unsigned char)*p) || *p == '_')) {
                if (len < (int)sizeof name - 1) name[len++] = *p;
                ++p;
            }
            name[len] = '\0';
            const char *out = name;
            if (!strcmp(name, "x")) out = xname;
            else if (!strcmp(name, "pi")) out = "3.14159265358979323846f";
            for (size_t i = 0; i < sizeof map / sizeof map[0]; ++i)
                if (!strcmp(name, map[i][0])) out = map[i][1];
            sb_add(s, "%s", out);
        } else {
            sb_add(s, "%c", *p++);
        }
    }
}

static void emit_pair_params(sbuf *s, int flags, int k, const char *pad) {
    if (flags & F_W) sb_add(s, "%sconst float2 wv_[1] = {make_float2(w%d[j], w%d[j + 1])};\n", pad, k, k);
    if (flags & F_BIAS) sb_add(s, "%sconst float2 bv_[1] = {make_float2(bias%d[j], bias%d[j + 1])};\n", pad, k, k);
}

static void emit_registry_forward(sbuf *s, const tkm_plasma_formula *f, int flags, int k, const char *v) {
    sb_add(s, "            /* the registry's code of this op */\n");
    sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; j += 2) {\n");
    sb_add(s, "                const float2 in_ = make_float2(%s[j], %s[j + 1]);\n", v, v);
    emit_pair_params(s, flags, k, "                ");
    sb_add(s, "                float2 out_;\n                {\n");
    sb_add(s, "                    float2 v = in_; const float fval = fv; const int tid = 0; (void)fval; (void)tid;\n");
    if (flags & F_W) sb_add(s, "                    const float2 *w_vec = wv_; (void)w_vec;\n");
    if (flags & F_BIAS) sb_add(s, "                    const float2 *b_vec = bv_; (void)b_vec;\n");
    if (f->expr) {
        sb_add(s, "                    v.x = ");
        emit_expr(s, f->fwd, "v.x");
        sb_add(s, ";\n                    v.y = ");
        emit_expr(s, f->fwd, "v.y");
        sb_add(s, ";\n");
    } else {
        sb_add(s, "                    %s\n", f->fwd);
    }
    sb_add(s, "                    out_ = v;\n                }\n");
    sb_add(s, "                %s[j] = out_.x;\n                %s[j + 1] = out_.y;\n            }\n", v, v);
}

static void emit_registry_backward(sbuf *s, const tkm_plasma_formula *f, int flags, int k, const char *gv,
                                   const char *pv) {
    sb_add(s, "            /* the registry's code of this op */\n");
    sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; j += 2) {\n");
    sb_add(s, "                const float2 gin_ = make_float2(%s[j], %s[j + 1]);\n", gv, gv);
    sb_add(s, "                const float2 pin_ = make_float2(%s[j], %s[j + 1]);\n", pv, pv);
    emit_pair_params(s, flags, k, "                ");
    sb_add(s, "                float2 gout_, aw_ = make_float2(0.f, 0.f), ab_ = make_float2(0.f, 0.f);\n");
    sb_add(s, "                (void)aw_; (void)ab_;\n                {\n");
    sb_add(s, "                    float2 dy = gin_; const float2 pre = pin_; const float fval = fv; const int tid = 0;\n");
    sb_add(s, "                    (void)pre; (void)fval; (void)tid;\n");
    sb_add(s, "                    float2 acc_dw = make_float2(0.f, 0.f), acc_db = make_float2(0.f, 0.f);\n");
    if (flags & F_W) sb_add(s, "                    const float2 *w_vec = wv_; (void)w_vec;\n");
    if (flags & F_BIAS) sb_add(s, "                    const float2 *b_vec = bv_; (void)b_vec;\n");
    if (f->expr) {
        sb_add(s, "                    dy.x *= ");
        emit_expr(s, f->bwd, "pre.x");
        sb_add(s, ";\n                    dy.y *= ");
        emit_expr(s, f->bwd, "pre.y");
        sb_add(s, ";\n");
    } else {
        sb_add(s, "                    %s\n", f->bwd);
    }
    sb_add(s, "                    gout_ = dy; aw_ = acc_dw; ab_ = acc_db;\n                }\n");
    sb_add(s, "                %s[j] = gout_.x;\n                %s[j + 1] = gout_.y;\n", gv, gv);
    if (flags & F_W) sb_add(s, "                if (live) { a_w%d[j] += aw_.x; a_w%d[j + 1] += aw_.y; }\n", k, k);
    if (flags & F_BIAS) sb_add(s, "                if (live) { a_bias%d[j] += ab_.x; a_bias%d[j + 1] += ab_.y; }\n", k, k);
    sb_add(s, "            }\n");
}

/* Forward of node k on v[TKM_CW]; `save` emits the stores of the norm state (forward pass only;
 * the backward replays norms from their saved xhat, emit_replay_norm). */
static void emit_node_forward(sbuf *s, const tkm_plasma_desc *d, const tkm_plasma_geom *g, int k, const char *v,
                              int save) {
    const tkm_plasma_node *n = node_at(d, k);
    const op_info *o = &OPS[n->op];
    sb_add(s, "        { /* node %d: %s */\n", k, o->name);
    sb_add(s, "            const float fv = %a; (void)fv;\n", (double)n->fval);
    if (o->flags & F_NORM) {
        const int ln = (n->op == TKM_OP_LN || n->op == TKM_OP_BN);
        {
            if (ln) {
                sb_add(s, "            float sm = 0.f, sq = 0.f;\n");
                sb_add(s, "            if (ok) {   /* lanes past the row end stay out of the sums */\n");
                sb_add(s, "#pragma unroll\n                for (int j = 0; j < TKM_CW; ++j) { sm += %s[j]; sq += %s[j] * %s[j]; }\n", v, v, v);
                sb_add(s, "            }\n");
                sb_add(s, "            sm = tkm_sum_lanes%d(sm); sq = tkm_sum_lanes%d(sq);\n", g->NGL, g->NGL);
                sb_add(s, "            const float m = sm * TKM_INV_C;\n");
                sb_add(s, "            const float is = rsqrtf(fmaxf(0.f, sq * TKM_INV_C - m * m) + fv);\n");
                sb_add(s, "            float xh[TKM_CW];\n");
                sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) xh[j] = (%s[j] - m) * is;\n", v);
            } else {
                sb_add(s, "            float sq = 0.f;\n");
                sb_add(s, "            if (ok) {   /* lanes past the row end stay out of the sums */\n");
                sb_add(s, "#pragma unroll\n                for (int j = 0; j < TKM_CW; ++j) sq += %s[j] * %s[j];\n", v, v);
                sb_add(s, "            }\n");
                sb_add(s, "            sq = tkm_sum_lanes%d(sq);\n", g->NGL);
                sb_add(s, "            const float is = rsqrtf(sq * TKM_INV_C + fv);\n");
                sb_add(s, "            float xh[TKM_CW];\n");
                sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) xh[j] = %s[j] * is;\n", v);
            }
            if (save) {
                sb_add(s, "            if (live) {\n");
                sb_add(s, "                xhat_%d[(size_t)r * TKM_CH + ch] = tkm_pack_%s(xh);\n", k, kind16(d));
                sb_add(s, "                if ((ch & (TKM_NGL - 1)) == 0) istd_%d[(size_t)r * TKM_NG + ch / 8] = is;\n", k);
                sb_add(s, "            }\n");
            }
            if (ln)
                sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) %s[j] = fmaf(w%d[j], xh[j], beta%d[j]);\n", v, k, k);
            else if (o->flags & F_W)
                sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) %s[j] = xh[j] * w%d[j];\n", v, k);
            else
                sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) %s[j] = xh[j];\n", v);
        }
    } else if (o->flags & F_MASK) {
        /* Drop (registry src/tkm_registry.c:426-434): one generator per channel pair, seeded with
         * step_seed ^ (node_id * 19937 + 1) at the pair's row-major index (src/tkm_codegen.c:310-313);
         * two draws per pair; the backward replays it from the saved keep bits. */
        sb_add(s, "            const float kp = 1.0f - fv, ikp = 1.0f / kp;\n");
        if (save) {
            sb_add(s, "            const uint32_t sd = seed_%d[0] ^ %uu;\n", k, (unsigned)n->node_id * 19937u + 1u);
            sb_add(s, "            uint32_t mk[TKM_CW / 2];\n");
            sb_add(s, "#pragma unroll\n            for (int p = 0; p < TKM_CW / 2; ++p) {\n");
            sb_add(s, "                %s rng;\n", rng_struct(n->rng_type));
            sb_add(s, "                rng_init(&rng, sd, (uint32_t)((size_t)r * (TKM_CW / 2 * TKM_CH) + TKM_CW / 2 * ch + p));\n");
            sb_add(s, "                const uint32_t k0 = rng_uniform(&rng) < kp ? 1u : 0u;\n");
            sb_add(s, "                const uint32_t k1 = rng_uniform(&rng) < kp ? 1u : 0u;\n");
            sb_add(s, "                %s[2 * p] = k0 ? %s[2 * p] * ikp : 0.0f;\n", v, v);
            sb_add(s, "                %s[2 * p + 1] = k1 ? %s[2 * p + 1] * ikp : 0.0f;\n", v, v);
            sb_add(s, "                mk[p] = k0 | (k1 << 8);\n");
            sb_add(s, "            }\n");
            if (g->CW == 8)
                sb_add(s, "            if (live) mask_%d[(size_t)r * TKM_CH + ch] = make_uint2(mk[0] | (mk[1] << 16), "
                          "mk[2] | (mk[3] << 16));\n", k);
            else
                sb_add(s, "            if (live) mask_%d[(size_t)r * TKM_CH + ch] = (uint16_t)mk[0];\n", k);
        } else {
            emit_mask_load(s, g, k);
            sb_add(s, "#pragma unroll\n            for (int p = 0; p < TKM_CW / 2; ++p) {\n");
            sb_add(s, "                const uint32_t m = tkm_mask_pair(mm, p);\n");
            sb_add(s, "                %s[2 * p] = (m & 0xffu) ? %s[2 * p] * ikp : 0.0f;\n", v, v);
            sb_add(s, "                %s[2 * p + 1] = (m >> 8) ? %s[2 * p + 1] * ikp : 0.0f;\n", v, v);
            sb_add(s, "            }\n");
        }
    } else if (o->flags & F_BRANCH) {
        sb_add(s, "            float bi[TKM_CW];\n");
        sb_add(s, "            tkm_unpack_%s(live ? branch_%d[(size_t)r * TKM_CH + ch] : TKM_ZERO(), bi);\n",
               kind16(d), k);
        sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) %s[j] += bi[j];\n", v);
    } else if (g->formulas && g->formulas[k].fwd) {
        emit_registry_forward(s, &g->formulas[k], o->flags, k, v);
    } else {
        sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) {\n");
        sb_add(s, "                float x = %s[j];\n", v);
        if (o->flags & F_W) sb_add(s, "                const float w = w%d[j];\n", k);
        if (o->flags & F_BIAS) sb_add(s, "                const float b = bias%d[j];\n", k);
        sb_add(s, "                %s\n", o->fwd);
        sb_add(s, "                %s[j] = x;\n", v);
        sb_add(s, "            }\n");
    }
    sb_add(s, "        }\n");
}

/* The replayed norm output needs the node index in two places; emit it directly. */
static void emit_replay_norm(sbuf *s, const tkm_plasma_desc *d, int k, const char *v) {
    const tkm_plasma_node *n = node_at(d, k);
    const op_info *o = &OPS[n->op];
    const int ln = (n->op == TKM_OP_LN || n->op == TKM_OP_BN);
    sb_add(s, "        { /* node %d: %s (replayed from xhat) */\n", k, o->name);
    sb_add(s, "            float xh[TKM_CW];\n");
    sb_add(s, "            tkm_unpack_%s(live ? xhat_%d[(size_t)r * TKM_CH + ch] : TKM_ZERO(), xh);\n",
           kind16(d), k);
    if (ln)
        sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) %s[j] = fmaf(w%d[j], xh[j], beta%d[j]);\n", v, k, k);
    else if (o->flags & F_W)
        sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) %s[j] = xh[j] * w%d[j];\n", v, k);
    else
        sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) %s[j] = xh[j];\n", v);
    sb_add(s, "        }\n");
}

/* Backward of node k: gradient gv[TKM_CW] in place; input (replayed) pv[TKM_CW]. */
static void emit_node_backward(sbuf *s, const tkm_plasma_desc *d, const tkm_plasma_geom *g, int k, const char *gv,
                               const char *pv) {
    const tkm_plasma_node *n = node_at(d, k);
    const op_info *o = &OPS[n->op];
    sb_add(s, "        { /* node %d: %s backward */\n", k, o->name);
    sb_add(s, "            const float fv = %a; (void)fv;\n", (double)n->fval);
    if (o->flags & F_NORM) {
        const int ln = (n->op == TKM_OP_LN || n->op == TKM_OP_BN);
        sb_add(s, "            float xh[TKM_CW], dxh[TKM_CW];\n");
        sb_add(s, "            tkm_unpack_%s(live ? xhat_%d[(size_t)r * TKM_CH + ch] : TKM_ZERO(), xh);\n",
               kind16(d), k);
        sb_add(s, "            float m1 = 0.f, m2 = 0.f;\n");
        sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) {\n");
        if (o->flags & F_W) {
            sb_add(s, "                if (live) a_w%d[j] += %s[j] * xh[j];\n", k, gv);
            sb_add(s, "                dxh[j] = %s[j] * w%d[j];\n", gv, k);
        } else {
            sb_add(s, "                dxh[j] = %s[j];\n", gv);
        }
        if (o->flags & F_BETA) sb_add(s, "                if (live) a_beta%d[j] += %s[j];\n", k, gv);
        if (ln) sb_add(s, "                m1 += ok ? dxh[j] : 0.f;\n");
        sb_add(s, "                m2 += ok ? dxh[j] * xh[j] : 0.f;\n");
        sb_add(s, "            }\n");
        if (ln) sb_add(s, "            m1 = tkm_sum_lanes%d(m1) * TKM_INV_C;\n", g->NGL);
        sb_add(s, "            m2 = tkm_sum_lanes%d(m2) * TKM_INV_C;\n", g->NGL);
        sb_add(s, "            const float is = live ? istd_%d[(size_t)r * TKM_NG + ch / 8] : 0.f;\n", k);
        sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) %s[j] = is * (dxh[j]%s - xh[j] * m2);\n", gv,
               ln ? " - m1" : "");
        (void)pv;
    } else if (o->flags & F_MASK) {
        sb_add(s, "            const float ikp = 1.0f / (1.0f - fv);\n");
        emit_mask_load(s, g, k);
        sb_add(s, "#pragma unroll\n            for (int p = 0; p < TKM_CW / 2; ++p) {\n");
        sb_add(s, "                const uint32_t m = tkm_mask_pair(mm, p);\n");
        sb_add(s, "                %s[2 * p] *= (m & 0xffu) ? ikp : 0.0f;\n", gv);
        sb_add(s, "                %s[2 * p + 1] *= (m >> 8) ? ikp : 0.0f;\n", gv);
        sb_add(s, "            }\n");
        (void)pv;
    } else if (o->flags & F_BRANCH) {
        sb_add(s, "            if (live) {\n");
        sb_add(s, "                float pb[TKM_CW];\n");
        sb_add(s, "                tkm_unpack_%s(acc_branch ? dbranch_%d[(size_t)r * TKM_CH + ch] : TKM_ZERO(), pb);\n",
               kind16(d), k);
        sb_add(s, "#pragma unroll\n                for (int j = 0; j < TKM_CW; ++j) pb[j] += %s[j];\n", gv);
        sb_add(s, "                dbranch_%d[(size_t)r * TKM_CH + ch] = tkm_pack_%s(pb);\n", k, kind16(d));
        sb_add(s, "            }\n");
    } else if (g->formulas && g->formulas[k].bwd) {
        emit_registry_backward(s, &g->formulas[k], o->flags, k, gv, pv);
    } else {
        sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) {\n");
        sb_add(s, "                float g = %s[j];\n", gv);
        sb_add(s, "                const float p = %s[j]; (void)p;\n", pv);
        if (o->flags & F_W) {
            sb_add(s, "                const float w = w%d[j];\n", k);
            sb_add(s, "                float aw = 0.f;\n");
        }
        if (o->flags & F_BIAS) sb_add(s, "                if (live) a_bias%d[j] += g;\n", k);
        sb_add(s, "                %s\n", o->bwd);
        if (o->flags & F_W) sb_add(s, "                if (live) a_w%d[j] += aw;\n", k);
        sb_add(s, "                %s[j] = g;\n", gv);
        sb_add(s, "            }\n");
    }
    sb_add(s, "        }\n");
}

static void emit_constants(sbuf *s, const tkm_plasma_desc *d, const tkm_plasma_geom *g) {
    sb_add(s, "/* plasma group %d: C=%d twin=%d nodes=%d %s */\n", d->group_id, d->channels, d->twin, g->n_nodes,
           kind16(d));
    sb_add(s, "#define TKM_CW %d      /* channels per lane chunk */\n", g->CW);
    sb_add(s, "#define TKM_CH %d      /* chunks per row */\n", g->CH);
    if (g->CW == 8)
        sb_add(s, "#define TKM_VEC uint4\n#define TKM_PVEC float4\n#define TKM_MVEC uint2\n#define TKM_ZERO tkm_zero4\n");
    else
        sb_add(s, "#define TKM_VEC uint32_t\n#define TKM_PVEC float2\n#define TKM_MVEC uint16_t\n"
                  "#define TKM_ZERO tkm_zero1\n");
    sb_add(s, "#define TKM_L %d       /* lanes per row */\n", g->L);
    sb_add(s, "#define TKM_RW %d      /* rows per wave */\n", g->RW);
    sb_add(s, "#define TKM_NGL %d     /* lanes per norm group */\n", g->NGL);
    sb_add(s, "#define TKM_NG %d      /* norm groups per row */\n", g->NG);
    sb_add(s, "#define TKM_INV_C %af\n", 1.0 / (double)(float)d->channels);
    sb_add(s, "#define TKM_PW %d      /* partial-sum row width */\n", g->part_width > 0 ? g->part_width : 1);
    if (g->CW == 8) {
        sb_add(s, "__device__ __forceinline__ void tkm_ld_param(const float4 *p, int ch, bool ok, float *v) {\n");
        sb_add(s, "    const float4 a = ok ? p[2 * ch] : make_float4(0.f, 0.f, 0.f, 0.f);\n");
        sb_add(s, "    const float4 b = ok ? p[2 * ch + 1] : make_float4(0.f, 0.f, 0.f, 0.f);\n");
        sb_add(s, "    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;\n");
    } else {
        sb_add(s, "__device__ __forceinline__ void tkm_ld_param(const float2 *p, int ch, bool ok, float *v) {\n");
        sb_add(s, "    const float2 a = ok ? p[ch] : make_float2(0.f, 0.f);\n");
        sb_add(s, "    v[0] = a.x; v[1] = a.y;\n");
    }
    sb_add(s, "}\n");
    sb_add(s, "__device__ __forceinline__ uint32_t tkm_mask_pair(unsigned long long mm, int p) {\n"
              "    return (uint32_t)(mm >> (16 * p)) & 0xffffu;\n}\n\n");
}

/* forward kernel */
static int emit_fwd(sbuf *s, const tkm_plasma_desc *d, const tkm_plasma_geom *g, const tkm_kplan *plan) {
    const char *k16 = kind16(d);
    if (emit_header(s, d, 0, plan)) return -1;
    emit_lane_map(s);
    emit_param_loads(s, d, g);
    const int RPI = TKM_PLASMA_FWD_RPI;
    sb_add(s, "    const int r0 = blockIdx.y * %d * 4 * TKM_RW + slot;\n", RPI);
    if (d->twin) sb_add(s, "    TKM_VEC xa[%d], xb[%d];\n", RPI, RPI);
    else sb_add(s, "    TKM_VEC xa[%d];\n", RPI);
    sb_add(s, "#pragma unroll\n    for (int k = 0; k < %d; ++k) {\n", RPI);
    sb_add(s, "        const int r = r0 + k * 4 * TKM_RW;\n");
    sb_add(s, "        const bool live = ok && r < rows;\n");
    if (d->twin) {
        sb_add(s, "        xa[k] = live ? in[(size_t)r * (2 * TKM_CH) + ch] : TKM_ZERO();\n");
        sb_add(s, "        xb[k] = live ? in[(size_t)r * (2 * TKM_CH) + TKM_CH + ch] : TKM_ZERO();\n");
    } else {
        sb_add(s, "        xa[k] = live ? in[(size_t)r * TKM_CH + ch] : TKM_ZERO();\n");
    }
    sb_add(s, "    }\n");
    sb_add(s, "#pragma unroll\n    for (int k = 0; k < %d; ++k) {\n", RPI);
    sb_add(s, "        const int r = r0 + k * 4 * TKM_RW;\n");
    sb_add(s, "        const bool live = ok && r < rows;\n");
    sb_add(s, "        float v[TKM_CW];\n");
    sb_add(s, "        tkm_unpack_%s(xa[k], v);\n", k16);
    int k0 = 0;
    if (d->twin) {
        sb_add(s, "        float u[TKM_CW];\n");
        sb_add(s, "        tkm_unpack_%s(xb[k], u);\n", k16);
        for (int k = 0; k < d->n_left; ++k) emit_node_forward(s, d, g, k, "v", 1);
        for (int k = 0; k < d->n_right; ++k) emit_node_forward(s, d, g, d->n_left + k, "u", 1);
        sb_add(s, "#pragma unroll\n        for (int j = 0; j < TKM_CW; ++j) v[j] *= u[j];\n");
        k0 = d->n_left + d->n_right;
    }
    for (int k = k0; k < g->n_nodes; ++k) emit_node_forward(s, d, g, k, "v", 1);
    sb_add(s, "        if (live) out[(size_t)r * TKM_CH + ch] = tkm_pack_%s(v);\n", k16);
    sb_add(s, "    }\n}\n\n");
    return 0;
}

/* backward kernel + partial-sum reduce */
static int emit_bwd(sbuf *s, const tkm_plasma_desc *d, const tkm_plasma_geom *g, const tkm_kplan *plan) {
    const char *k16 = kind16(d);
    if (emit_header(s, d, 1, plan)) return -1;
    sb_add(s, "    (void)part;\n");
    emit_lane_map(s);
    emit_param_loads(s, d, g);
    sb_add(s, "    const bool acc_din = (acc_flags & 1) != 0, acc_branch = (acc_flags & 4) != 0;\n");
    sb_add(s, "    (void)acc_branch;\n");
    for (int p = 0; p < g->n_par; ++p) {
        const char *nm = g->par[p].kind == TKM_ARG_DWEIGHT ? "w" : g->par[p].kind == TKM_ARG_DBETA ? "beta" : "bias";
        sb_add(s, "    float a_%s%d[TKM_CW] = {};\n", nm, g->par[p].node);
    }
    sb_add(s, "    const int rbeg = blockIdx.y * band, rend = min(rows, rbeg + band);\n");
    sb_add(s, "    for (int r = rbeg + slot; r < rbeg + band; r += 4 * TKM_RW) {\n");
    sb_add(s, "        const bool live = ok && r < rend;\n");
    /* replay: the input of every node */
    const int nn = g->n_nodes;
    if (d->twin) {
        sb_add(s, "        float v[TKM_CW], u[TKM_CW];\n");
        sb_add(s, "        tkm_unpack_%s(live ? in[(size_t)r * (2 * TKM_CH) + ch] : TKM_ZERO(), v);\n", k16);
        sb_add(s, "        tkm_unpack_%s(live ? in[(size_t)r * (2 * TKM_CH) + TKM_CH + ch] : TKM_ZERO(), u);\n", k16);
    } else {
        sb_add(s, "        float v[TKM_CW];\n");
        sb_add(s, "        tkm_unpack_%s(live ? in[(size_t)r * TKM_CH + ch] : TKM_ZERO(), v);\n", k16);
    }
    for (int k = 0; k < nn; ++k) {
        const int is_right = d->twin && k >= d->n_left && k < d->n_left + d->n_right;
        const char *src = is_right ? "u" : "v";
        if (d->twin && k == d->n_left + d->n_right) {
            /* product of the two gates */
            sb_add(s, "        float gl[TKM_CW], gr[TKM_CW];\n");
            sb_add(s, "#pragma unroll\n        for (int j = 0; j < TKM_CW; ++j) { gl[j] = v[j]; gr[j] = u[j]; v[j] *= u[j]; }\n");
        }
        sb_add(s, "        float pre%d[TKM_CW];\n", k);
        sb_add(s, "#pragma unroll\n        for (int j = 0; j < TKM_CW; ++j) pre%d[j] = %s[j];\n", k, src);
        if (OPS[node_at(d, k)->op].flags & F_NORM) emit_replay_norm(s, d, k, src);
        else emit_node_forward(s, d, g, k, src, 0);
    }
    if (d->twin && nn == d->n_left + d->n_right) {
        sb_add(s, "        float gl[TKM_CW], gr[TKM_CW];\n");
        sb_add(s, "#pragma unroll\n        for (int j = 0; j < TKM_CW; ++j) { gl[j] = v[j]; gr[j] = u[j]; }\n");
    }
    /* backward in reverse */
    sb_add(s, "        float dy[TKM_CW];\n");
    sb_add(s, "        tkm_unpack_%s(live ? dout[(size_t)r * TKM_CH + ch] : TKM_ZERO(), dy);\n", k16);
    const int kpost = d->twin ? d->n_left + d->n_right : 0;
    for (int k = nn - 1; k >= kpost; --k) {
        char pv[16];
        snprintf(pv, sizeof pv, "pre%d", k);
        emit_node_backward(s, d, g, k, "dy", pv);
    }
    if (d->twin) {
        sb_add(s, "        float dl[TKM_CW], dr[TKM_CW];\n");
        sb_add(s, "#pragma unroll\n        for (int j = 0; j < TKM_CW; ++j) { dl[j] = dy[j] * gr[j]; dr[j] = dy[j] * gl[j]; }\n");
        for (int k = d->n_left + d->n_right - 1; k >= d->n_left; --k) {
            char pv[16];
            snprintf(pv, sizeof pv, "pre%d", k);
            emit_node_backward(s, d, g, k, "dr", pv);
        }
        for (int k = d->n_left - 1; k >= 0; --k) {
            char pv[16];
            snprintf(pv, sizeof pv, "pre%d", k);
            emit_node_backward(s, d, g, k, "dl", pv);
        }
        sb_add(s, "        if (live) {\n");
        sb_add(s, "            float pa[TKM_CW], pb[TKM_CW];\n");
        sb_add(s, "            tkm_unpack_%s(acc_din ? din[(size_t)r * (2 * TKM_CH) + ch] : TKM_ZERO(), pa);\n", k16);
        sb_add(s, "            tkm_unpack_%s(acc_din ? din[(size_t)r * (2 * TKM_CH) + TKM_CH + ch] : TKM_ZERO(), pb);\n", k16);
        sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) { pa[j] += dl[j]; pb[j] += dr[j]; }\n");
        sb_add(s, "            din[(size_t)r * (2 * TKM_CH) + ch] = tkm_pack_%s(pa);\n", k16);
        sb_add(s, "            din[(size_t)r * (2 * TKM_CH) + TKM_CH + ch] = tkm_pack_%s(pb);\n", k16);
        sb_add(s, "        }\n");
    } else {
        sb_add(s, "        if (live) {\n");
        sb_add(s, "            float pa[TKM_CW];\n");
        sb_add(s, "            tkm_unpack_%s(acc_din ? din[(size_t)r * TKM_CH + ch] : TKM_ZERO(), pa);\n", k16);
        sb_add(s, "#pragma unroll\n            for (int j = 0; j < TKM_CW; ++j) pa[j] += dy[j];\n");
        sb_add(s, "            din[(size_t)r * TKM_CH + ch] = tkm_pack_%s(pa);\n", k16);
        sb_add(s, "        }\n");
    }
    sb_add(s, "    }\n");
    if (g->n_par > 0) {
        /* combine the 4 x RW lane slots of the block in slot order, one partial row per band */
        sb_add(s, "    __shared__ float red[4 * TKM_RW][TKM_CW][TKM_L];\n");
        sb_add(s, "    const int cl = lane & (TKM_L - 1);\n");
        for (int p = 0; p < g->n_par; ++p) {
            const char *nm = g->par[p].kind == TKM_ARG_DWEIGHT ? "w" : g->par[p].kind == TKM_ARG_DBETA ? "beta" : "bias";
            if (p) sb_add(s, "    __syncthreads();\n");
            sb_add(s, "#pragma unroll\n    for (int j = 0; j < TKM_CW; ++j) red[slot][j][cl] = a_%s%d[j];\n", nm, g->par[p].node);
            sb_add(s, "    __syncthreads();\n");
            sb_add(s, "    if (slot == 0 && ok) {\n");
            sb_add(s, "        float t[TKM_CW];\n");
            sb_add(s, "#pragma unroll\n        for (int j = 0; j < TKM_CW; ++j) {\n");
            sb_add(s, "            float acc = red[0][j][cl];\n");
            sb_add(s, "            for (int q = 1; q < 4 * TKM_RW; ++q) acc += red[q][j][cl];\n");
            sb_add(s, "            t[j] = acc;\n");
            sb_add(s, "        }\n");
            if (g->CW == 8) {
                sb_add(s, "        float4 *pp = (float4 *)(part + (size_t)blockIdx.y * TKM_PW + %d + 8 * ch);\n", p * g->C);
                sb_add(s, "        pp[0] = make_float4(t[0], t[1], t[2], t[3]);\n");
                sb_add(s, "        pp[1] = make_float4(t[4], t[5], t[6], t[7]);\n");
            } else {
                sb_add(s, "        float2 *pp = (float2 *)(part + (size_t)blockIdx.y * TKM_PW + %d + 2 * ch);\n", p * g->C);
                sb_add(s, "        pp[0] = make_float2(t[0], t[1]);\n");
            }
            sb_add(s, "    }\n");
        }
    }
    sb_add(s, "}\n\n");

    if (g->n_par > 0) {
        sb_add(s, "extern \"C\" __global__ __launch_bounds__(1024) void tkm_plasma_bwd_g%d_reduce(\n", d->group_id);
        sb_add(s, "    const float *__restrict__ part, int bands, int acc_params");
        for (int p = 0; p < g->n_par; ++p) sb_add(s, ", float *__restrict__ dst%d", p);
        sb_add(s, ")\n{\n");
        sb_add(s, "    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;\n");
        sb_add(s, "    const int c = blockIdx.x * 64 + lane;\n");
        sb_add(s, "    float acc = 0.f;\n");
        sb_add(s, "    if (c < TKM_PW) {\n");
        sb_add(s, "#pragma unroll 4\n");
        sb_add(s, "        for (int b = wave; b < bands; b += 16) acc += part[(size_t)b * TKM_PW + c];\n");
        sb_add(s, "    }\n");
        sb_add(s, "    __shared__ float red[16][64];\n");
        sb_add(s, "    red[wave][lane] = acc;\n");
        sb_add(s, "    __syncthreads();\n");
        sb_add(s, "    if (wave != 0 || c >= TKM_PW) return;\n");
        sb_add(s, "    float t = red[0][lane];\n");
        sb_add(s, "    for (int q = 1; q < 16; ++q) t += red[q][lane];\n");
        sb_add(s, "    const int p = c / %d, o = c - p * %d;\n", g->C, g->C);
        sb_add(s, "    float *dst = ");
        for (int p = 0; p < g->n_par; ++p) sb_add(s, "%sp == %d ? dst%d", p ? " : " : "", p, p);
        sb_add(s, " : dst0;\n");
        sb_add(s, "    dst[o] = acc_params ? dst[o] + t : t;\n");
        sb_add(s, "}\n");
    }
    return 0;
}

int tkm_plasma_emit(tkm_sbuf *s, const tkm_plasma_desc *d, const tkm_kplan *fwd_plan, const tkm_kplan *bwd_plan,
                    int scoped, const tkm_plasma_formula *formulas) {
    int rc = tkm_plasma_check_desc_f(d, formulas);
    if (rc) return rc;
    tkm_plasma_geom g;
    tkm_plasma_geometry(d, &g);
    g.formulas = formulas;
    if (scoped) sb_add(s, "namespace tkm_g%d {\n", d->group_id);
    emit_constants(s, d, &g);
    if (emit_fwd(s, d, &g, fwd_plan) || emit_bwd(s, d, &g, bwd_plan))
        return tkm_set_error(TKM_ATTN_EINVAL, "plasma group %d: a kernel argument is missing from its plan",
                             d->group_id);
    if (scoped) {
        sb_add(s, "}  /* namespace tkm_g%d */\n", d->group_id);
        sb_add(s, "#undef TKM_CW\n#undef TKM_CH\n#undef TKM_L\n#undef TKM_RW\n#undef TKM_NGL\n#undef TKM_NG\n"
                  "#undef TKM_INV_C\n#undef TKM_PW\n#undef TKM_VEC\n#undef TKM_PVEC\n#undef TKM_MVEC\n#undef TKM_ZERO\n\n");
    }
    return s->failed ? tkm_set_error(TKM_ATTN_EINVAL, "out of host memory while emitting source") : TKM_ATTN_OK;
}

char *tkm_plasma_source(const tkm_plasma_desc *d) {
    sbuf s = {0};
    sb_add(&s, "%s", tkm_hip_prelude());
    if (tkm_plasma_emit(&s, d, NULL, NULL, 0, NULL) != TKM_ATTN_OK) {
        free(s.buf);
        return NULL;
    }
    return s.buf;
}
