/*
 * Whole-graph HIP code generator: tkm_codegen_cuda_string (include/tkm.h) for hipRTC, gfx950.
 *
 * Counterpart of the reference's table-driven NVRTC generator (src/tkm_codegen.c:627-634,
 * emit_plasma_group 484-625, emit_qkv_prep_plasma_group 211-295).  For every PlasmaGroup of a
 * TkmGraph (the reference front end's output) it maps the group onto this build's generators:
 *
 *   - the qkv_prep group (the fused QKV GEMM's epilogue: bias, QKNorm, RoPE; the node fields
 *     written by the 3-way rule, src/tkm_registry.c:750-768) -> tkm_prep_desc;
 *   - plain and twin groups (src/tkm_core.c:509-537) -> tkm_plasma_desc, ops mapped from the
 *     node's TkmOpType (user-formula ops by their registry index);
 *
 * and emits their kernels under the reference's names tkm_plasma_{fwd,bwd}_g<N> with the
 * parameters of the group's TkmKernelSig, in its order, with its C types and names
 * (src/tkm_core.c:289-382), followed by the extra parameters this build's kernels take
 * (rows, the backward's partial-sum workspace, band, accumulation flags, and any pointer the
 * backward reads that the reference's signature lacks).  Parameters the kernels do not read
 * (the reference's replay_in_0 and b_vec in a qkv-prep backward, the d(param) outputs that the
 * separate reduce kernel writes) stay in the list, unused.  Each group also emits
 * tkm_plasma_bwd_g<N>_reduce, the deterministic parameter-gradient reduction.
 *
 * Launch geometry is this build's (2-D grids, 16-byte lanes), not the signature's grid_x /
 * block_x: the runtime (tkm_hip.c) launches the kernels it generated.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tkm.h"
#include "tkm_codegen_internal.h"
#include "tkm_hip.h"
#include "tkm_plasma_internal.h"

/* Registry indices of the user-formula ops (OP_USER_FLUID nodes carry spec_id; reference
 * src/tkm_registry.c:445-455); pinned against the registry by tests/test_tkm_runtime_cpu.py. */
enum { SPEC_SOFTPLUS = 62, SPEC_SNAKE = 63 };

/* The registry (the reference's tkm_registry.c) is part of the front end, which the
 * application links; without it the generator uses this build's own op formulas. */
#pragma weak tkm_find_spec_by_node

static int g_registry_code = 1;

void tkm_hip_use_registry_code(int mode) { g_registry_code = mode < 0 ? 0 : (mode > 2 ? 2 : mode); }

int tkm_hip_registry_linked(void) { return tkm_find_spec_by_node != NULL; }

static const TkmOpSpec *registry_spec(const TkmNode *n) {
    return tkm_find_spec_by_node ? tkm_find_spec_by_node(n) : NULL;
}

/* A pointwise op of the registry with code the generator can paste (CUDA snippets or a user
 * formula, both directions). */
static int has_pointwise_code(const TkmOpSpec *sp) {
    return sp && sp->cat == CAT_FLUID && ((sp->fwd_cuda && sp->bwd_cuda) || (sp->fwd_expr && sp->bwd_expr));
}

/* An op this build has no formula of its own for: the registry's code, by its parameters. */
static int formula_op(const TkmNode *n) {
    const TkmOpSpec *sp = registry_spec(n);
    if (!has_pointwise_code(sp)) return -1;
    switch (sp->res_flags) {
        case RES_NONE: return TKM_OP_FORMULA;
        case RES_PARAM_WEIGHT: return TKM_OP_FORMULA_W;
        case RES_PARAM_BIAS: return TKM_OP_FORMULA_B;
        default: return -1;
    }
}

int tkm_hip_plasma_op(const TkmNode *n) {
    if (g_registry_code == 2) {         /* every pointwise op as an op unknown to this build */
        const int f = formula_op(n);
        if (f >= 0) return f;
    }
    switch (n->op) {
        case OP_BIAS: return TKM_OP_BIAS;
        case OP_RMSNORM: return TKM_OP_RMSNORM;
        case OP_LN: return TKM_OP_LN;
        case OP_BN: return TKM_OP_BN;
        case OP_L2NORM: return TKM_OP_L2NORM;
        case OP_SILU: return TKM_OP_SILU;
        case OP_RELU: return TKM_OP_RELU;
        case OP_RELU2: return TKM_OP_RELU2;
        case OP_LEAKY_RELU: return TKM_OP_LEAKY_RELU;
        case OP_ELU: return TKM_OP_ELU;
        case OP_GELU: return TKM_OP_GELU;
        case OP_MISH: return TKM_OP_MISH;
        case OP_HARDSWISH: return TKM_OP_HARDSWISH;
        case OP_HARDSIGMOID: return TKM_OP_HARDSIGMOID;
        case OP_TANH: return TKM_OP_TANH;
        case OP_SIGMOID: return TKM_OP_SIGMOID;
        case OP_SWISH_BETA: return TKM_OP_SWISH_BETA;
        case OP_SIN: return TKM_OP_SIN;
        case OP_COSGATE: return TKM_OP_COSGATE;
        case OP_SOFTCAP: return TKM_OP_SOFTCAP;
        case OP_CLAMP: return TKM_OP_CLAMP;
        case OP_SCALE: return TKM_OP_SCALE;
        case OP_LAYERSCALE: return TKM_OP_LAYERSCALE;
        case OP_DYT: return TKM_OP_DYT;
        case OP_PRELU: return TKM_OP_PRELU;
        case OP_XATLU: return TKM_OP_XATLU;
        case OP_ADD: return TKM_OP_ADD;
        case OP_DROP: return TKM_OP_DROP;
        case OP_USER_FLUID:
            if (n->spec_id == SPEC_SOFTPLUS) return TKM_OP_SOFTPLUS;
            if (n->spec_id == SPEC_SNAKE) return TKM_OP_SNAKE;
            return formula_op(n);
        default: return formula_op(n);
    }
}

/* The registry's code of each chain position's op (g_registry_code and the front end linked),
 * for the pointwise ops that have it; all-NULL otherwise. */
static void group_formulas(const TkmGraph *g, const tkm_plasma_desc *d, const int *map, int nm,
                           tkm_plasma_formula *out) {
    memset(out, 0, sizeof(tkm_plasma_formula) * 3 * TKM_PLASMA_MAX_NODES);
    for (int k = 0; k < nm; ++k) {
        const TkmNode *n = &g->nodes[map[k]];
        const int op = k < (d->twin ? d->n_left : 0) ? d->left_ops[k].op
                       : k < (d->twin ? d->n_left + d->n_right : 0) ? d->right_ops[k - d->n_left].op
                       : d->main_ops[k - (d->twin ? d->n_left + d->n_right : 0)].op;
        const TkmOpSpec *sp = registry_spec(n);
        const int forced = op == TKM_OP_FORMULA || op == TKM_OP_FORMULA_W || op == TKM_OP_FORMULA_B;
        if (!has_pointwise_code(sp) || !tkm_plasma_op_pointwise(op) || (!g_registry_code && !forced)) continue;
        out[k].expr = sp->fwd_cuda ? 0 : 1;
        out[k].fwd = sp->fwd_cuda ? sp->fwd_cuda : sp->fwd_expr;
        out[k].bwd = sp->bwd_cuda ? sp->bwd_cuda : sp->bwd_expr;
    }
}

static int is_prep_group(const TkmGraph *g, const PlasmaGroup *pg) {
    return pg->is_qkv_prep && pg->count == 1 && g->nodes[pg->node_ids[0]].op == OP_QKNORM;
}

int tkm_hip_group_kind(const TkmGraph *g, int gid) {
    if (!g || gid < 0 || gid >= g->num_groups) return -1;
    const PlasmaGroup *pg = &g->groups[gid];
    if (pg->is_coord_group) return -1;
    if (is_prep_group(g, pg)) return TKM_HIP_GROUP_PREP;
    return TKM_HIP_GROUP_PLASMA;
}

int tkm_hip_prep_desc(const TkmGraph *g, int gid, int dtype, tkm_prep_desc *d) {
    if (!g || !d || tkm_hip_group_kind(g, gid) != TKM_HIP_GROUP_PREP)
        return tkm_set_error(TKM_ATTN_EINVAL, "group %d is not a qkv-prep group", gid);
    const PlasmaGroup *pg = &g->groups[gid];
    const TkmNode *n = &g->nodes[pg->node_ids[0]];
    tkm_prep_desc_init(d);
    d->group_id = pg->id;
    d->seq_len = pg->H * pg->W;       /* RoPE position = row % (H*W) (src/tkm_codegen.c:215) */
    d->q_heads = n->q_heads;
    d->kv_heads = n->kv_heads;
    d->head_dim = n->head_dim;
    d->has_qknorm = n->has_qknorm ? 1 : 0;
    d->has_rope = n->has_rope ? 1 : 0;
    d->rope_theta = n->rope_theta;
    d->rope_scale = n->rope_scale;
    d->rope_low_freq_factor = n->rope_low_freq_factor;
    d->rope_high_freq_factor = n->rope_high_freq_factor;
    d->rope_original_context_length = n->rope_original_context_length;
    d->dtype = dtype;
    if (n->q_c != n->q_heads * n->head_dim || n->k_c != n->kv_heads * n->head_dim || n->v_c != n->k_c ||
        pg->C != n->q_c + n->k_c + n->v_c)
        return tkm_set_error(TKM_ATTN_EINVAL, "qkv-prep group %d: widths q_c=%d k_c=%d v_c=%d C=%d do not match "
                             "%d + 2 x %d heads of %d", gid, n->q_c, n->k_c, n->v_c, pg->C, n->q_heads,
                             n->kv_heads, n->head_dim);
    return tkm_prep_check_desc(d);
}

static int set_node(const TkmGraph *g, int nid, tkm_plasma_node *out) {
    const TkmNode *n = &g->nodes[nid];
    const int op = tkm_hip_plasma_op(n);
    if (op < 0) return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "node %d (%s): op %d has no HIP epilogue", nid, n->tag,
                                     (int)n->op);
    out->op = op;
    out->fval = n->fval;
    out->rng_type = (int)n->rng_type;
    out->node_id = n->id;
    return TKM_ATTN_OK;
}

int tkm_hip_plasma_desc(const TkmGraph *g, int gid, int dtype, tkm_plasma_desc *d, int *chain_nodes) {
    if (!g || !d || tkm_hip_group_kind(g, gid) != TKM_HIP_GROUP_PLASMA)
        return tkm_set_error(TKM_ATTN_EINVAL, "group %d is not a plain or twin epilogue group", gid);
    const PlasmaGroup *pg = &g->groups[gid];
    memset(d, 0, sizeof *d);
    d->group_id = pg->id;
    d->channels = pg->C;
    d->dtype = dtype;
    int map[3 * TKM_PLASMA_MAX_NODES], nm = 0, rc = 0;
    if (pg->is_twin_epilogue) {
        const TkmNode *mul = &g->nodes[pg->node_ids[0]];
        if (mul->op != OP_MUL || mul->left_len > TKM_PLASMA_MAX_NODES || mul->right_len > TKM_PLASMA_MAX_NODES ||
            pg->count - 1 > TKM_PLASMA_MAX_NODES)
            return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "twin group %d: chains too long or no Mul", gid);
        d->twin = 1;
        d->n_left = mul->left_len;
        d->n_right = mul->right_len;
        d->n_main = pg->count - 1;
        for (int i = 0; i < mul->left_len && !rc; ++i) {
            rc = set_node(g, mul->left_nodes[i], &d->left_ops[i]);
            map[nm++] = mul->left_nodes[i];
        }
        for (int i = 0; i < mul->right_len && !rc; ++i) {
            rc = set_node(g, mul->right_nodes[i], &d->right_ops[i]);
            map[nm++] = mul->right_nodes[i];
        }
        for (int i = 1; i < pg->count && !rc; ++i) {
            rc = set_node(g, pg->node_ids[i], &d->main_ops[i - 1]);
            map[nm++] = pg->node_ids[i];
        }
    } else {
        if (pg->count > TKM_PLASMA_MAX_NODES)
            return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "group %d: %d ops, at most %d", gid, pg->count,
                                 TKM_PLASMA_MAX_NODES);
        d->n_main = pg->count;
        for (int i = 0; i < pg->count && !rc; ++i) {
            rc = set_node(g, pg->node_ids[i], &d->main_ops[i]);
            map[nm++] = pg->node_ids[i];
        }
    }
    if (rc) return rc;
    if (chain_nodes)
        for (int i = 0; i < nm; ++i) chain_nodes[i] = map[i];
    tkm_plasma_formula f[3 * TKM_PLASMA_MAX_NODES];
    group_formulas(g, d, map, nm, f);
    return tkm_plasma_check_desc_f(d, f);
}

/* Internal (kind, chain index) of a signature argument, or TKM_KP_UNUSED.  map: chain index ->
 * graph node id; nm entries. */
static void sig_to_internal(const TkmGraph *g, const TkmKernelArg *a, const int *map, int nm, int is_prep,
                            int bwd, int *kind, int *node) {
    *node = -1;
    int k = -1;
    for (int i = 0; i < nm; ++i)
        if (map[i] == a->node_id) k = i;
    switch (a->kind) {
        case KARG_IN_MAIN: *kind = (is_prep && bwd) ? TKM_KP_UNUSED : TKM_ARG_IN; return;
        case KARG_OUT_MAIN: *kind = TKM_ARG_OUT; return;
        case KARG_DOUT_MAIN: *kind = TKM_ARG_DOUT; return;
        case KARG_DIN_MAIN: *kind = TKM_ARG_DIN; return;
        case KARG_BIAS: *kind = (is_prep && bwd) ? TKM_KP_UNUSED : TKM_ARG_BIAS; *node = k; break;
        case KARG_WEIGHT_VEC: *kind = TKM_ARG_WEIGHT; *node = k; break;
        case KARG_BETA: *kind = TKM_ARG_BETA; *node = k; break;
        case KARG_SAVE_ISTD: *kind = TKM_ARG_SAVE_ISTD; *node = k; break;
        case KARG_SAVE_XHAT: *kind = TKM_ARG_SAVE_XHAT; *node = k; break;
        case KARG_SAVE_MASK: *kind = TKM_ARG_SAVE_MASK; *node = k; break;
        case KARG_STEP_SEED: *kind = TKM_ARG_SEED; *node = k; break;
        case KARG_BRANCH_IN:
        case KARG_DBRANCH_OUT:
            /* node_id is the Add's branch source (its in1): find the Add */
            *kind = a->kind == KARG_BRANCH_IN ? TKM_ARG_BRANCH_IN : TKM_ARG_DBRANCH;
            for (int i = 0; i < nm; ++i)
                if (g->nodes[map[i]].op == OP_ADD && g->nodes[map[i]].in1 == a->node_id) *node = i;
            return;
        default: *kind = TKM_KP_UNUSED; return;  /* d(param): written by the reduce kernel */
    }
    if (*node < 0) *kind = TKM_KP_UNUSED;
}

static const char *internal_prefix(int kind) {
    switch (kind) {
        case TKM_ARG_BRANCH_IN: return "x_branch";
        case TKM_ARG_DBRANCH: return "x_dbranch";
        case TKM_ARG_SAVE_MASK: return "x_mask";
        case TKM_ARG_SEED: return "x_seed";
        case TKM_ARG_WEIGHT: return "x_w";
        case TKM_ARG_BIAS: return "x_bias";
        case TKM_ARG_BETA: return "x_beta";
        case TKM_ARG_SAVE_XHAT: return "x_xhat";
        case TKM_ARG_SAVE_ISTD: return "x_istd";
        default: return "x_arg";
    }
}

int tkm_hip_group_plan(const TkmGraph *g, int gid, int pass, int dtype, tkm_kplan *plan, int *chain_nodes,
                       int *n_chain) {
    const int kind = tkm_hip_group_kind(g, gid);
    if (kind < 0) return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "group %d has no HIP kernels (coordinate group)", gid);
    const PlasmaGroup *pg = &g->groups[gid];
    int map[3 * TKM_PLASMA_MAX_NODES], nm = 0, rc;
    tkm_kparam need[TKM_KPLAN_MAX];
    int n_need;
    if (kind == TKM_HIP_GROUP_PREP) {
        tkm_prep_desc d;
        rc = tkm_hip_prep_desc(g, gid, dtype, &d);
        if (rc) return rc;
        map[nm++] = pg->node_ids[0];
        n_need = tkm_prep_need(pass, need);
    } else {
        tkm_plasma_desc d;
        rc = tkm_hip_plasma_desc(g, gid, dtype, &d, map);
        if (rc) return rc;
        nm = d.twin ? d.n_left + d.n_right + d.n_main : d.n_main;
        n_need = tkm_plasma_need(&d, pass, need);
    }
    const TkmKernelSig *sig = pass ? &pg->bwd_sig : &pg->fwd_sig;
    plan->n = 0;
    for (int i = 0; i < sig->num_args; ++i) {
        int k, node;
        sig_to_internal(g, &sig->args[i], map, nm, kind == TKM_HIP_GROUP_PREP, pass, &k, &node);
        /* an internal argument the kernel does not read is passed but unused */
        int used = 0;
        for (int j = 0; j < n_need && k != TKM_KP_UNUSED; ++j)
            if (need[j].kind == k && need[j].node == node) used = 1;
        if (!used) {
            k = TKM_KP_UNUSED;
            node = -1;
        }
        for (int j = 0; j < plan->n && k != TKM_KP_UNUSED; ++j)
            if (plan->p[j].kind == k && plan->p[j].node == node) k = TKM_KP_UNUSED;  /* listed twice */
        if (tkm_kplan_add(plan, k, k == TKM_KP_UNUSED ? -1 : node, sig->args[i].c_type, sig->args[i].c_name))
            return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "group %d: too many kernel parameters", gid);
    }
    /* extras: internal arguments the signature does not carry */
    for (int j = 0; j < n_need; ++j) {
        int found = 0;
        for (int i = 0; i < plan->n; ++i)
            if (plan->p[i].kind == need[j].kind && plan->p[i].node == need[j].node) found = 1;
        if (found) continue;
        char name[40];
        if (need[j].kind >= TKM_KP_ROWS) snprintf(name, sizeof name, "%s", need[j].name);
        else if (need[j].node < 0) snprintf(name, sizeof name, "x_%s", need[j].name);
        else snprintf(name, sizeof name, "%s_%d", internal_prefix(need[j].kind), need[j].node);
        if (tkm_kplan_add(plan, need[j].kind, need[j].node, need[j].decl, name))
            return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "group %d: too many kernel parameters", gid);
    }
    if (chain_nodes)
        for (int i = 0; i < nm; ++i) chain_nodes[i] = map[i];
    if (n_chain) *n_chain = nm;
    return TKM_ATTN_OK;
}

char *tkm_codegen_hip_source(const TkmGraph *g, int dtype) {
    if (!g) {
        tkm_set_error(TKM_ATTN_EINVAL, "tkm_codegen_hip_source: graph is NULL");
        return NULL;
    }
    tkm_sbuf s = {0};
    tkm_sb_add(&s, "/* generated by tkm_codegen_hip.c: %d groups, %s */\n\n", g->num_groups,
               dtype == TKM_ATTN_BF16 ? "bf16" : "fp16");
    for (int gid = 0; gid < g->num_groups; ++gid) {
        const int kind = tkm_hip_group_kind(g, gid);
        if (kind < 0) {
            tkm_sb_add(&s, "/* group %d: coordinate/augmentation group, no HIP kernels in this build */\n\n", gid);
            continue;
        }
        tkm_kplan fp, bp;
        int rc = tkm_hip_group_plan(g, gid, 0, dtype, &fp, NULL, NULL);
        if (!rc) rc = tkm_hip_group_plan(g, gid, 1, dtype, &bp, NULL, NULL);
        if (!rc) {
            if (kind == TKM_HIP_GROUP_PREP) {
                tkm_prep_desc d;
                rc = tkm_hip_prep_desc(g, gid, dtype, &d);
                if (!rc) rc = tkm_prep_emit(&s, &d, &fp, &bp, 1);
            } else {
                tkm_plasma_desc d;
                int map[3 * TKM_PLASMA_MAX_NODES];
                tkm_plasma_formula f[3 * TKM_PLASMA_MAX_NODES];
                rc = tkm_hip_plasma_desc(g, gid, dtype, &d, map);
                if (!rc) {
                    group_formulas(g, &d, map, d.twin ? d.n_left + d.n_right + d.n_main : d.n_main, f);
                    rc = tkm_plasma_emit(&s, &d, &fp, &bp, 1, f);
                }
            }
        }
        if (rc) {
            free(s.buf);
            return NULL;
        }
    }
    if (s.failed) {
        free(s.buf);
        tkm_set_error(TKM_ATTN_EINVAL, "out of host memory while emitting source");
        return NULL;
    }
    return s.buf;
}

char *tkm_codegen_cuda_string(const TkmGraph *g) {
    char *src = tkm_codegen_hip_source(g, TKM_ATTN_F16);
    if (!src) fprintf(stderr, "[TKM HIP] code generation failed: %s\n", tkm_attn_last_error());
    return src;
}
