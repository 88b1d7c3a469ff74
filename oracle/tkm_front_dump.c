/*
 * tkm_front_dump.c -- test infrastructure (not product code).
 *
 * Linked with the reference's unchanged front end (src/tkm_core.c, src/tkm_registry.c,
 * src/tkm_codegen.c, compiled from /root/reference by oracle/Makefile's `ref` target into
 * oracle/_ref/), it writes the fixtures that pin this build's runtime (tkm_hip.c) and HIP code
 * generator against the reference's graph IR:
 *
 *   tkm_front_dump graph <model.tkm> <batch> <out_prefix>
 *       runs tkm_parse_dsl -> tkm_optimize_and_bind -> tkm_plan_memory (the path of the
 *       reference's tkm_load_buffer, src/tkm_gpu.cu:1428-1448) and writes <out_prefix>.bin
 *       (the TkmGraph struct, byte for byte) and <out_prefix>.json (nodes, groups and their
 *       TkmKernelSig argument lists and grids)
 *   tkm_front_dump registry
 *       prints the op registry (index, name, op, category, resource flags, default constant)
 *   tkm_front_dump layout
 *       prints sizeof / offsetof of every struct of tkm.h (also built against this build's
 *       include/tkm.h by the CPU tests, which compare the two)
 */
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tkm.h"

#ifndef TKM_LAYOUT_ONLY

static char *read_file(const char *path) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    char *s = (char *)malloc((size_t)n + 1);
    if (fread(s, 1, (size_t)n, f) != (size_t)n) {
        fclose(f);
        free(s);
        return NULL;
    }
    s[n] = '\0';
    fclose(f);
    return s;
}

static void json_str(FILE *o, const char *s) {
    fputc('"', o);
    for (; *s; s++) {
        if (*s == '"' || *s == '\\') fputc('\\', o);
        if (*s == '\n') { fputs("\\n", o); continue; }
        fputc(*s, o);
    }
    fputc('"', o);
}

static void dump_sig(FILE *o, const TkmKernelSig *s) {
    fprintf(o, "{\"func_name\": ");
    json_str(o, s->func_name);
    fprintf(o, ", \"grid_x\": %d, \"block_x\": %d, \"args\": [", s->grid_x, s->block_x);
    for (int i = 0; i < s->num_args; i++) {
        const TkmKernelArg *a = &s->args[i];
        fprintf(o, "%s{\"kind\": %d, \"node_id\": %d, \"c_type\": ", i ? ", " : "", (int)a->kind, a->node_id);
        json_str(o, a->c_type);
        fprintf(o, ", \"c_name\": ");
        json_str(o, a->c_name);
        fprintf(o, "}");
    }
    fprintf(o, "]}");
}

static int dump_graph(const char *path, int batch, const char *prefix) {
    char *text = read_file(path);
    if (!text) {
        fprintf(stderr, "cannot read %s\n", path);
        return 1;
    }
    TkmGraph *g = (TkmGraph *)calloc(1, sizeof(TkmGraph));
    tkm_parse_dsl(g, text, batch);
    tkm_optimize_and_bind(g);
    tkm_plan_memory(g);

    char fn[1024];
    snprintf(fn, sizeof fn, "%s.bin", prefix);
    FILE *b = fopen(fn, "wb");
    fwrite(g, sizeof(TkmGraph), 1, b);
    fclose(b);

    snprintf(fn, sizeof fn, "%s.json", prefix);
    FILE *o = fopen(fn, "w");
    fprintf(o, "{\"num_nodes\": %d, \"num_groups\": %d, \"batch_size\": %d, \"default_rng\": %d, "
               "\"total_arena_bytes\": %zu, \"naive_arena_bytes\": %zu, \"sizeof_graph\": %zu,\n",
            g->num_nodes, g->num_groups, g->batch_size, (int)g->default_rng, g->total_arena_bytes,
            g->naive_arena_bytes, sizeof(TkmGraph));
    fprintf(o, "\"nodes\": [\n");
    for (int i = 0; i < g->num_nodes; i++) {
        const TkmNode *n = &g->nodes[i];
        fprintf(o, "%s{\"id\": %d, \"spec_id\": %d, \"tag\": ", i ? ",\n" : "", n->id, n->spec_id);
        json_str(o, n->tag);
        fprintf(o, ", \"op\": %d, \"cat\": %d, \"dead\": %d, \"in0\": %d, \"in1\": %d, \"in2\": %d, "
                   "\"users\": %d, \"plasma_grp\": %d, \"c_out\": %d, \"q_c\": %d, \"k_c\": %d, \"v_c\": %d, "
                   "\"q_heads\": %d, \"kv_heads\": %d, \"head_dim\": %d, \"has_qknorm\": %d, \"has_rope\": %d, "
                   "\"causal\": %d, \"fval\": %.9g, \"fval2\": %.9g, \"rope_theta\": %.9g, \"rope_scale\": %.9g, "
                   "\"rope_low_freq_factor\": %.9g, \"rope_high_freq_factor\": %.9g, "
                   "\"rope_original_context_length\": %.9g, \"rng_type\": %d, \"H\": %d, \"W\": %d, \"C\": %d, "
                   "\"out_buf_id\": %d, \"out_offset\": %zu, \"out_bytes\": %zu, \"left\": [",
                (int)n->op, (int)n->cat, n->dead, n->in0, n->in1, n->in2, n->users, n->plasma_grp,
                n->c_out, n->q_c, n->k_c, n->v_c, n->q_heads, n->kv_heads, n->head_dim, n->has_qknorm,
                n->has_rope, n->causal, n->fval, n->fval2, n->rope_theta, n->rope_scale,
                n->rope_low_freq_factor, n->rope_high_freq_factor, n->rope_original_context_length,
                (int)n->rng_type, n->H, n->W, n->C, n->out_buf_id, n->out_offset, n->out_bytes);
        for (int k = 0; k < n->left_len; k++) fprintf(o, "%s%d", k ? ", " : "", n->left_nodes[k]);
        fprintf(o, "], \"right\": [");
        for (int k = 0; k < n->right_len; k++) fprintf(o, "%s%d", k ? ", " : "", n->right_nodes[k]);
        fprintf(o, "]}");
    }
    fprintf(o, "],\n\"groups\": [\n");
    for (int i = 0; i < g->num_groups; i++) {
        const PlasmaGroup *pg = &g->groups[i];
        fprintf(o, "%s{\"id\": %d, \"anchor_id\": %d, \"nodes\": [", i ? ",\n" : "", pg->id, pg->anchor_id);
        for (int k = 0; k < pg->count; k++) fprintf(o, "%s%d", k ? ", " : "", pg->node_ids[k]);
        fprintf(o, "], \"has_norm\": %d, \"is_twin_epilogue\": %d, \"is_coord_group\": %d, "
                   "\"is_qkv_prep\": %d, \"use_reflect_border\": %d, \"out_node_id\": %d, "
                   "\"H\": %d, \"W\": %d, \"C\": %d, \"fwd_sig\": ",
                pg->has_norm, pg->is_twin_epilogue, pg->is_coord_group, pg->is_qkv_prep,
                pg->use_reflect_border, pg->out_node_id, pg->H, pg->W, pg->C);
        dump_sig(o, &pg->fwd_sig);
        fprintf(o, ", \"bwd_sig\": ");
        dump_sig(o, &pg->bwd_sig);
        fprintf(o, "}");
    }
    fprintf(o, "]}\n");
    fclose(o);
    free(g);
    free(text);
    return 0;
}

static int dump_registry(void) {
    printf("[\n");
    for (int i = 0; i < tkm_get_spec_count(); i++) {
        const TkmOpSpec *s = tkm_find_spec_by_index(i);
        printf("%s{\"index\": %d, \"name\": ", i ? ",\n" : "", i);
        json_str(stdout, s->dsl_name);
        printf(", \"op\": %d, \"cat\": %d, \"res_flags\": %u, \"default_fval\": %.9g, "
               "\"fwd_cuda\": %d, \"fwd_expr\": %d}",
               (int)s->op, (int)s->cat, s->res_flags, s->default_fval, s->fwd_cuda != NULL,
               s->fwd_expr != NULL);
    }
    printf("]\n");
    return 0;
}
#endif /* TKM_LAYOUT_ONLY */

#define F(T, m) printf("  \"%s.%s\": [%zu, %zu],\n", #T, #m, offsetof(T, m), sizeof(((T *)0)->m))
static int dump_layout(void) {
    printf("{\n");
    printf("  \"sizeof.TkmOpSpec\": %zu, \"sizeof.TkmKernelArg\": %zu, \"sizeof.TkmKernelSig\": %zu,\n",
           sizeof(TkmOpSpec), sizeof(TkmKernelArg), sizeof(TkmKernelSig));
    printf("  \"sizeof.TkmNode\": %zu, \"sizeof.PlasmaGroup\": %zu, \"sizeof.TkmGraph\": %zu,\n",
           sizeof(TkmNode), sizeof(PlasmaGroup), sizeof(TkmGraph));
    printf("  \"sizeof.TkmFusionRule\": %zu,\n", sizeof(TkmFusionRule));
    F(TkmOpSpec, op); F(TkmOpSpec, dsl_name); F(TkmOpSpec, cat); F(TkmOpSpec, res_flags);
    F(TkmOpSpec, default_fval); F(TkmOpSpec, fwd_cuda); F(TkmOpSpec, bwd_cuda); F(TkmOpSpec, fwd_expr);
    F(TkmOpSpec, bwd_expr);
    F(TkmKernelArg, kind); F(TkmKernelArg, node_id); F(TkmKernelArg, c_type); F(TkmKernelArg, c_name);
    F(TkmKernelSig, func_name); F(TkmKernelSig, args); F(TkmKernelSig, num_args); F(TkmKernelSig, grid_x);
    F(TkmKernelSig, block_x);
    F(TkmNode, id); F(TkmNode, spec_id); F(TkmNode, tag); F(TkmNode, op); F(TkmNode, cat); F(TkmNode, dead);
    F(TkmNode, in0); F(TkmNode, in1); F(TkmNode, in2); F(TkmNode, users); F(TkmNode, plasma_grp);
    F(TkmNode, c_out); F(TkmNode, k); F(TkmNode, s); F(TkmNode, p); F(TkmNode, q_c); F(TkmNode, k_c);
    F(TkmNode, v_c); F(TkmNode, q_heads); F(TkmNode, kv_heads); F(TkmNode, head_dim);
    F(TkmNode, has_qknorm); F(TkmNode, has_rope); F(TkmNode, causal); F(TkmNode, qkv_prep_nid);
    F(TkmNode, fval); F(TkmNode, fval2); F(TkmNode, rope_theta); F(TkmNode, rope_scale);
    F(TkmNode, rope_low_freq_factor); F(TkmNode, rope_high_freq_factor);
    F(TkmNode, rope_original_context_length); F(TkmNode, rng_type); F(TkmNode, left_nodes);
    F(TkmNode, left_len); F(TkmNode, right_nodes); F(TkmNode, right_len); F(TkmNode, H); F(TkmNode, W);
    F(TkmNode, C); F(TkmNode, out_buf_id); F(TkmNode, out_offset); F(TkmNode, out_bytes);
    F(PlasmaGroup, id); F(PlasmaGroup, anchor_id); F(PlasmaGroup, node_ids); F(PlasmaGroup, count);
    F(PlasmaGroup, has_norm); F(PlasmaGroup, is_twin_epilogue); F(PlasmaGroup, is_coord_group);
    F(PlasmaGroup, is_qkv_prep); F(PlasmaGroup, use_reflect_border); F(PlasmaGroup, out_node_id);
    F(PlasmaGroup, H); F(PlasmaGroup, W); F(PlasmaGroup, C); F(PlasmaGroup, fwd_sig); F(PlasmaGroup, bwd_sig);
    F(TkmGraph, nodes); F(TkmGraph, num_nodes); F(TkmGraph, groups); F(TkmGraph, num_groups);
    F(TkmGraph, batch_size); F(TkmGraph, default_rng); F(TkmGraph, total_arena_bytes);
    F(TkmGraph, naive_arena_bytes);
    F(TkmFusionRule, name); F(TkmFusionRule, match); F(TkmFusionRule, apply);
    printf("  \"enum.OP_COUNT\": [%d, 0], \"enum.OP_GQA_ATTN\": [%d, 0], \"enum.OP_DROP\": [%d, 0],\n",
           (int)OP_COUNT, (int)OP_GQA_ATTN, (int)OP_DROP);
    printf("  \"enum.KARG_STEP_SEED\": [%d, 0], \"enum.RES_AUG_COLOR\": [%d, 0], \"enum.CAT_FLUID\": [%d, 0],\n",
           (int)KARG_STEP_SEED, (int)RES_AUG_COLOR, (int)CAT_FLUID);
    printf("  \"enum.RNG_PHILOX\": [%d, 0], \"const.TKM_MAX_KARGS\": [%d, 0], \"const.TKM_MAX_GROUPS\": [%d, 0]\n",
           (int)RNG_PHILOX, TKM_MAX_KARGS, TKM_MAX_GROUPS);
    printf("}\n");
    return 0;
}

int main(int argc, char **argv) {
    if (argc >= 2 && !strcmp(argv[1], "layout")) return dump_layout();
#ifndef TKM_LAYOUT_ONLY
    if (argc >= 2 && !strcmp(argv[1], "registry")) return dump_registry();
    if (argc >= 5 && !strcmp(argv[1], "graph")) return dump_graph(argv[2], atoi(argv[3]), argv[4]);
#endif
    fprintf(stderr, "usage: %s layout | registry | graph <model.tkm> <batch> <out_prefix>\n", argv[0]);
    return 2;
}
