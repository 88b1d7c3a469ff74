/*
 * tkm_hip.c -- the HIP runtime behind the public API of tkm.h (section 5) on one MI355X
 * (gfx950).  It replaces the host half of the reference's src/tkm_gpu.cu:
 *
 *   ignite: module, arena, parameters, saved state   tkm_gpu.cu:901-1140
 *   forward node walk                                tkm_gpu.cu:1176-1289
 *   recorded step (clear, forward, backward, SGD)    tkm_gpu.cu:1291-1421
 *   load / step / eval / forward / probes / I/O      tkm_gpu.cu:1423-1999
 *
 * with this build's kernels: the generated qkv-prep and plasma epilogues (tkm_codegen_hip.c,
 * compiled by hipRTC for gfx950), the attention kernels (include/tkm_attn.h), hipBLASLt GEMMs
 * (tkm_gemm.hip) and the runtime's own kernels (tkm_rt_kernels.hip).  The step is captured
 * once into a hipGraph and replayed, as the reference does.  Host code is C; HIP is called
 * through its C API.
 *
 * Scope: the transformer family of the op set (FC and its fused twin / QKV forms, GQA
 * attention, every row-wise epilogue op including Drop, Softmax and the three softmax losses,
 * Flatten).  The CNN family (Conv, MixPool, AvgPool and the coordinate / augmentation groups)
 * is outside the attention path this build serves: ignite names the first such node and
 * returns NULL.
 *
 * Differences from the reference, on purpose:
 *   - labels may be int32 per row (tkm_hip.h), and activations bf16, both opt-in;
 *   - parameter gradients, losses and accuracy counts are reduced in a fixed order (no float
 *     atomics), so a step is bitwise reproducible;
 *   - the per-step clears are fill kernels (no memset nodes in the step graph);
 *   - weights are initialized from a seeded PCG32 (Box-Muller), not the C library's rand();
 *   - HIP and hipBLASLt failures are reported (stderr) and make the call fail instead of
 *     exit(1) where the API can return a failure; the reference's float-returning calls return
 *     NAN then.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "tkm.h"
#include "tkm_attn.h"
#include "tkm_codegen_internal.h"
#include "tkm_gemm.h"
#include "tkm_hip.h"
#include "tkm_plasma_internal.h"
#include "tkm_prep_internal.h"
#include "tkm_rt_kernels.h"

/* The front end (the reference's src/tkm_core.c) is linked in by the application; the
 * tkm_load_* functions need it, everything else takes a TkmGraph. */
#pragma weak tkm_parse_dsl
#pragma weak tkm_optimize_and_bind
#pragma weak tkm_plan_memory
#pragma weak tkm_find_spec_by_node

#define TKM_GEMM_MAX_WS (64u << 20)
#define TKM_ALIGN(x) (((x) + 255) & ~(size_t)255)

enum { T_GEMM_W = 0, T_BIAS = 1, T_WVEC = 2, T_BETA = 3 };

typedef struct {
    float *master, *vel, *grad;
    void *w16;
    size_t n;
    int node, kind;
} rt_tensor;

typedef struct {
    int in_dim, out_dim, rows;
    int t_w, t_bias, t_wvec, t_beta;   /* tensor indices, -1 if none */
    float *istd;
    void *xhat;
    void *mask;
    float *lse;
    tkm_gemm *g_fwd, *g_dw, *g_dx;
    int dx_first;                       /* GEMM dX is the first writer of grad(in0): beta 0 */
} rt_node;

typedef struct {
    int kind;                           /* TKM_HIP_GROUP_*, or -1 */
    void *fwd, *bwd, *reduce;           /* hipFunction_t */
    tkm_kplan plan[2];
    int chain[3 * TKM_PLASMA_MAX_NODES], n_chain;
    int rows, twin;
    int din_first, branch_first;        /* first writer of the gradient slot: overwrite instead of += */
    unsigned gx, gy_fwd, bands, band, gx_red;
    int n_par;                          /* reduce targets (plasma: geometry order; prep: dbias, dgamma) */
    int par_kind[3 * 3 * TKM_PLASMA_MAX_NODES], par_node[3 * 3 * TKM_PLASMA_MAX_NODES];
    size_t part_bytes, part_off;        /* this group's band partials in the partials block */
    int pw, chan;                       /* partial row width; channels (prep: C, then QK) */
} rt_group;

struct TkmRuntime {
    TkmGraph graph;
    tkm_runtime_opts opts;
    int dt, training;
    hipStream_t stream;
    /* Training: the weight-gradient GEMMs run on `side` with their own workspace, forked from
     * `stream` at each GEMM node of the backward walk and joined before the reductions. */
    hipStream_t side;
    hipEvent_t ev_fork, ev_join;
    void *lt;
    void *gemm_ws, *gemm_ws_side;
    size_t gemm_ws_bytes;
    hipModule_t module;
    rt_group *groups;
    rt_node *nodes;
    rt_tensor *tensors;
    int n_tensors;
    long long total_elems, sgd_blocks;
    size_t (*clear)[2];                 /* gradient-arena ranges (offset, bytes) a step clears */
    int n_clear;
    TkmSgdTensor *d_sgd;
    void *param_block;           /* masters, velocities, GEMM gradients, 16-bit copies */
    float *pgrad_block;          /* gradients of the parameter vectors: cleared each step */
    size_t pgrad_bytes;
    void *save_block;
    uint8_t *arena, *grad_arena;
    float *d_input_f32;
    size_t in_elems;
    void *d_labels;
    size_t n_labels;
    float *d_lr, *d_loss, *d_epoch_loss;
    int *d_correct;
    uint32_t *d_seed;
    float *row_loss;
    int *row_correct;
    void *attn_ws;
    size_t attn_ws_bytes;
    void *part_ws;
    size_t part_ws_bytes;
    TkmReduceChunk *d_red;              /* parameter-gradient reductions, one launch per step */
    int n_red;
    float *h_pin_lr, *h_pin_loss;
    hipGraph_t step_graph[2];        /* [0] clears the loss, [1] accumulates it (epochs) */
    hipGraphExec_t step_exec[2];
    float *d_out_f32;                /* tkm_runtime_forward's fp32 copy of the output node */
    float *h_stage_in;               /* pinned batch staging of the callback loops */
    uint8_t *h_stage_lbl;
    float last_lr;
    int kernel_count, counting;
    int failed;                      /* a launch failed while recording */
};

struct TkmDataset {
    TkmRuntime *rt;
    const float *h_images;           /* caller-owned, NHWC fp32, and one uint8 label per sample */
    const uint8_t *h_labels;
    size_t num_samples, sample_elems;
    int resident;
    uint32_t *h_order;               /* pinned: the epoch's sample order */
    /* resident: the samples in the runtime's 16-bit type, the labels, the order */
    void *d_images;
    uint8_t *d_labels;
    uint32_t *d_order;
    /* streaming: two staging slots (pinned host rows and labels, their device copies), filled
     * on the host while the other slot's batch runs; `copy` moves a slot to the device while
     * `rt->stream` trains on the previous one */
    float *h_in[2], *d_in[2];
    uint8_t *h_lbl[2], *d_lbl[2];
    hipStream_t copy;
    hipEvent_t copied[2], consumed[2];
    int used[2];
};

/* ---- errors ------------------------------------------------------------------------------ */

static int hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return 1;
    fprintf(stderr, "[TKM HIP] %s failed: %s\n", what, hipGetErrorString(e));
    return 0;
}
#define HIP_OK(call) hip_ok((call), #call)

static void note(TkmRuntime *rt, int rc, const char *what) {
    if (rc != 0) {
        if (!rt->failed) fprintf(stderr, "[TKM HIP] %s failed: %s\n", what, tkm_attn_last_error());
        rt->failed = 1;
    }
    if (rt->counting) rt->kernel_count++;
}

/* Work enqueued on `waiter` from now on runs after everything enqueued on `on` so far. */
static void depend(TkmRuntime *rt, hipStream_t waiter, hipStream_t on, hipEvent_t ev) {
    if (!HIP_OK(hipEventRecord(ev, on)) || !HIP_OK(hipStreamWaitEvent(waiter, ev, 0))) rt->failed = 1;
}

/* ---- op resources (the registry's resource flags, src/tkm_registry.c:43-456) -------------- */

uint32_t tkm_hip_res_flags(const TkmNode *n) {
    /* with the front end linked, the registry's own flags (equal for every op this table
     * knows: tests/test_tkm_runtime_cpu.py; also those of ops it does not) */
    const TkmOpSpec *sp = tkm_find_spec_by_node ? tkm_find_spec_by_node(n) : NULL;
    if (sp) return sp->res_flags;
    switch (n->op) {
        case OP_BN: case OP_LN: return RES_PARAM_WEIGHT | RES_PARAM_BETA | RES_SAVE_ISTD | RES_SAVE_XHAT;
        case OP_RMSNORM: return RES_PARAM_WEIGHT | RES_SAVE_ISTD | RES_SAVE_XHAT;
        case OP_L2NORM: return RES_SAVE_ISTD | RES_SAVE_XHAT;
        case OP_QKNORM: return RES_PARAM_BIAS | RES_PARAM_WEIGHT | RES_SAVE_ISTD | RES_SAVE_XHAT;
        case OP_BIAS: return RES_PARAM_BIAS;
        case OP_LAYERSCALE: case OP_DYT: case OP_PRELU: case OP_XATLU: return RES_PARAM_WEIGHT;
        case OP_DROP: return RES_SAVE_MASK | RES_RNG_SEED;
        case OP_ADD: return RES_BRANCH_IN;
        case OP_RAND_SHIFT: case OP_RAND_ROTATE: case OP_RAND_SCALE: case OP_RAND_FLIPX: case OP_RAND_FLIPY:
        case OP_RAND_ELASTIC: return RES_RNG_SEED;
        case OP_RAND_NOISE: case OP_RAND_CUTOUT: case OP_RAND_BRIGHTNESS: case OP_RAND_CONTRAST:
        case OP_RAND_SOLARIZE: case OP_RAND_ERASING: return RES_RNG_SEED | RES_AUG_PIXEL;
        case OP_RAND_SATURATION: case OP_RAND_HUE: case OP_RAND_GRAYSCALE: case OP_RAND_CHANNEL_SCALE:
            return RES_RNG_SEED | RES_AUG_COLOR;
        default: return RES_NONE;
    }
}

static int is_gemm(TkmOpType op) { return op == OP_FC || op == OP_FC_TWIN_FUSED || op == OP_FC_QKV_FUSED; }
static int is_loss(TkmOpType op) { return op == OP_SOFTMAX_CE || op == OP_SOFTMAX_FOCAL || op == OP_SOFTMAX_MSE; }

/* ---- weight initialization: PCG32 (O'Neill) + Box-Muller ---------------------------------- */

typedef struct {
    uint64_t state, inc;
} pcg32;

static uint32_t pcg_next(pcg32 *r) {
    const uint64_t old = r->state;
    r->state = old * 6364136223846793005ULL + r->inc;
    const uint32_t xsh = (uint32_t)(((old >> 18u) ^ old) >> 27u), rot = (uint32_t)(old >> 59u);
    return (xsh >> rot) | (xsh << ((32u - rot) & 31u));
}

static void pcg_seed(pcg32 *r, uint64_t seed, uint64_t seq) {
    r->state = 0;
    r->inc = (seq << 1u) | 1u;
    (void)pcg_next(r);
    r->state += seed;
    (void)pcg_next(r);
}

static void init_values(float *h, size_t n, float scale, float value, uint64_t seed, int index) {
    if (scale <= 0.0f) {
        for (size_t i = 0; i < n; ++i) h[i] = value;
        return;
    }
    pcg32 r;
    pcg_seed(&r, seed, (uint64_t)index + 1);
    for (size_t i = 0; i < n; ++i) {
        const double u1 = ((pcg_next(&r) >> 8) + 1.0) / 16777216.0, u2 = (pcg_next(&r) >> 8) / 16777216.0;
        h[i] = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2)) * scale;
    }
}

/* ---- graph checks ------------------------------------------------------------------------- */

static int check_graph(const TkmGraph *g) {
    if (g->num_nodes < 1 || g->num_nodes > TKM_MAX_NODES || g->num_groups < 0 || g->num_groups > TKM_MAX_GROUPS ||
        g->batch_size < 1) {
        fprintf(stderr, "[TKM HIP] malformed graph (%d nodes, %d groups, batch %d)\n", g->num_nodes, g->num_groups,
                g->batch_size);
        return 0;
    }
    for (int i = 1; i < g->num_nodes; ++i) {
        const TkmNode *n = &g->nodes[i];
        if (n->dead) continue;
        if (n->plasma_grp >= 0) {
            if (n->plasma_grp >= g->num_groups || tkm_hip_group_kind(g, n->plasma_grp) < 0) {
                fprintf(stderr, "[TKM HIP] node #%d (%s) is in a coordinate/augmentation group: the CNN family is "
                        "outside this runtime\n", i, n->tag);
                return 0;
            }
            continue;
        }
        if (is_gemm(n->op) || n->op == OP_GQA_ATTN || n->op == OP_FLATTEN || n->op == OP_SOFTMAX || is_loss(n->op))
            continue;
        fprintf(stderr, "[TKM HIP] node #%d (%s, op %d) has no HIP implementation here: the CNN family "
                "(Conv, pooling, augmentation) is outside this runtime\n", i, n->tag, (int)n->op);
        return 0;
    }
    return 1;
}

/* ---- ignite ------------------------------------------------------------------------------- */

void tkm_runtime_opts_init(tkm_runtime_opts *o) {
    if (!o) return;
    memset(o, 0, sizeof *o);
    o->dtype = TKM_ATTN_F16;
    o->training = 1;
    o->init_seed = 0x7417u;
    o->verbose = 1;
}

static size_t rows_of(const TkmGraph *g, const TkmNode *n) { return (size_t)g->batch_size * n->H * n->W; }

/* Allocates the learnable tensors in TKM1 order: every node (dead ones too, as the reference
 * does: src/tkm_gpu.cu:1109-1118), a GEMM's weight, then bias, weight vector and beta. */
static int alloc_params(TkmRuntime *rt) {
    const TkmGraph *g = &rt->graph;
    int cap = 4 * g->num_nodes + 4, nt = 0;
    rt->tensors = (rt_tensor *)calloc((size_t)cap, sizeof(rt_tensor));
    if (!rt->tensors) return 0;
    size_t master_bytes = 0, w16_bytes = 0, gemm_grad_bytes = 0, pgrad = 0;
    for (int pass = 0; pass < 2; ++pass) {
        nt = 0;
        size_t mo = 0, w16o = 0, ggo = 0, pgo = 0;
        for (int i = 0; i < g->num_nodes; ++i) {
            const TkmNode *n = &g->nodes[i];
            rt_node *st = &rt->nodes[i];
            if (pass == 0) st->t_w = st->t_bias = st->t_wvec = st->t_beta = -1;
            if (n->C <= 0) continue;
            int kinds[4], nk = 0;
            size_t sizes[4];
            if (is_gemm(n->op) && n->in0 >= 0) {
                kinds[nk] = T_GEMM_W;
                sizes[nk++] = (size_t)g->nodes[n->in0].C * n->C;
            }
            const uint32_t f = tkm_hip_res_flags(n);
            if (f & RES_PARAM_BIAS) { kinds[nk] = T_BIAS; sizes[nk++] = (size_t)n->C; }
            if (f & RES_PARAM_WEIGHT) { kinds[nk] = T_WVEC; sizes[nk++] = (size_t)n->C; }
            if (f & RES_PARAM_BETA) { kinds[nk] = T_BETA; sizes[nk++] = (size_t)n->C; }
            for (int k = 0; k < nk; ++k, ++nt) {
                rt_tensor *t = &rt->tensors[nt];
                const size_t b = TKM_ALIGN(sizes[k] * sizeof(float));
                if (pass == 1) {
                    uint8_t *base = (uint8_t *)rt->param_block;
                    t->n = sizes[k];
                    t->node = i;
                    t->kind = kinds[k];
                    t->master = (float *)(base + mo);
                    t->vel = (float *)(base + master_bytes + mo);
                    if (kinds[k] == T_GEMM_W) {
                        t->grad = (float *)(base + 2 * master_bytes + ggo);
                        t->w16 = base + 2 * master_bytes + gemm_grad_bytes + w16o;
                    } else {
                        t->grad = (float *)((uint8_t *)rt->pgrad_block + pgo);
                        t->w16 = NULL;
                    }
                    if (kinds[k] == T_GEMM_W) st->t_w = nt;
                    if (kinds[k] == T_BIAS) st->t_bias = nt;
                    if (kinds[k] == T_WVEC) st->t_wvec = nt;
                    if (kinds[k] == T_BETA) st->t_beta = nt;
                }
                mo += b;
                if (kinds[k] == T_GEMM_W) {
                    ggo += b;
                    w16o += TKM_ALIGN(sizes[k] * 2);
                } else {
                    pgo += b;
                }
            }
        }
        if (pass == 0) {
            master_bytes = mo;
            w16_bytes = w16o;
            gemm_grad_bytes = ggo;
            pgrad = pgo;
            const size_t total = 2 * master_bytes + gemm_grad_bytes + w16_bytes;
            if (total && !HIP_OK(hipMalloc(&rt->param_block, total))) return 0;
            if (pgrad && !HIP_OK(hipMalloc((void **)&rt->pgrad_block, pgrad))) return 0;
            rt->pgrad_bytes = pgrad;
            if (total && !HIP_OK(hipMemset(rt->param_block, 0, total))) return 0;
            if (pgrad && !HIP_OK(hipMemset(rt->pgrad_block, 0, pgrad))) return 0;
        }
    }
    rt->n_tensors = nt;
    /* initial values (host), uploaded once */
    long long off = 0, blocks = 0;
    TkmSgdTensor *h = (TkmSgdTensor *)calloc((size_t)(nt > 0 ? nt : 1), sizeof(TkmSgdTensor));
    if (!h) return 0;
    for (int k = 0; k < nt; ++k) {
        rt_tensor *t = &rt->tensors[k];
        float *v = (float *)malloc(t->n * sizeof(float));
        if (!v) { free(h); return 0; }
        if (t->kind == T_GEMM_W)
            init_values(v, t->n, sqrtf(2.0f / (float)g->nodes[g->nodes[t->node].in0].C), 0.0f, rt->opts.init_seed, k);
        else
            init_values(v, t->n, 0.0f, t->kind == T_WVEC ? 1.0f : 0.0f, rt->opts.init_seed, k);
        int ok = HIP_OK(hipMemcpy(t->master, v, t->n * sizeof(float), hipMemcpyHostToDevice));
        free(v);
        if (!ok) { free(h); return 0; }
        if (t->w16 && tkm_rt_f32_to_16(t->master, t->w16, t->n, rt->dt, rt->stream)) { free(h); return 0; }
        h[k].master = t->master;
        h[k].w16 = t->w16;
        h[k].vel = t->vel;
        h[k].grad = t->grad;
        h[k].offset = off;
        h[k].size = (long long)t->n;
        h[k].block0 = blocks;
        off += (long long)t->n;
        blocks += ((long long)t->n + TKM_SGD_CHUNK - 1) / TKM_SGD_CHUNK;
    }
    rt->total_elems = off;
    rt->sgd_blocks = blocks;
    if (nt > 0) {
        if (!HIP_OK(hipMalloc((void **)&rt->d_sgd, (size_t)nt * sizeof(TkmSgdTensor))) ||
            !HIP_OK(hipMemcpy(rt->d_sgd, h, (size_t)nt * sizeof(TkmSgdTensor), hipMemcpyHostToDevice))) {
            free(h);
            return 0;
        }
    }
    free(h);
    return HIP_OK(hipStreamSynchronize(rt->stream));
}

/* Saved state of the live nodes, sized for this build's kernels. */
static int alloc_saves(TkmRuntime *rt) {
    const TkmGraph *g = &rt->graph;
    const int bytes16 = 2;
    size_t total = 0;
    for (int pass = 0; pass < 2; ++pass) {
        size_t off = 0;
        for (int i = 0; i < g->num_nodes; ++i) {
            const TkmNode *n = &g->nodes[i];
            rt_node *st = &rt->nodes[i];
            if (n->dead || n->C <= 0) continue;
            const size_t rows = rows_of(g, n);
            size_t b_istd = 0, b_xhat = 0, b_mask = 0, b_lse = 0;
            if (n->op == OP_QKNORM && n->q_c > 0 && n->plasma_grp >= 0) {
                if (n->has_qknorm) {
                    b_istd = rows * (size_t)(n->q_heads + n->kv_heads) * 4;
                    b_xhat = rows * (size_t)(n->q_c + n->k_c) * bytes16;
                }
            } else if (n->op == OP_GQA_ATTN) {
                b_lse = rows * (size_t)n->q_heads * 4;
            } else if (n->plasma_grp >= 0) {
                const uint32_t f = tkm_hip_res_flags(n);
                if (f & RES_SAVE_ISTD) b_istd = rows * (size_t)((n->C + 63) / 64) * 4;
                if (f & RES_SAVE_XHAT) b_xhat = rows * (size_t)n->C * bytes16;
                if (f & RES_SAVE_MASK) b_mask = rows * (size_t)(n->C / 2) * 2;
            }
            uint8_t *base = (uint8_t *)rt->save_block;
            if (b_istd) { if (pass) st->istd = (float *)(base + off); off += TKM_ALIGN(b_istd); }
            if (b_xhat) { if (pass) st->xhat = base + off; off += TKM_ALIGN(b_xhat); }
            if (b_mask) { if (pass) st->mask = base + off; off += TKM_ALIGN(b_mask); }
            if (b_lse) { if (pass) st->lse = (float *)(base + off); off += TKM_ALIGN(b_lse); }
        }
        if (pass == 0) {
            total = off;
            if (total && (!HIP_OK(hipMalloc(&rt->save_block, total)) || !HIP_OK(hipMemset(rt->save_block, 0, total))))
                return 0;
        }
    }
    return 1;
}

/* Which kernel writes each gradient slot first in the backward walk (the order record_step
 * records).  The reference clears the whole gradient arena every step and lets every writer
 * accumulate; here the first writer of a slot overwrites it instead (GEMM dX with beta 0, a
 * group's din or residual gradient without its accumulate flag), and only the slots whose
 * first writer must accumulate, or that are read before any write, are cleared.  A group
 * whose residual Add reads its own anchor (din and the branch gradient land in one slot)
 * keeps accumulating. */
static int plan_grad_writes(TkmRuntime *rt) {
    const TkmGraph *g = &rt->graph;
    if (!rt->training) return 1;
    unsigned char *written = (unsigned char *)calloc((size_t)g->num_nodes, 1);
    unsigned char *clear = (unsigned char *)calloc((size_t)g->num_nodes, 1);
    unsigned char done[TKM_MAX_GROUPS] = {0};
    if (!written || !clear) {
        free(written);
        free(clear);
        return 0;
    }
#define TKM_READ(nid) do { if (!written[nid]) { clear[nid] = 1; written[nid] = 1; } } while (0)
#define TKM_ACCUM(nid) do { if (!written[nid]) { clear[nid] = 1; written[nid] = 1; } } while (0)
    for (int i = 1; i < g->num_nodes; ++i)      /* the loss writes dlogits in the forward walk */
        if (!g->nodes[i].dead && is_loss(g->nodes[i].op)) written[g->nodes[i].in0] = 1;
    for (int i = g->num_nodes - 1; i >= 1; --i) {
        const TkmNode *n = &g->nodes[i];
        if (n->dead || is_loss(n->op)) continue;
        if (n->plasma_grp >= 0) {
            const int gid = n->plasma_grp;
            if (done[gid]) continue;
            done[gid] = 1;
            rt_group *G = &rt->groups[gid];
            const PlasmaGroup *pg = &g->groups[gid];
            G->din_first = G->branch_first = 0;
            if (G->kind < 0) continue;
            TKM_READ(pg->out_node_id);
            const int a = pg->anchor_id;
            int self_branch = 0, n_add = 0, adds_unwritten = 0;
            if (G->kind == TKM_HIP_GROUP_PLASMA)
                for (int k = 0; k < G->n_chain; ++k) {
                    const TkmNode *c = &g->nodes[G->chain[k]];
                    if (c->op != OP_ADD) continue;
                    ++n_add;
                    if (c->in1 == a) self_branch = 1;
                    for (int k2 = 0; k2 < k; ++k2)
                        if (g->nodes[G->chain[k2]].op == OP_ADD && g->nodes[G->chain[k2]].in1 == c->in1) self_branch = 1;
                    if (!written[c->in1]) ++adds_unwritten;
                }
            /* residual gradients (written before din inside the kernel) */
            if (n_add > 0) {
                if (!self_branch && adds_unwritten == n_add) {
                    G->branch_first = 1;
                    for (int k = 0; k < G->n_chain; ++k)
                        if (g->nodes[G->chain[k]].op == OP_ADD) written[g->nodes[G->chain[k]].in1] = 1;
                } else {
                    for (int k = 0; k < G->n_chain; ++k)
                        if (g->nodes[G->chain[k]].op == OP_ADD) TKM_ACCUM(g->nodes[G->chain[k]].in1);
                }
            }
            if (G->kind == TKM_HIP_GROUP_PLASMA && G->twin) {
                written[a] = 1;                 /* a twin group overwrites din */
            } else if (!written[a] && !self_branch) {
                G->din_first = 1;
                written[a] = 1;
            } else {
                TKM_ACCUM(a);
            }
            continue;
        }
        rt_node *st = &rt->nodes[i];
        if (is_gemm(n->op)) {
            TKM_READ(i);
            st->dx_first = !written[n->in0];
            written[n->in0] = 1;
        } else if (n->op == OP_GQA_ATTN) {
            TKM_READ(i);
            written[n->in0] = 1;
        } else if (n->op == OP_FLATTEN) {
            TKM_READ(i);
            if (n->out_offset != g->nodes[n->in0].out_offset) written[n->in0] = 1;
        } else if (n->op == OP_SOFTMAX) {
            TKM_READ(i);
            TKM_ACCUM(n->in0);
        }
    }
#undef TKM_READ
#undef TKM_ACCUM
    /* the slots to clear, as merged byte ranges of the gradient arena */
    rt->clear = (size_t(*)[2])calloc((size_t)g->num_nodes + 1, sizeof *rt->clear);
    int nc = 0;
    if (rt->clear) {
        for (int i = 0; i < g->num_nodes; ++i) {
            if (!clear[i] || g->nodes[i].out_bytes == 0) continue;
            const size_t lo = g->nodes[i].out_offset & ~(size_t)15;
            const size_t hi = (g->nodes[i].out_offset + g->nodes[i].out_bytes + 15) & ~(size_t)15;
            int merged = 0;
            for (int c = 0; c < nc && !merged; ++c)
                if (lo <= rt->clear[c][0] + rt->clear[c][1] && hi >= rt->clear[c][0]) {
                    const size_t a0 = lo < rt->clear[c][0] ? lo : rt->clear[c][0];
                    const size_t a1 = hi > rt->clear[c][0] + rt->clear[c][1] ? hi : rt->clear[c][0] + rt->clear[c][1];
                    rt->clear[c][0] = a0;
                    rt->clear[c][1] = a1 - a0;
                    merged = 1;
                }
            if (!merged) {
                rt->clear[nc][0] = lo;
                rt->clear[nc][1] = hi - lo;
                ++nc;
            }
        }
    }
    rt->n_clear = nc;
    if (rt->clear && rt->opts.clear_all_grads && g->total_arena_bytes >= 4) {
        rt->clear[0][0] = 0;
        rt->clear[0][1] = g->total_arena_bytes & ~(size_t)3;
        rt->n_clear = 1;
    }
    free(written);
    free(clear);
    return rt->clear != NULL;
}

static int plan_gemms(TkmRuntime *rt) {
    const TkmGraph *g = &rt->graph;
    const int ab = rt->dt == TKM_ATTN_BF16 ? TKM_GEMM_BF16 : TKM_GEMM_F16;
    size_t ws = 0;
    for (int i = 1; i < g->num_nodes; ++i) {
        const TkmNode *n = &g->nodes[i];
        if (n->dead || !is_gemm(n->op) || n->plasma_grp >= 0) continue;
        rt_node *st = &rt->nodes[i];
        const int K = g->nodes[n->in0].C, N = n->C, rows = (int)rows_of(g, n);
        st->in_dim = K;
        st->out_dim = N;
        st->rows = rows;
        if (tkm_gemm_create(&st->g_fwd, rt->lt, 0, 0, N, rows, K, N, K, N, ab, ab, 0.0f, TKM_GEMM_MAX_WS)) goto fail;
        if (ws < tkm_gemm_workspace(st->g_fwd)) ws = tkm_gemm_workspace(st->g_fwd);
        if (rt->training) {
            if (tkm_gemm_create(&st->g_dw, rt->lt, 0, 1, N, K, rows, N, K, N, ab, TKM_GEMM_F32, 0.0f, TKM_GEMM_MAX_WS))
                goto fail;
            if (tkm_gemm_create(&st->g_dx, rt->lt, 1, 0, K, rows, N, N, N, K, ab, ab, st->dx_first ? 0.0f : 1.0f,
                                TKM_GEMM_MAX_WS))
                goto fail;
            if (ws < tkm_gemm_workspace(st->g_dw)) ws = tkm_gemm_workspace(st->g_dw);
            if (ws < tkm_gemm_workspace(st->g_dx)) ws = tkm_gemm_workspace(st->g_dx);
        }
        continue;
    fail:
        fprintf(stderr, "[TKM HIP] GEMM of node #%d (%s, %d x %d x %d): %s\n", i, n->tag, N, rows, K,
                tkm_gemm_last_error());
        return 0;
    }
    rt->gemm_ws_bytes = ws;
    if (ws && !HIP_OK(hipMalloc(&rt->gemm_ws, ws))) return 0;
    if (ws && rt->training && !HIP_OK(hipMalloc(&rt->gemm_ws_side, ws))) return 0;
    return 1;
}

static int plan_groups(TkmRuntime *rt) {
    const TkmGraph *g = &rt->graph;
    size_t part = 0;
    for (int gid = 0; gid < g->num_groups; ++gid) {
        rt_group *G = &rt->groups[gid];
        const PlasmaGroup *pg = &g->groups[gid];
        G->kind = tkm_hip_group_kind(g, gid);
        if (G->kind < 0) continue;
        for (int pass = 0; pass < 2; ++pass)
            if (tkm_hip_group_plan(g, gid, pass, rt->dt, &G->plan[pass], G->chain, &G->n_chain)) {
                fprintf(stderr, "[TKM HIP] group %d: %s\n", gid, tkm_attn_last_error());
                return 0;
            }
        G->rows = g->batch_size * pg->H * pg->W;
        char name[96];
        snprintf(name, sizeof name, "tkm_plasma_fwd_g%d", gid);
        if (tkm_rtc_function(rt->module, name, &G->fwd)) return 0;
        snprintf(name, sizeof name, "tkm_plasma_bwd_g%d", gid);
        if (tkm_rtc_function(rt->module, name, &G->bwd)) return 0;
        if (G->kind == TKM_HIP_GROUP_PREP) {
            tkm_prep_desc d;
            tkm_prep_geom geo;
            tkm_hip_prep_desc(g, gid, rt->dt, &d);
            tkm_prep_geometry(&d, &geo);
            G->gx = (unsigned)((geo.CH + 63) / 64);
            G->gy_fwd = (unsigned)((G->rows + 4 * TKM_PREP_FWD_RPW - 1) / (4 * TKM_PREP_FWD_RPW));
            G->bands = (unsigned)tkm_bwd_bands(G->rows, (int)G->gx);
            G->gx_red = (unsigned)((geo.part_width + 63) / 64);
            G->part_bytes = TKM_ALIGN((size_t)G->bands * geo.part_width * sizeof(float));
            G->pw = geo.part_width;
            G->chan = geo.C;
            G->n_par = 1 + (d.has_qknorm ? 1 : 0);
            G->par_kind[0] = TKM_ARG_DBIAS;
            G->par_kind[1] = TKM_ARG_DWEIGHT;
            G->par_node[0] = G->par_node[1] = 0;
        } else {
            tkm_plasma_desc d;
            tkm_plasma_geom geo;
            tkm_hip_plasma_desc(g, gid, rt->dt, &d, NULL);
            tkm_plasma_geometry(&d, &geo);
            G->twin = d.twin;
            G->gx = (unsigned)geo.XB;
            const int rpb = TKM_PLASMA_FWD_RPI * 4 * geo.RW;
            G->gy_fwd = (unsigned)((G->rows + rpb - 1) / rpb);
            G->bands = (unsigned)tkm_bwd_bands(G->rows, geo.XB);
            G->gx_red = (unsigned)((geo.part_width + 63) / 64);
            G->part_bytes = geo.n_par ? TKM_ALIGN((size_t)G->bands * geo.part_width * sizeof(float)) : 0;
            G->pw = geo.part_width;
            G->chan = geo.C;
            G->n_par = geo.n_par;
            for (int p = 0; p < geo.n_par; ++p) {
                G->par_kind[p] = geo.par[p].kind;
                G->par_node[p] = geo.par[p].node;
            }
        }
        G->band = (G->rows + G->bands - 1) / G->bands;
        if (G->n_par > 0) {
            snprintf(name, sizeof name, "tkm_plasma_bwd_g%d_reduce", gid);
            if (tkm_rtc_function(rt->module, name, &G->reduce)) return 0;
        }
        G->part_off = part;                 /* each group's partials stay until the step's reduction */
        part += G->part_bytes;
    }
    rt->part_ws_bytes = part;
    if (part && !HIP_OK(hipMalloc(&rt->part_ws, part))) return 0;
    return 1;
}

static void free_runtime(TkmRuntime *rt);
static int plan_reductions(TkmRuntime *rt);

TkmRuntime *tkm_runtime_ignite_ex(const TkmGraph *g, const char *src, const tkm_runtime_opts *o) {
    if (!g) return NULL;
    tkm_runtime_opts opts;
    if (o) opts = *o;
    else tkm_runtime_opts_init(&opts);
    if (opts.dtype != TKM_ATTN_F16 && opts.dtype != TKM_ATTN_BF16) {
        fprintf(stderr, "[TKM HIP] unknown dtype %d\n", opts.dtype);
        return NULL;
    }
    if (opts.dataset_mode < 0 || opts.dataset_mode > 2) {
        fprintf(stderr, "[TKM HIP] unknown dataset_mode %d\n", opts.dataset_mode);
        return NULL;
    }
    if (!check_graph(g)) return NULL;
    TkmRuntime *rt = (TkmRuntime *)calloc(1, sizeof(TkmRuntime));
    if (!rt) return NULL;
    rt->graph = *g;
    rt->opts = opts;
    rt->dt = opts.dtype;
    rt->training = opts.training ? 1 : 0;
    rt->last_lr = -1.0f;
    rt->nodes = (rt_node *)calloc(TKM_MAX_NODES, sizeof(rt_node));
    rt->groups = (rt_group *)calloc(TKM_MAX_GROUPS, sizeof(rt_group));
    TkmGraph *G = &rt->graph;
    char *own_src = NULL;
    if (!rt->nodes || !rt->groups) goto fail;
    /* a node without a shape takes its input's (src/tkm_gpu.cu:1111-1116) */
    for (int i = 0; i < G->num_nodes; ++i) {
        TkmNode *n = &G->nodes[i];
        if (n->C == 0 && n->in0 >= 0) {
            const TkmNode *p = &G->nodes[n->in0];
            n->H = p->H;
            n->W = p->W;
            n->C = p->c_out > 0 ? p->c_out : p->C;
        }
    }
    if (tkm_attn_init() != TKM_ATTN_OK) {
        fprintf(stderr, "[TKM HIP] %s\n", tkm_attn_last_error());
        goto fail;
    }
    if (!HIP_OK(hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking))) goto fail;
    if (!HIP_OK(hipStreamCreateWithFlags(&rt->side, hipStreamNonBlocking))) goto fail;
    if (!HIP_OK(hipEventCreateWithFlags(&rt->ev_fork, hipEventDisableTiming))) goto fail;
    if (!HIP_OK(hipEventCreateWithFlags(&rt->ev_join, hipEventDisableTiming))) goto fail;
    if (tkm_gemm_handle_create(&rt->lt)) goto fail;
    /* generated kernels: prelude + source, hipRTC for gfx950 (src/tkm_gpu.cu:1047-1078) */
    if (!src) src = own_src = tkm_codegen_hip_source(G, rt->dt);
    if (!src) goto fail;
    {
        const char *pre = tkm_hip_prelude();
        size_t n = strlen(pre) + strlen(src) + 2;
        char *full = (char *)malloc(n);
        if (!full) goto fail;
        snprintf(full, n, "%s\n%s", pre, src);
        void *mod = NULL;
        int rc = tkm_rtc_load(full, "tkm_graph.hip", &mod);
        free(full);
        if (rc) {
            fprintf(stderr, "[TKM HIP] compiling the generated kernels failed: %s\n", tkm_attn_last_error());
            goto fail;
        }
        rt->module = (hipModule_t)mod;
    }
    /* arenas (one slot per planned node, src/tkm_core.c:540-559) */
    if (!HIP_OK(hipMalloc((void **)&rt->arena, G->total_arena_bytes ? G->total_arena_bytes : 256)) ||
        !HIP_OK(hipMemset(rt->arena, 0, G->total_arena_bytes ? G->total_arena_bytes : 256)))
        goto fail;
    if (rt->training && (!HIP_OK(hipMalloc((void **)&rt->grad_arena, G->total_arena_bytes ? G->total_arena_bytes : 256)) ||
                         !HIP_OK(hipMemset(rt->grad_arena, 0, G->total_arena_bytes ? G->total_arena_bytes : 256))))
        goto fail;
    rt->in_elems = (size_t)G->batch_size * G->nodes[0].H * G->nodes[0].W * G->nodes[0].C;
    rt->n_labels = (size_t)G->batch_size * G->nodes[0].H * G->nodes[0].W;
    if (!HIP_OK(hipMalloc((void **)&rt->d_input_f32, rt->in_elems * sizeof(float) + 16)) ||
        !HIP_OK(hipMalloc(&rt->d_labels, rt->n_labels * 4 + 16)) ||
        !HIP_OK(hipMemset(rt->d_labels, 0, rt->n_labels * 4 + 16)))
        goto fail;
    {
        int max_rows = 1;
        size_t attn_ws = 0;
        for (int i = 1; i < G->num_nodes; ++i) {
            const TkmNode *n = &G->nodes[i];
            if (n->dead) continue;
            if (is_loss(n->op) && (int)rows_of(G, n) > max_rows) max_rows = (int)rows_of(G, n);
            if (n->op == OP_GQA_ATTN) {
                const size_t w = tkm_attn_bwd_workspace_bytes(G->batch_size, n->H * n->W, n->q_heads);
                if (w > attn_ws) attn_ws = w;
            }
        }
        if (!HIP_OK(hipMalloc((void **)&rt->row_loss, (size_t)max_rows * 4)) ||
            !HIP_OK(hipMalloc((void **)&rt->row_correct, (size_t)max_rows * 4)))
            goto fail;
        rt->attn_ws_bytes = attn_ws;
        if (attn_ws && !HIP_OK(hipMalloc(&rt->attn_ws, attn_ws))) goto fail;
    }
    {
        float *scal = NULL;
        if (!HIP_OK(hipMalloc((void **)&scal, 256))) goto fail;
        rt->d_lr = scal;
        rt->d_loss = scal + 1;
        rt->d_epoch_loss = scal + 2;
        rt->d_correct = (int *)(scal + 3);
        rt->d_seed = (uint32_t *)(scal + 4);
        const float init[5] = {1e-3f, 0.0f, 0.0f, 0.0f, 0.0f};
        const uint32_t seed0 = 0x13579BDFu;   /* the reference's initial step seed */
        if (!HIP_OK(hipMemcpy(scal, init, sizeof init, hipMemcpyHostToDevice)) ||
            !HIP_OK(hipMemcpy(rt->d_seed, &seed0, 4, hipMemcpyHostToDevice)))
            goto fail;
        if (!HIP_OK(hipHostMalloc((void **)&rt->h_pin_lr, 64, hipHostMallocDefault))) goto fail;
        rt->h_pin_loss = rt->h_pin_lr + 1;
        *rt->h_pin_lr = 1e-3f;
    }
    if (!alloc_params(rt) || !alloc_saves(rt) || !plan_groups(rt) || !plan_grad_writes(rt) || !plan_gemms(rt) ||
        (rt->training && !plan_reductions(rt)))
        goto fail;
    free(own_src);
    if (opts.verbose)
        printf("  [TKM HIP Engine] Ignited %d hipRTC kernels | %d Learnable Tensors (%lld params) | %.2f MB Arena "
               "| %s\n", G->num_groups * 2, rt->n_tensors, rt->total_elems, G->total_arena_bytes / (1024.0 * 1024.0),
               rt->dt == TKM_ATTN_BF16 ? "bf16" : "fp16");
    return rt;
fail:
    free(own_src);
    free_runtime(rt);
    return NULL;
}

TkmRuntime *tkm_runtime_ignite(const TkmGraph *g, const char *cuda_src) {
    tkm_runtime_opts o;
    tkm_runtime_opts_init(&o);
    return tkm_runtime_ignite_ex(g, cuda_src, &o);
}

TkmRuntime *tkm_runtime_ignite_inference(const TkmGraph *g, const char *cuda_src) {
    tkm_runtime_opts o;
    tkm_runtime_opts_init(&o);
    o.training = 0;
    return tkm_runtime_ignite_ex(g, cuda_src, &o);
}

/* ---- launches ----------------------------------------------------------------------------- */

static uint8_t *act(TkmRuntime *rt, int nid) { return rt->arena + rt->graph.nodes[nid].out_offset; }
static uint8_t *grd(TkmRuntime *rt, int nid) { return rt->grad_arena + rt->graph.nodes[nid].out_offset; }

static float *tensor_master(TkmRuntime *rt, int t) { return t >= 0 ? rt->tensors[t].master : NULL; }
static float *tensor_grad(TkmRuntime *rt, int t) { return t >= 0 ? rt->tensors[t].grad : NULL; }

/* Resolves a plan parameter (the reference's resolve_arg_ptr, src/tkm_gpu.cu:1142-1164). */
static void resolve(TkmRuntime *rt, const rt_group *G, const PlasmaGroup *pg, const tkm_kparam *p, int bwd,
                    void **val, int *ival) {
    const TkmGraph *g = &rt->graph;
    const int nid = p->node >= 0 ? G->chain[p->node] : -1;
    const rt_node *st = nid >= 0 ? &rt->nodes[nid] : NULL;
    *val = NULL;
    switch (p->kind) {
        case TKM_ARG_IN: *val = act(rt, pg->anchor_id); break;
        case TKM_ARG_OUT: *val = act(rt, pg->out_node_id); break;
        case TKM_ARG_DOUT: *val = grd(rt, pg->out_node_id); break;
        case TKM_ARG_DIN: *val = grd(rt, pg->anchor_id); break;
        case TKM_ARG_WEIGHT: *val = tensor_master(rt, st->t_wvec); break;
        case TKM_ARG_BETA: *val = tensor_master(rt, st->t_beta); break;
        case TKM_ARG_BIAS: *val = tensor_master(rt, st->t_bias); break;
        case TKM_ARG_SAVE_XHAT: *val = st->xhat; break;
        case TKM_ARG_SAVE_ISTD: *val = st->istd; break;
        case TKM_ARG_SAVE_MASK: *val = st->mask; break;
        case TKM_ARG_SEED: *val = rt->d_seed; break;
        case TKM_ARG_BRANCH_IN: *val = act(rt, g->nodes[nid].in1); break;
        case TKM_ARG_DBRANCH: *val = grd(rt, g->nodes[nid].in1); break;
        case TKM_KP_PART: *val = (uint8_t *)rt->part_ws + G->part_off; break;
        case TKM_KP_ROWS: *ival = G->rows; break;
        case TKM_KP_BAND: *ival = (int)G->band; break;
        case TKM_KP_ACC:
            /* plain groups and the qkv-prep accumulate din, a twin group overwrites it
             * (src/tkm_codegen.c:601-614), residual and parameter gradients accumulate; a
             * group that writes a gradient slot first overwrites it (plan_grad_writes) */
            if (G->kind == TKM_HIP_GROUP_PREP) *ival = G->din_first ? 0 : 1;
            else *ival = (G->twin || G->din_first ? 0 : TKM_PLASMA_ACC_DIN) | TKM_PLASMA_ACC_PARAMS |
                         (G->branch_first ? 0 : TKM_PLASMA_ACC_BRANCH);
            break;
        default: break;
    }
    (void)bwd;
}

static void launch_group(TkmRuntime *rt, int gid, int bwd) {
    rt_group *G = &rt->groups[gid];
    const PlasmaGroup *pg = &rt->graph.groups[gid];
    const tkm_kplan *plan = &G->plan[bwd];
    void *vals[TKM_KPLAN_MAX];
    int ivals[TKM_KPLAN_MAX];
    void *kargs[TKM_KPLAN_MAX];
    for (int i = 0; i < plan->n; ++i) {
        const int k = plan->p[i].kind;
        resolve(rt, G, pg, &plan->p[i], bwd, &vals[i], &ivals[i]);
        kargs[i] = (k == TKM_KP_ROWS || k == TKM_KP_BAND || k == TKM_KP_ACC) ? (void *)&ivals[i] : (void *)&vals[i];
    }
    char what[64];
    snprintf(what, sizeof what, "group %d %s", gid, bwd ? "backward" : "forward");
    note(rt, tkm_rtc_launch(bwd ? G->bwd : G->fwd, G->gx, bwd ? G->bands : G->gy_fwd, 256, kargs, rt->stream, what),
         what);
}

/* The table of parameter-gradient reductions: each group's band partials (its own slice of the
 * partials block) into its parameters' gradients, 64 columns per entry.  Plasma groups lay
 * parameter p out at columns [p*C, (p+1)*C); the qkv-prep d(bias) at [0, C), d(gamma) after. */
static int plan_reductions(TkmRuntime *rt) {
    const TkmGraph *g = &rt->graph;
    int n = 0, cap = 0;
    TkmReduceChunk *h = NULL;
    for (int pass = 0; pass < 2; ++pass) {
        for (int gid = 0; gid < g->num_groups; ++gid) {
            const rt_group *G = &rt->groups[gid];
            if (G->kind < 0 || G->n_par == 0) continue;
            for (int p = 0; p < G->n_par; ++p) {
                const rt_node *st = &rt->nodes[G->chain[G->par_node[p]]];
                const int t = G->par_kind[p] == TKM_ARG_DWEIGHT ? st->t_wvec
                              : G->par_kind[p] == TKM_ARG_DBETA ? st->t_beta : st->t_bias;
                const int col0 = G->kind == TKM_HIP_GROUP_PREP ? (p == 0 ? 0 : G->chan) : p * G->chan;
                const int ncols = G->kind == TKM_HIP_GROUP_PREP ? (p == 0 ? G->chan : G->pw - G->chan) : G->chan;
                float *dst = tensor_grad(rt, t);
                if (!dst) continue;
                for (int c = 0; c < ncols; c += 64, ++n) {
                    if (pass == 0) continue;
                    h[n].part = (const float *)((uint8_t *)rt->part_ws + G->part_off);
                    h[n].dst = dst + c;
                    h[n].pw = G->pw;
                    h[n].bands = (int)G->bands;
                    h[n].col0 = col0 + c;
                    h[n].ncols = ncols - c < 64 ? ncols - c : 64;
                }
            }
        }
        if (pass == 0) {
            cap = n;
            n = 0;
            if (cap == 0) break;
            h = (TkmReduceChunk *)calloc((size_t)cap, sizeof *h);
            if (!h) return 0;
        }
    }
    rt->n_red = n;
    int ok = 1;
    if (n > 0)
        ok = HIP_OK(hipMalloc((void **)&rt->d_red, (size_t)n * sizeof *h)) &&
             HIP_OK(hipMemcpy(rt->d_red, h, (size_t)n * sizeof *h, hipMemcpyHostToDevice));
    free(h);
    return ok;
}

static float attn_scale(int D) { return 1.0f / sqrtf((float)D); }

/* The forward node walk (src/tkm_gpu.cu:1176-1289). */
static void forward_pass(TkmRuntime *rt, int is_eval, int valid_examples) {
    const TkmGraph *g = &rt->graph;
    const int B = g->batch_size;
    unsigned char done[TKM_MAX_GROUPS] = {0};
    for (int i = 1; i < g->num_nodes; ++i) {
        const TkmNode *n = &g->nodes[i];
        if (n->dead) continue;
        if (n->plasma_grp >= 0) {
            if (!done[n->plasma_grp]) {
                done[n->plasma_grp] = 1;
                launch_group(rt, n->plasma_grp, 0);
            }
            continue;
        }
        rt_node *st = &rt->nodes[i];
        void *in = act(rt, n->in0), *out = act(rt, i);
        const int rows = (int)rows_of(g, n);
        if (is_gemm(n->op)) {
            note(rt, tkm_gemm_run(st->g_fwd, rt->tensors[st->t_w].w16, in, out, rt->gemm_ws, rt->gemm_ws_bytes,
                                  rt->stream), "GEMM forward");
        } else if (n->op == OP_GQA_ATTN) {
            note(rt, tkm_attn_fwd(in, out, st->lse, NULL, B, n->H * n->W, n->q_heads, n->kv_heads, n->head_dim,
                                  attn_scale(n->head_dim), n->causal ? 1 : 0, rt->dt, rt->stream),
                 "attention forward");
        } else if (n->op == OP_FLATTEN) {
            if (out != in) note(rt, hipMemcpyAsync(out, in, n->out_bytes, hipMemcpyDeviceToDevice, rt->stream)
                                        == hipSuccess ? 0 : -1, "flatten copy");
        } else if (n->op == OP_SOFTMAX) {
            note(rt, tkm_rt_softmax_fwd(in, out, rows, n->C, rt->dt, rt->stream), "softmax forward");
        } else if (is_loss(n->op)) {
            const int kind = n->op == OP_SOFTMAX_FOCAL ? 1 : (n->op == OP_SOFTMAX_MSE ? 2 : 0);
            void *dlogits = rt->grad_arena ? grd(rt, n->in0) : act(rt, i);
            const int valid = is_eval ? (valid_examples * rows + B - 1) / B : rows;
            note(rt, tkm_rt_softmax_loss(in, rt->dt, rt->d_labels, rt->opts.token_labels, dlogits, rt->row_loss,
                                         rt->row_correct, rows, g->nodes[n->in0].C, is_eval, valid, kind, n->fval,
                                         rt->d_loss, rt->d_correct, 1, 1, rt->stream), "softmax loss");
        }
    }
}

/* The whole training step (src/tkm_gpu.cu:1291-1421): clears, forward, backward, SGD. */
static void record_step(TkmRuntime *rt, int clear_loss) {
    const TkmGraph *g = &rt->graph;
    const int B = g->batch_size;
    if (clear_loss) note(rt, tkm_rt_fill_u32(rt->d_loss, 4, 0, rt->stream), "loss clear");
    for (int c = 0; c < rt->n_clear; ++c)
        note(rt, tkm_rt_fill_u32(rt->grad_arena + rt->clear[c][0], rt->clear[c][1], 0, rt->stream),
             "gradient slot clear");
    forward_pass(rt, 0, B);
    unsigned char done[TKM_MAX_GROUPS] = {0};
    for (int i = g->num_nodes - 1; i >= 1; --i) {
        const TkmNode *n = &g->nodes[i];
        if (n->dead || is_loss(n->op)) continue;
        if (n->plasma_grp >= 0) {
            if (!done[n->plasma_grp]) {
                done[n->plasma_grp] = 1;
                launch_group(rt, n->plasma_grp, 1);
            }
            continue;
        }
        rt_node *st = &rt->nodes[i];
        void *in_act = act(rt, n->in0), *out_act = act(rt, i), *dout = grd(rt, i), *din = grd(rt, n->in0);
        if (is_gemm(n->op)) {
            /* dW on the side stream: its inputs (this node's gradient, complete once every
             * consumer's backward ran, and the saved input activation) are never written again
             * in the step, and only SGD reads its output */
            rt_tensor *t = &rt->tensors[st->t_w];
            depend(rt, rt->side, rt->stream, rt->ev_fork);
            note(rt, tkm_gemm_run(st->g_dw, dout, in_act, t->grad, rt->gemm_ws_side, rt->gemm_ws_bytes, rt->side),
                 "GEMM dW");
            note(rt, tkm_gemm_run(st->g_dx, t->w16, dout, din, rt->gemm_ws, rt->gemm_ws_bytes, rt->stream), "GEMM dX");
        } else if (n->op == OP_GQA_ATTN) {
            note(rt, tkm_attn_bwd(in_act, out_act, dout, st->lse, din, NULL, B, n->H * n->W, n->q_heads, n->kv_heads,
                                  n->head_dim, attn_scale(n->head_dim), n->causal ? 1 : 0, rt->dt, rt->attn_ws,
                                  rt->attn_ws_bytes, rt->stream), "attention backward");
        } else if (n->op == OP_FLATTEN) {
            if (din != dout)
                note(rt, hipMemcpyAsync(din, dout, g->nodes[n->in0].out_bytes, hipMemcpyDeviceToDevice, rt->stream)
                             == hipSuccess ? 0 : -1, "flatten copy");
        } else if (n->op == OP_SOFTMAX) {
            note(rt, tkm_rt_softmax_bwd(out_act, dout, din, (int)rows_of(g, n), n->C, rt->dt, rt->stream),
                 "softmax backward");
        }
    }
    depend(rt, rt->stream, rt->side, rt->ev_join);
    /* parameter gradients: every group's band partials, summed in one launch (each gradient
     * has one producer and is overwritten; gradients nothing writes stay zero) */
    note(rt, tkm_rt_reduce_parts(rt->d_red, rt->n_red, rt->stream), "parameter-gradient reductions");
    if (rt->total_elems > 0)
        note(rt, tkm_rt_sgd(rt->d_sgd, rt->n_tensors, rt->sgd_blocks, rt->d_lr, 0.9f, 1e-4f, rt->d_seed, rt->dt,
                            rt->stream), "SGD");
}

/* Captures the step once per variant (src/tkm_gpu.cu:1498-1508). */
static int ensure_step_graph(TkmRuntime *rt, int variant) {
    if (rt->step_exec[variant]) return 1;
    if (!HIP_OK(hipStreamSynchronize(rt->stream))) return 0;
    if (!HIP_OK(hipStreamBeginCapture(rt->stream, hipStreamCaptureModeGlobal))) return 0;
    rt->failed = 0;
    rt->counting = 1;
    rt->kernel_count = 0;
    record_step(rt, variant == 0);
    rt->counting = 0;
    hipGraph_t gr = NULL;
    if (!HIP_OK(hipStreamEndCapture(rt->stream, &gr))) return 0;
    if (rt->failed) {
        hipGraphDestroy(gr);
        return 0;
    }
    if (!HIP_OK(hipGraphInstantiate(&rt->step_exec[variant], gr, NULL, NULL, 0))) {
        hipGraphDestroy(gr);
        return 0;
    }
    rt->step_graph[variant] = gr;
    if (rt->opts.verbose)
        printf("  [HIP Graph] Full Fwd+Bwd+SGD step captured into one hipGraphExec (%d launches)\n", rt->kernel_count);
    return 1;
}

/* The learning rate goes to the device as a fill kernel's argument: the value is taken at
 * launch, so steps enqueued back to back (epochs, tkm_runtime_step_device) each read their own
 * rate, which a copy from one reused host word would not guarantee. */
static int set_lr(TkmRuntime *rt, float lr) {
    if (lr == rt->last_lr) return 1;
    rt->last_lr = lr;
    uint32_t bits;
    memcpy(&bits, &lr, sizeof bits);
    return tkm_rt_fill_u32(rt->d_lr, sizeof(float), bits, rt->stream) == 0;
}

int tkm_runtime_upload(TkmRuntime *rt, const float *h_input, const void *h_labels, size_t n_labels) {
    if (!rt) return -1;
    if (h_input) {
        if (!HIP_OK(hipMemcpyAsync(rt->d_input_f32, h_input, rt->in_elems * sizeof(float), hipMemcpyHostToDevice,
                                   rt->stream)))
            return -1;
        if (tkm_rt_f32_to_16(rt->d_input_f32, act(rt, 0), rt->in_elems, rt->dt, rt->stream)) return -1;
    }
    if (h_labels && n_labels) {
        const size_t esz = rt->opts.token_labels ? 4 : 1;
        if (n_labels > rt->n_labels) n_labels = rt->n_labels;
        if (!HIP_OK(hipMemcpyAsync(rt->d_labels, h_labels, n_labels * esz, hipMemcpyHostToDevice, rt->stream)))
            return -1;
    }
    return 0;
}

static float step_common(TkmRuntime *rt, const float *h_input, const void *h_labels, size_t n_labels, float lr) {
    if (!rt || !rt->training) {
        fprintf(stderr, "[TKM API Error] tkm_runtime_step needs a training runtime.\n");
        return NAN;
    }
    if (!set_lr(rt, lr) || tkm_runtime_upload(rt, h_input, h_labels, n_labels)) return NAN;
    if (!ensure_step_graph(rt, 0)) return NAN;
    if (!HIP_OK(hipGraphLaunch(rt->step_exec[0], rt->stream))) return NAN;
    float loss = 0.0f;
    if (h_input) {   /* the reference reads the loss back only when it uploaded an input */
        if (!HIP_OK(hipMemcpyAsync(rt->h_pin_loss, rt->d_loss, 4, hipMemcpyDeviceToHost, rt->stream)) ||
            !HIP_OK(hipStreamSynchronize(rt->stream)))
            return NAN;
        loss = *rt->h_pin_loss;
    }
    return loss;
}

float tkm_runtime_step(TkmRuntime *rt, const float *h_input, const uint8_t *h_labels, float lr) {
    if (rt && rt->opts.token_labels) {
        fprintf(stderr, "[TKM API Error] this runtime takes int32 labels: use tkm_runtime_step_tokens.\n");
        return NAN;
    }
    /* the reference uploads B labels (src/tkm_gpu.cu:1495) */
    return step_common(rt, h_input, h_labels, rt ? (size_t)rt->graph.batch_size : 0, lr);
}

float tkm_runtime_step_tokens(TkmRuntime *rt, const float *h_input, const int32_t *h_labels, float lr) {
    if (!rt || !rt->opts.token_labels) {
        fprintf(stderr, "[TKM API Error] tkm_runtime_step_tokens needs a runtime ignited with token_labels.\n");
        return NAN;
    }
    return step_common(rt, h_input, h_labels, rt->n_labels, lr);
}

int tkm_runtime_step_device(TkmRuntime *rt, float lr) {
    if (!rt || !rt->training || !set_lr(rt, lr) || !ensure_step_graph(rt, 0)) return -1;
    return HIP_OK(hipGraphLaunch(rt->step_exec[0], rt->stream)) ? 0 : -1;
}

float tkm_runtime_last_loss(TkmRuntime *rt) {
    if (!rt) return NAN;
    float l = NAN;
    if (!HIP_OK(hipStreamSynchronize(rt->stream)) || !HIP_OK(hipMemcpy(&l, rt->d_loss, 4, hipMemcpyDeviceToHost)))
        return NAN;
    return l;
}

/* ---- eval, forward, probes ------------------------------------------------------------------ */

static int output_node(const TkmGraph *g) {
    for (int i = g->num_nodes - 1; i >= 0; --i)
        if (!g->nodes[i].dead) return i;
    return -1;
}

/* One runtime batch of inference (docs/C_API.md 6.2): 0 unless the graph ends in a tensor and
 * h_output holds all of it.  The output node's 16-bit rows are widened on the device into a
 * buffer the runtime keeps for later calls, then copied out. */
size_t tkm_runtime_forward(TkmRuntime *rt, const float *h_input, float *h_output, size_t output_capacity) {
    const char *why = NULL;
    const size_t n = rt ? tkm_runtime_output_elements(rt) : 0;
    if (!rt || !h_input || !h_output) why = "a runtime, an input and an output buffer are required";
    else if (n == 0) why = "the graph ends in a loss, which has no inference output";
    else if (output_capacity < n) why = "the output buffer is smaller than tkm_runtime_output_elements()";
    if (why) {
        fprintf(stderr, "[TKM HIP] tkm_runtime_forward: %s\n", why);
        return 0;
    }
    if (!rt->d_out_f32 && !HIP_OK(hipMalloc((void **)&rt->d_out_f32, n * sizeof(float)))) return 0;
    if (tkm_runtime_upload(rt, h_input, NULL, 0)) return 0;
    rt->failed = 0;
    forward_pass(rt, 1, rt->graph.batch_size);
    if (rt->failed || tkm_rt_16_to_f32(act(rt, output_node(&rt->graph)), rt->d_out_f32, n, rt->dt, rt->stream) ||
        !HIP_OK(hipMemcpyAsync(h_output, rt->d_out_f32, n * sizeof(float), hipMemcpyDeviceToHost, rt->stream)) ||
        !HIP_OK(hipStreamSynchronize(rt->stream)))
        return 0;
    return n;
}

float tkm_eval_current_loss(TkmRuntime *rt) {
    if (!rt) return NAN;
    if (tkm_rt_fill_u32(rt->d_loss, 4, 0, rt->stream)) return NAN;
    rt->failed = 0;
    forward_pass(rt, 0, rt->graph.batch_size);
    if (rt->failed) return NAN;
    return tkm_runtime_last_loss(rt);
}

void tkm_perturb_tensor(TkmRuntime *rt, int node_id, int elem_idx, float delta) {
    if (!rt || node_id < 0 || node_id >= rt->graph.num_nodes || elem_idx < 0) return;
    tkm_rt_perturb(act(rt, node_id), elem_idx, delta, rt->dt, rt->stream);
    HIP_OK(hipStreamSynchronize(rt->stream));
}

float tkm_get_grad_sample(TkmRuntime *rt, int node_id, int elem_idx) {
    if (!rt || !rt->grad_arena || node_id < 0 || node_id >= rt->graph.num_nodes || elem_idx < 0) return NAN;
    uint16_t b = 0;
    if (!HIP_OK(hipStreamSynchronize(rt->stream)) ||
        !HIP_OK(hipMemcpy(&b, grd(rt, node_id) + (size_t)elem_idx * 2, 2, hipMemcpyDeviceToHost)))
        return NAN;
    if (rt->dt == TKM_ATTN_BF16) {
        const uint32_t u = (uint32_t)b << 16;
        float f;
        memcpy(&f, &u, 4);
        return f;
    }
    /* fp16 -> fp32 */
    const uint32_t s = (b >> 15) & 1u, e = (b >> 10) & 31u, m = b & 1023u;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 1024u), (int)e - 25);
    return s ? -v : v;
}

int tkm_runtime_eval(TkmRuntime *rt, const float *h_input, const uint8_t *h_labels, int count) {
    if (!rt || !h_input || !h_labels || count <= 0 || rt->opts.token_labels) return 0;
    const TkmGraph *g = &rt->graph;
    const int B = g->batch_size;
    const size_t per = rt->in_elems / (size_t)B;
    float *h_batch = (float *)calloc(rt->in_elems, sizeof(float));
    uint8_t *h_lbl = (uint8_t *)calloc((size_t)B, 1);
    if (!h_batch || !h_lbl) { free(h_batch); free(h_lbl); return 0; }
    tkm_rt_fill_u32(rt->d_correct, 4, 0, rt->stream);
    rt->failed = 0;
    for (int off = 0; off < count; off += B) {
        const int valid = count - off < B ? count - off : B;
        memset(h_batch, 0, rt->in_elems * sizeof(float));
        memset(h_lbl, 0, (size_t)B);
        memcpy(h_batch, h_input + (size_t)off * per, (size_t)valid * per * sizeof(float));
        memcpy(h_lbl, h_labels + off, (size_t)valid);
        if (tkm_runtime_upload(rt, h_batch, h_lbl, (size_t)B)) break;
        forward_pass(rt, 1, valid);
        HIP_OK(hipStreamSynchronize(rt->stream));   /* the host buffers are reused */
    }
    int correct = 0;
    HIP_OK(hipMemcpy(&correct, rt->d_correct, 4, hipMemcpyDeviceToHost));
    free(h_batch);
    free(h_lbl);
    return rt->failed ? 0 : correct;
}

size_t tkm_runtime_input_elements(const TkmRuntime *rt) { return rt ? rt->in_elems : 0; }

size_t tkm_runtime_output_elements(const TkmRuntime *rt) {
    if (!rt) return 0;
    const int out = output_node(&rt->graph);
    if (out < 0 || is_loss(rt->graph.nodes[out].op)) return 0;
    return rows_of(&rt->graph, &rt->graph.nodes[out]) * (size_t)rt->graph.nodes[out].C;
}

/* ---- weights: the reference's TKM1 layout (src/tkm_gpu.cu:1652-1765) ------------------------
 * u32 magic 0x544B4D31 ("TKM1" little-endian 1MKT), u32 tensor count, then per tensor u32 count
 * and that many fp32 master values, in the order of alloc_params. */

#define TKM_WEIGHT_MAGIC 0x544B4D31u

size_t tkm_runtime_weight_bytes(const TkmRuntime *rt) {
    if (!rt) return 0;
    size_t b = 8;
    for (int i = 0; i < rt->n_tensors; ++i) b += 4 + rt->tensors[i].n * 4;
    return b;
}

int tkm_save_weights_buffer(TkmRuntime *rt, void *buffer, size_t capacity, size_t *out_size) {
    if (out_size) *out_size = 0;
    if (!rt) return 0;
    const size_t need = tkm_runtime_weight_bytes(rt);
    if (out_size) *out_size = need;
    if (!buffer || capacity < need) return 0;
    if (!HIP_OK(hipStreamSynchronize(rt->stream))) return 0;
    uint8_t *d = (uint8_t *)buffer;
    const uint32_t magic = TKM_WEIGHT_MAGIC, nt = (uint32_t)rt->n_tensors;
    memcpy(d, &magic, 4);
    memcpy(d + 4, &nt, 4);
    d += 8;
    for (int i = 0; i < rt->n_tensors; ++i) {
        const uint32_t n = (uint32_t)rt->tensors[i].n;
        memcpy(d, &n, 4);
        d += 4;
        if (!HIP_OK(hipMemcpy(d, rt->tensors[i].master, (size_t)n * 4, hipMemcpyDeviceToHost))) return 0;
        d += (size_t)n * 4;
    }
    return 1;
}

int tkm_load_weights_buffer(TkmRuntime *rt, const void *buffer, size_t size) {
    if (!rt || !buffer || size < 8) return 0;
    const uint8_t *s = (const uint8_t *)buffer;
    uint32_t magic, nt;
    memcpy(&magic, s, 4);
    memcpy(&nt, s + 4, 4);
    if (magic != TKM_WEIGHT_MAGIC || nt != (uint32_t)rt->n_tensors) return 0;
    s += 8;
    size -= 8;
    /* validate the whole layout before writing anything */
    const uint8_t *p = s;
    size_t left = size;
    for (int i = 0; i < rt->n_tensors; ++i) {
        uint32_t n;
        if (left < 4) return 0;
        memcpy(&n, p, 4);
        if (n != (uint32_t)rt->tensors[i].n || (size_t)n > (left - 4) / 4) return 0;
        p += 4 + (size_t)n * 4;
        left -= 4 + (size_t)n * 4;
    }
    if (!HIP_OK(hipStreamSynchronize(rt->stream))) return 0;
    for (int i = 0; i < rt->n_tensors; ++i) {
        rt_tensor *t = &rt->tensors[i];
        s += 4;
        if (!HIP_OK(hipMemcpy(t->master, s, t->n * 4, hipMemcpyHostToDevice))) return 0;
        if (t->w16 && tkm_rt_f32_to_16(t->master, t->w16, t->n, rt->dt, rt->stream)) return 0;
        s += t->n * 4;
    }
    return HIP_OK(hipStreamSynchronize(rt->stream));
}

/* ---- host files ---------------------------------------------------------------------------- */

/* The whole file at `path` in a malloc'd buffer with one spare byte past its end (set to 0), its
 * size in *size; NULL if it cannot be read or is empty (the reason goes to stderr). */
static char *file_slurp(const char *path, size_t *size) {
    char *data = NULL;
    long len = -1;
    FILE *f = fopen(path, "rb");
    if (f && fseek(f, 0, SEEK_END) == 0) len = ftell(f);
    if (f && len > 0 && fseek(f, 0, SEEK_SET) == 0 && (data = (char *)malloc((size_t)len + 1)) != NULL &&
        fread(data, 1, (size_t)len, f) == (size_t)len) {
        data[len] = '\0';
        *size = (size_t)len;
    } else {
        fprintf(stderr, "[TKM HIP] cannot read '%s'%s\n", path, f ? "" : " (open failed)");
        free(data);
        data = NULL;
    }
    if (f) fclose(f);
    return data;
}

/* Writes n bytes to `path` (created or truncated); 1 on success. */
static int file_write(const char *path, const void *data, size_t n) {
    FILE *f = fopen(path, "wb");
    const int ok = f && fwrite(data, 1, n, f) == n;
    if (f && fclose(f) != 0) return 0;
    if (!ok) fprintf(stderr, "[TKM HIP] cannot write '%s'\n", path);
    return ok;
}

/* Checkpoint files hold exactly the bytes of tkm_save_weights_buffer (docs/C_API.md 6.4). */
int tkm_save_weights(TkmRuntime *rt, const char *bin_path) {
    const size_t n = rt && bin_path ? tkm_runtime_weight_bytes(rt) : 0;
    void *buf = n ? malloc(n) : NULL;
    const int ok = buf && tkm_save_weights_buffer(rt, buf, n, NULL) && file_write(bin_path, buf, n);
    free(buf);
    if (ok && rt->opts.verbose)
        printf("  [TKM HIP] checkpoint '%s': %zu bytes, %d tensors\n", bin_path, n, rt->n_tensors);
    return ok;
}

int tkm_load_weights(TkmRuntime *rt, const char *bin_path) {
    size_t n = 0;
    char *buf = rt && bin_path ? file_slurp(bin_path, &n) : NULL;
    const int ok = buf && tkm_load_weights_buffer(rt, buf, n);
    free(buf);
    if (ok && rt->opts.verbose)
        printf("  [TKM HIP] checkpoint '%s' loaded: %d tensors\n", bin_path, rt->n_tensors);
    return ok;
}

/* ---- loading from .tkm text ---------------------------------------------------------------
 * The front end (parsing, fusion, arena plan) is the reference's own code, which the
 * application links in; this library only generates, compiles and runs what it produces. */

/* A training runtime from NUL-terminated .tkm text, which it takes over and frees. */
static TkmRuntime *runtime_from_text(char *text, int batch_size) {
    TkmRuntime *rt = NULL;
    TkmGraph *g = NULL;
    char *src = NULL;
    if (!tkm_parse_dsl || !tkm_optimize_and_bind || !tkm_plan_memory)
        fprintf(stderr, "[TKM HIP] tkm_load_*: link the .tkm front end (tkm_core.c, tkm_registry.c) to load text\n");
    else if ((g = (TkmGraph *)calloc(1, sizeof *g)) != NULL) {
        tkm_parse_dsl(g, text, batch_size);
        tkm_optimize_and_bind(g);
        tkm_plan_memory(g);
        if ((src = tkm_codegen_cuda_string(g)) != NULL) rt = tkm_runtime_ignite(g, src);
    }
    free(src);
    free(g);
    free(text);
    return rt;
}

TkmRuntime *tkm_load_buffer(const char *dsl_data, size_t dsl_size, int batch_size) {
    char *text = NULL;
    if (dsl_data && dsl_size > 0 && dsl_size < SIZE_MAX && batch_size > 0 && (text = (char *)malloc(dsl_size + 1))) {
        memcpy(text, dsl_data, dsl_size);   /* the caller may free its bytes on return */
        text[dsl_size] = '\0';
        return runtime_from_text(text, batch_size);
    }
    return NULL;
}

TkmRuntime *tkm_load_string(const char *dsl_text, int batch_size) {
    return dsl_text ? tkm_load_buffer(dsl_text, strlen(dsl_text), batch_size) : NULL;
}

TkmRuntime *tkm_load_file(const char *tkm_path, int batch_size) {
    size_t n = 0;
    char *text = tkm_path && batch_size > 0 ? file_slurp(tkm_path, &n) : NULL;
    return text ? runtime_from_text(text, batch_size) : NULL;
}

/* ---- batches from a caller's loader (docs/C_API.md 6.5) -------------------------------------
 * One loop serves training and evaluation: it asks the loader for a batch into the runtime's
 * pinned staging rows, checks the count against the mode's rule (training: exactly B;
 * evaluation: 1..B), and hands the batch to the mode's step. */

typedef struct {
    int train;
    float lr;
    double total;        /* training: sum of the batch losses; evaluation: correct samples */
    size_t batches, samples;
} batch_loop;

static int loop_batches(TkmRuntime *rt, TkmDatasetNext next, void *user, size_t max_batches, batch_loop *L) {
    const size_t B = (size_t)rt->graph.batch_size;
    if ((!rt->h_stage_in && !HIP_OK(hipHostMalloc((void **)&rt->h_stage_in, rt->in_elems * sizeof(float),
                                                  hipHostMallocDefault))) ||
        (!rt->h_stage_lbl && !HIP_OK(hipHostMalloc((void **)&rt->h_stage_lbl, B, hipHostMallocDefault))))
        return 0;
    while (max_batches == 0 || L->batches < max_batches) {
        size_t got = 0;
        const int more = next(user, rt->h_stage_in, rt->h_stage_lbl, B, &got);
        if (more == 0) break;                                    /* end of the dataset */
        if (more < 0 || got == 0 || got > B || (L->train && got != B)) return 0;
        if (L->train) {
            const float loss = tkm_runtime_step(rt, rt->h_stage_in, rt->h_stage_lbl, L->lr);
            if (!isfinite(loss)) return 0;
            L->total += loss;
        } else {
            L->total += tkm_runtime_eval(rt, rt->h_stage_in, rt->h_stage_lbl, (int)got);
            if (rt->failed) return 0;
        }
        L->batches++;
        L->samples += got;
    }
    return L->batches > 0;
}

int tkm_runtime_train_dataset(TkmRuntime *rt, TkmDatasetNext next_batch, void *user, size_t max_batches, float lr,
                              float *out_average_loss) {
    batch_loop L = {1, lr, 0.0, 0, 0};
    const int ok = rt && next_batch && rt->training && !rt->opts.token_labels &&
                   loop_batches(rt, next_batch, user, max_batches, &L);
    if (out_average_loss) *out_average_loss = ok ? (float)(L.total / (double)L.batches) : 0.0f;
    return ok;
}

int tkm_runtime_eval_dataset(TkmRuntime *rt, TkmDatasetNext next_batch, void *user, size_t max_batches,
                             int *out_correct, size_t *out_samples) {
    batch_loop L = {0, 0.0f, 0.0, 0, 0};
    const int ok = rt && next_batch && !rt->opts.token_labels && loop_batches(rt, next_batch, user, max_batches, &L);
    if (out_correct) *out_correct = (int)L.total;
    if (out_samples) *out_samples = L.samples;
    return ok;
}

/* lr of a step: linear warm-up, then cosine decay to min_lr_ratio (src/tkm_gpu.cu:1793-1800) */
static float epoch_lr(float peak_lr, float min_lr_ratio, size_t step, size_t total_steps, size_t warmup_steps) {
    const float warmup = (warmup_steps > 0 && step < warmup_steps) ? (float)(step + 1) / (float)warmup_steps : 1.0f;
    const float progress = total_steps > 1 ? fminf((float)step / (float)(total_steps - 1), 1.0f) : 1.0f;
    const float cosine = 0.5f * (1.0f + cosf(3.14159265358979323846f * progress));
    return peak_lr * warmup * (min_lr_ratio + (1.0f - min_lr_ratio) * cosine);
}

/* Resident (the samples converted once to the runtime's 16-bit type in device memory) when
 * that copy fits in half the free device memory, else streaming (docs/C_API.md 6.2); the
 * runtime's dataset_mode option can force either. */
TkmDataset *tkm_dataset_create(TkmRuntime *rt, const float *h_images, const uint8_t *h_labels, size_t num_samples) {
    if (!rt || !rt->training || rt->opts.token_labels || !h_images || !h_labels || num_samples == 0) return NULL;
    const size_t per = rt->in_elems / (size_t)rt->graph.batch_size;
    if (num_samples > SIZE_MAX / 4 / per) return NULL;
    TkmDataset *ds = (TkmDataset *)calloc(1, sizeof *ds);
    if (!ds) return NULL;
    *ds = (TkmDataset){.rt = rt, .h_images = h_images, .h_labels = h_labels, .num_samples = num_samples,
                       .sample_elems = per};
    size_t free_b = 0, total_b = 0;
    if (!HIP_OK(hipMemGetInfo(&free_b, &total_b))) goto fail;
    ds->resident = rt->opts.dataset_mode == 1 ||
                   (rt->opts.dataset_mode == 0 && num_samples * (per * 2 + 1) <= free_b / 2);
    if (!HIP_OK(hipHostMalloc((void **)&ds->h_order, num_samples * 4, hipHostMallocDefault))) goto fail;
    if (ds->resident) {
        const size_t total = num_samples * per;
        if (!HIP_OK(hipMalloc(&ds->d_images, total * 2)) || !HIP_OK(hipMalloc((void **)&ds->d_labels, num_samples)) ||
            !HIP_OK(hipMalloc((void **)&ds->d_order, num_samples * 4)))
            goto fail;
        /* through the runtime's fp32 input rows, one batch's worth at a time (after any work
         * still queued on them) */
        if (!HIP_OK(hipStreamSynchronize(rt->stream))) goto fail;
        for (size_t off = 0; off < total; off += rt->in_elems) {
            const size_t n = total - off < rt->in_elems ? total - off : rt->in_elems;
            if (!HIP_OK(hipMemcpy(rt->d_input_f32, h_images + off, n * 4, hipMemcpyHostToDevice)) ||
                tkm_rt_f32_to_16(rt->d_input_f32, (uint8_t *)ds->d_images + off * 2, n, rt->dt, rt->stream) ||
                !HIP_OK(hipStreamSynchronize(rt->stream)))
                goto fail;
        }
        if (!HIP_OK(hipMemcpy(ds->d_labels, h_labels, num_samples, hipMemcpyHostToDevice))) goto fail;
    } else {
        const size_t B = (size_t)rt->graph.batch_size;
        if (!HIP_OK(hipStreamCreateWithFlags(&ds->copy, hipStreamNonBlocking))) goto fail;
        for (int k = 0; k < 2; ++k)
            if (!HIP_OK(hipHostMalloc((void **)&ds->h_in[k], rt->in_elems * 4, hipHostMallocDefault)) ||
                !HIP_OK(hipHostMalloc((void **)&ds->h_lbl[k], B, hipHostMallocDefault)) ||
                !HIP_OK(hipMalloc((void **)&ds->d_in[k], rt->in_elems * 4)) ||
                !HIP_OK(hipMalloc((void **)&ds->d_lbl[k], B)) ||
                !HIP_OK(hipEventCreateWithFlags(&ds->copied[k], hipEventDisableTiming)) ||
                !HIP_OK(hipEventCreateWithFlags(&ds->consumed[k], hipEventDisableTiming)))
                goto fail;
    }
    return ds;
fail:
    tkm_dataset_free(ds);
    return NULL;
}

void tkm_dataset_free(TkmDataset *ds) {
    if (!ds) return;
    if (ds->copy) hipStreamSynchronize(ds->copy);
    if (ds->rt) hipStreamSynchronize(ds->rt->stream);
    for (int k = 0; k < 2; ++k) {
        if (ds->h_in[k]) hipHostFree(ds->h_in[k]);
        if (ds->h_lbl[k]) hipHostFree(ds->h_lbl[k]);
        hipFree(ds->d_in[k]);
        hipFree(ds->d_lbl[k]);
        if (ds->copied[k]) hipEventDestroy(ds->copied[k]);
        if (ds->consumed[k]) hipEventDestroy(ds->consumed[k]);
    }
    if (ds->copy) hipStreamDestroy(ds->copy);
    hipFree(ds->d_images);
    hipFree(ds->d_labels);
    hipFree(ds->d_order);
    if (ds->h_order) hipHostFree(ds->h_order);
    free(ds);
}

int tkm_dataset_is_resident(const TkmDataset *ds) { return ds ? ds->resident : 0; }

/* Batch b of a streaming epoch into the runtime's input rows and labels, on rt->stream.  Slot
 * b & 1 is refilled on the host once the batch that last used it has been converted (its
 * `consumed` event), copied to the device on the copy stream (which first waits for that same
 * event, since the device slot is reused too), and converted into the input node on rt->stream
 * after the copy.  So the host gathers batch b + 1 and the copy engine moves it while
 * rt->stream trains on batch b. */
static int stream_batch(TkmDataset *ds, size_t b) {
    TkmRuntime *rt = ds->rt;
    const size_t B = (size_t)rt->graph.batch_size, per = ds->sample_elems;
    const int k = (int)(b & 1);
    if (ds->used[k] && !HIP_OK(hipEventSynchronize(ds->consumed[k]))) return 0;
    for (size_t r = 0; r < B; ++r) {
        const uint32_t src = ds->h_order[b * B + r];
        memcpy(ds->h_in[k] + r * per, ds->h_images + (size_t)src * per, per * 4);
        ds->h_lbl[k][r] = ds->h_labels[src];
    }
    if ((ds->used[k] && !HIP_OK(hipStreamWaitEvent(ds->copy, ds->consumed[k], 0))) ||
        !HIP_OK(hipMemcpyAsync(ds->d_in[k], ds->h_in[k], rt->in_elems * 4, hipMemcpyHostToDevice, ds->copy)) ||
        !HIP_OK(hipMemcpyAsync(ds->d_lbl[k], ds->h_lbl[k], B, hipMemcpyHostToDevice, ds->copy)) ||
        !HIP_OK(hipEventRecord(ds->copied[k], ds->copy)) ||
        !HIP_OK(hipStreamWaitEvent(rt->stream, ds->copied[k], 0)) ||
        tkm_rt_f32_to_16(ds->d_in[k], act(rt, 0), rt->in_elems, rt->dt, rt->stream) ||
        !HIP_OK(hipMemcpyAsync(rt->d_labels, ds->d_lbl[k], B, hipMemcpyDeviceToDevice, rt->stream)) ||
        !HIP_OK(hipEventRecord(ds->consumed[k], rt->stream)))
        return 0;
    ds->used[k] = 1;
    return 1;
}

int tkm_runtime_train_epoch(TkmRuntime *rt, TkmDataset *ds, const uint32_t *h_order, float peak_lr,
                            float min_lr_ratio, size_t global_step_start, size_t total_steps, size_t warmup_steps,
                            float *out_average_loss) {
    if (out_average_loss) *out_average_loss = 0.0f;
    if (!rt || !ds || ds->rt != rt || total_steps == 0 || peak_lr <= 0.0f || min_lr_ratio < 0.0f ||
        min_lr_ratio > 1.0f)
        return 0;
    const size_t B = (size_t)rt->graph.batch_size, full = ds->num_samples / B;
    if (full == 0) return 0;
    /* the previous epoch's last copies must be done before its order is overwritten */
    if (!HIP_OK(hipStreamSynchronize(rt->stream))) return 0;
    for (size_t i = 0; i < ds->num_samples; ++i) {
        ds->h_order[i] = h_order ? h_order[i] : (uint32_t)i;
        if (ds->h_order[i] >= ds->num_samples) return 0;
    }
    if (!ensure_step_graph(rt, 1)) return 0;
    if (tkm_rt_fill_u32(rt->d_loss, 4, 0, rt->stream)) return 0;
    if (ds->resident &&
        !HIP_OK(hipMemcpyAsync(ds->d_order, ds->h_order, ds->num_samples * 4, hipMemcpyHostToDevice, rt->stream)))
        return 0;
    for (size_t b = 0; b < full; ++b) {
        const int staged = ds->resident ? !tkm_rt_gather(ds->d_images, ds->d_labels, ds->d_order, (long long)(b * B),
                                                         (int)B, ds->sample_elems, act(rt, 0),
                                                         (uint8_t *)rt->d_labels, rt->stream)
                                        : stream_batch(ds, b);
        if (!staged || !set_lr(rt, epoch_lr(peak_lr, min_lr_ratio, global_step_start + b, total_steps, warmup_steps)) ||
            !HIP_OK(hipGraphLaunch(rt->step_exec[1], rt->stream)))
            return 0;
    }
    float sum = NAN;
    if (!HIP_OK(hipStreamSynchronize(rt->stream)) || !HIP_OK(hipMemcpy(&sum, rt->d_loss, 4, hipMemcpyDeviceToHost)))
        return 0;
    if (out_average_loss) *out_average_loss = sum / (float)full;
    return 1;
}

/* ---- accessors (tkm_hip.h) ------------------------------------------------------------------- */

void *tkm_runtime_stream(TkmRuntime *rt) { return rt ? (void *)rt->stream : NULL; }

void *tkm_runtime_node_device(TkmRuntime *rt, int node_id, int grad) {
    if (!rt || node_id < 0 || node_id >= rt->graph.num_nodes || (grad && !rt->grad_arena)) return NULL;
    return grad ? (void *)grd(rt, node_id) : (void *)act(rt, node_id);
}

int tkm_runtime_num_tensors(const TkmRuntime *rt) { return rt ? rt->n_tensors : -1; }

int tkm_runtime_tensor(TkmRuntime *rt, int i, float **master, void **w16, float **grad, size_t *n, int *node_id) {
    if (!rt || i < 0 || i >= rt->n_tensors) return -1;
    const rt_tensor *t = &rt->tensors[i];
    if (master) *master = t->master;
    if (w16) *w16 = t->w16;
    if (grad) *grad = t->grad;
    if (n) *n = t->n;
    if (node_id) *node_id = t->node;
    return 0;
}

void *tkm_runtime_node_save(TkmRuntime *rt, int node_id, int kind) {
    if (!rt || node_id < 0 || node_id >= rt->graph.num_nodes) return NULL;
    const rt_node *st = &rt->nodes[node_id];
    switch (kind) {
        case 0: return st->istd;
        case 1: return st->xhat;
        case 2: return st->mask;
        case 3: return st->lse;
        default: return NULL;
    }
}

int tkm_runtime_step_kernel_count(const TkmRuntime *rt) { return rt ? rt->kernel_count : -1; }

/* ---- teardown ---------------------------------------------------------------------------------- */

static void free_runtime(TkmRuntime *rt) {
    if (!rt) return;
    if (rt->stream) hipStreamSynchronize(rt->stream);
    for (int v = 0; v < 2; ++v) {
        if (rt->step_exec[v]) hipGraphExecDestroy(rt->step_exec[v]);
        if (rt->step_graph[v]) hipGraphDestroy(rt->step_graph[v]);
    }
    if (rt->nodes)
        for (int i = 0; i < TKM_MAX_NODES; ++i) {
            tkm_gemm_destroy(rt->nodes[i].g_fwd);
            tkm_gemm_destroy(rt->nodes[i].g_dw);
            tkm_gemm_destroy(rt->nodes[i].g_dx);
        }
    tkm_gemm_handle_destroy(rt->lt);
    if (rt->module) tkm_rtc_unload(rt->module);
    hipFree(rt->arena);
    hipFree(rt->grad_arena);
    hipFree(rt->d_input_f32);
    hipFree(rt->d_labels);
    hipFree(rt->d_lr);
    hipFree(rt->row_loss);
    hipFree(rt->row_correct);
    hipFree(rt->attn_ws);
    hipFree(rt->part_ws);
    hipFree(rt->d_red);
    hipFree(rt->gemm_ws);
    hipFree(rt->gemm_ws_side);
    hipFree(rt->param_block);
    hipFree(rt->pgrad_block);
    hipFree(rt->save_block);
    hipFree(rt->d_sgd);
    free(rt->clear);
    hipFree(rt->d_out_f32);
    if (rt->h_stage_in) hipHostFree(rt->h_stage_in);
    if (rt->h_stage_lbl) hipHostFree(rt->h_stage_lbl);
    if (rt->h_pin_lr) hipHostFree(rt->h_pin_lr);
    if (rt->ev_fork) hipEventDestroy(rt->ev_fork);
    if (rt->ev_join) hipEventDestroy(rt->ev_join);
    if (rt->side) hipStreamDestroy(rt->side);
    if (rt->stream) hipStreamDestroy(rt->stream);
    free(rt->tensors);
    free(rt->nodes);
    free(rt->groups);
    free(rt);
}

void tkm_runtime_free(TkmRuntime *rt) { free_runtime(rt); }
