// SPDX-License-Identifier: MPL-2.0-no-copyleft-exception
// Copyright (c) 2026 BSODsystem32
// (The declarations below restate the reference's public interface, include/tkm.h, member for
// member, so they carry its notice; the comments are this build's.)

/*
 * tkm.h -- the public C interface of the Tokamak runtime, declared for this build's HIP runtime
 * (tokamak_amd/csrc/tkm_hip.c) and HIP code generator (tkm_codegen_hip.c).
 *
 * The north star keeps the reference's public API, op registry and .tkm format unchanged,
 * so every type, enumerator, struct member and function below has the reference's name,
 * order, type and meaning (reference include/tkm.h:31-271).  The struct layouts must be
 * identical byte for byte: the graph IR (TkmGraph) is produced by the reference's front end
 * (tkm_parse_dsl / tkm_optimize_and_bind / tkm_plan_memory in src/tkm_core.c and
 * src/tkm_registry.c) and consumed here.  tests/test_tkm_runtime_cpu.py compares sizeof and
 * offsetof of every member with a fixture dumped from the reference header.
 *
 * What this build implements (libtkm_hip.so): tkm_codegen_cuda_string (emits HIP for
 * hipRTC, gfx950) and the 25 runtime functions of section 5.  The front end (parsing,
 * fusion, memory planning, registry lookups, tkm_verify_registry, tkm_dump_summary) is the
 * reference's own code, linked in by the application.
 */
#ifndef TKM_H
#define TKM_H

#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(_WIN32)
#define TKM_API
#else
#define TKM_API __attribute__((visibility("default")))
#endif

/* Capacities of the fixed-size graph IR (reference include/tkm.h:31-36). */
#define TKM_MAX_NODES 1024
#define TKM_MAX_GROUPS 256
#define TKM_MAX_BUFFERS 512
#define TKM_MAX_CHAIN 8
#define TKM_MAX_KARGS 28
#define TKM_MAX_TENSORS 512

/* Random generators a node or graph may select (include/tkm.h:38-44). */
typedef enum { RNG_DEFAULT = 0, RNG_XORSHIFT32, RNG_WANG_XORSHIFT32, RNG_PCG32, RNG_PHILOX } TkmRngType;

/* Per-op resources (include/tkm.h:46-57): parameters, saved state, seeds, side inputs. */
typedef enum {
    RES_NONE = 0,
    RES_PARAM_BIAS = 1 << 0,
    RES_PARAM_WEIGHT = 1 << 1,
    RES_PARAM_BETA = 1 << 2,
    RES_SAVE_ISTD = 1 << 3,
    RES_SAVE_XHAT = 1 << 4,
    RES_SAVE_MASK = 1 << 5,
    RES_RNG_SEED = 1 << 6,
    RES_BRANCH_IN = 1 << 7,
    RES_AUG_PIXEL = 1 << 8,
    RES_AUG_COLOR = 1 << 9
} TkmResourceFlags;

/* Op categories (include/tkm.h:59-66). */
typedef enum { CAT_META = 0, CAT_ANCHOR, CAT_SPATIAL, CAT_COORD, CAT_NORM, CAT_FLUID } TkmOpCat;

/* Op types, in the reference's order (include/tkm.h:68-93). */
typedef enum {
    OP_NONE = 0, OP_INPUT,
    OP_CONV, OP_FC, OP_FC_TWIN_FUSED, OP_FC_QKV_FUSED, OP_GQA_ATTN,
    OP_MIXPOOL, OP_AVGPOOL, OP_FLATTEN,
    OP_BORDER_REFLECT,
    OP_RAND_SHIFT, OP_RAND_ROTATE, OP_RAND_SCALE, OP_RAND_FLIPX, OP_RAND_FLIPY,
    OP_RAND_ELASTIC, OP_RAND_NOISE, OP_RAND_CUTOUT, OP_RAND_BRIGHTNESS, OP_RAND_CONTRAST,
    OP_RAND_SATURATION, OP_RAND_HUE, OP_RAND_GRAYSCALE, OP_RAND_CHANNEL_SCALE,
    OP_RAND_SOLARIZE, OP_RAND_ERASING,
    OP_BN, OP_LN, OP_RMSNORM, OP_L2NORM, OP_QKNORM,
    OP_BIAS, OP_SILU, OP_RELU, OP_RELU2, OP_LEAKY_RELU, OP_ELU,
    OP_GELU, OP_MISH, OP_HARDSWISH, OP_HARDSIGMOID, OP_TANH, OP_SIGMOID,
    OP_SWISH_BETA, OP_SIN, OP_COSGATE, OP_SOFTCAP, OP_CLAMP,
    OP_SCALE, OP_LAYERSCALE, OP_DYT, OP_PRELU, OP_XATLU,
    OP_ROPE, OP_DROP, OP_ADD, OP_MUL,
    OP_SOFTMAX, OP_SOFTMAX_CE, OP_SOFTMAX_FOCAL, OP_SOFTMAX_MSE,
    OP_USER_FLUID,
    OP_COUNT
} TkmOpType;

/* One registry entry (include/tkm.h:95-105). */
typedef struct {
    TkmOpType op;
    const char *dsl_name;
    TkmOpCat cat;
    uint32_t res_flags;
    float default_fval;
    const char *fwd_cuda;
    const char *bwd_cuda;
    const char *fwd_expr;
    const char *bwd_expr;
} TkmOpSpec;

/* What a generated kernel argument points at (include/tkm.h:107-112). */
typedef enum {
    KARG_IN_MAIN = 0, KARG_OUT_MAIN, KARG_DOUT_MAIN, KARG_DIN_MAIN,
    KARG_BRANCH_IN, KARG_DBRANCH_OUT,
    KARG_BIAS, KARG_DBIAS, KARG_WEIGHT_VEC, KARG_DWEIGHT_VEC, KARG_BETA, KARG_DBETA,
    KARG_SAVE_ISTD, KARG_SAVE_XHAT, KARG_SAVE_MASK, KARG_STEP_SEED
} TkmArgKind;

typedef struct {
    TkmArgKind kind;
    int node_id;
    char c_type[32];
    char c_name[32];
} TkmKernelArg;

/* A generated kernel's name, ordered argument list and 1-D launch shape
 * (include/tkm.h:114-126). */
typedef struct {
    char func_name[64];
    TkmKernelArg args[TKM_MAX_KARGS];
    int num_args;
    int grid_x, block_x;
} TkmKernelSig;

/* A graph node (include/tkm.h:128-159). */
typedef struct {
    int id;
    int spec_id;
    char tag[32];
    TkmOpType op;
    TkmOpCat cat;
    int dead;

    int in0, in1, in2;
    int users;
    int plasma_grp;

    int c_out, k, s, p;
    int q_c, k_c, v_c;
    int q_heads, kv_heads, head_dim;
    int has_qknorm, has_rope, causal;
    int qkv_prep_nid;
    float fval;
    float fval2;
    float rope_theta, rope_scale, rope_low_freq_factor, rope_high_freq_factor;
    float rope_original_context_length;
    TkmRngType rng_type;

    int left_nodes[TKM_MAX_CHAIN];
    int left_len;
    int right_nodes[TKM_MAX_CHAIN];
    int right_len;

    int H, W, C;
    int out_buf_id;
    size_t out_offset, out_bytes;
} TkmNode;

/* A fused epilogue group: one generated forward and one backward kernel
 * (include/tkm.h:161-176). */
typedef struct {
    int id;
    int anchor_id;
    int node_ids[16];
    int count;
    int has_norm;
    int is_twin_epilogue;
    int is_coord_group;
    int is_qkv_prep;
    int use_reflect_border;
    int out_node_id;
    int H, W, C;
    TkmKernelSig fwd_sig;
    TkmKernelSig bwd_sig;
} PlasmaGroup;

/* The whole graph (include/tkm.h:178-186). */
typedef struct TkmGraph {
    TkmNode nodes[TKM_MAX_NODES];
    int num_nodes;
    PlasmaGroup groups[TKM_MAX_GROUPS];
    int num_groups;
    int batch_size;
    TkmRngType default_rng;
    size_t total_arena_bytes;
    size_t naive_arena_bytes;
} TkmGraph;

typedef struct {
    const char *name;
    int (*match)(const TkmGraph *g, int node_id);
    void (*apply)(TkmGraph *g, int node_id);
} TkmFusionRule;

/* Registry and front end: provided by the reference's src/tkm_registry.c and src/tkm_core.c
 * (include/tkm.h:194-211). */
const TkmOpSpec *tkm_find_spec_by_op(TkmOpType op);
const TkmOpSpec *tkm_find_spec_by_name(const char *dsl_name);
const TkmOpSpec *tkm_find_spec_by_index(int index);
const TkmOpSpec *tkm_find_spec_by_node(const TkmNode *node);
int tkm_get_spec_index(const TkmOpSpec *spec);
int tkm_get_spec_count(void);
int tkm_eval_math_expr(const char *expr, float x, float fval, float *out_value);
const TkmFusionRule *tkm_get_fusion_rules(int *out_count);
const char *tkm_rng_name(TkmRngType r);
const char *tkm_rng_struct_name(TkmRngType r);
TkmRngType tkm_parse_rng_name(const char *s);

TKM_API int tkm_verify_registry(void);
TKM_API void tkm_parse_dsl(TkmGraph *g, const char *dsl_text, int batch_size);
TKM_API void tkm_infer_shapes(TkmGraph *g);
TKM_API void tkm_optimize_and_bind(TkmGraph *g);
TKM_API void tkm_plan_memory(TkmGraph *g);
TKM_API void tkm_dump_summary(const TkmGraph *g, FILE *out);

/* This build: the HIP source (hipRTC, gfx950) of every group's kernels, without the prelude
 * (the runtime prepends it, as the reference prepends its NVRTC prelude).  Heap string; the
 * caller frees it with free().  Reference include/tkm.h:212, src/tkm_codegen.c:627-634. */
TKM_API char *tkm_codegen_cuda_string(const TkmGraph *g);

/* 5. Runtime (include/tkm.h:214-271); this build: tokamak_amd/csrc/tkm_hip.c. */
typedef struct TkmRuntime TkmRuntime;
typedef struct TkmDataset TkmDataset;

/* Fills up to `capacity` samples; returns > 0 for a batch, 0 at the end, < 0 on error.
 * Training loaders return exactly the batch size; evaluation loaders may return fewer. */
typedef int (*TkmDatasetNext)(void *user, float *h_input, uint8_t *h_labels, size_t capacity,
                              size_t *out_count);

TKM_API TkmRuntime *tkm_runtime_ignite(const TkmGraph *g, const char *cuda_src);
TKM_API TkmRuntime *tkm_runtime_ignite_inference(const TkmGraph *g, const char *cuda_src);
TKM_API TkmRuntime *tkm_load_file(const char *tkm_path, int batch_size);
TKM_API TkmRuntime *tkm_load_string(const char *dsl_text, int batch_size);
TKM_API TkmRuntime *tkm_load_buffer(const char *dsl_data, size_t dsl_size, int batch_size);
TKM_API float tkm_runtime_step(TkmRuntime *rt, const float *h_input, const uint8_t *h_labels, float lr);
TKM_API int tkm_runtime_eval(TkmRuntime *rt, const float *h_input, const uint8_t *h_labels, int count);
TKM_API size_t tkm_runtime_forward(TkmRuntime *rt, const float *h_input, float *h_output,
                                   size_t output_capacity);
TKM_API size_t tkm_runtime_input_elements(const TkmRuntime *rt);
TKM_API size_t tkm_runtime_output_elements(const TkmRuntime *rt);
TKM_API size_t tkm_runtime_weight_bytes(const TkmRuntime *rt);
TKM_API int tkm_runtime_train_dataset(TkmRuntime *rt, TkmDatasetNext next_batch, void *user,
                                      size_t max_batches, float lr, float *out_average_loss);
TKM_API TkmDataset *tkm_dataset_create(TkmRuntime *rt, const float *h_images,
                                       const uint8_t *h_labels, size_t num_samples);
TKM_API void tkm_dataset_free(TkmDataset *ds);
TKM_API int tkm_dataset_is_resident(const TkmDataset *ds);
TKM_API int tkm_runtime_train_epoch(TkmRuntime *rt, TkmDataset *ds, const uint32_t *h_order,
                                    float peak_lr, float min_lr_ratio, size_t global_step_start,
                                    size_t total_steps, size_t warmup_steps,
                                    float *out_average_loss);
TKM_API int tkm_runtime_eval_dataset(TkmRuntime *rt, TkmDatasetNext next_batch, void *user,
                                     size_t max_batches, int *out_correct, size_t *out_samples);
TKM_API int tkm_save_weights(TkmRuntime *rt, const char *bin_path);
TKM_API int tkm_load_weights(TkmRuntime *rt, const char *bin_path);
TKM_API int tkm_save_weights_buffer(TkmRuntime *rt, void *buffer, size_t capacity, size_t *out_size);
TKM_API int tkm_load_weights_buffer(TkmRuntime *rt, const void *buffer, size_t size);
TKM_API void tkm_runtime_free(TkmRuntime *rt);

/* Finite-difference gradient check probes (include/tkm.h:267-270). */
TKM_API float tkm_get_grad_sample(TkmRuntime *rt, int node_id, int elem_idx);
TKM_API void tkm_perturb_tensor(TkmRuntime *rt, int node_id, int elem_idx, float delta);
TKM_API float tkm_eval_current_loss(TkmRuntime *rt);

#ifdef __cplusplus
}
#endif

#endif /* TKM_H */
