/*
 * tkm_hip.h -- extensions of this build's HIP runtime (libtkm_hip.so) beyond the unchanged
 * public API of tkm.h.  None has a reference counterpart unless stated; none changes tkm.h or
 * the .tkm grammar.
 *
 *   - the graph-to-kernel mapping the generator and the runtime share (the qkv_prep node and
 *     the plasma groups as descriptors of include/tkm_prep.h and include/tkm_plasma.h);
 *   - run-time options: bf16 storage (fp32 master weights either way), int32 per-row labels
 *     (a language model's next-token loss; the reference uploads B uint8 labels,
 *     src/tkm_gpu.cu:1495), the weight-initialization seed;
 *   - a step on inputs already in device memory (benchmarks, resident data);
 *   - accessors of device buffers for tests.
 */
#ifndef TKM_HIP_H
#define TKM_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "tkm.h"
#include "tkm_plasma.h"
#include "tkm_prep.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- the graph's groups as this build's generator descriptors ----------------------------- */

enum { TKM_HIP_GROUP_PREP = 0, TKM_HIP_GROUP_PLASMA = 1 };

/* TKM_HIP_GROUP_PREP (the qkv_prep group), TKM_HIP_GROUP_PLASMA (plain or twin), or -1 for a
 * group without HIP kernels here (the coordinate / augmentation groups of the CNN family). */
TKM_API int tkm_hip_group_kind(const TkmGraph *g, int gid);

/* The qkv_prep node of group gid (fields written by the 3-way rule, reference
 * src/tkm_registry.c:750-768) as a tkm_prep_desc: heads, D, S = H*W, QKNorm / RoPE flags and
 * parameters.  Returns TKM_ATTN_OK or a status. */
TKM_API int tkm_hip_prep_desc(const TkmGraph *g, int gid, int dtype, tkm_prep_desc *d);

/* A plain or twin group as a tkm_plasma_desc; chain_nodes (if not NULL, 24 entries) receives
 * the graph node of every chain position (twin: left, right, then post ops). */
TKM_API int tkm_hip_plasma_desc(const TkmGraph *g, int gid, int dtype, tkm_plasma_desc *d, int *chain_nodes);

/* The TKM_OP_* of a node (user-formula ops by registry index), -1 if none. */
TKM_API int tkm_hip_plasma_op(const TkmNode *n);

/* tkm_codegen_cuda_string for a 16-bit type: TKM_ATTN_F16 (what tkm_codegen_cuda_string
 * emits) or TKM_ATTN_BF16.  Free with free(). */
TKM_API char *tkm_codegen_hip_source(const TkmGraph *g, int dtype);

/* The resource flags (TkmResourceFlags) of a node's op, as the reference's registry declares
 * them (src/tkm_registry.c:43-456); the runtime allocates parameters and saved state by them. */
TKM_API uint32_t tkm_hip_res_flags(const TkmNode *n);

/* Pointwise ops' code.  With the front end linked, the generator pastes each pointwise op's
 * code as the registry holds it (TkmOpSpec fwd_cuda / bwd_cuda, or the user formulas
 * fwd_expr / bwd_expr), as the reference's generator does, and takes ops it has no formula of
 * its own for (TKM_OP_FORMULA*); without the front end it uses this build's own formulas of
 * the ops it knows.  mode 1 (default): as described; 0: this build's formulas for every op it
 * knows; 2: every pointwise op as an op unknown to this build (the TKM_OP_FORMULA* path a new
 * registry op takes).  Process-wide; read when a source is generated (tkm_codegen_*, ignite). */
TKM_API void tkm_hip_use_registry_code(int mode);
/* 1 when the registry is linked (tkm_find_spec_by_node resolves). */
TKM_API int tkm_hip_registry_linked(void);

/* ---- run-time options ------------------------------------------------------------------- */

typedef struct {
    int dtype;             /* TKM_ATTN_F16 (default) or TKM_ATTN_BF16: activations, gradients,
                              GEMM weight copies; master weights are fp32 either way */
    int training;          /* 1 (default): gradients and SGD; 0: inference only */
    int token_labels;      /* 0 (default): uint8 labels, the reference's B per step; 1: one int32
                              label per row (B*H*W), uploaded by tkm_runtime_step_tokens */
    uint64_t init_seed;    /* weight initialization (N(0,1)*sqrt(2/fan_in) for GEMM weights) */
    int verbose;           /* 1: print the ignite summary line */
    int dataset_mode;      /* tkm_dataset_create: 0 (default) resident when the 16-bit copy fits in
                              half the free device memory, else streaming (the reference's rule);
                              1 always resident; 2 always streaming */
    int clear_all_grads;   /* debug: 1 clears the whole gradient arena at every step, as the
                              reference does, instead of only the slots whose first writer
                              accumulates (0, the default); the results must not change */
} tkm_runtime_opts;

TKM_API void tkm_runtime_opts_init(tkm_runtime_opts *o);

/* tkm_runtime_ignite / _inference with options.  src = NULL generates the source for o's
 * dtype (tkm_codegen_hip_source); a given src must have been generated for that dtype. */
TKM_API TkmRuntime *tkm_runtime_ignite_ex(const TkmGraph *g, const char *src, const tkm_runtime_opts *o);

/* tkm_runtime_step with int32 labels, one per row (B*H*W), for token_labels runtimes. */
TKM_API float tkm_runtime_step_tokens(TkmRuntime *rt, const float *h_input, const int32_t *h_labels, float lr);

/* Replays the captured step on the input rows and labels already in device memory (written
 * by an earlier step, tkm_runtime_upload or through tkm_runtime_device_*).  No host copy but
 * the learning rate's when it changed, no synchronization.  Returns 0 or -1. */
TKM_API int tkm_runtime_step_device(TkmRuntime *rt, float lr);

/* Copies input rows (fp32, converted to the runtime's 16-bit type) and labels (uint8 or int32
 * per the options; NULL leaves them) to the device, asynchronously.  Returns 0 or -1. */
TKM_API int tkm_runtime_upload(TkmRuntime *rt, const float *h_input, const void *h_labels, size_t n_labels);

/* Loss of the last step (synchronizes). */
TKM_API float tkm_runtime_last_loss(TkmRuntime *rt);

/* Device buffers: the runtime's stream; a node's activation (grad = 0) or gradient (grad = 1)
 * slot of the arena; learnable tensor i (in TKM1 file order): master, 16-bit copy (or NULL),
 * gradient, element count, owning node.  Return NULL / -1 when out of range. */
TKM_API void *tkm_runtime_stream(TkmRuntime *rt);
TKM_API void *tkm_runtime_node_device(TkmRuntime *rt, int node_id, int grad);
TKM_API int tkm_runtime_num_tensors(const TkmRuntime *rt);
TKM_API int tkm_runtime_tensor(TkmRuntime *rt, int i, float **master, void **w16, float **grad, size_t *n,
                               int *node_id);
/* The saved state of node_id: kind 0 istd, 1 xhat, 2 mask, 3 LSE (attention). */
TKM_API void *tkm_runtime_node_save(TkmRuntime *rt, int node_id, int kind);
/* Kernels launched by one captured step (GEMMs, generated kernels, attention, runtime). */
TKM_API int tkm_runtime_step_kernel_count(const TkmRuntime *rt);

#ifdef __cplusplus
}
#endif

#endif /* TKM_HIP_H */
