/*
 * tkm_plasma.h -- C ABI of the generated "plasma" epilogues: chains of row-wise ops fused
 * behind a GEMM (libtkm_attn.so).
 *
 * The reference vertically fuses the pointwise, normalization, residual and gated ops that
 * follow an anchor GEMM into one generated kernel pair per group (emit_plasma_group, reference
 * src/tkm_codegen.c:484-625, per-op code 297-482, op registry src/tkm_registry.c:186-456).
 * Here a descriptor lists the chain, tkm_plasma_source emits HIP C for it, tkm_plasma_create
 * compiles it with hipRTC for gfx950, and tkm_plasma_fwd / tkm_plasma_bwd launch it.
 *
 * A group works on `rows` rows of C channels (16-bit, fp16 or bf16):
 *   plain: out = chain(in)                               in, out: [rows][C]
 *   twin : out = post(left(in[:, :C]) * right(in[:, C:])) in: [rows][2C], out: [rows][C]
 *          (the gated FFN epilogue, e.g. SiLU(gate) * up; tkm_codegen.c:509-515)
 * Op semantics follow the registry, with these rules kept from the reference:
 *   - Norms reduce over aligned 64-channel groups when C > 64 (the whole row when C <= 64) and
 *     divide by C, not by the group size (tkm_codegen.c:490-496, registry 229-245).
 *   - The backward recomputes each op's input from the group input ("replay"); a norm's
 *     output is replayed from its saved 16-bit xhat (tkm_codegen.c:464-482).
 * Differences, on purpose:
 *   - istd is saved per (row, 64-channel group): [rows][ceil(C/64)].  The reference saves one
 *     value per row (group 0's) and its backward applies it to every group.
 *   - The replay applies a residual Add (re-reading branch_in); the reference skips it, which
 *     feeds later ops the wrong input.
 *   - Parameter gradients are reduced without atomics, in a fixed order (bitwise reproducible).
 *   - Twin chains hold pointwise and parameterized pointwise ops only (no norm, no Add).
 *   - The replay also applies Drop from its saved mask; the reference's replay skips Drop
 *     (src/tkm_codegen.c:478-479), so ops after a Drop would see its input.
 *
 * Kernel arguments are resolved by the caller, as the reference's resolve_arg_ptr does
 * (src/tkm_gpu.cu:1142-1164): tkm_plasma_num_args / tkm_plasma_arg describe the pointer list
 * of each pass, in order, and the caller passes the pointers in that order.
 */
#ifndef TKM_PLASMA_H
#define TKM_PLASMA_H

#include "tkm_prep.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Ops (registry names in comments; fval is the op's constant, e.g. the norm's epsilon). */
enum {
    TKM_OP_BIAS = 0,        /* Bias        x + b                                   (param b) */
    TKM_OP_RMSNORM,         /* RMSNorm     x * rsqrt(sum_g x^2 / C + fval) * w      (param w) */
    TKM_OP_LN,              /* LN          (x - m) * rsqrt(var + fval) * w + beta   (w, beta) */
    TKM_OP_BN,              /* BN          as LN (a row statistic in plasma groups)  (w, beta) */
    TKM_OP_L2NORM,          /* L2Norm      x * rsqrt(sum_g x^2 / C + fval)                    */
    TKM_OP_SILU, TKM_OP_RELU, TKM_OP_RELU2, TKM_OP_LEAKY_RELU, TKM_OP_ELU, TKM_OP_GELU,
    TKM_OP_MISH, TKM_OP_HARDSWISH, TKM_OP_HARDSIGMOID, TKM_OP_TANH, TKM_OP_SIGMOID,
    TKM_OP_SWISH_BETA, TKM_OP_SIN, TKM_OP_COSGATE, TKM_OP_SOFTCAP, TKM_OP_CLAMP, TKM_OP_SCALE,
    TKM_OP_LAYERSCALE,      /* x * w                                                 (param w) */
    TKM_OP_DYT,             /* tanh(fval x) * w                                      (param w) */
    TKM_OP_PRELU,           /* x > 0 ? x : x * w * fval                              (param w) */
    TKM_OP_XATLU,           /* x * (w * sigmoid(x) + 1 - w)                          (param w) */
    TKM_OP_SOFTPLUS,        /* log(1 + exp(x))                                                */
    TKM_OP_SNAKE,           /* x + sin^2(fval x) / fval                                       */
    TKM_OP_ADD,             /* residual: x + branch_in                       (branch tensor)  */
    TKM_OP_DROP,            /* Drop: keep with probability 1 - fval, scaled by 1 / (1 - fval); the
                               mask is drawn per channel pair from the node's generator, seeded by
                               the step seed (registry src/tkm_registry.c:426-434)  (mask, seed) */
    TKM_OP_FORMULA,         /* a pointwise op of the reference registry that this build has no
                               formula of its own for: its TkmOpSpec code (fwd_cuda / bwd_cuda,
                               or fwd_expr / bwd_expr) is emitted as the registry holds it.  Only
                               the whole-graph generator (tkm_codegen_hip.c, front end linked)
                               can give it; the descriptor API rejects it                    */
    TKM_OP_FORMULA_W,       /* the same with a weight vector                          (param w) */
    TKM_OP_FORMULA_B,       /* the same with a bias vector                            (param b) */
    TKM_OP_COUNT
};

/* Argument kinds of the generated kernels. */
enum {
    TKM_ARG_IN = 0,         /* group input rows; in the backward: the replay input */
    TKM_ARG_OUT,            /* group output rows */
    TKM_ARG_DOUT,           /* gradient of the output */
    TKM_ARG_DIN,            /* gradient of the input (written, or accumulated) */
    TKM_ARG_WEIGHT,         /* C floats */
    TKM_ARG_BETA,           /* C floats */
    TKM_ARG_BIAS,           /* C floats */
    TKM_ARG_SAVE_XHAT,      /* [rows][C] 16-bit */
    TKM_ARG_SAVE_ISTD,      /* [rows][ceil(C/64)] floats */
    TKM_ARG_BRANCH_IN,      /* [rows][C] 16-bit residual input */
    TKM_ARG_DBRANCH,        /* [rows][C] 16-bit gradient of the residual input */
    TKM_ARG_DWEIGHT,        /* C floats */
    TKM_ARG_DBETA,          /* C floats */
    TKM_ARG_DBIAS,          /* C floats */
    TKM_ARG_SAVE_MASK,      /* [rows][C/2] uint16: Drop's keep bits of a channel pair (bit 0 of
                               byte 0: even channel, byte 1: odd channel) */
    TKM_ARG_SEED            /* one uint32: the step seed (advanced by the runtime's SGD) */
};

/* Accumulation flags of tkm_plasma_bwd (the reference: a plain group accumulates din, a twin
 * group overwrites it; parameter gradients and residual gradients always accumulate). */
enum { TKM_PLASMA_ACC_DIN = 1, TKM_PLASMA_ACC_PARAMS = 2, TKM_PLASMA_ACC_BRANCH = 4 };

#define TKM_PLASMA_MAX_NODES 8

typedef struct tkm_plasma_node {
    int op;                 /* TKM_OP_* */
    float fval;             /* the op's constant (registry default if unsure) */
    int rng_type;           /* Drop: generator, the TkmRngType values 1..4 (xorshift32,
                               wang_xorshift32, pcg32, philox); 0 = wang_xorshift32 */
    int node_id;            /* Drop: the graph node id; the generator is seeded with
                               step_seed ^ (node_id * 19937 + 1) (src/tkm_codegen.c:310-313) */
} tkm_plasma_node;

typedef struct tkm_plasma_desc {
    int group_id;           /* N of tkm_plasma_{fwd,bwd}_g<N> */
    int channels;           /* C: a multiple of 8 */
    int twin;               /* 0 or 1 */
    int n_main;             /* plain: the chain; twin: the ops after the product */
    int n_left, n_right;    /* twin: the two gate chains */
    tkm_plasma_node main_ops[TKM_PLASMA_MAX_NODES];
    tkm_plasma_node left_ops[TKM_PLASMA_MAX_NODES];
    tkm_plasma_node right_ops[TKM_PLASMA_MAX_NODES];
    int dtype;              /* TKM_ATTN_F16 or TKM_ATTN_BF16 */
} tkm_plasma_desc;

typedef struct tkm_plasma tkm_plasma;

/* The registry's default constant of an op (reference src/tkm_registry.c), 0 if none. */
TKM_ATTN_API float tkm_plasma_default_fval(int op);

/* HIP source (prelude included) for d, or NULL on a bad descriptor; free with tkm_free. */
TKM_ATTN_API char *tkm_plasma_source(const tkm_plasma_desc *d);

/* Emit + hipRTC-compile + load on the current (gfx950) device.  Not capturable. */
TKM_ATTN_API int tkm_plasma_create(const tkm_plasma_desc *d, tkm_plasma **out);
TKM_ATTN_API void tkm_plasma_destroy(tkm_plasma *p);

/* Pointer list of a pass (0 = forward, 1 = backward): count, then kind and node of entry i.
 * node is the op's index in the chain (left ops first, then right, then main, for a twin
 * group), -1 for the group tensors (IN, OUT, DOUT, DIN). */
TKM_ATTN_API int tkm_plasma_num_args(const tkm_plasma *p, int pass);
TKM_ATTN_API int tkm_plasma_arg(const tkm_plasma *p, int pass, int i, int *kind, int *node);

TKM_ATTN_API int tkm_plasma_fwd(const tkm_plasma *p, void *const *args, int rows, void *stream);
TKM_ATTN_API size_t tkm_plasma_bwd_workspace_bytes(const tkm_plasma *p, int rows);
TKM_ATTN_API int tkm_plasma_bwd(const tkm_plasma *p, void *const *args, int rows, int acc_flags,
                                void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TKM_PLASMA_H */
