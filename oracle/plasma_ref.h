/*
 * plasma_ref.h -- CPU oracle of the plasma epilogues (chains of row-wise ops).
 * TEST INFRASTRUCTURE ONLY; semantics and reference citations in plasma_ref.c.
 */
#ifndef TKM_PLASMA_REF_H
#define TKM_PLASMA_REF_H

#ifdef __cplusplus
extern "C" {
#endif

/* op codes, in the order of the product's TKM_OP_* (include/tkm_plasma.h) */
enum {
    PR_BIAS = 0, PR_RMSNORM, PR_LN, PR_BN, PR_L2NORM, PR_SILU, PR_RELU, PR_RELU2, PR_LEAKY_RELU, PR_ELU,
    PR_GELU, PR_MISH, PR_HARDSWISH, PR_HARDSIGMOID, PR_TANH, PR_SIGMOID, PR_SWISH_BETA, PR_SIN, PR_COSGATE,
    PR_SOFTCAP, PR_CLAMP, PR_SCALE, PR_LAYERSCALE, PR_DYT, PR_PRELU, PR_XATLU, PR_SOFTPLUS, PR_SNAKE, PR_ADD,
    PR_DROP, PR_OP_COUNT
};
#define PR_MAX_NODES 24

typedef struct { int op; float fval; } pr_node;

/* Per-node parameter arrays, indexed by node (NULL where a node has none): C floats each;
 * branch: [rows][C] residual input of an Add node. */
typedef struct {
    const float *const *w, *const *beta, *const *bias, *const *branch;
    const unsigned char *const *keep;   /* Drop nodes: [rows][C] keep bits (0 or 1) */
} pr_params;

/* The generators of the reference's NVRTC prelude (src/tkm_gpu.cu:751-800): type 1
 * xorshift32, 2 Wang hash + xorshift32, 3 PCG32, 4 the 7-round multiply-xor counter generator
 * (0 = 2).  Writes n successive rng_u32 draws after rng_init(seed, idx). */
int pr_rng_u32(int type, unsigned seed, unsigned idx, int n, unsigned *out);
/* Drop's keep bits of a [rows][C] tensor (registry src/tkm_registry.c:426-434, seeding as
 * src/tkm_codegen.c:310-313): the pair (2t, 2t+1) of row r draws from a generator initialized
 * with (step_seed ^ (node_id * 19937 + 1), r * C/2 + t); keep = uniform < 1 - p. */
int pr_drop_keep(int rows, int C, unsigned step_seed, int node_id, int rng_type, float p, unsigned char *keep);

int pr_op_flags(int op);
double pr_op_fwd(int op, double fv, double x, double w, double b);
double pr_op_grad(int op, double fv, double p, double w, double *dw);

/* in: [rows][C] or, twin, [rows][2C]; out: [rows][C]; xhat[k]: [rows][C], istd[k]:
 * [rows][ceil(C/64)] for norm nodes k.  Nodes: twin = left, right, then main. */
int pr_fwd(const float *in, int rows, int C, int twin, const pr_node *nodes, int n_left, int n_right,
           int n_main, const pr_params *P, int dtype, float *out, float *const *xhat, float *const *istd);

/* acc_flags: 1 din accumulates (din holds the previous values), 2 parameter gradients
 * accumulate, 4 residual gradients accumulate; otherwise they are overwritten. */
int pr_bwd(const float *dout, const float *in, int rows, int C, int twin, const pr_node *nodes, int n_left,
           int n_right, int n_main, const pr_params *P, const float *const *xhat, const float *const *istd,
           int dtype, int acc_flags, float *din, float *const *dbranch, double *const *dw, double *const *dbeta,
           double *const *dbias);

#ifdef __cplusplus
}
#endif

#endif
