/* Internal declarations of the plasma-epilogue generator and runtime (not installed). */
#ifndef TKM_PLASMA_INTERNAL_H
#define TKM_PLASMA_INTERNAL_H

#include "tkm_plasma.h"
#include "tkm_codegen_internal.h"
#include "tkm_prep_internal.h"

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TKM_PLASMA_FWD_RPI = 4,        /* forward: rows per lane slot per block */
    TKM_PLASMA_MAX_ARGS = 4 + 7 * 3 * TKM_PLASMA_MAX_NODES
};

typedef struct {
    int kind, node;
} tkm_plasma_argd;

/* A chain op's code as the reference registry holds it (TkmOpSpec): the CUDA snippets of a
 * pointwise op (fwd_cuda / bwd_cuda, on the channel pair v / pre / dy, with fval, w_vec[tid],
 * b_vec[tid], acc_dw, acc_db), or a user formula (fwd_expr / bwd_expr in x and fval, expr = 1).
 * fwd = NULL: the op's own formula of this build. */
typedef struct {
    const char *fwd, *bwd;
    int expr;
} tkm_plasma_formula;

typedef struct {
    int C, CW, CH;      /* channels, channels per lane chunk (8, or 2 when C % 8 != 0), chunks per row */
    int L, RW, XB;      /* lanes per row, rows per wave, blocks across a row */
    int NGL, NG;        /* lanes per norm group, norm groups per row */
    int n_nodes;
    int n_fwd, n_bwd, n_par;
    tkm_plasma_argd fwd[TKM_PLASMA_MAX_ARGS], bwd[TKM_PLASMA_MAX_ARGS], par[TKM_PLASMA_MAX_ARGS];
    int part_width;     /* n_par * C */
    const tkm_plasma_formula *formulas;   /* per chain position, or NULL (set while emitting) */
} tkm_plasma_geom;

TKM_HIDDEN int tkm_plasma_check_desc(const tkm_plasma_desc *d);
/* The descriptor's checks with the registry code of its chain (formulas may be NULL): an op of
 * the TKM_OP_FORMULA family needs both snippets. */
TKM_HIDDEN int tkm_plasma_check_desc_f(const tkm_plasma_desc *d, const tkm_plasma_formula *formulas);
/* 1 for an op computed element by element that may take registry code (no norm, mask or branch). */
TKM_HIDDEN int tkm_plasma_op_pointwise(int op);
TKM_HIDDEN void tkm_plasma_geometry(const tkm_plasma_desc *d, tkm_plasma_geom *g);

/* Internal argument list of the forward (pass 0) or backward (pass 1) kernel: pointer
 * arguments, then the scalars (forward: rows; backward: part, rows, band, acc_flags).
 * `out` holds TKM_KPLAN_MAX entries; returns the count. */
TKM_HIDDEN int tkm_plasma_need(const tkm_plasma_desc *d, int pass, tkm_kparam *out);
/* Appends the group's constants and kernels to s (no prelude); plans may be NULL (internal
 * order); `scoped` confines helpers and macros so that many groups share one source. */
TKM_HIDDEN int tkm_plasma_emit(tkm_sbuf *s, const tkm_plasma_desc *d, const tkm_kplan *fwd_plan,
                               const tkm_kplan *bwd_plan, int scoped, const tkm_plasma_formula *formulas);

#ifdef __cplusplus
}
#endif

#endif
