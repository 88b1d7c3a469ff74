/* Internal declarations shared by the HIP code generators (qkv-prep, plasma, whole graph). */
#ifndef TKM_CODEGEN_INTERNAL_H
#define TKM_CODEGEN_INTERNAL_H

#include <stddef.h>

#include "tkm_prep.h"
#include "tkm_prep_internal.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Growable text buffer; `failed` latches on allocation failure. */
typedef struct {
    char *buf;
    size_t len, cap;
    int failed;
} tkm_sbuf;

TKM_HIDDEN void tkm_sb_add(tkm_sbuf *s, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

/* Parameter plans.  A generated kernel body refers to its arguments by internal names (kind,
 * chain node).  A plan lists the kernel's parameters in launch order, each with its declared C
 * type and name and the internal argument it carries; the body then reads its internal names
 * through casts of the plan's parameters.  The standalone APIs (tkm_prep_*, tkm_plasma_*) use
 * plans that are the internal lists themselves; the whole-graph generator
 * (tkm_codegen_cuda_string) uses the reference's TkmKernelSig order, names and types, followed
 * by the extra arguments this build's kernels take (rows, workspace, ...). */
enum {
    TKM_KP_UNUSED = -1,           /* a parameter the kernel does not read */
    TKM_KP_ROWS = 100,            /* int rows */
    TKM_KP_PART = 101,            /* float * partial sums (backward workspace) */
    TKM_KP_BAND = 102,            /* int rows per band */
    TKM_KP_ACC = 103              /* int accumulation flags */
};

#define TKM_KPLAN_MAX 192

typedef struct {
    int kind, node;
    char decl[48];
    char name[40];
} tkm_kparam;

typedef struct {
    int n;
    tkm_kparam p[TKM_KPLAN_MAX];
} tkm_kplan;

/* Appends a parameter; returns 0, or -1 when the plan is full. */
TKM_HIDDEN int tkm_kplan_add(tkm_kplan *pl, int kind, int node, const char *decl, const char *name);

/* Emits `(\n decl name, ...)\n{\n` for the plan, then, for every internal argument of `need`
 * (n_need entries) whose plan parameter has another name, a local of the internal declaration
 * and name cast from that parameter, and `(void)` for unused parameters.  Returns 0, or -1
 * when an internal argument has no parameter in the plan. */
TKM_HIDDEN int tkm_emit_plan_params(tkm_sbuf *s, const tkm_kplan *plan, const tkm_kparam *need, int n_need);

/* qkv-prep generator (tkm_prep_codegen.c): internal argument list of pass 0 / 1 (kinds of
 * include/tkm_plasma.h, node 0 = the qkv_prep node), and the group's emission (no prelude). */
TKM_HIDDEN int tkm_prep_need(int pass, tkm_kparam *out);
TKM_HIDDEN int tkm_prep_emit(tkm_sbuf *s, const tkm_prep_desc *d, const tkm_kplan *fwd_plan,
                             const tkm_kplan *bwd_plan, int scoped);

/* Whole-graph generator (tkm_codegen_hip.c): the parameter plan of group gid's forward (pass
 * 0) or backward (pass 1) kernel -- the TkmKernelSig's parameters, then this build's extras --
 * and the graph node of every chain position (n_chain entries).  Needs tkm.h's TkmGraph. */
struct TkmGraph;
TKM_HIDDEN int tkm_hip_group_plan(const struct TkmGraph *g, int gid, int pass, int dtype, tkm_kplan *plan,
                                  int *chain_nodes, int *n_chain);

#ifdef __cplusplus
}
#endif

#endif
