/* Internal declarations of the plasma-epilogue generator and runtime (not installed). */
#ifndef TKM_PLASMA_INTERNAL_H
#define TKM_PLASMA_INTERNAL_H

#include "tkm_plasma.h"
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

typedef struct {
    int C, CH;          /* channels, 8-channel chunks per row */
    int L, RW, XB;      /* lanes per row, rows per wave, blocks across a row */
    int NGL, NG;        /* lanes per norm group, norm groups per row */
    int n_nodes;
    int n_fwd, n_bwd, n_par;
    tkm_plasma_argd fwd[TKM_PLASMA_MAX_ARGS], bwd[TKM_PLASMA_MAX_ARGS], par[TKM_PLASMA_MAX_ARGS];
    int part_width;     /* n_par * C */
} tkm_plasma_geom;

TKM_HIDDEN int tkm_plasma_check_desc(const tkm_plasma_desc *d);
TKM_HIDDEN void tkm_plasma_geometry(const tkm_plasma_desc *d, tkm_plasma_geom *g);

#ifdef __cplusplus
}
#endif

#endif
