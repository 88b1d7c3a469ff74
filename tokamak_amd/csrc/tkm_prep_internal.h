/* Internal declarations shared by the host sources of libtkm_attn.so (not installed). */
#ifndef TKM_PREP_INTERNAL_H
#define TKM_PREP_INTERNAL_H

#include <stdarg.h>

#include "tkm_prep.h"

#ifdef __cplusplus
extern "C" {
#endif

#define TKM_HIDDEN __attribute__((visibility("hidden")))

/* Records a formatted message as the calling thread's last error and returns status. */
TKM_HIDDEN int tkm_set_error(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
TKM_HIDDEN int tkm_vset_error(int status, const char *fmt, va_list ap);

/* Launch geometry of the generated qkv-prep kernels. */
enum {
    TKM_PREP_FWD_RPW = 4,          /* forward: rows per wave per block */
    TKM_PREP_BWD_BATCH = 4,        /* backward: rows per wave loaded before the arithmetic */
    TKM_BWD_TARGET_BLOCKS = 2048,  /* backward: bands are chosen to give about this many blocks */
    TKM_BWD_MIN_BAND = 4,          /* backward: rows per band, at least (one row per wave:
                                    * at 4096 x 512 the rows a wave walks one after the other
                                    * cost more than the 4x larger partial rows' reduction) */
    TKM_REDUCE_WAVES = 16          /* partial-row reduction: waves per block (1024 threads) */
};

typedef struct {
    int D, C, QK, CH, QKCH, NH, G, part_width;
} tkm_prep_geom;

TKM_HIDDEN int tkm_prep_check_desc(const tkm_prep_desc *d);
TKM_HIDDEN void tkm_prep_geometry(const tkm_prep_desc *d, tkm_prep_geom *g);
/* Bands (block rows of a backward with per-band parameter partials) for `rows` rows and
 * `xblocks` blocks across a row: about TKM_BWD_TARGET_BLOCKS blocks, at least
 * TKM_BWD_MIN_BAND rows per band. */
TKM_HIDDEN int tkm_bwd_bands(int rows, int xblocks);
TKM_HIDDEN float tkm_rope_inv_freq(const tkm_prep_desc *d, int i);

/* Checks that the current device is gfx950, compiles src with hipRTC and loads it; *module
 * receives the hipModule_t. */
TKM_HIDDEN int tkm_rtc_load(const char *src, const char *name, void **module);
TKM_HIDDEN int tkm_rtc_function(void *module, const char *name, void **fn);
TKM_HIDDEN void tkm_rtc_unload(void *module);
TKM_HIDDEN int tkm_rtc_launch(void *fn, unsigned gx, unsigned gy, unsigned block, void **args, void *stream,
                              const char *what);

#ifdef __cplusplus
}
#endif

#endif
