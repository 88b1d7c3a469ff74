/* Per-thread last-error message of libtkm_attn.so (tkm_attn_last_error, include/tkm_attn.h). */
#include <stdio.h>

#include "tkm_prep_internal.h"

static _Thread_local char g_err[256] = "";

int tkm_vset_error(int status, const char *fmt, va_list ap) {
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    return status;
}

int tkm_set_error(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    tkm_vset_error(status, fmt, ap);
    va_end(ap);
    return status;
}

const char *tkm_attn_last_error(void) { return g_err; }
