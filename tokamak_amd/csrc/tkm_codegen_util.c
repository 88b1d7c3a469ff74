/* Text buffer and parameter plans shared by the HIP code generators (tkm_codegen_internal.h). */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tkm_codegen_internal.h"

void tkm_sb_add(tkm_sbuf *s, const char *fmt, ...) {
    if (s->failed) return;
    for (;;) {
        va_list ap;
        va_start(ap, fmt);
        int n = vsnprintf(s->buf ? s->buf + s->len : NULL, s->buf ? s->cap - s->len : 0, fmt, ap);
        va_end(ap);
        if (n < 0) {
            s->failed = 1;
            return;
        }
        if (s->buf && (size_t)n < s->cap - s->len) {
            s->len += (size_t)n;
            return;
        }
        size_t cap = (s->cap + (size_t)n + 1) * 2;
        char *nb = (char *)realloc(s->buf, cap);
        if (!nb) {
            s->failed = 1;
            return;
        }
        s->buf = nb;
        s->cap = cap;
    }
}

int tkm_kplan_add(tkm_kplan *pl, int kind, int node, const char *decl, const char *name) {
    if (pl->n >= TKM_KPLAN_MAX) return -1;
    tkm_kparam *p = &pl->p[pl->n++];
    p->kind = kind;
    p->node = node;
    snprintf(p->decl, sizeof p->decl, "%s", decl);
    snprintf(p->name, sizeof p->name, "%s", name);
    return 0;
}

int tkm_emit_plan_params(tkm_sbuf *s, const tkm_kplan *plan, const tkm_kparam *need, int n_need) {
    tkm_sb_add(s, "(\n");
    for (int i = 0; i < plan->n; ++i)
        tkm_sb_add(s, "    %s %s%s\n", plan->p[i].decl, plan->p[i].name, i + 1 < plan->n ? "," : "");
    tkm_sb_add(s, ")\n{\n");
    for (int k = 0; k < n_need; ++k) {
        const tkm_kparam *q = &need[k];
        int found = -1;
        for (int i = 0; i < plan->n && found < 0; ++i)
            if (plan->p[i].kind == q->kind && plan->p[i].node == q->node) found = i;
        if (found < 0) return -1;
        if (strcmp(plan->p[found].name, q->name) != 0)
            tkm_sb_add(s, "    %s %s = (%s)%s;\n", q->decl, q->name, q->decl, plan->p[found].name);
    }
    for (int i = 0; i < plan->n; ++i)
        if (plan->p[i].kind == TKM_KP_UNUSED) tkm_sb_add(s, "    (void)%s;\n", plan->p[i].name);
    return 0;
}
