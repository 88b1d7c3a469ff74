/*
 * plasma_ref.c -- CPU oracle of the plasma epilogues (chains of row-wise ops behind a GEMM).
 * TEST INFRASTRUCTURE ONLY: tests/ compare the generated HIP kernels against it; no product
 * code path links, loads or calls it.
 *
 * Semantics restated from the reference (no CPU version exists there):
 *   chain forward / output store      src/tkm_codegen.c:484-518 (emit_plasma_group)
 *   per-op forward and backward       src/tkm_registry.c:186-456 (op registry), norms as
 *                                     emitted at src/tkm_codegen.c:297-353, 411-444
 *   backward with replayed inputs     src/tkm_codegen.c:519-625, 464-482 (norm outputs are
 *                                     replayed from the saved 16-bit xhat)
 *   twin (gated) groups               src/tkm_codegen.c:509-515, 548-584
 * Norm statistics (F7): sums over aligned 64-channel groups when C > 64 (the whole row when
 * C <= 64), divided by C.  Deliberate differences: istd per (row, group) (the reference keeps
 * group 0's value per row); a residual Add and a Drop are applied in the replay (the reference
 * skips both, src/tkm_codegen.c:478-479).  Drop (registry src/tkm_registry.c:426-434) takes
 * its keep bits from pr_drop_keep, which restates the prelude's generators.
 *
 * Arithmetic in double from the rounded inputs; outputs rounded once to the storage type.
 * dtype: 0 fp16, 1 bf16, 2 fp32.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "plasma_ref.h"
#include "qkv_prep_ref.h"

#include <stdint.h>

enum { F_W = 1, F_BETA = 2, F_BIAS = 4, F_NORM = 8, F_BRANCH = 16, F_MASK = 32 };

static int op_flags(int op) {
    switch (op) {
        case PR_BIAS: return F_BIAS;
        case PR_RMSNORM: return F_NORM | F_W;
        case PR_LN: case PR_BN: return F_NORM | F_W | F_BETA;
        case PR_L2NORM: return F_NORM;
        case PR_LAYERSCALE: case PR_DYT: case PR_PRELU: case PR_XATLU: return F_W;
        case PR_ADD: return F_BRANCH;
        case PR_DROP: return F_MASK;
        default: return 0;
    }
}

int pr_op_flags(int op) { return op >= 0 && op < PR_OP_COUNT ? op_flags(op) : -1; }

/* ---- the prelude's generators (reference src/tkm_gpu.cu:751-800), restated ----------
 * Pinned bit for bit to the reference's own generator code (tests/golden/rng_vectors.npz,
 * written by running src/tkm_gpu.cu:751-794 through oracle/ref_rng_harness.hip). */
typedef struct {
    int type;
    uint32_t s;                 /* xorshift32 state */
    uint64_t state, inc;        /* PCG32 */
    uint32_t ctr, key, sub;     /* counter generator */
} pr_rng;

static uint32_t xorshift32(uint32_t x) {  /* Marsaglia's (13, 17, 5) */
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    return x;
}

static uint32_t pcg_step(pr_rng *r) {      /* PCG32 XSH-RR (O'Neill) */
    const uint64_t old = r->state;
    r->state = old * 6364136223846793005ULL + r->inc;
    const uint32_t xsh = (uint32_t)(((old >> 18u) ^ old) >> 27u), rot = (uint32_t)(old >> 59u);
    return (xsh >> rot) | (xsh << ((32u - rot) & 31u));
}

static void rng_init(pr_rng *r, int type, uint32_t seed, uint32_t idx) {
    memset(r, 0, sizeof *r);
    r->type = type;
    switch (type) {
        case 1: {
            const uint32_t x = seed ^ (idx * 0x9E3779B9u + 0x7F4A7C15u);
            r->s = x ? x : 1u;
            break;
        }
        case 3:   /* pcg32_srandom(seed ^ 0x853C49E6748FEA9B, idx) */
            r->inc = ((uint64_t)idx << 1u) | 1u;
            (void)pcg_step(r);
            r->state += (uint64_t)seed ^ 0x853C49E6748FEA9BULL;
            (void)pcg_step(r);
            break;
        case 4:
            r->ctr = idx;
            r->key = seed;
            r->sub = 0;
            break;
        default: {  /* Thomas Wang's 32-bit integer hash of seed ^ idx */
            r->type = 2;
            uint32_t k = seed ^ idx;
            k = ~k + (k << 18);
            k ^= k >> 31;
            k = (k + (k << 2)) + (k << 4);
            k ^= k >> 11;
            k += k << 6;
            k ^= k >> 22;
            r->s = k ? k : 1u;
        }
    }
}

static uint32_t rng_next(pr_rng *r) {
    if (r->type == 3) return pcg_step(r);
    if (r->type == 4) {
        uint32_t c0 = r->ctr, c1 = r->sub++, k0 = r->key;
        for (int i = 0; i < 7; i++) {
            const uint64_t prod = (uint64_t)0xD2511F53u * c0;
            const uint32_t hi = (uint32_t)(prod >> 32), lo = (uint32_t)prod;
            c0 = hi ^ c1 ^ k0;
            c1 = lo;
            k0 += 0x9E3779B9u;
        }
        return c0;
    }
    return r->s = xorshift32(r->s);
}

int pr_rng_u32(int type, unsigned seed, unsigned idx, int n, unsigned *out) {
    if (!out || n < 0 || type < 0 || type > 4) return -1;
    pr_rng r;
    rng_init(&r, type, seed, idx);
    for (int i = 0; i < n; ++i) out[i] = rng_next(&r);
    return 0;
}

int pr_drop_keep(int rows, int C, unsigned step_seed, int node_id, int rng_type, float p, unsigned char *keep) {
    if (!keep || rows < 0 || C <= 0 || C % 2 || !(p >= 0.0f && p < 1.0f) || rng_type < 0 || rng_type > 4) return -1;
    const float kp = 1.0f - p;
    const uint32_t sd = (uint32_t)step_seed ^ ((uint32_t)node_id * 19937u + 1u);
    for (int r = 0; r < rows; ++r)
        for (int t = 0; t < C / 2; ++t) {
            pr_rng g;
            rng_init(&g, rng_type, sd, (uint32_t)((size_t)r * (C / 2) + t));
            for (int e = 0; e < 2; ++e) {
                const float u = (float)(rng_next(&g) >> 8) * (1.0f / 16777216.0f);
                keep[(size_t)r * C + 2 * t + e] = u < kp;
            }
        }
    return 0;
}

/* Drop's scale 1 / (1 - p), as the fp32 constant of the registry's snippet */
static double drop_scale(double p) { return (double)(1.0f / (1.0f - (float)p)); }

static double sigm(double x) { return 1.0 / (1.0 + exp(-x)); }

/* y = f(x) of a pointwise op (w: weight element, b: bias element) */
double pr_op_fwd(int op, double fv, double x, double w, double b) {
    const double k = 0.79788456, a = 0.044715;
    switch (op) {
        case PR_BIAS: return x + b;
        case PR_SILU: return x * sigm(x);
        case PR_RELU: return x > 0 ? x : 0.0;
        case PR_RELU2: return x > 0 ? x * x : 0.0;
        case PR_LEAKY_RELU: return x > 0 ? x : x * fv;
        case PR_ELU: return x > 0 ? x : fv * (exp(x) - 1.0);
        case PR_GELU: return 0.5 * x * (1.0 + tanh(k * (x + a * x * x * x)));
        case PR_MISH: return x * tanh(x > 20.0 ? x : log1p(exp(x)));
        case PR_HARDSWISH: return x * fmin(fmax(x + 3.0, 0.0), 6.0) / 6.0;
        case PR_HARDSIGMOID: return fmin(fmax((x + 3.0) / 6.0, 0.0), 1.0);
        case PR_TANH: return tanh(x);
        case PR_SIGMOID: return sigm(x);
        case PR_SWISH_BETA: return x * sigm(fv * x);
        case PR_SIN: return sin(fv * x);
        case PR_COSGATE: return x * cos(x);
        case PR_SOFTCAP: return fv * tanh(x / fv);
        case PR_CLAMP: return fmin(fmax(x, -fv), fv);
        case PR_SCALE: return x * fv;
        case PR_LAYERSCALE: return x * w;
        case PR_DYT: return tanh(fv * x) * w;
        case PR_PRELU: return x > 0 ? x : x * w * fv;
        case PR_XATLU: return x * (w * sigm(x) + 1.0 - w);
        /* the reference's user formula log(1.0 + exp(x)) (tkm_registry.c:446-448) runs in
           float: expf overflows above ln(FLT_MAX) and the result is +inf */
        case PR_SOFTPLUS: { const double e = exp(x); return isinf((float)e) ? INFINITY : log1p(e); }
        case PR_SNAKE: { const double s = sin(fv * x); return x + s * s / fv; }
        default: return x;
    }
}

/* dy/dx at p, and (through *dw) dy/dw */
double pr_op_grad(int op, double fv, double p, double w, double *dw) {
    const double k = 0.79788456, a = 0.044715;
    *dw = 0.0;
    switch (op) {
        case PR_BIAS: return 1.0;
        case PR_SILU: { const double s = sigm(p); return s * (1.0 + p * (1.0 - s)); }
        case PR_RELU: return p > 0 ? 1.0 : 0.0;
        case PR_RELU2: return p > 0 ? 2.0 * p : 0.0;
        case PR_LEAKY_RELU: return p > 0 ? 1.0 : fv;
        case PR_ELU: return p > 0 ? 1.0 : fv * exp(p);
        case PR_GELU: {
            const double t = tanh(k * (p + a * p * p * p));
            return 0.5 * (1.0 + t) + 0.5 * p * (1.0 - t * t) * k * (1.0 + 3.0 * a * p * p);
        }
        case PR_MISH: {
            const double t = tanh(p > 20.0 ? p : log1p(exp(p)));
            return t + p * (1.0 - t * t) * sigm(p);
        }
        case PR_HARDSWISH: return p <= -3.0 ? 0.0 : (p >= 3.0 ? 1.0 : (2.0 * p + 3.0) / 6.0);
        case PR_HARDSIGMOID: return (p > -3.0 && p < 3.0) ? 1.0 / 6.0 : 0.0;
        case PR_TANH: { const double t = tanh(p); return 1.0 - t * t; }
        case PR_SIGMOID: { const double s = sigm(p); return s * (1.0 - s); }
        case PR_SWISH_BETA: { const double s = sigm(fv * p); return s * (1.0 + fv * p * (1.0 - s)); }
        case PR_SIN: return fv * cos(fv * p);
        case PR_COSGATE: return cos(p) - p * sin(p);
        case PR_SOFTCAP: { const double t = tanh(p / fv); return 1.0 - t * t; }
        case PR_CLAMP: return (p > -fv && p < fv) ? 1.0 : 0.0;
        case PR_SCALE: return fv;
        case PR_LAYERSCALE: *dw = p; return w;
        case PR_DYT: { const double t = tanh(fv * p); *dw = t; return w * fv * (1.0 - t * t); }
        case PR_PRELU: if (p <= 0) *dw = p * fv; return p > 0 ? 1.0 : w * fv;
        case PR_XATLU: {
            const double s = sigm(p);
            *dw = p * (s - 1.0);
            return (1.0 - w) + w * s * (1.0 + p * (1.0 - s));
        }
        case PR_SOFTPLUS: return sigm(p);
        case PR_SNAKE: return 1.0 + sin(2.0 * fv * p);
        default: return 1.0;
    }
}

static int nodes_ok(const pr_node *nodes, int n) {
    for (int k = 0; k < n; ++k)
        if (nodes[k].op < 0 || nodes[k].op >= PR_OP_COUNT) return 0;
    return 1;
}

/* Norm of one row in place: groups of 64 (or the row), sums / C; stores xhat (rounded) and istd. */
static void norm_fwd(int op, double eps, double *v, int C, const float *w, const float *beta, int dtype,
                     float *xhat_row, float *istd_row) {
    const int G = C <= 64 ? C : 64;
    for (int g0 = 0, gi = 0; g0 < C; g0 += G, ++gi) {
        const int g1 = g0 + G < C ? g0 + G : C;
        double sm = 0.0, sq = 0.0;
        for (int c = g0; c < g1; ++c) {
            sm += v[c];
            sq += v[c] * v[c];
        }
        const int ln = (op == PR_LN || op == PR_BN);
        const double m = ln ? sm / C : 0.0;
        const double var = ln ? fmax(0.0, sq / C - m * m) : sq / C;
        const double is = 1.0 / sqrt(var + eps);
        istd_row[gi] = (float)is;
        for (int c = g0; c < g1; ++c) {
            const double xh = (v[c] - m) * is;
            xhat_row[c] = (float)qp_round(xh, dtype);
            v[c] = ln ? xh * w[c] + beta[c] : (op == PR_RMSNORM ? xh * w[c] : xh);
        }
    }
}

static void apply_node(const pr_node *n, int k, double *v, int C, int r, const pr_params *P, int dtype,
                       float *const *xhat, float *const *istd, int NG) {
    const int f = op_flags(n->op);
    if (f & F_NORM) {
        norm_fwd(n->op, n->fval, v, C, P->w[k], P->beta[k], dtype, xhat[k] + (size_t)r * C, istd[k] + (size_t)r * NG);
    } else if (f & F_BRANCH) {
        for (int c = 0; c < C; ++c) v[c] += P->branch[k][(size_t)r * C + c];
    } else if (f & F_MASK) {
        const double ikp = drop_scale(n->fval);
        for (int c = 0; c < C; ++c) v[c] = P->keep[k][(size_t)r * C + c] ? v[c] * ikp : 0.0;
    } else {
        for (int c = 0; c < C; ++c)
            v[c] = pr_op_fwd(n->op, n->fval, v[c], (f & F_W) ? P->w[k][c] : 0.0, (f & F_BIAS) ? P->bias[k][c] : 0.0);
    }
}

int pr_fwd(const float *in, int rows, int C, int twin, const pr_node *nodes, int n_left, int n_right,
           int n_main, const pr_params *P, int dtype, float *out, float *const *xhat, float *const *istd) {
    const int nn = twin ? n_left + n_right + n_main : n_main;
    if (!in || !out || !P || rows < 0 || C <= 0 || !nodes_ok(nodes, nn)) return -1;
    const int NG = (C + 63) / 64;
    double *v = (double *)malloc(sizeof(double) * 2 * (size_t)C);
    if (!v) return -1;
    double *u = v + C;
    for (int r = 0; r < rows; ++r) {
        const int W = twin ? 2 * C : C;
        for (int c = 0; c < C; ++c) v[c] = in[(size_t)r * W + c];
        int k = 0;
        if (twin) {
            for (int c = 0; c < C; ++c) u[c] = in[(size_t)r * W + C + c];
            for (; k < n_left; ++k) apply_node(&nodes[k], k, v, C, r, P, dtype, xhat, istd, NG);
            for (; k < n_left + n_right; ++k) apply_node(&nodes[k], k, u, C, r, P, dtype, xhat, istd, NG);
            for (int c = 0; c < C; ++c) v[c] *= u[c];
        }
        for (; k < nn; ++k) apply_node(&nodes[k], k, v, C, r, P, dtype, xhat, istd, NG);
        for (int c = 0; c < C; ++c) out[(size_t)r * C + c] = (float)qp_round(v[c], dtype);
    }
    free(v);
    return 0;
}

int pr_bwd(const float *dout, const float *in, int rows, int C, int twin, const pr_node *nodes, int n_left,
           int n_right, int n_main, const pr_params *P, const float *const *xhat, const float *const *istd,
           int dtype, int acc_flags, float *din, float *const *dbranch, double *const *dw, double *const *dbeta,
           double *const *dbias) {
    const int nn = twin ? n_left + n_right + n_main : n_main;
    if (!dout || !in || !din || !P || rows < 0 || C <= 0 || nn > PR_MAX_NODES || !nodes_ok(nodes, nn)) return -1;
    const int NG = (C + 63) / 64, G = C <= 64 ? C : 64;
    const int W = twin ? 2 * C : C;
    const int kpost = twin ? n_left + n_right : 0;
    double *buf = (double *)malloc(sizeof(double) * (size_t)C * (2 * PR_MAX_NODES + 8));
    if (!buf) return -1;
    double *pre = buf;                                   /* [nn][C]: input of each node */
    double *v = buf + (size_t)PR_MAX_NODES * C, *u = v + C, *gl = u + C, *gr = gl + C, *g = gr + C, *g2 = g + C;
    if (!(acc_flags & 2)) {
        for (int k = 0; k < nn; ++k) {
            const int f = op_flags(nodes[k].op);
            for (int c = 0; c < C; ++c) {
                if (f & F_W) dw[k][c] = 0.0;
                if (f & F_BETA) dbeta[k][c] = 0.0;
                if (f & F_BIAS) dbias[k][c] = 0.0;
            }
        }
    }
    for (int r = 0; r < rows; ++r) {
        /* replay */
        for (int c = 0; c < C; ++c) v[c] = in[(size_t)r * W + c];
        if (twin)
            for (int c = 0; c < C; ++c) u[c] = in[(size_t)r * W + C + c];
        for (int k = 0; k < nn; ++k) {
            if (twin && k == kpost) {
                memcpy(gl, v, sizeof(double) * C);
                memcpy(gr, u, sizeof(double) * C);
                for (int c = 0; c < C; ++c) v[c] *= u[c];
            }
            double *x = (twin && k >= n_left && k < kpost) ? u : v;
            memcpy(pre + (size_t)k * C, x, sizeof(double) * C);
            const pr_node *n = &nodes[k];
            const int f = op_flags(n->op);
            if (f & F_NORM) {
                const float *xh = xhat[k] + (size_t)r * C;
                for (int c = 0; c < C; ++c)
                    x[c] = (n->op == PR_LN || n->op == PR_BN) ? xh[c] * (double)P->w[k][c] + P->beta[k][c]
                           : (n->op == PR_RMSNORM ? xh[c] * (double)P->w[k][c] : xh[c]);
            } else if (f & F_BRANCH) {
                for (int c = 0; c < C; ++c) x[c] += P->branch[k][(size_t)r * C + c];
            } else if (f & F_MASK) {   /* replayed from the saved keep bits */
                const double ikp = drop_scale(n->fval);
                for (int c = 0; c < C; ++c) x[c] = P->keep[k][(size_t)r * C + c] ? x[c] * ikp : 0.0;
            } else {
                for (int c = 0; c < C; ++c)
                    x[c] = pr_op_fwd(n->op, n->fval, x[c], (f & F_W) ? P->w[k][c] : 0.0, (f & F_BIAS) ? P->bias[k][c] : 0.0);
            }
        }
        if (twin && nn == kpost) {
            memcpy(gl, v, sizeof(double) * C);
            memcpy(gr, u, sizeof(double) * C);
        }
        /* backward */
        for (int c = 0; c < C; ++c) g[c] = dout[(size_t)r * C + c];
        for (int pass = 0; pass < (twin ? 3 : 1); ++pass) {
            int k_hi, k_lo;
            double *gg;
            if (!twin) { k_hi = nn - 1; k_lo = 0; gg = g; }
            else if (pass == 0) { k_hi = nn - 1; k_lo = kpost; gg = g; }
            else if (pass == 1) {
                for (int c = 0; c < C; ++c) { g2[c] = g[c] * gl[c]; g[c] = g[c] * gr[c]; }
                k_hi = kpost - 1; k_lo = n_left; gg = g2;       /* right chain gets dy * left */
            } else { k_hi = n_left - 1; k_lo = 0; gg = g; }      /* left chain gets dy * right */
            for (int k = k_hi; k >= k_lo; --k) {
                const pr_node *n = &nodes[k];
                const int f = op_flags(n->op);
                const double *p = pre + (size_t)k * C;
                if (f & F_NORM) {
                    const float *xh = xhat[k] + (size_t)r * C;
                    const int ln = (n->op == PR_LN || n->op == PR_BN);
                    for (int g0 = 0, gi = 0; g0 < C; g0 += G, ++gi) {
                        const int g1 = g0 + G < C ? g0 + G : C;
                        double m1 = 0.0, m2 = 0.0;
                        for (int c = g0; c < g1; ++c) {
                            const double dxh = (f & F_W) ? gg[c] * P->w[k][c] : gg[c];
                            if (f & F_W) dw[k][c] += gg[c] * xh[c];
                            if (f & F_BETA) dbeta[k][c] += gg[c];
                            m1 += dxh;
                            m2 += dxh * xh[c];
                        }
                        m1 /= C;
                        m2 /= C;
                        const double is = istd[k][(size_t)r * NG + gi];
                        for (int c = g0; c < g1; ++c) {
                            const double dxh = (f & F_W) ? gg[c] * P->w[k][c] : gg[c];
                            gg[c] = is * (dxh - (ln ? m1 : 0.0) - xh[c] * m2);
                        }
                    }
                } else if (f & F_BRANCH) {
                    for (int c = 0; c < C; ++c) {
                        const size_t i = (size_t)r * C + c;
                        const double prev = (acc_flags & 4) ? dbranch[k][i] : 0.0;
                        dbranch[k][i] = (float)qp_round(prev + gg[c], dtype);
                    }
                } else if (f & F_MASK) {
                    const double ikp = drop_scale(n->fval);
                    for (int c = 0; c < C; ++c) gg[c] *= P->keep[k][(size_t)r * C + c] ? ikp : 0.0;
                } else {
                    for (int c = 0; c < C; ++c) {
                        double dwe;
                        const double d = pr_op_grad(n->op, n->fval, p[c], (f & F_W) ? P->w[k][c] : 0.0, &dwe);
                        if (f & F_BIAS) dbias[k][c] += gg[c];
                        if (f & F_W) dw[k][c] += gg[c] * dwe;
                        gg[c] *= d;
                    }
                }
            }
        }
        for (int c = 0; c < C; ++c) {
            const size_t i = (size_t)r * W + c;
            din[i] = (float)qp_round(((acc_flags & 1) ? din[i] : 0.0) + g[c], dtype);
            if (twin) din[i + C] = (float)qp_round(((acc_flags & 1) ? din[i + C] : 0.0) + g2[c], dtype);
        }
    }
    free(buf);
    return 0;
}
