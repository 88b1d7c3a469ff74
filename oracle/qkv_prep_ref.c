/*
 * qkv_prep_ref.c -- CPU oracle for the qkv-prep epilogue (bias + QKNorm + RoPE) that feeds
 * the attention kernels.  TEST INFRASTRUCTURE ONLY: tests/ compare the generated HIP kernels
 * against it; no product code path links, loads or calls it.
 *
 * Semantics restated from the reference generator (the reference has no CPU version):
 *   forward   /root/reference/src/tkm_codegen.c:211-251   bias, QKNorm, RoPE, fp16 store
 *   backward  /root/reference/src/tkm_codegen.c:253-294   inverse RoPE, QKNorm backward,
 *                                                         d(gamma), d(bias), din (+)= dy
 *   RoPE      /root/reference/src/tkm_codegen.c:43-70     inverse frequency, rescaling, rotation
 *   defaults  /root/reference/src/tkm_core.c:56-60        theta, scale, factors, context length
 * with one deliberate difference: istd is kept per (row, head).  The reference stores one istd
 * per row that every head overwrites (tkm_codegen.c:243, 280), which makes its QKNorm backward
 * wrong with more than one head.
 *
 * Arithmetic: everything in double from the (already rounded) 16-bit inputs, rounded once to
 * the storage type at the end.  The one fp32 step kept on purpose is part of the reference's
 * formula: the RoPE angle is the fp32 product (float)pos * inv_freq (tkm_codegen.c:63) with
 * inv_freq the fp32 value of the expression at tkm_codegen.c:45-62.
 *
 * Layout: rows = B*S row-major rows of C = (Hq + 2*Hkv)*D channels (Q heads | K heads | V
 * heads, tkm_registry.c:736-748); QK = (Hq + Hkv)*D; NH = Hq + Hkv; head of channel c < QK is
 * c / D; the RoPE pair of channels (c, c+1), c even, has index i = (c % D) / 2; pos = row % S.
 * dtype: 0 = fp16, 1 = bf16, 2 = fp32 (round to float only; for finite-difference checks).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "qkv_prep_ref.h"

/* Round x to the nearest value of a binary format with p significand bits, minimum normal
 * exponent emin and largest finite value maxv, ties to even. */
static double round_format(double x, int p, int emin, double maxv) {
    if (x == 0.0 || !isfinite(x)) return x;
    int k;
    frexp(x, &k);                      /* |x| = m * 2^k, m in [0.5, 1) */
    int e = k - 1;
    if (e < emin) e = emin;
    const double ulp = ldexp(1.0, e - (p - 1));
    const double r = nearbyint(x / ulp) * ulp;
    if (fabs(r) > maxv) return x > 0 ? INFINITY : -INFINITY;
    return r;
}

double qp_round(double x, int dtype) {
    switch (dtype) {
        case 0: return round_format(x, 11, -14, 65504.0);
        case 1: return round_format(x, 8, -126, 0x1.fep127);
        default: return (double)(float)x;
    }
}

/* fp32 value of the reference's inverse-frequency expression for pair i (tkm_codegen.c:45-62). */
float qp_inv_freq(float theta, float scale, float low, float high, float ocl, int D, int i) {
    volatile float t = -logf(theta) * (float)i;
    float inv_freq = expf(t / (float)D);
    if (scale > 1.0f) {
        const float wavelen = 6.283185307179586f / inv_freq;
        const float low_wavelen = ocl / low;
        const float high_wavelen = ocl / high;
        if (wavelen > low_wavelen) {
            inv_freq /= scale;
        } else if (wavelen >= high_wavelen) {
            const float smooth = (ocl / wavelen - low) / (high - low);
            volatile float f = 1.0f - smooth * (1.0f - 1.0f / scale);
            inv_freq *= f;
        }
    }
    return inv_freq;
}

static void angle(int pos, float inv_freq, double *s, double *c) {
    volatile float a = (float)pos * inv_freq;        /* fp32 product, tkm_codegen.c:63 */
    *s = sin((double)a);
    *c = cos((double)a);
}

/* Forward.  in, out: [rows][C]; bias: C; gamma: QK; inv_freq: D/2 (used when has_rope);
 * xhat: [rows][QK], istd: [rows][NH] (written when has_qknorm; may be NULL otherwise). */
int qp_fwd(const float *in, const float *bias, const float *gamma, const float *inv_freq,
           int rows, int S, int Hq, int Hkv, int D, int has_qknorm, int has_rope, int dtype,
           float *out, float *xhat, float *istd) {
    if (!in || !bias || !out || rows < 0 || S < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || (D != 64 && D != 128))
        return -1;
    if (has_qknorm && (!gamma || !xhat || !istd)) return -1;
    if (has_rope && !inv_freq) return -1;
    const int C = (Hq + 2 * Hkv) * D, QK = (Hq + Hkv) * D, NH = Hq + Hkv;
    double *v = (double *)malloc(sizeof(double) * (size_t)C);
    if (!v) return -1;
    for (int r = 0; r < rows; ++r) {
        const float *x = in + (size_t)r * C;
        for (int c = 0; c < C; ++c) v[c] = (double)x[c] + (double)bias[c];
        if (has_qknorm) {
            for (int h = 0; h < NH; ++h) {
                double sq = 0.0;
                for (int j = 0; j < D; ++j) sq += v[h * D + j] * v[h * D + j];
                const double is = 1.0 / sqrt(sq / D + 1e-5);
                istd[(size_t)r * NH + h] = (float)is;
                for (int j = 0; j < D; ++j) {
                    const int c = h * D + j;
                    const double xh = v[c] * is;
                    xhat[(size_t)r * QK + c] = (float)qp_round(xh, dtype);
                    v[c] = xh * (double)gamma[c];
                }
            }
        }
        if (has_rope) {
            const int pos = r % S;
            for (int c = 0; c < QK; c += 2) {
                double s, co;
                angle(pos, inv_freq[(c % D) / 2], &s, &co);
                const double a = v[c], b = v[c + 1];
                v[c] = a * co - b * s;
                v[c + 1] = a * s + b * co;
            }
        }
        for (int c = 0; c < C; ++c) out[(size_t)r * C + c] = (float)qp_round(v[c], dtype);
    }
    free(v);
    return 0;
}

/* Backward.  dout, din: [rows][C]; din_prev: NULL to overwrite din, else the values din
 * accumulates onto (may equal din); xhat, istd, gamma as saved / used by the forward;
 * dgamma: QK, dbias: C, double sums over rows (overwritten). */
int qp_bwd(const float *dout, const float *xhat, const float *istd, const float *gamma,
           const float *inv_freq, const float *din_prev, int rows, int S, int Hq, int Hkv, int D,
           int has_qknorm, int has_rope, int dtype, float *din, double *dgamma, double *dbias) {
    if (!dout || !din || !dbias || rows < 0 || S < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || (D != 64 && D != 128))
        return -1;
    if (has_qknorm && (!xhat || !istd || !gamma || !dgamma)) return -1;
    if (has_rope && !inv_freq) return -1;
    const int C = (Hq + 2 * Hkv) * D, QK = (Hq + Hkv) * D, NH = Hq + Hkv;
    double *dy = (double *)malloc(sizeof(double) * (size_t)C);
    if (!dy) return -1;
    for (int c = 0; c < C; ++c) dbias[c] = 0.0;
    if (has_qknorm)
        for (int c = 0; c < QK; ++c) dgamma[c] = 0.0;
    for (int r = 0; r < rows; ++r) {
        for (int c = 0; c < C; ++c) dy[c] = (double)dout[(size_t)r * C + c];
        if (has_rope) {
            const int pos = r % S;
            for (int c = 0; c < QK; c += 2) {
                double s, co;
                angle(pos, inv_freq[(c % D) / 2], &s, &co);
                const double a = dy[c], b = dy[c + 1];
                dy[c] = a * co + b * s;
                dy[c + 1] = b * co - a * s;
            }
        }
        if (has_qknorm) {
            for (int h = 0; h < NH; ++h) {
                const float *xh = xhat + (size_t)r * QK + h * D;
                double m2 = 0.0;
                for (int j = 0; j < D; ++j) {
                    const int c = h * D + j;
                    dgamma[c] += dy[c] * xh[j];
                    m2 += dy[c] * gamma[c] * xh[j];
                }
                m2 /= D;
                const double is = istd[(size_t)r * NH + h];
                for (int j = 0; j < D; ++j) {
                    const int c = h * D + j;
                    dy[c] = is * (dy[c] * gamma[c] - xh[j] * m2);
                }
            }
        }
        for (int c = 0; c < C; ++c) {
            dbias[c] += dy[c];
            const double prev = din_prev ? (double)din_prev[(size_t)r * C + c] : 0.0;
            din[(size_t)r * C + c] = (float)qp_round(prev + dy[c], dtype);
        }
    }
    free(dy);
    return 0;
}
