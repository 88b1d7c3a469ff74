/*
 * attn_ref.c -- CPU oracle for the Tokamak GQA attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP kernels are compared against,
 * never part of the product path.  Semantics, layout and citations are in
 * attn_ref.h.  The computation is the plain definition, row by row:
 *   s_ij  = scale * <q_i, k_j>                       tkm_gpu.cu:376-392
 *   m_i   = max_j s_ij, l_i = sum_j exp(s_ij - m_i)  tkm_gpu.cu:387-411
 *   O_i   = sum_j exp(s_ij - m_i) v_j / l_i          tkm_gpu.cu:414-435
 *   LSE_i = m_i + ln l_i                             tkm_gpu.cu:430
 *   D_i   = <O_i, dO_i>                              tkm_gpu.cu:503-512
 *   P_ij  = exp(s_ij - LSE_i), dS_ij = P_ij (<dO_i, v_j> - D_i)
 *                                                    tkm_gpu.cu:545-553
 *   dQ_i  = scale sum_j dS_ij k_j                    tkm_gpu.cu:557-564
 *   dK_j  = scale sum_i dS_ij q_i, dV_j = sum_i P_ij dO_i   (true gradient)
 * with the visibility rule of tkm_gpu.cu:393 extended by kv_len.
 */
#include "attn_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ PCG32 */
uint32_t ar_pcg32_next(ar_pcg32 *rng) {
    uint64_t old = rng->state;
    rng->state = old * 6364136223846793005ULL + rng->inc;
    uint32_t xs = (uint32_t)(((old >> 18u) ^ old) >> 27u);
    uint32_t rot = (uint32_t)(old >> 59u);
    return (xs >> rot) | (xs << ((32u - rot) & 31u));
}

void ar_pcg32_seed(ar_pcg32 *rng, uint64_t initstate, uint64_t initseq) {
    rng->state = 0u;
    rng->inc = (initseq << 1u) | 1u;
    ar_pcg32_next(rng);
    rng->state += initstate;
    ar_pcg32_next(rng);
}

void ar_fill_normal(float *out, size_t n, uint64_t seed, uint64_t seq, float mul) {
    ar_pcg32 rng;
    ar_pcg32_seed(&rng, seed, seq);
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        uint32_t r1 = ar_pcg32_next(&rng), r2 = ar_pcg32_next(&rng);
        double u1 = ((double)(r1 >> 8) + 1.0) * (1.0 / 16777216.0);
        double u2 = (double)(r2 >> 8) * (1.0 / 16777216.0);
        double rad = sqrt(-2.0 * log(u1));
        out[i] = (float)(rad * cos(two_pi * u2)) * mul;
        if (i + 1 < n) out[i + 1] = (float)(rad * sin(two_pi * u2)) * mul;
    }
}

/* ------------------------------------------------ fp16 / bf16 rounding */
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16 from binary32, round to nearest even, with subnormals,
 * overflow to inf and NaN preserved. */
static uint16_t f32_to_f16_bits(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) return (uint16_t)(sign | (absx > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 */
    if (absx < 0x38800000u) {                                 /* below 2^-14: subnormal */
        /* value * 2^24 rounded to an integer (ties to even) is the mantissa */
        float v = u2f(absx) * 16777216.0f;                   /* exact scaling */
        float r = nearbyintf(v);                              /* default mode = RNE */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t mant = absx & 0x7fffffu;
    int32_t e = (int32_t)(absx >> 23) - 127 + 15;
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

static float f16_bits_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

static uint16_t f32_to_bf16_bits(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

void ar_round_f16(float *x, uint16_t *out16, size_t n) {
    for (size_t i = 0; i < n; i++) {
        uint16_t h = f32_to_f16_bits(x[i]);
        if (out16) out16[i] = h;
        x[i] = f16_bits_to_f32(h);
    }
}
void ar_round_bf16(float *x, uint16_t *out16, size_t n) {
    for (size_t i = 0; i < n; i++) {
        uint16_t h = f32_to_bf16_bits(x[i]);
        if (out16) out16[i] = h;
        x[i] = u2f((uint32_t)h << 16);
    }
}
void ar_widen_f16(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = f16_bits_to_f32(in[i]);
}
void ar_widen_bf16(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = u2f((uint32_t)in[i] << 16);
}

/* ---------------------------------------------------------------- threads */
static int g_threads = 0;
int ar_online_cpus(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}
void ar_set_threads(int n) { g_threads = n; }
int ar_get_threads(void) { return g_threads > 0 ? g_threads : ar_online_cpus(); }

static int check_args(const void *qkv, const void *out, int B, int S, int Hq, int Hkv, int D) {
    if (!qkv || !out || B < 1 || S < 1 || Hq < 1 || Hkv < 1 || D < 1) return -1;
    if (Hq % Hkv) return -1;
    return 0;
}

static int visible_len(const int32_t *kv_len, int b, int S) {
    if (!kv_len) return S;
    int n = kv_len[b];
    return n < 0 ? 0 : (n > S ? S : n);
}

/* ------------------------------------------------------------------ kernels
 * Written once as a macro body and instantiated for ACC = float and double. */
#define AR_DEFINE_FWD(NAME, ACC, EXP, LOG, GUARD)                                  \
static void NAME(const float *qkv, float *o, float *lse, const int32_t *kv_len,   \
                 int B, int S, int Hq, int Hkv, int D, float scale, int causal) { \
    const int g = Hq / Hkv;                                                        \
    const size_t ld = (size_t)(Hq + 2 * Hkv) * D, ldo = (size_t)Hq * D;            \
    const long total = (long)B * Hq * S;                                           \
    _Pragma("omp parallel num_threads(ar_get_threads())")                          \
    {                                                                              \
        ACC *s = (ACC *)malloc(sizeof(ACC) * (size_t)S);                           \
        ACC *acc = (ACC *)malloc(sizeof(ACC) * (size_t)D);                         \
        _Pragma("omp for schedule(dynamic, 16)")                                   \
        for (long t = 0; t < total; t++) {                                         \
            int i = (int)(t % S), h = (int)((t / S) % Hq), b = (int)(t / ((long)S * Hq)); \
            int kh = h / g, kvl = visible_len(kv_len, b, S);                       \
            int jend = causal ? (i + 1 < kvl ? i + 1 : kvl) : kvl;                 \
            const float *base = qkv + (size_t)b * S * ld;                          \
            const float *q = base + (size_t)i * ld + (size_t)h * D;                \
            float *orow = o + ((size_t)b * S + i) * ldo + (size_t)h * D;           \
            float *lrow = lse ? lse + ((size_t)b * Hq + h) * S + i : NULL;         \
            if (jend <= 0) {                                                       \
                for (int d = 0; d < D; d++) orow[d] = 0.0f;                        \
                if (lrow) *lrow = -INFINITY;                                       \
                continue;                                                          \
            }                                                                      \
            ACC m = -INFINITY;                                                     \
            for (int j = 0; j < jend; j++) {                                       \
                const float *k = base + (size_t)j * ld + (size_t)(Hq + kh) * D;    \
                ACC dot = 0;                                                       \
                _Pragma("omp simd reduction(+:dot)")                               \
                for (int d = 0; d < D; d++) dot += (ACC)q[d] * (ACC)k[d];          \
                s[j] = dot * (ACC)scale;                                           \
                if (s[j] > m) m = s[j];                                            \
            }                                                                      \
            for (int d = 0; d < D; d++) acc[d] = 0;                                \
            ACC l = 0;                                                             \
            for (int j = 0; j < jend; j++) {                                       \
                const float *v = base + (size_t)j * ld + (size_t)(Hq + Hkv + kh) * D; \
                ACC p = EXP(s[j] - m);                                             \
                l += p;                                                            \
                _Pragma("omp simd")                                                \
                for (int d = 0; d < D; d++) acc[d] += p * (ACC)v[d];               \
            }                                                                      \
            ACC inv = (ACC)1 / (l + (ACC)GUARD);                                   \
            for (int d = 0; d < D; d++) orow[d] = (float)(acc[d] * inv);           \
            if (lrow) *lrow = (float)(m + LOG(l + (ACC)GUARD));                    \
        }                                                                          \
        free(s);                                                                   \
        free(acc);                                                                 \
    }                                                                              \
}

#define AR_DEFINE_BWD(NAME, ACC, EXP)                                              \
static void NAME(const float *qkv, const float *o, const float *dout,             \
                 const float *lse, float *dqkv, const int32_t *kv_len,            \
                 int B, int S, int Hq, int Hkv, int D, float scale, int causal) { \
    const int g = Hq / Hkv;                                                        \
    const size_t ld = (size_t)(Hq + 2 * Hkv) * D, ldo = (size_t)Hq * D;            \
    const long tasks = (long)B * Hkv;                                              \
    _Pragma("omp parallel num_threads(ar_get_threads())")                          \
    {                                                                              \
        ACC *dk = (ACC *)malloc(sizeof(ACC) * (size_t)S * D);                      \
        ACC *dv = (ACC *)malloc(sizeof(ACC) * (size_t)S * D);                      \
        ACC *dq = (ACC *)malloc(sizeof(ACC) * (size_t)D);                          \
        _Pragma("omp for schedule(dynamic, 1)")                                    \
        for (long t = 0; t < tasks; t++) {                                         \
            int kh = (int)(t % Hkv), b = (int)(t / Hkv);                           \
            int kvl = visible_len(kv_len, b, S);                                   \
            const float *base = qkv + (size_t)b * S * ld;                          \
            float *dbase = dqkv + (size_t)b * S * ld;                              \
            memset(dk, 0, sizeof(ACC) * (size_t)S * D);                            \
            memset(dv, 0, sizeof(ACC) * (size_t)S * D);                            \
            for (int h = kh * g; h < kh * g + g; h++) {                            \
                for (int i = 0; i < S; i++) {                                      \
                    int jend = causal ? (i + 1 < kvl ? i + 1 : kvl) : kvl;         \
                    const float *q = base + (size_t)i * ld + (size_t)h * D;        \
                    const float *orow = o + ((size_t)b * S + i) * ldo + (size_t)h * D;   \
                    const float *dorow = dout + ((size_t)b * S + i) * ldo + (size_t)h * D; \
                    ACC Di = 0;                                                    \
                    _Pragma("omp simd reduction(+:Di)")                            \
                    for (int d = 0; d < D; d++) Di += (ACC)orow[d] * (ACC)dorow[d]; \
                    ACC L = (ACC)lse[((size_t)b * Hq + h) * S + i];                \
                    for (int d = 0; d < D; d++) dq[d] = 0;                         \
                    for (int j = 0; j < jend; j++) {                               \
                        const float *k = base + (size_t)j * ld + (size_t)(Hq + kh) * D;       \
                        const float *v = base + (size_t)j * ld + (size_t)(Hq + Hkv + kh) * D; \
                        ACC sd = 0, pd = 0;                                        \
                        _Pragma("omp simd reduction(+:sd,pd)")                     \
                        for (int d = 0; d < D; d++) {                              \
                            sd += (ACC)q[d] * (ACC)k[d];                           \
                            pd += (ACC)dorow[d] * (ACC)v[d];                       \
                        }                                                          \
                        ACC p = EXP(sd * (ACC)scale - L);                          \
                        ACC ds = p * (pd - Di);                                    \
                        ACC *dkj = dk + (size_t)j * D, *dvj = dv + (size_t)j * D;  \
                        _Pragma("omp simd")                                        \
                        for (int d = 0; d < D; d++) {                              \
                            dq[d] += ds * (ACC)k[d];                               \
                            dkj[d] += ds * (ACC)q[d];                              \
                            dvj[d] += p * (ACC)dorow[d];                           \
                        }                                                          \
                    }                                                              \
                    float *dqrow = dbase + (size_t)i * ld + (size_t)h * D;         \
                    for (int d = 0; d < D; d++) dqrow[d] = (float)(dq[d] * (ACC)scale); \
                }                                                                  \
            }                                                                      \
            for (int j = 0; j < S; j++) {                                          \
                float *dkrow = dbase + (size_t)j * ld + (size_t)(Hq + kh) * D;     \
                float *dvrow = dbase + (size_t)j * ld + (size_t)(Hq + Hkv + kh) * D; \
                for (int d = 0; d < D; d++) {                                      \
                    dkrow[d] = (float)(dk[(size_t)j * D + d] * (ACC)scale);        \
                    dvrow[d] = (float)dv[(size_t)j * D + d];                       \
                }                                                                  \
            }                                                                      \
        }                                                                          \
        free(dk);                                                                  \
        free(dv);                                                                  \
        free(dq);                                                                  \
    }                                                                              \
}

AR_DEFINE_FWD(fwd_f32, float, expf, logf, 1e-8f)
AR_DEFINE_FWD(fwd_f64, double, exp, log, 0.0)
AR_DEFINE_BWD(bwd_f32, float, expf)
AR_DEFINE_BWD(bwd_f64, double, exp)

/* Forward as the reference's kernel orders it (tkm_gpu.cu:359-435), in double apart from
 * the one rounding it adds: keys in tiles of 16 (kv_base, 359); per tile the running max
 * m' = max(m, tile scores) with m starting at -1e30 (356, 388-395), alpha = exp(m - m')
 * (397), p = exp(s - m') accumulated into the row sum unrounded (399-403, 409) but rounded
 * to fp16 for the PV product (402, 414-424), O *= alpha (406-408); at the end
 * O = acc / (l + 1e-8), LSE = m + ln(l + 1e-8) (429-430).  Masked keys (key >= kv_len, or
 * causal and key > row: 393 with this build's kv_len) add nothing; tiles past the last
 * visible key are skipped, which changes nothing since their p are exactly 0 and alpha 1. */
static void fwd_pround(const float *qkv, float *o, float *lse, const int32_t *kv_len,
                       int B, int S, int Hq, int Hkv, int D, float scale, int causal) {
    const int g = Hq / Hkv;
    const size_t ld = (size_t)(Hq + 2 * Hkv) * D, ldo = (size_t)Hq * D;
    const long total = (long)B * Hq * S;
    _Pragma("omp parallel num_threads(ar_get_threads())")
    {
        double *acc = (double *)malloc(sizeof(double) * (size_t)D);
        _Pragma("omp for schedule(dynamic, 16)")
        for (long t = 0; t < total; t++) {
            int i = (int)(t % S), h = (int)((t / S) % Hq), b = (int)(t / ((long)S * Hq));
            int kh = h / g, kvl = visible_len(kv_len, b, S);
            int jend = causal ? (i + 1 < kvl ? i + 1 : kvl) : kvl;
            const float *base = qkv + (size_t)b * S * ld;
            const float *q = base + (size_t)i * ld + (size_t)h * D;
            float *orow = o + ((size_t)b * S + i) * ldo + (size_t)h * D;
            float *lrow = lse ? lse + ((size_t)b * Hq + h) * S + i : NULL;
            if (jend <= 0) {
                for (int d = 0; d < D; d++) orow[d] = 0.0f;
                if (lrow) *lrow = -INFINITY;
                continue;
            }
            double m = -1e30, l = 0.0, sc[16];
            for (int d = 0; d < D; d++) acc[d] = 0.0;
            for (int j0 = 0; j0 < jend; j0 += 16) {
                int n = jend - j0 < 16 ? jend - j0 : 16;
                double mt = m;
                for (int c = 0; c < n; c++) {
                    const float *k = base + (size_t)(j0 + c) * ld + (size_t)(Hq + kh) * D;
                    double dot = 0.0;
                    for (int d = 0; d < D; d++) dot += (double)q[d] * (double)k[d];
                    sc[c] = dot * (double)scale;
                    if (sc[c] > mt) mt = sc[c];
                }
                double alpha = exp(m - mt), rs = 0.0;
                for (int d = 0; d < D; d++) acc[d] *= alpha;
                for (int c = 0; c < n; c++) {
                    double pe = exp(sc[c] - mt);
                    float p16 = (float)pe;
                    ar_round_f16(&p16, NULL, 1);
                    rs += pe;
                    const float *v = base + (size_t)(j0 + c) * ld + (size_t)(Hq + Hkv + kh) * D;
                    for (int d = 0; d < D; d++) acc[d] += (double)p16 * (double)v[d];
                }
                l = l * alpha + rs;
                m = mt;
            }
            double inv = 1.0 / (l + 1e-8);
            for (int d = 0; d < D; d++) orow[d] = (float)(acc[d] * inv);
            if (lrow) *lrow = (float)(m + log(l + 1e-8));
        }
        free(acc);
    }
}

int ar_attn_fwd_pround(const float *qkv, float *o, float *lse, const int32_t *kv_len,
                       int B, int S, int Hq, int Hkv, int D, float scale, int causal) {
    if (check_args(qkv, o, B, S, Hq, Hkv, D)) return -1;
    fwd_pround(qkv, o, lse, kv_len, B, S, Hq, Hkv, D, scale, causal);
    return 0;
}

int ar_attn_fwd(const float *qkv, float *o, float *lse, const int32_t *kv_len,
                int B, int S, int Hq, int Hkv, int D, float scale, int causal,
                int acc_f64) {
    if (check_args(qkv, o, B, S, Hq, Hkv, D)) return -1;
    if (acc_f64) fwd_f64(qkv, o, lse, kv_len, B, S, Hq, Hkv, D, scale, causal);
    else         fwd_f32(qkv, o, lse, kv_len, B, S, Hq, Hkv, D, scale, causal);
    return 0;
}

int ar_attn_bwd(const float *qkv, const float *o, const float *dout,
                const float *lse, float *dqkv, const int32_t *kv_len,
                int B, int S, int Hq, int Hkv, int D, float scale, int causal,
                int acc_f64) {
    if (check_args(qkv, dqkv, B, S, Hq, Hkv, D) || !o || !dout || !lse) return -1;
    if (acc_f64) bwd_f64(qkv, o, dout, lse, dqkv, kv_len, B, S, Hq, Hkv, D, scale, causal);
    else         bwd_f32(qkv, o, dout, lse, dqkv, kv_len, B, S, Hq, Hkv, D, scale, causal);
    return 0;
}
