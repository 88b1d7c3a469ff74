/*
 * qkv-prep code generator: HIP C for the bias + QKNorm + RoPE epilogue between the fused
 * QKV GEMM and attention (semantics in include/tkm_prep.h; reference generator
 * src/tkm_codegen.c:43-70, 211-295).
 *
 * Layout of the generated kernels (gfx950, 64-lane waves, 256 threads = 4 waves per block):
 *   - a lane owns one 8-channel chunk of a row: one 16-byte load / store per tensor per row,
 *     64 consecutive chunks = 1 KiB contiguous per wave instruction;
 *   - block (x, y) covers chunks [64x, 64x + 64) and a band of rows; wave w takes the rows
 *     band_start + w + 4k;
 *   - a head of D channels is D/8 consecutive lanes (8 or 16, aligned), so the QKNorm sums
 *     are DPP reductions inside a lane row (tkm_sum_lanes8/16), no LDS;
 *   - bias, gamma and the RoPE frequencies of the chunk are loaded once per lane;
 *   - forward: 4 rows per wave, all loads issued before the arithmetic;
 *   - backward: the d(bias) / d(gamma) sums stay in registers over the band (about 2048
 *     blocks in all, at least 16 rows per band), then the 4 waves combine through LDS in a
 *     fixed order into one partial per band; a second kernel (16 waves per column group)
 *     adds the partials in band order.  No atomics: bitwise reproducible.
 * The RoPE inverse frequencies are computed here, on the host, in fp32 with the reference's
 * expression, and baked into the source as exact hexadecimal literals.
 */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tkm_prep.h"
#include "tkm_codegen_internal.h"
#include "tkm_plasma.h"
#include "tkm_prep_internal.h"

typedef tkm_sbuf sbuf;
#define sb_add tkm_sb_add

void tkm_prep_desc_init(tkm_prep_desc *d) {
    if (!d) return;
    memset(d, 0, sizeof(*d));
    d->seq_len = 1;
    d->q_heads = 1;
    d->kv_heads = 1;
    d->head_dim = 64;
    d->rope_theta = 10000.0f;
    d->rope_scale = 1.0f;
    d->rope_low_freq_factor = 1.0f;
    d->rope_high_freq_factor = 4.0f;
    d->rope_original_context_length = 8192.0f;
    d->dtype = TKM_ATTN_F16;
}

int tkm_prep_check_desc(const tkm_prep_desc *d) {
    if (!d) return tkm_set_error(TKM_ATTN_EINVAL, "descriptor is NULL");
    if (d->head_dim != 64 && d->head_dim != 128)
        return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "head_dim %d: must be 64 or 128", d->head_dim);
    if (d->q_heads <= 0 || d->kv_heads <= 0 || d->q_heads % d->kv_heads != 0)
        return tkm_set_error(TKM_ATTN_EINVAL, "heads Hq=%d Hkv=%d: need Hq, Hkv > 0 and Hq %% Hkv == 0",
                             d->q_heads, d->kv_heads);
    if ((long long)(d->q_heads + 2 * d->kv_heads) * d->head_dim > (1 << 20))
        return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "row width (Hq + 2 Hkv) * D above 2^20 channels");
    if (d->seq_len <= 0) return tkm_set_error(TKM_ATTN_EINVAL, "seq_len %d must be positive", d->seq_len);
    if (d->group_id < 0) return tkm_set_error(TKM_ATTN_EINVAL, "group_id %d must be >= 0", d->group_id);
    if ((d->has_qknorm != 0 && d->has_qknorm != 1) || (d->has_rope != 0 && d->has_rope != 1))
        return tkm_set_error(TKM_ATTN_EINVAL, "has_qknorm / has_rope must be 0 or 1");
    if (d->dtype != TKM_ATTN_F16 && d->dtype != TKM_ATTN_BF16)
        return tkm_set_error(TKM_ATTN_EUNSUPPORTED, "dtype %d", d->dtype);
    if (d->has_rope) {
        /* reference src/tkm_core.c:405-412 */
        if (!(d->rope_theta > 0.0f) || !(d->rope_scale >= 1.0f) || !(d->rope_low_freq_factor > 0.0f) ||
            !(d->rope_high_freq_factor > d->rope_low_freq_factor) || !(d->rope_original_context_length > 0.0f) ||
            !isfinite(d->rope_theta) || !isfinite(d->rope_scale) || !isfinite(d->rope_high_freq_factor) ||
            !isfinite(d->rope_original_context_length))
            return tkm_set_error(TKM_ATTN_EINVAL, "RoPE needs theta > 0, scale >= 1, 0 < low_freq_factor < "
                                 "high_freq_factor and original_context_length > 0 (all finite)");
    }
    return TKM_ATTN_OK;
}

/* Inverse frequency of pair i, in fp32, by the reference's expression (src/tkm_codegen.c:45-62):
 * exp(-ln(theta) * i / D), then, if scale > 1, the band-wise rescaling.  The reference's middle
 * band multiplies by 1 - smooth * (1 - 1/scale); that is kept as is. */
float tkm_rope_inv_freq(const tkm_prep_desc *d, int i) {
    volatile float t = -logf(d->rope_theta) * (float)i;   /* fp32 product, then fp32 quotient */
    float inv_freq = expf(t / (float)d->head_dim);
    if (d->rope_scale > 1.0f) {
        const float wavelen = 6.283185307179586f / inv_freq;
        const float low_wavelen = d->rope_original_context_length / d->rope_low_freq_factor;
        const float high_wavelen = d->rope_original_context_length / d->rope_high_freq_factor;
        if (wavelen > low_wavelen) {
            inv_freq /= d->rope_scale;
        } else if (wavelen >= high_wavelen) {
            const float smooth = (d->rope_original_context_length / wavelen - d->rope_low_freq_factor) /
                                 (d->rope_high_freq_factor - d->rope_low_freq_factor);
            volatile float f = 1.0f - smooth * (1.0f - 1.0f / d->rope_scale);
            inv_freq *= f;
        }
    }
    return inv_freq;
}

void tkm_prep_geometry(const tkm_prep_desc *d, tkm_prep_geom *g) {
    g->D = d->head_dim;
    g->C = (d->q_heads + 2 * d->kv_heads) * d->head_dim;
    g->QK = (d->q_heads + d->kv_heads) * d->head_dim;
    g->CH = g->C / 8;
    g->QKCH = g->QK / 8;
    g->NH = d->q_heads + d->kv_heads;
    g->G = d->head_dim / 8;
    g->part_width = g->C + (d->has_qknorm ? g->QK : 0);
}

int tkm_bwd_bands(int rows, int xblocks) {
    int bands = (TKM_BWD_TARGET_BLOCKS + xblocks - 1) / xblocks;
    const int most = (rows + TKM_BWD_MIN_BAND - 1) / TKM_BWD_MIN_BAND;
    if (bands > most) bands = most;
    return bands < 1 ? 1 : bands;
}

static const char *kind(const tkm_prep_desc *d) { return d->dtype == TKM_ATTN_BF16 ? "bf16" : "f16"; }

static void emit_constants(sbuf *s, const tkm_prep_desc *d, const tkm_prep_geom *g) {
    sb_add(s, "/* qkv-prep group %d: Hq=%d Hkv=%d D=%d S=%d qknorm=%d rope=%d %s */\n", d->group_id,
           d->q_heads, d->kv_heads, d->head_dim, d->seq_len, d->has_qknorm, d->has_rope, kind(d));
    sb_add(s, "#define TKM_CH %d      /* 8-channel chunks per row */\n", g->CH);
    sb_add(s, "#define TKM_QKCH %d    /* chunks holding Q and K */\n", g->QKCH);
    sb_add(s, "#define TKM_NH %d      /* Q + K heads */\n", g->NH);
    sb_add(s, "#define TKM_G %d       /* lanes per head */\n", g->G);
    sb_add(s, "#define TKM_S %d\n", d->seq_len);
    sb_add(s, "#define TKM_PW %d      /* partial-sum row width */\n", g->part_width);
    sb_add(s, "#define TKM_C %d\n", g->C);
    if (d->has_rope) {
        sb_add(s, "__constant__ float tkm_inv_freq_g%d[%d] = {", d->group_id, g->D / 2);
        for (int i = 0; i < g->D / 2; ++i)
            sb_add(s, "%s%af", i == 0 ? "\n    " : (i % 4 ? ", " : ",\n    "), (double)tkm_rope_inv_freq(d, i));
        sb_add(s, "\n};\n");
    }
    sb_add(s, "\n");
}

/* RoPE of the lane's 4 pairs (pair index i0 + p of its head) at position pos. */
static void emit_rope(sbuf *s, const char *var, int inverse) {
    sb_add(s, "            {\n");
    sb_add(s, "                const float fpos = (float)(r %% TKM_S);\n");
    sb_add(s, "#pragma unroll\n");
    sb_add(s, "                for (int p = 0; p < 4; ++p) {\n");
    sb_add(s, "                    const float ang = fpos * fr[p];\n");
    sb_add(s, "                    float sn, cs;\n");
    sb_add(s, "                    sincosf(ang, &sn, &cs);\n");
    sb_add(s, "                    const float x = %s[2 * p], y = %s[2 * p + 1];\n", var, var);
    if (inverse) {
        sb_add(s, "                    %s[2 * p] = x * cs + y * sn;\n", var);
        sb_add(s, "                    %s[2 * p + 1] = y * cs - x * sn;\n", var);
    } else {
        sb_add(s, "                    %s[2 * p] = x * cs - y * sn;\n", var);
        sb_add(s, "                    %s[2 * p + 1] = x * sn + y * cs;\n", var);
    }
    sb_add(s, "                }\n");
    sb_add(s, "            }\n");
}

static void emit_lane_setup(sbuf *s, const tkm_prep_desc *d, int need_bias) {
    sb_add(s, "    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;\n");
    sb_add(s, "    const int ch = blockIdx.x * 64 + lane;\n");
    sb_add(s, "    const bool ok = ch < TKM_CH;\n");
    sb_add(s, "    const bool qk = ch < TKM_QKCH;\n");
    if (need_bias) {
        sb_add(s, "    float b[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};\n");
        sb_add(s, "    if (ok) {\n");
        sb_add(s, "        const float4 b0 = bias[2 * ch], b1 = bias[2 * ch + 1];\n");
        sb_add(s, "        b[0] = b0.x; b[1] = b0.y; b[2] = b0.z; b[3] = b0.w;\n");
        sb_add(s, "        b[4] = b1.x; b[5] = b1.y; b[6] = b1.z; b[7] = b1.w;\n");
        sb_add(s, "    }\n");
    }
    if (d->has_qknorm) {
        sb_add(s, "    float g[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};\n");
        sb_add(s, "    if (qk) {\n");
        sb_add(s, "        const float4 g0 = gamma[2 * ch], g1 = gamma[2 * ch + 1];\n");
        sb_add(s, "        g[0] = g0.x; g[1] = g0.y; g[2] = g0.z; g[3] = g0.w;\n");
        sb_add(s, "        g[4] = g1.x; g[5] = g1.y; g[6] = g1.z; g[7] = g1.w;\n");
        sb_add(s, "    }\n");
    }
    if (d->has_rope) {
        sb_add(s, "    float fr[4] = {0.f, 0.f, 0.f, 0.f};\n");
        sb_add(s, "    if (qk) {\n");
        sb_add(s, "        const int i0 = (ch %% TKM_G) * 4;   /* first pair of the chunk within its head */\n");
        sb_add(s, "#pragma unroll\n");
        sb_add(s, "        for (int p = 0; p < 4; ++p) fr[p] = tkm_inv_freq_g%d[i0 + p];\n", d->group_id);
        sb_add(s, "    }\n");
    }
}

/* Internal argument lists of the two kernels (kinds of include/tkm_plasma.h, node 0 = the
 * qkv_prep node), in the order of the standalone API. */
int tkm_prep_need(int pass, tkm_kparam *out) {
    static const tkm_kparam fwd[] = {
        {TKM_ARG_IN, -1, "const uint4 *", "in"},
        {TKM_ARG_OUT, -1, "uint4 *", "out"},
        {TKM_ARG_BIAS, 0, "const float4 *__restrict__", "bias"},
        {TKM_ARG_WEIGHT, 0, "const float4 *__restrict__", "gamma"},
        {TKM_ARG_SAVE_ISTD, 0, "float *__restrict__", "save_istd"},
        {TKM_ARG_SAVE_XHAT, 0, "uint4 *__restrict__", "save_xhat"},
        {TKM_KP_ROWS, -1, "int", "rows"}};
    static const tkm_kparam bwd[] = {
        {TKM_ARG_DOUT, -1, "const uint4 *__restrict__", "dout"},
        {TKM_ARG_DIN, -1, "uint4 *__restrict__", "din"},
        {TKM_ARG_SAVE_XHAT, 0, "const uint4 *__restrict__", "save_xhat"},
        {TKM_ARG_SAVE_ISTD, 0, "const float *__restrict__", "save_istd"},
        {TKM_ARG_WEIGHT, 0, "const float4 *__restrict__", "gamma"},
        {TKM_KP_PART, -1, "float *__restrict__", "part"},
        {TKM_KP_ROWS, -1, "int", "rows"},
        {TKM_KP_BAND, -1, "int", "band"},
        {TKM_KP_ACC, -1, "int", "accumulate"}};
    const tkm_kparam *src = pass ? bwd : fwd;
    const int n = pass ? (int)(sizeof bwd / sizeof bwd[0]) : (int)(sizeof fwd / sizeof fwd[0]);
    for (int i = 0; i < n; ++i) out[i] = src[i];
    return n;
}

static int emit_header(sbuf *s, const tkm_prep_desc *d, int pass, const tkm_kplan *plan) {
    tkm_kparam need[16];
    const int n = tkm_prep_need(pass, need);
    tkm_kplan def;
    if (!plan) {
        def.n = 0;
        for (int i = 0; i < n; ++i) tkm_kplan_add(&def, need[i].kind, need[i].node, need[i].decl, need[i].name);
        plan = &def;
    }
    sb_add(s, "extern \"C\" __global__ __launch_bounds__(256) void tkm_plasma_%s_g%d", pass ? "bwd" : "fwd",
           d->group_id);
    return tkm_emit_plan_params(s, plan, need, n);
}

static int emit_fwd(sbuf *s, const tkm_prep_desc *d, const tkm_prep_geom *g, const tkm_kplan *plan) {
    const char *k = kind(d);
    if (emit_header(s, d, 0, plan)) return -1;
    if (!d->has_qknorm) sb_add(s, "    (void)gamma; (void)save_istd; (void)save_xhat;\n");
    emit_lane_setup(s, d, 1);
    sb_add(s, "    const int r0 = blockIdx.y * %d + wave;\n", 4 * TKM_PREP_FWD_RPW);
    sb_add(s, "    uint4 x[%d];\n", TKM_PREP_FWD_RPW);
    sb_add(s, "#pragma unroll\n");
    sb_add(s, "    for (int k = 0; k < %d; ++k) {\n", TKM_PREP_FWD_RPW);
    sb_add(s, "        const int r = r0 + 4 * k;\n");
    sb_add(s, "        x[k] = (ok && r < rows) ? in[(size_t)r * TKM_CH + ch] : tkm_zero4();\n");
    sb_add(s, "    }\n");
    sb_add(s, "#pragma unroll\n");
    sb_add(s, "    for (int k = 0; k < %d; ++k) {\n", TKM_PREP_FWD_RPW);
    sb_add(s, "        const int r = r0 + 4 * k;\n");
    sb_add(s, "        if (r >= rows) break;\n");
    sb_add(s, "        float v[8];\n");
    sb_add(s, "        tkm_unpack_%s(x[k], v);\n", k);
    sb_add(s, "#pragma unroll\n");
    sb_add(s, "        for (int j = 0; j < 8; ++j) v[j] += b[j];\n");
    if (d->has_qknorm || d->has_rope) {
        sb_add(s, "        if (qk) {   /* whole heads: the branch never splits a lane group */\n");
        if (d->has_qknorm) {
            sb_add(s, "            float sq = 0.f;\n");
            sb_add(s, "#pragma unroll\n");
            sb_add(s, "            for (int j = 0; j < 8; ++j) sq += v[j] * v[j];\n");
            sb_add(s, "            sq = tkm_sum_lanes%d(sq);\n", g->G);
            sb_add(s, "            const float istd = rsqrtf(sq * %af + 1e-5f);\n", 1.0 / (double)g->D);
            sb_add(s, "            float xh[8];\n");
            sb_add(s, "#pragma unroll\n");
            sb_add(s, "            for (int j = 0; j < 8; ++j) xh[j] = v[j] * istd;\n");
            sb_add(s, "            save_xhat[(size_t)r * TKM_QKCH + ch] = tkm_pack_%s(xh);\n", k);
            sb_add(s, "            if ((lane & (TKM_G - 1)) == 0) save_istd[(size_t)r * TKM_NH + ch / TKM_G] = istd;\n");
            sb_add(s, "#pragma unroll\n");
            sb_add(s, "            for (int j = 0; j < 8; ++j) v[j] = xh[j] * g[j];\n");
        }
        if (d->has_rope) emit_rope(s, "v", 0);
        sb_add(s, "        }\n");
    }
    sb_add(s, "        if (ok) out[(size_t)r * TKM_CH + ch] = tkm_pack_%s(v);\n", k);
    sb_add(s, "    }\n}\n\n");
    return 0;
}

static int emit_bwd(sbuf *s, const tkm_prep_desc *d, const tkm_prep_geom *g, const tkm_kplan *plan) {
    const char *k = kind(d);
    const int B = TKM_PREP_BWD_BATCH;
    if (emit_header(s, d, 1, plan)) return -1;
    if (!d->has_qknorm) sb_add(s, "    (void)save_xhat; (void)save_istd; (void)gamma;\n");
    emit_lane_setup(s, d, 0);
    sb_add(s, "    float adb[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};\n");
    if (d->has_qknorm) sb_add(s, "    float adw[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};\n");
    sb_add(s, "    const int rbeg = blockIdx.y * band;\n");
    sb_add(s, "    const int rend = min(rows, rbeg + band);\n");
    sb_add(s, "    for (int rb = rbeg + wave; rb < rend; rb += %d) {\n", 4 * B);
    sb_add(s, "        uint4 dyr[%d], pv[%d];\n", B, B);
    if (d->has_qknorm) sb_add(s, "        uint4 xhr[%d];\n", B);
    sb_add(s, "#pragma unroll\n");
    sb_add(s, "        for (int k = 0; k < %d; ++k) {\n", B);
    sb_add(s, "            const int r = rb + 4 * k;\n");
    sb_add(s, "            const bool live = ok && r < rend;\n");
    sb_add(s, "            dyr[k] = live ? dout[(size_t)r * TKM_CH + ch] : tkm_zero4();\n");
    sb_add(s, "            pv[k] = (live && accumulate) ? din[(size_t)r * TKM_CH + ch] : tkm_zero4();\n");
    if (d->has_qknorm) sb_add(s, "            xhr[k] = (live && qk) ? save_xhat[(size_t)r * TKM_QKCH + ch] : tkm_zero4();\n");
    sb_add(s, "        }\n");
    sb_add(s, "#pragma unroll\n");
    sb_add(s, "        for (int k = 0; k < %d; ++k) {\n", B);
    sb_add(s, "            const int r = rb + 4 * k;\n");
    sb_add(s, "            if (r >= rend) break;\n");
    sb_add(s, "            float dy[8];\n");
    sb_add(s, "            tkm_unpack_%s(dyr[k], dy);\n", k);
    if (d->has_qknorm || d->has_rope) {
        sb_add(s, "            if (qk) {\n");
        if (d->has_rope) emit_rope(s, "dy", 1);
        if (d->has_qknorm) {
            sb_add(s, "                float xh[8], dxh[8];\n");
            sb_add(s, "                tkm_unpack_%s(xhr[k], xh);\n", k);
            sb_add(s, "                float m2 = 0.f;\n");
            sb_add(s, "#pragma unroll\n");
            sb_add(s, "                for (int j = 0; j < 8; ++j) {\n");
            sb_add(s, "                    adw[j] += dy[j] * xh[j];\n");
            sb_add(s, "                    dxh[j] = dy[j] * g[j];\n");
            sb_add(s, "                    m2 += dxh[j] * xh[j];\n");
            sb_add(s, "                }\n");
            sb_add(s, "                m2 = tkm_sum_lanes%d(m2) * %af;\n", g->G, 1.0 / (double)g->D);
            sb_add(s, "                const float istd = save_istd[(size_t)r * TKM_NH + ch / TKM_G];\n");
            sb_add(s, "#pragma unroll\n");
            sb_add(s, "                for (int j = 0; j < 8; ++j) dy[j] = istd * (dxh[j] - xh[j] * m2);\n");
        }
        sb_add(s, "            }\n");
    }
    sb_add(s, "            float pr[8];\n");
    sb_add(s, "            tkm_unpack_%s(pv[k], pr);\n", k);
    sb_add(s, "#pragma unroll\n");
    sb_add(s, "            for (int j = 0; j < 8; ++j) {\n");
    sb_add(s, "                adb[j] += dy[j];\n");
    sb_add(s, "                pr[j] = accumulate ? pr[j] + dy[j] : dy[j];\n");
    sb_add(s, "            }\n");
    sb_add(s, "            if (ok) din[(size_t)r * TKM_CH + ch] = tkm_pack_%s(pr);\n", k);
    sb_add(s, "        }\n");
    sb_add(s, "    }\n");
    /* combine the 4 waves in wave order, one partial row per block row */
    const int NV = d->has_qknorm ? 16 : 8;
    sb_add(s, "    __shared__ float red[4][%d][64];\n", NV);
    sb_add(s, "#pragma unroll\n");
    sb_add(s, "    for (int j = 0; j < 8; ++j) red[wave][j][lane] = adb[j];\n");
    if (d->has_qknorm) {
        sb_add(s, "#pragma unroll\n");
        sb_add(s, "    for (int j = 0; j < 8; ++j) red[wave][8 + j][lane] = adw[j];\n");
    }
    sb_add(s, "    __syncthreads();\n");
    sb_add(s, "    if (wave == 0 && ok) {\n");
    sb_add(s, "        float t[%d];\n", NV);
    sb_add(s, "#pragma unroll\n");
    sb_add(s, "        for (int j = 0; j < %d; ++j) t[j] = ((red[0][j][lane] + red[1][j][lane]) + red[2][j][lane]) + red[3][j][lane];\n", NV);
    sb_add(s, "        float4 *pb = (float4 *)(part + (size_t)blockIdx.y * TKM_PW + 8 * ch);\n");
    sb_add(s, "        pb[0] = make_float4(t[0], t[1], t[2], t[3]);\n");
    sb_add(s, "        pb[1] = make_float4(t[4], t[5], t[6], t[7]);\n");
    if (d->has_qknorm) {
        sb_add(s, "        if (qk) {\n");
        sb_add(s, "            float4 *pw = (float4 *)(part + (size_t)blockIdx.y * TKM_PW + TKM_C + 8 * ch);\n");
        sb_add(s, "            pw[0] = make_float4(t[8], t[9], t[10], t[11]);\n");
        sb_add(s, "            pw[1] = make_float4(t[12], t[13], t[14], t[15]);\n");
        sb_add(s, "        }\n");
    }
    sb_add(s, "    }\n}\n\n");

    /* partial rows -> dbias | dgamma: column c of the partials, summed over the bands in order.
     * 16 waves split the bands round-robin and combine in wave order. */
    sb_add(s, "extern \"C\" __global__ __launch_bounds__(1024) void tkm_plasma_bwd_g%d_reduce(\n", d->group_id);
    sb_add(s, "    const float *__restrict__ part, float *__restrict__ dbias, float *__restrict__ dgamma,\n");
    sb_add(s, "    int bands, int accumulate)\n{\n");
    if (!d->has_qknorm) sb_add(s, "    (void)dgamma;\n");
    sb_add(s, "    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;\n");
    sb_add(s, "    const int c = blockIdx.x * 64 + lane;\n");
    sb_add(s, "    float acc = 0.f;\n");
    sb_add(s, "    if (c < TKM_PW) {\n");
    sb_add(s, "#pragma unroll 4\n");
    sb_add(s, "        for (int b = wave; b < bands; b += 16) acc += part[(size_t)b * TKM_PW + c];\n");
    sb_add(s, "    }\n");
    sb_add(s, "    __shared__ float red[16][64];\n");
    sb_add(s, "    red[wave][lane] = acc;\n");
    sb_add(s, "    __syncthreads();\n");
    sb_add(s, "    if (wave != 0 || c >= TKM_PW) return;\n");
    sb_add(s, "    float t = red[0][lane];\n");
    sb_add(s, "    for (int q = 1; q < 16; ++q) t += red[q][lane];\n");
    if (d->has_qknorm)
        sb_add(s, "    float *dst = c < TKM_C ? dbias + c : dgamma + (c - TKM_C);\n");
    else
        sb_add(s, "    float *dst = dbias + c;\n");
    sb_add(s, "    *dst = accumulate ? *dst + t : t;\n");
    sb_add(s, "}\n");
    return 0;
}

int tkm_prep_emit(tkm_sbuf *s, const tkm_prep_desc *d, const tkm_kplan *fwd_plan, const tkm_kplan *bwd_plan,
                  int scoped) {
    int rc = tkm_prep_check_desc(d);
    if (rc) return rc;
    tkm_prep_geom g;
    tkm_prep_geometry(d, &g);
    if (scoped) sb_add(s, "namespace tkm_g%d {\n", d->group_id);
    emit_constants(s, d, &g);
    if (emit_fwd(s, d, &g, fwd_plan) || emit_bwd(s, d, &g, bwd_plan))
        return tkm_set_error(TKM_ATTN_EINVAL, "qkv-prep group %d: a kernel argument is missing from its plan",
                             d->group_id);
    if (scoped) {
        sb_add(s, "}  /* namespace tkm_g%d */\n", d->group_id);
        sb_add(s, "#undef TKM_CH\n#undef TKM_QKCH\n#undef TKM_NH\n#undef TKM_G\n#undef TKM_S\n#undef TKM_PW\n"
                  "#undef TKM_C\n\n");
    }
    return s->failed ? tkm_set_error(TKM_ATTN_EINVAL, "out of host memory while emitting source") : TKM_ATTN_OK;
}

char *tkm_prep_source(const tkm_prep_desc *d) {
    sbuf s = {0};
    sb_add(&s, "%s", tkm_hip_prelude());
    if (tkm_prep_emit(&s, d, NULL, NULL, 0) != TKM_ATTN_OK) {
        free(s.buf);
        return NULL;
    }
    return s.buf;
}

void tkm_free(void *p) { free(p); }
