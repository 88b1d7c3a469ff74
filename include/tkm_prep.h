/*
 * tkm_prep.h -- C ABI of the generated kernels that feed the attention kernels, of the
 * run-time compiler behind them, and of step-graph capture (libtkm_attn.so).
 *
 * 1. qkv-prep epilogue.  In the reference the fused QKV GEMM is followed by one generated
 *    "plasma" kernel pair that finishes Q|K|V for attention: bias, optional per-head
 *    QKNorm, optional RoPE (emit_qkv_prep_plasma_group + emit_rope_rotation, reference
 *    src/tkm_codegen.c:43-70 and 211-295).  Here tkm_prep_source emits HIP C for the same
 *    operation, tkm_prep_create compiles it with hipRTC for gfx950 and loads it (the
 *    NVRTC -> cuModuleLoadDataEx -> cuModuleGetFunction sequence of src/tkm_gpu.cu:1047-1078),
 *    and tkm_prep_fwd / tkm_prep_bwd launch it (launch_plasma_sig, src/tkm_gpu.cu:1166-1174).
 *
 *    Semantics, per row r of rows = B*S and channel c of C = (Hq + 2*Hkv)*D
 *    (Q heads | K heads | V heads, src/tkm_registry.c:736-748):
 *      v = in[r][c] + bias[c]                                     (tkm_codegen.c:235-236)
 *      Q and K channels (c < QK = (Hq + Hkv)*D) of head h = c / D:
 *        QKNorm: istd = rsqrt(sum_{head} v^2 / D + 1e-5); xhat = v * istd;
 *                v = xhat * gamma[c]                              (tkm_codegen.c:237-245)
 *        RoPE on the pair (c, c+1), c even, i = (c % D) / 2, pos = r % S:
 *                inv_freq = exp(-ln(theta) * i / D)   -- exponent i/D, not the usual 2i/D
 *                (optionally rescaled as tkm_codegen.c:47-62 does when scale > 1);
 *                (v0, v1) <- (v0 cos - v1 sin, v0 sin + v1 cos), angle pos * inv_freq
 *                                                                 (tkm_codegen.c:43-70, 246-250)
 *      out[r][c] = round-to-nearest-even(v)
 *    The backward applies the transposes in reverse order: inverse rotation, QKNorm backward
 *    using the saved xhat (16-bit) and istd, then d(bias) and d(in) (tkm_codegen.c:253-294).
 *    Differences from the reference, on purpose:
 *      - istd is saved per (row, head): save_istd [rows][Hq + Hkv].  The reference keeps one
 *        value per row that all heads overwrite (tkm_codegen.c:243, 280), so its QKNorm
 *        backward is wrong with more than one head.
 *      - d(gamma) and d(bias) are reduced without atomics, in a fixed order: results do not
 *        change from run to run.  The reference uses float atomicAdd (tkm_codegen.c:287-294).
 *      - QKNorm is accepted for D = 128 as well (the reference accepts only D = 64,
 *        tkm_registry.c:728-731), normalizing over the whole head.
 *      - 16-bit storage may be fp16 (the reference's) or bf16.
 *
 * 2. Step graphs.  tkm_graph_begin / tkm_graph_end / tkm_graph_launch capture everything
 *    enqueued on a stream once and replay it per step, as tkm_runtime_step does
 *    (src/tkm_gpu.cu:1498-1508).  Every entry point of this library and of tkm_attn.h is
 *    capturable: none allocates, copies, synchronizes or enqueues a memset.
 *
 * Device pointers; 16-bit tensors, bias, gamma and the workspace 16-byte aligned; save_istd,
 * dgamma and dbias 16-byte aligned.  Calls are asynchronous on `stream` (hipStream_t, NULL =
 * null stream).  Return TKM_ATTN_OK or a negative TKM_ATTN_* status; tkm_attn_last_error()
 * describes the last failure of the calling thread.
 */
#ifndef TKM_PREP_H
#define TKM_PREP_H

#include "tkm_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* What the runtime copies out of the reference's qkv_prep TkmNode (tkm_registry.c:750-765)
 * and its plasma group (tkm_core.c:494-505). */
typedef struct tkm_prep_desc {
    int group_id;               /* N of the kernel names tkm_plasma_{fwd,bwd}_g<N> */
    int seq_len;                /* S (= H*W of the group): RoPE position is row % S */
    int q_heads, kv_heads;      /* Hq, Hkv: q_c = Hq*D, k_c = v_c = Hkv*D */
    int head_dim;               /* D: 64 or 128 */
    int has_qknorm, has_rope;   /* 0 or 1 */
    float rope_theta;           /* > 0 */
    float rope_scale;           /* >= 1; > 1 enables the frequency rescaling */
    float rope_low_freq_factor, rope_high_freq_factor;   /* 0 < low < high */
    float rope_original_context_length;                   /* > 0 */
    int dtype;                  /* TKM_ATTN_F16 or TKM_ATTN_BF16 */
} tkm_prep_desc;

typedef struct tkm_prep tkm_prep;
typedef struct tkm_graph tkm_graph;

/* Fills the defaults of a parsed RoPE node (theta 10000, scale 1, low 1, high 4, original
 * context 8192: reference src/tkm_core.c:56-60), no QKNorm, no RoPE, fp16, group 0. */
TKM_ATTN_API void tkm_prep_desc_init(tkm_prep_desc *d);

/* The HIP source of the kernels for d (the prelude included), or NULL on a bad descriptor.
 * The caller frees it with tkm_free.  Counterpart of tkm_codegen_cuda_string for this group
 * (reference include/tkm.h:212). */
TKM_ATTN_API char *tkm_prep_source(const tkm_prep_desc *d);
TKM_ATTN_API void tkm_free(void *p);

/* Emits, compiles (hipRTC, gfx950) and loads the kernels on the current device.
 * Not capturable (it compiles and loads a module); call it once, before capture. */
TKM_ATTN_API int tkm_prep_create(const tkm_prep_desc *d, tkm_prep **out);
TKM_ATTN_API void tkm_prep_destroy(tkm_prep *p);

/* Forward over `rows` rows.  in/out: [rows][C]; bias: C floats; gamma: (Hq+Hkv)*D floats;
 * save_istd: [rows][Hq+Hkv] floats; save_xhat: [rows][(Hq+Hkv)*D] 16-bit.  gamma, save_istd
 * and save_xhat are used only with QKNorm (may be NULL otherwise).  in and out may be the
 * same buffer.  rows = 0 launches nothing (pointers are not inspected). */
TKM_ATTN_API int tkm_prep_fwd(const tkm_prep *p, const void *in, void *out, const float *bias,
                              const float *gamma, float *save_istd, void *save_xhat, int rows,
                              void *stream);

/* Bytes of workspace tkm_prep_bwd needs for `rows` rows (per-block partial sums). */
TKM_ATTN_API size_t tkm_prep_bwd_workspace_bytes(const tkm_prep *p, int rows);

/* Backward.  dout: [rows][C] (the gradient of out); din: [rows][C] 16-bit; dbias: C floats;
 * dgamma: (Hq+Hkv)*D floats (QKNorm only).  accumulate = 1 adds to din, dbias and dgamma
 * (the reference's semantics: its gradient arena is zeroed at the start of the step);
 * accumulate = 0 overwrites them.  din must not alias dout.  With rows = 0 the row tensors
 * may be NULL and only dbias / dgamma are written (cleared, or kept when accumulating). */
TKM_ATTN_API int tkm_prep_bwd(const tkm_prep *p, const void *dout, void *din,
                              const void *save_xhat, const float *save_istd, const float *gamma,
                              float *dgamma, float *dbias, int rows, int accumulate,
                              void *workspace, size_t workspace_bytes, void *stream);

/* The prelude every generated source starts with (static storage, do not free).
 * Counterpart of NVRTC_STANDALONE_PRELUDE, reference src/tkm_gpu.cu:722-827. */
TKM_ATTN_API const char *tkm_hip_prelude(void);

/* Compiles `src` with hipRTC for gfx950 (works without a GPU).  On success *code (free with
 * tkm_free) holds the code object of *code_bytes bytes.  *log, if log != NULL, receives the
 * compiler log (free with tkm_free; may be NULL when empty). */
TKM_ATTN_API int tkm_rtc_compile(const char *src, const char *name, void **code,
                                 size_t *code_bytes, char **log);

/* Step graphs (reference tkm_runtime_step, src/tkm_gpu.cu:1498-1508).  begin starts a
 * global-mode capture on `stream`; end stops it and instantiates the graph; launch replays
 * it on `stream`. */
TKM_ATTN_API int tkm_graph_begin(void *stream);
TKM_ATTN_API int tkm_graph_end(void *stream, tkm_graph **out);
TKM_ATTN_API int tkm_graph_launch(const tkm_graph *g, void *stream);
TKM_ATTN_API void tkm_graph_destroy(tkm_graph *g);

#ifdef __cplusplus
}
#endif

#endif /* TKM_PREP_H */
