/*
 * tkm_attn.h -- C ABI of the MI355X (gfx950) attention kernels (libtkm_attn.so).
 *
 * This is the inner boundary the Tokamak runtime dispatches GQA attention to.  In the
 * reference it is implicit: the OP_GQA_ATTN cases of execute_forward_pass and of the
 * backward node walk launch k_gqa_flash_attn_tc_fwd / _bwd directly
 * (reference src/tkm_gpu.cu:1252-1265 and 1389-1404, kernels at 302-438 and 440-598).
 * The host runtime (tkm_hip.c) calls these functions at those two sites instead.
 *
 * Conventions (unchanged from the reference):
 *   - all tensors are device pointers, row-major, 16-bit elements (fp16 or bf16):
 *       qkv  [B][S][(Hq + 2*Hkv) * D]  Q heads | K heads | V heads   (tkm_registry.c:736-748)
 *       o    [B][S][Hq * D]
 *       lse  [B][Hq][S] fp32, natural log of the row sum of exp(scaled scores) (tkm_gpu.cu:430)
 *       dout [B][S][Hq * D],  dqkv has the layout of qkv and is overwritten
 *   - q-head h attends with kv-head h / (Hq / Hkv)                (tkm_gpu.cu:315-316)
 *   - scores are scale * <q_i, k_j>; the runtime passes scale = 1/sqrtf(D) (tkm_gpu.cu:1258);
 *     scale must be positive and finite
 *   - key j is visible from query i iff j < S and (!causal || j <= i) (tkm_gpu.cu:393)
 * Extension (reference has none, its GQA op has no key-length input):
 *   - kv_len: optional device array of B int32; keys j >= kv_len[b] are masked.  Values are
 *     clamped to [0, S]; a query row with no visible key gets O = 0, LSE = -inf and zero
 *     gradients.  NULL means kv_len[b] = S.
 *   - dtype TKM_ATTN_BF16 in addition to the reference's fp16.
 *
 * All calls are asynchronous on `stream` (a hipStream_t, NULL = null stream), allocate
 * nothing and never synchronize, so they may be captured into a hipGraph.  D must be 64 or
 * 128 (the reference accepts exactly these, tkm_core.c:392-404).  16-bit tensors and the
 * workspace must be 16-byte aligned; lse 4-byte aligned.
 * Return value: TKM_ATTN_OK or a negative status; tkm_attn_last_error() describes the last
 * failure of the calling thread.  Nothing is launched when a call fails validation.
 */
#ifndef TKM_ATTN_H
#define TKM_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(_WIN32)
#define TKM_ATTN_API
#else
#define TKM_ATTN_API __attribute__((visibility("default")))
#endif

enum { TKM_ATTN_F16 = 0, TKM_ATTN_BF16 = 1 };

enum {
    TKM_ATTN_OK = 0,
    TKM_ATTN_EINVAL = -1,       /* null pointer, non-positive size, Hq % Hkv != 0, bad flag */
    TKM_ATTN_EUNSUPPORTED = -2, /* D not in {64, 128}, unknown dtype, size beyond int range */
    TKM_ATTN_EALIGN = -3,       /* misaligned pointer */
    TKM_ATTN_EWORKSPACE = -4,   /* workspace missing or smaller than required */
    TKM_ATTN_ELAUNCH = -5,      /* the HIP runtime rejected a kernel launch */
    TKM_ATTN_ECOMPILE = -6,     /* hipRTC rejected a generated source */
    TKM_ATTN_EDEVICE = -7       /* no device current, a HIP module/graph call failed, or the
                                   gfx950 assembly kernels failed to load */
};

/* Backward stages.  Two valid schedules:
 *   DELTA, then DKDV and DQ (independent of each other: they may run on two streams);
 *   DQ_DELTA, then DKDV (one stream, one pass over O and dO fewer; what tkm_attn_bwd runs).
 * DELTA writes D = <O, dO> per row into the workspace; DQ_DELTA computes D inside the dQ
 * pass and writes it there; DKDV and DQ read it.  Both also write the row pairs
 * (-LSE*log2(e), -D) that DKDV reads. */
enum { TKM_ATTN_BWD_DELTA = 0, TKM_ATTN_BWD_DKDV = 1, TKM_ATTN_BWD_DQ = 2, TKM_ATTN_BWD_DQ_DELTA = 3 };

/* Forward: O and (if lse != NULL) LSE.
 * Replaces k_gqa_flash_attn_tc_fwd + dispatch, reference src/tkm_gpu.cu:302-438, 1252-1265. */
TKM_ATTN_API int tkm_attn_fwd(const void *qkv, void *o, float *lse, const int32_t *kv_len,
                              int B, int S, int Hq, int Hkv, int D, float scale, int causal,
                              int dtype, void *stream);

/* Bytes of device workspace tkm_attn_bwd needs: the per-row D = <O, dO> vector, and the same
 * rows' -LSE*log2(e) and -D values in tiles of 32 rows per (batch, head), for the dK/dV pass.
 * Replaces the per-node save buffer sizing of init_node_resources, src/tkm_gpu.cu:1000-1001. */
TKM_ATTN_API size_t tkm_attn_bwd_workspace_bytes(int B, int S, int Hq);

/* Backward: dqkv (dQ | dK | dV), overwritten.  lse is the forward's LSE.
 * Replaces k_gqa_flash_attn_tc_bwd + dispatch, reference src/tkm_gpu.cu:440-598, 1389-1404
 * (with the true dK/dV; the reference writes dK := dQ and dV := dO, tkm_gpu.cu:588-596). */
TKM_ATTN_API int tkm_attn_bwd(const void *qkv, const void *o, const void *dout,
                              const float *lse, void *dqkv, const int32_t *kv_len,
                              int B, int S, int Hq, int Hkv, int D, float scale, int causal,
                              int dtype, void *workspace, size_t workspace_bytes, void *stream);

/* tkm_attn_bwd without a workspace argument and without any allocation: the workspace is a
 * static device array of TKM_ATTN_NOALLOC_SCRATCH_BYTES (16 MiB) that each GPU holds from
 * the library's first use on it until the process ends.  No reference counterpart: it is
 * for callers that cannot allocate (code under graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Results equal tkm_attn_bwd's bit for bit.
 * Limits: tkm_attn_bwd_workspace_bytes(B, S, Hq) must not exceed the scratch size (about
 * 1.4 million (batch, head, row) triples; config 5's 524288 fit), else TKM_ATTN_EWORKSPACE
 * and nothing runs.  Every call on one GPU shares that GPU's array: calls that overlap on
 * one GPU (other streams, other threads) race, so serialize them.  Nothing needs clearing
 * between calls (the dQ stage writes all the dK/dV stage reads).  tkm_attn_init sets the
 * array up per device; call it before capturing, else the first call on a device does. */
#define TKM_ATTN_NOALLOC_SCRATCH_BYTES (16 << 20)
TKM_ATTN_API int tkm_attn_bwd_noalloc(const void *qkv, const void *o, const void *dout,
                                      const float *lse, void *dqkv, const int32_t *kv_len,
                                      int B, int S, int Hq, int Hkv, int D, float scale,
                                      int causal, int dtype, void *stream);

/* One stage of tkm_attn_bwd (same arguments), for callers that split the backward across
 * streams or time its kernels separately.  No reference counterpart (the reference backward
 * is a single kernel). */
TKM_ATTN_API int tkm_attn_bwd_stage(int stage, const void *qkv, const void *o, const void *dout,
                                    const float *lse, void *dqkv, const int32_t *kv_len,
                                    int B, int S, int Hq, int Hkv, int D, float scale, int causal,
                                    int dtype, void *workspace, size_t workspace_bytes,
                                    void *stream);

/* Loads this library's gfx950 assembly kernels (D = 128, fp16 and bf16) on the current device.  Call
 * it once per device before capturing a graph, as the runtime does at ignite; otherwise the
 * first call on a device loads them (inside a capture, with the thread's capture mode
 * relaxed so that nothing is recorded).  Returns TKM_ATTN_OK (also on a device that is not
 * gfx950, where the HIP kernels serve every shape) or TKM_ATTN_EDEVICE when a code object
 * fails to load; the calls that need them then fail with TKM_ATTN_EDEVICE too, they never
 * switch to the slower kernels.  No reference counterpart (the reference JIT-compiles its
 * generated kernels at ignite, src/tkm_gpu.cu:1047-1078; its attention kernels are
 * compiled ahead of time). */
TKM_ATTN_API int tkm_attn_init(void);

/* 1 if the assembly kernels are loaded on the current device (gfx950), else 0. */
TKM_ATTN_API int tkm_attn_asm_available(void);

/* Kernels launched by the calling thread's last tkm_attn_fwd / _bwd / _bwd_stage call
 * (OR of the bits below; 0 after a call that failed validation).  No reference counterpart. */
enum {
    TKM_ATTN_K_FWD_ASM = 1,     /* tkm_fa_fwd_d128_f16 (assembly) */
    TKM_ATTN_K_FWD_HIP = 2,     /* fa_fwd_kernel (HIP) */
    TKM_ATTN_K_DQ_ASM = 4,      /* tkm_fa_bwd_dq_d128_f16 (assembly) */
    TKM_ATTN_K_DQ_HIP = 8,      /* fa_bwd_dq_kernel (HIP) */
    TKM_ATTN_K_DKDV_ASM = 16,   /* tkm_fa_bwd_dkdv_d128_f16 (assembly) */
    TKM_ATTN_K_DKDV_HIP = 32,   /* fa_bwd_dkdv_kernel (HIP) */
    TKM_ATTN_K_DELTA_HIP = 64   /* fa_bwd_delta_kernel (HIP) */
};
TKM_ATTN_API unsigned tkm_attn_last_kernels(void);

/* Static description of a status code, and the last failure message of this thread. */
TKM_ATTN_API const char *tkm_attn_status_string(int status);
TKM_ATTN_API const char *tkm_attn_last_error(void);

/* ABI version: major * 10000 + minor * 100 + patch. */
TKM_ATTN_API int tkm_attn_version(void);

#ifdef __cplusplus
}
#endif
#endif /* TKM_ATTN_H */
