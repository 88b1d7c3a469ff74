/*
 * attn_ref.h -- CPU oracle for the Tokamak GQA attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP kernels
 * are compared against (tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py).  No product code path links, loads or calls it.
 *
 * Semantics restated from the reference GPU kernels (the reference ships no
 * CPU attention):
 *   forward  : /root/reference/src/tkm_gpu.cu:302-438  (k_gqa_flash_attn_tc_fwd)
 *   backward : /root/reference/src/tkm_gpu.cu:440-598  (k_gqa_flash_attn_tc_bwd),
 *              dQ path only (503-564); dK/dV follow the true gradient because
 *              the reference writes dK := dQ, dV := dO at 588-596.
 *   dispatch : /root/reference/src/tkm_gpu.cu:1252-1265, 1389-1404
 *              (scale = 1/sqrtf(D), grid over B*Hq heads).
 *   packing  : /root/reference/src/tkm_registry.c:736-748 (Q | K | V heads).
 *
 * Layout (all row-major, elements are float here; the GPU path stores the
 * same values as fp16/bf16):
 *   qkv  [B][S][(Hq + 2*Hkv) * D]   Q heads, then K heads, then V heads
 *   o    [B][S][Hq * D]
 *   lse  [B][Hq][S]                 natural log, in units of scaled scores
 *   dqkv [B][S][(Hq + 2*Hkv) * D]   overwritten
 * q-head h reads kv-head h / (Hq / Hkv)            (tkm_gpu.cu:315-316)
 * key j is visible from query i iff j < kv_len[b] and (!causal || j <= i);
 * kv_len == NULL means every key < S is visible  (tkm_gpu.cu:393).
 * A query row with no visible key produces O = 0 and LSE = -inf (the
 * reference leaves this case undefined; it cannot arise without kv_len).
 */
#ifndef TKM_ATTN_REF_H
#define TKM_ATTN_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic inputs ------------------------------------------------
 * PCG32 (XSH-RR, 64-bit LCG state), M. E. O'Neill, "PCG: A Family of Simple
 * Fast Space-Efficient Statistically Good Algorithms for Random Number
 * Generation" (2014); seeding as pcg32_srandom_r.  The same recurrence is
 * used by /root/reference/examples/cifar10_bin.c:108-127.
 */
typedef struct { uint64_t state, inc; } ar_pcg32;
void     ar_pcg32_seed(ar_pcg32 *rng, uint64_t initstate, uint64_t initseq);
uint32_t ar_pcg32_next(ar_pcg32 *rng);

/* n samples of N(0,1) * mul from stream (seed, seq) by the Box-Muller
 * transform: u1 = ((r1 >> 8) + 1) * 2^-24, u2 = (r2 >> 8) * 2^-24,
 * z0 = sqrt(-2 ln u1) cos(2 pi u2), z1 = sqrt(-2 ln u1) sin(2 pi u2),
 * evaluated in double and rounded to float. */
void ar_fill_normal(float *out, size_t n, uint64_t seed, uint64_t seq, float mul);

/* Round floats in place to the nearest fp16 / bf16 value (ties to even);
 * out16 (optional) receives the raw 16-bit patterns. */
void ar_round_f16(float *x, uint16_t *out16, size_t n);
void ar_round_bf16(float *x, uint16_t *out16, size_t n);
void ar_widen_f16(const uint16_t *in, float *out, size_t n);
void ar_widen_bf16(const uint16_t *in, float *out, size_t n);

/* ---- attention ------------------------------------------------------------
 * acc_f64 = 0: fp32 accumulation (mirrors the reference's fp32 WMMA
 * accumulators and its +1e-8 guard on the row sum, tkm_gpu.cu:429-430).
 * acc_f64 = 1: fp64 accumulation, no guard; the high-precision check.
 * Return 0 on success, -1 on invalid arguments. */
int ar_attn_fwd(const float *qkv, float *o, float *lse, const int32_t *kv_len,
                int B, int S, int Hq, int Hkv, int D, float scale, int causal,
                int acc_f64);

/* The forward with the reference kernel's order of work and its fp16 P: online softmax
 * over tiles of 16 keys with a running max, each p = exp(s - m) rounded to fp16 before
 * the PV product while the row sum adds the unrounded p (tkm_gpu.cu:359-435); double
 * elsewhere.  It differs from ar_attn_fwd only by that rounding of P. */
int ar_attn_fwd_pround(const float *qkv, float *o, float *lse, const int32_t *kv_len,
                       int B, int S, int Hq, int Hkv, int D, float scale, int causal);

/* Backward: D_i = sum_d O_id dO_id from the given (stored) O; P recomputed
 * from lse; dS = P (dP - D); dQ = scale dS K; dK = scale dS^T Q and
 * dV = P^T dO summed over the q-heads of each kv group. */
int ar_attn_bwd(const float *qkv, const float *o, const float *dout,
                const float *lse, float *dqkv, const int32_t *kv_len,
                int B, int S, int Hq, int Hkv, int D, float scale, int causal,
                int acc_f64);

/* Threads used by the two functions above (OpenMP); 0 = all online CPUs. */
void ar_set_threads(int n);
int  ar_get_threads(void);
int  ar_online_cpus(void);

#ifdef __cplusplus
}
#endif
#endif
