/*
 * qkv_prep_ref.h -- CPU oracle of the qkv-prep epilogue (bias + QKNorm + RoPE).
 * TEST INFRASTRUCTURE ONLY; semantics and reference citations in qkv_prep_ref.c.
 */
#ifndef TKM_QKV_PREP_REF_H
#define TKM_QKV_PREP_REF_H

#ifdef __cplusplus
extern "C" {
#endif

/* x rounded to fp16 (dtype 0), bf16 (1) or fp32 (2), ties to even */
double qp_round(double x, int dtype);
/* fp32 inverse frequency of RoPE pair i (reference src/tkm_codegen.c:45-62) */
float qp_inv_freq(float theta, float scale, float low, float high, float ocl, int D, int i);
int qp_fwd(const float *in, const float *bias, const float *gamma, const float *inv_freq,
           int rows, int S, int Hq, int Hkv, int D, int has_qknorm, int has_rope, int dtype,
           float *out, float *xhat, float *istd);
int qp_bwd(const float *dout, const float *xhat, const float *istd, const float *gamma,
           const float *inv_freq, const float *din_prev, int rows, int S, int Hq, int Hkv, int D,
           int has_qknorm, int has_rope, int dtype, float *din, double *dgamma, double *dbias);

#ifdef __cplusplus
}
#endif

#endif
