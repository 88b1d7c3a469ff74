/* Launchers of the runtime's own kernels (tkm_rt_kernels.hip), used by tkm_hip.c.  Each
 * enqueues on `stream` (a hipStream_t) and returns 0, or -1 when the launch failed.  16-bit
 * tensors are fp16 (dtype 0) or bf16 (dtype 1). */
#ifndef TKM_RT_KERNELS_H
#define TKM_RT_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One learnable tensor for the SGD kernel (device-resident table). */
typedef struct {
    float *master;      /* fp32 master values */
    void *w16;          /* 16-bit copy read by the GEMMs, or NULL */
    float *vel;         /* momentum */
    const float *grad;  /* gradient */
    long long offset;   /* first element in the concatenation of all tensors */
    long long size;
    long long block0;   /* first SGD block (TKM_SGD_CHUNK elements per block) of this tensor */
} TkmSgdTensor;

/* Elements one SGD block updates (256 threads x 8). */
#define TKM_SGD_CHUNK 2048

/* Up to 64 columns of one group's band partials of parameter gradients: dst[c] = sum over
 * bands b of part[b * pw + col0 + c], c < ncols (overwritten). */
typedef struct {
    const float *part;
    float *dst;
    int pw, bands, col0, ncols;
} TkmReduceChunk;

int tkm_rt_f32_to_16(const float *src, void *dst, size_t n, int dtype, void *stream);
int tkm_rt_16_to_f32(const void *src, float *dst, size_t n, int dtype, void *stream);
int tkm_rt_fill_u32(void *dst, size_t bytes, uint32_t value, void *stream);
/* Softmax + loss per row (loss_kind 0 CE, 1 focal with gamma, 2 MSE on the probabilities);
 * labels are uint8 or (label_i32) int32, one per row, or NULL (label 0).  Writes dlogits
 * (overwritten) unless is_eval, then loss_out / correct_out (added to them when acc_*). */
int tkm_rt_softmax_loss(const void *logits, int dtype, const void *labels, int label_i32, void *dlogits,
                        float *row_loss, int *row_correct, int rows, int cols, int is_eval, int valid_rows,
                        int loss_kind, float gamma, float *loss_out, int *correct_out, int acc_loss,
                        int acc_correct, void *stream);
int tkm_rt_softmax_fwd(const void *x, void *y, int rows, int cols, int dtype, void *stream);
int tkm_rt_softmax_bwd(const void *p, const void *dp, void *din, int rows, int cols, int dtype, void *stream);
/* Momentum SGD over every tensor: n_blocks = sum over tensors of ceil(size / TKM_SGD_CHUNK),
 * block0 the prefix sums. */
int tkm_rt_sgd(const TkmSgdTensor *tensors, int nt, long long n_blocks, const float *d_lr, float momentum, float wd,
               uint32_t *d_seed, int dtype, void *stream);
/* Every chunk of the table, one block each (the band sums in the order of the generated
 * per-group reduce kernels). */
int tkm_rt_reduce_parts(const TkmReduceChunk *chunks, int n, void *stream);
int tkm_rt_perturb(void *p, long long i, float delta, int dtype, void *stream);
int tkm_rt_add_f32(float *acc, const float *v, void *stream);
int tkm_rt_gather(const void *images, const uint8_t *labels, const uint32_t *order, long long first, int B,
                  size_t elems, void *dst, uint8_t *dst_labels, void *stream);

#ifdef __cplusplus
}
#endif

#endif
