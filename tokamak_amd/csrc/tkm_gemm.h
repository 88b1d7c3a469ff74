/* The runtime's GEMMs (tkm_gemm.hip, hipBLASLt): column-major C = op(A) . op(B) with
 * alpha = 1 and a fixed beta, the algorithm chosen at creation.  Returns 0 or -1 with
 * tkm_gemm_last_error(). */
#ifndef TKM_GEMM_H
#define TKM_GEMM_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { TKM_GEMM_F16 = 0, TKM_GEMM_BF16 = 1, TKM_GEMM_F32 = 2 };

typedef struct tkm_gemm tkm_gemm;

int tkm_gemm_handle_create(void **handle);
void tkm_gemm_handle_destroy(void *handle);
/* m x n result C (ldc), inner dimension k; A stored m x k (k x m if trans_a), B stored k x n
 * (n x k if trans_b); A and B of type ab_type, C of c_type. */
int tkm_gemm_create(tkm_gemm **out, void *handle, int trans_a, int trans_b, int m, int n, int k, int lda, int ldb,
                    int ldc, int ab_type, int c_type, float beta, size_t max_workspace);
size_t tkm_gemm_workspace(const tkm_gemm *g);
int tkm_gemm_run(const tkm_gemm *g, const void *A, const void *B, void *C, void *workspace, size_t ws_bytes,
                 void *stream);
void tkm_gemm_destroy(tkm_gemm *g);
const char *tkm_gemm_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
