// tkm_gemm.hip -- the runtime's FC GEMMs through hipBLASLt (host code; the C runtime calls the
// extern "C" functions of tkm_gemm.h).  They replace the reference's cublasGemmEx calls
// (src/tkm_gpu.cu:1207-1217 forward, 1330-1345 backward), with the same column-major
// operands: a weight W is stored as the column-major N_out x K matrix (ld N_out), i.e. the
// row-major [K][N_out] array the TKM1 files hold.
//   forward   out[N x rows]  = W[N x K] . in[K x rows]                       (N, N), beta 0
//   dW        dW[N x K] fp32 = dout[N x rows] . in^T                         (N, T), beta 0
//   dX        din[K x rows] += W^T . dout                                    (T, N), beta 1
// The algorithm is chosen once, at ignite (hipblasLtMatmulAlgoGetHeuristic); a launch then
// enqueues one hipblasLtMatmul on the runtime's stream with a caller-owned workspace, so a
// captured step replays it without allocation.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>
#include <stdio.h>
#include <stdlib.h>

#include "tkm_gemm.h"

struct tkm_gemm {
    hipblasLtHandle_t lt;
    hipblasLtMatmulDesc_t desc;
    hipblasLtMatrixLayout_t a, b, c;
    hipblasLtMatmulAlgo_t algo;
    float alpha, beta;
    size_t ws_needed;
};

namespace {
char g_err[256];

int fail(const char* what, int st) {
    snprintf(g_err, sizeof g_err, "%s failed with hipBLAS status %d", what, st);
    return -1;
}

hipDataType dtype_of(int t) { return t == TKM_GEMM_BF16 ? HIP_R_16BF : (t == TKM_GEMM_F32 ? HIP_R_32F : HIP_R_16F); }
}  // namespace

extern "C" {

const char* tkm_gemm_last_error(void) { return g_err; }

int tkm_gemm_handle_create(void** handle) {
    hipblasLtHandle_t h = nullptr;
    hipblasStatus_t st = hipblasLtCreate(&h);
    if (st != HIPBLAS_STATUS_SUCCESS) return fail("hipblasLtCreate", (int)st);
    *handle = h;
    return 0;
}

void tkm_gemm_handle_destroy(void* handle) {
    if (handle) hipblasLtDestroy((hipblasLtHandle_t)handle);
}

int tkm_gemm_create(tkm_gemm** out, void* handle, int trans_a, int trans_b, int m, int n, int k, int lda, int ldb,
                    int ldc, int ab_type, int c_type, float beta, size_t max_workspace) {
    *out = nullptr;
    tkm_gemm* g = (tkm_gemm*)calloc(1, sizeof(tkm_gemm));
    if (!g) return fail("calloc", -1);
    g->lt = (hipblasLtHandle_t)handle;
    g->alpha = 1.0f;
    g->beta = beta;
    hipblasStatus_t st = hipblasLtMatmulDescCreate(&g->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (st != HIPBLAS_STATUS_SUCCESS) { free(g); return fail("hipblasLtMatmulDescCreate", (int)st); }
    hipblasOperation_t ta = trans_a ? HIPBLAS_OP_T : HIPBLAS_OP_N, tb = trans_b ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    hipblasLtMatmulDescSetAttribute(g->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
    hipblasLtMatmulDescSetAttribute(g->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
    // stored shapes (column-major): A is m x k (or k x m transposed), B is k x n (or n x k)
    const hipDataType tab = dtype_of(ab_type), tc = dtype_of(c_type);
    hipblasLtMatrixLayoutCreate(&g->a, tab, trans_a ? k : m, trans_a ? m : k, lda);
    hipblasLtMatrixLayoutCreate(&g->b, tab, trans_b ? n : k, trans_b ? k : n, ldb);
    hipblasLtMatrixLayoutCreate(&g->c, tc, m, n, ldc);
    hipblasLtMatmulPreference_t pref;
    hipblasLtMatmulPreferenceCreate(&pref);
    uint64_t ws = max_workspace;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
    hipblasLtMatmulHeuristicResult_t res[1];
    int found = 0;
    st = hipblasLtMatmulAlgoGetHeuristic(g->lt, g->desc, g->a, g->b, g->c, g->c, pref, 1, res, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || found < 1) {
        snprintf(g_err, sizeof g_err,
                 "no hipBLASLt algorithm for m=%d n=%d k=%d trans=%d%d types %d/%d (status %d, found %d)", m, n, k,
                 trans_a, trans_b, ab_type, c_type, (int)st, found);
        tkm_gemm_destroy(g);
        return -1;
    }
    g->algo = res[0].algo;
    g->ws_needed = res[0].workspaceSize;
    *out = g;
    return 0;
}

size_t tkm_gemm_workspace(const tkm_gemm* g) { return g ? g->ws_needed : 0; }

int tkm_gemm_run(const tkm_gemm* g, const void* A, const void* B, void* C, void* workspace, size_t ws_bytes,
                 void* stream) {
    hipblasStatus_t st = hipblasLtMatmul(g->lt, g->desc, &g->alpha, A, g->a, B, g->b, &g->beta, C, g->c, C, g->c,
                                         &g->algo, workspace, ws_bytes, (hipStream_t)stream);
    return st == HIPBLAS_STATUS_SUCCESS ? 0 : fail("hipblasLtMatmul", (int)st);
}

void tkm_gemm_destroy(tkm_gemm* g) {
    if (!g) return;
    if (g->a) hipblasLtMatrixLayoutDestroy(g->a);
    if (g->b) hipblasLtMatrixLayoutDestroy(g->b);
    if (g->c) hipblasLtMatrixLayoutDestroy(g->c);
    if (g->desc) hipblasLtMatmulDescDestroy(g->desc);
    free(g);
}

}  // extern "C"
