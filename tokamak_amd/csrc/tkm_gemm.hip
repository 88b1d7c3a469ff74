// tkm_gemm.hip -- the runtime's FC GEMMs through hipBLASLt (host code; the C runtime calls the
// extern "C" functions of tkm_gemm.h).  They replace the reference's cublasGemmEx calls
// (src/tkm_gpu.cu:1207-1217 forward, 1330-1345 backward), with the same column-major
// operands: a weight W is stored as the column-major N_out x K matrix (ld N_out), i.e. the
// row-major [K][N_out] array the TKM1 files hold.
//   forward   out[N x rows]  = W[N x K] . in[K x rows]                       (N, N), beta 0
//   dW        dW[N x K] fp32 = dout[N x rows] . in^T                         (N, T), beta 0
//   dX        din[K x rows] += W^T . dout                                    (T, N), beta 1
// The algorithm is chosen once, at ignite: hipblasLtMatmulAlgoGetHeuristic proposes up to
// TKM_GEMM_CANDIDATES, and tkm_gemm_tune times them on the runtime's own buffers and keeps the
// fastest (once per distinct problem in a process).  A launch then enqueues one
// hipblasLtMatmul on the runtime's stream with a caller-owned workspace, so a captured step
// replays it without allocation.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>
#include <stdio.h>
#include <stdlib.h>

#include "tkm_gemm.h"

#define TKM_GEMM_CANDIDATES 8

struct tkm_gemm {
    hipblasLtHandle_t lt;
    hipblasLtMatmulDesc_t desc;
    hipblasLtMatrixLayout_t a, b, c;
    hipblasLtMatmulAlgo_t algo;
    float alpha, beta;
    size_t ws_needed;
    hipblasLtMatmulAlgo_t cand[TKM_GEMM_CANDIDATES];
    size_t cand_ws[TKM_GEMM_CANDIDATES];
    int n_cand;
    int key[10];              // the problem: transposes, sizes, leading dimensions, types, beta
};

namespace {
char g_err[256];

int fail(const char* what, int st) {
    snprintf(g_err, sizeof g_err, "%s failed with hipBLAS status %d", what, st);
    return -1;
}

hipDataType dtype_of(int t) { return t == TKM_GEMM_BF16 ? HIP_R_16BF : (t == TKM_GEMM_F32 ? HIP_R_32F : HIP_R_16F); }

// problems already tuned in this process: key -> candidate index
struct tuned_entry {
    int key[10];
    int pick;
};
tuned_entry g_tuned[256];
int g_n_tuned = 0;

int find_tuned(const int* key) {
    for (int i = 0; i < g_n_tuned; ++i) {
        bool same = true;
        for (int j = 0; j < 10; ++j) same = same && g_tuned[i].key[j] == key[j];
        if (same) return g_tuned[i].pick;
    }
    return -1;
}
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
    hipblasLtMatmulHeuristicResult_t res[TKM_GEMM_CANDIDATES];
    int found = 0;
    st = hipblasLtMatmulAlgoGetHeuristic(g->lt, g->desc, g->a, g->b, g->c, g->c, pref, TKM_GEMM_CANDIDATES, res,
                                         &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || found < 1) {
        snprintf(g_err, sizeof g_err,
                 "no hipBLASLt algorithm for m=%d n=%d k=%d trans=%d%d types %d/%d (status %d, found %d)", m, n, k,
                 trans_a, trans_b, ab_type, c_type, (int)st, found);
        tkm_gemm_destroy(g);
        return -1;
    }
    g->n_cand = found < TKM_GEMM_CANDIDATES ? found : TKM_GEMM_CANDIDATES;
    for (int i = 0; i < g->n_cand; ++i) {
        g->cand[i] = res[i].algo;
        g->cand_ws[i] = res[i].workspaceSize;
    }
    g->algo = res[0].algo;
    g->ws_needed = res[0].workspaceSize;
    const int key[10] = {trans_a, trans_b, m, n, k, lda, ldb, ldc, ab_type * 4 + c_type, beta != 0.0f};
    for (int j = 0; j < 10; ++j) g->key[j] = key[j];
    *out = g;
    return 0;
}

size_t tkm_gemm_workspace(const tkm_gemm* g) {
    if (!g) return 0;
    size_t w = g->ws_needed;
    for (int i = 0; i < g->n_cand; ++i)
        if (g->cand_ws[i] > w) w = g->cand_ws[i];
    return w;
}

int tkm_gemm_tune(tkm_gemm* g, const void* A, const void* B, void* C, void* workspace, size_t ws_bytes,
                  void* stream) {
    if (!g || g->n_cand <= 1) return 0;
    int pick = find_tuned(g->key);
    if (pick < 0) {
        hipStream_t st = (hipStream_t)stream;
        hipEvent_t e0, e1;
        if (hipEventCreate(&e0) != hipSuccess) return fail("hipEventCreate", -1);
        if (hipEventCreate(&e1) != hipSuccess) {
            hipEventDestroy(e0);
            return fail("hipEventCreate", -1);
        }
        float best = 0.0f;
        for (int i = 0; i < g->n_cand; ++i) {
            if (g->cand_ws[i] > ws_bytes) continue;
            // one untimed run (also rejects a candidate the library cannot launch), then 5 timed
            if (hipblasLtMatmul(g->lt, g->desc, &g->alpha, A, g->a, B, g->b, &g->beta, C, g->c, C, g->c, &g->cand[i],
                                workspace, ws_bytes, st) != HIPBLAS_STATUS_SUCCESS)
                continue;
            hipEventRecord(e0, st);
            bool ok = true;
            for (int r = 0; r < 5 && ok; ++r)
                ok = hipblasLtMatmul(g->lt, g->desc, &g->alpha, A, g->a, B, g->b, &g->beta, C, g->c, C, g->c,
                                     &g->cand[i], workspace, ws_bytes, st) == HIPBLAS_STATUS_SUCCESS;
            hipEventRecord(e1, st);
            float ms = 0.0f;
            if (!ok || hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) continue;
            if (pick < 0 || ms < best) {
                best = ms;
                pick = i;
            }
        }
        hipEventDestroy(e0);
        hipEventDestroy(e1);
        if (pick < 0) pick = 0;
        if (g_n_tuned < (int)(sizeof g_tuned / sizeof g_tuned[0])) {
            for (int j = 0; j < 10; ++j) g_tuned[g_n_tuned].key[j] = g->key[j];
            g_tuned[g_n_tuned++].pick = pick;
        }
    }
    if (pick >= g->n_cand) pick = 0;
    g->algo = g->cand[pick];
    g->ws_needed = g->cand_ws[pick];
    return 0;
}

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
