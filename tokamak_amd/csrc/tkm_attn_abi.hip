// tkm_attn_abi.hip -- the extern "C" entry points declared in include/tkm_attn.h:
// argument validation, workspace checks and dispatch to the kernel launchers.
#include <stdarg.h>
#include <stdio.h>
#include <math.h>
#include <string.h>

#include <mutex>

#include <hip/hip_runtime.h>

#include "attn_launch.h"
#include "tkm_attn.h"
#include "tkm_prep_internal.h"

namespace tkm {
namespace {
thread_local unsigned t_kernels = 0;  // kernels launched by this thread's current/last call
}  // namespace
void note_kernels(unsigned bits) { t_kernels |= bits; }
}  // namespace tkm

// Backward workspace of tkm_attn_bwd_noalloc: a static device array, one per GPU (each
// device holds its own copy, at its own address, until the process ends).  Host code never
// uses the name `scratch` as an address (on the host it is only a stand-in symbol): it uses
// the per-device address that hipGetSymbolAddress returns, kept in g_scratch_ptr.  Nothing
// in it needs to start at zero: the dQ stage writes every byte the dK/dV stage reads.
static __device__ __align__(256) unsigned char scratch[TKM_ATTN_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch` on each device
}  // namespace

namespace {

int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    tkm_vset_error(status, fmt, ap);
    va_end(ap);
    return status;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Backward workspace: D per row (B*Hq*S floats), then at this 256-byte aligned offset the
// per-row pairs (-LSE*log2(e), -D), B*Hq rows each padded to a multiple of 32.
size_t tkm_ws_pairs_offset(int B, int S, int Hq) {
    const size_t n = (size_t)B * Hq * S * sizeof(float);
    return (n + 255) & ~(size_t)255;
}

// Shape checks shared by forward and backward (reference rules: tkm_core.c:392-404).
int check_shape(int B, int S, int Hq, int Hkv, int D, int causal, int dtype) {
    if (B < 1 || S < 1 || Hq < 1 || Hkv < 1)
        return fail(TKM_ATTN_EINVAL, "sizes must be positive (B=%d S=%d Hq=%d Hkv=%d)", B, S, Hq, Hkv);
    if (Hq % Hkv != 0) return fail(TKM_ATTN_EINVAL, "Hq=%d is not a multiple of Hkv=%d", Hq, Hkv);
    if (D != 64 && D != 128) return fail(TKM_ATTN_EUNSUPPORTED, "head dim D=%d (supported: 64, 128)", D);
    if (dtype != TKM_ATTN_F16 && dtype != TKM_ATTN_BF16)
        return fail(TKM_ATTN_EUNSUPPORTED, "dtype %d (supported: TKM_ATTN_F16, TKM_ATTN_BF16)", dtype);
    if (causal != 0 && causal != 1) return fail(TKM_ATTN_EINVAL, "causal must be 0 or 1, got %d", causal);
    // Every element offset must fit in int64 and every grid dimension in 31 bits.
    const double elems = (double)B * S * (Hq + 2.0 * Hkv) * D;
    if (elems > 9.0e15) return fail(TKM_ATTN_EUNSUPPORTED, "tensor too large");
    const double wgs = (double)B * Hq * ((S + 127) / 128 + 1);
    if (wgs > 2147483647.0) return fail(TKM_ATTN_EUNSUPPORTED, "grid too large");
    // Tiles are addressed through 32-bit buffer offsets: 128 rows of qkv must span < 2^31 bytes.
    if ((double)(Hq + 2 * Hkv) * D * 2.0 * 128.0 >= 2147483648.0)
        return fail(TKM_ATTN_EUNSUPPORTED, "row of qkv too wide ((Hq+2*Hkv)*D = %d)", (Hq + 2 * Hkv) * D);
    return TKM_ATTN_OK;
}

// Status of a launcher (0, -1 launch error, -2 code objects failed to load) as an ABI status.
int launch_status(int rc, const char* what) {
    if (rc == 0) return TKM_ATTN_OK;
    if (rc == -2)
        return fail(TKM_ATTN_EDEVICE, "%s: gfx950 assembly kernels failed to load (%s)", what,
                    tkm::asm_load_error());
    return fail(TKM_ATTN_ELAUNCH, "%s: kernel launch failed", what);
}

int run_bwd_stage(int stage, const tkm::BwdArgs& a) {
    int rc = 0;
    switch (stage) {
        case TKM_ATTN_BWD_DELTA: rc = tkm::launch_bwd_delta(a); break;
        case TKM_ATTN_BWD_DKDV: rc = tkm::launch_bwd_dkdv(a); break;
        case TKM_ATTN_BWD_DQ: rc = tkm::launch_bwd_dq(a); break;
        case TKM_ATTN_BWD_DQ_DELTA: rc = tkm::launch_bwd_dq_delta(a); break;
        default: return fail(TKM_ATTN_EINVAL, "unknown backward stage %d", stage);
    }
    if (rc == 0) return TKM_ATTN_OK;
    char what[48];
    snprintf(what, sizeof what, "backward stage %d", stage);
    return launch_status(rc, what);
}

// Checks of the backward's arguments other than the workspace.
int check_bwd_args(const void* qkv, const void* o, const void* dout, const float* lse,
                   void* dqkv, const int32_t* kv_len, int B, int S, int Hq, int Hkv, int D,
                   float scale, int causal, int dtype) {
    if (!qkv || !o || !dout || !lse || !dqkv)
        return fail(TKM_ATTN_EINVAL, "qkv, o, dout, lse and dqkv must be non-null");
    int rc = check_shape(B, S, Hq, Hkv, D, causal, dtype);
    if (rc) return rc;
    if (!aligned(qkv, 16) || !aligned(o, 16) || !aligned(dout, 16) || !aligned(dqkv, 16) ||
        !aligned(lse, 4) || (kv_len && !aligned(kv_len, 4)))
        return fail(TKM_ATTN_EALIGN, "16-bit tensors must be 16-byte aligned, lse/kv_len 4-byte");
    if (!(scale > 0.f) || scale == INFINITY) return fail(TKM_ATTN_EINVAL, "scale must be positive and finite");
    return TKM_ATTN_OK;
}

int prepare_bwd(tkm::BwdArgs& a, const void* qkv, const void* o, const void* dout,
                const float* lse, void* dqkv, const int32_t* kv_len, int B, int S, int Hq,
                int Hkv, int D, float scale, int causal, int dtype, void* workspace,
                size_t workspace_bytes, void* stream) {
    int rc = check_bwd_args(qkv, o, dout, lse, dqkv, kv_len, B, S, Hq, Hkv, D, scale, causal, dtype);
    if (rc) return rc;
    const size_t need = tkm_attn_bwd_workspace_bytes(B, S, Hq);
    if (!workspace || workspace_bytes < need)
        return fail(TKM_ATTN_EWORKSPACE, "workspace of %zu bytes required, %zu given", need,
                    workspace ? workspace_bytes : (size_t)0);
    if (!aligned(workspace, 16)) return fail(TKM_ATTN_EALIGN, "workspace must be 16-byte aligned");
    a = tkm::BwdArgs{qkv, o, dout, lse, dqkv, kv_len, (float*)workspace,
                     (float*)((char*)workspace + tkm_ws_pairs_offset(B, S, Hq)),
                     B, S, Hq, Hkv, D, scale, causal, dtype, stream};
    return TKM_ATTN_OK;
}

// Resolves the current device's address of `scratch` once (with that device current).
int scratch_setup(int dev) {
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(TKM_ATTN_EDEVICE, "device %d beyond the %d the scratch table holds", dev,
                    kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev]) return TKM_ATTN_OK;
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return fail(TKM_ATTN_EDEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                    hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
    return TKM_ATTN_OK;
}

}  // namespace

extern "C" {

TKM_ATTN_API int tkm_attn_fwd(const void* qkv, void* o, float* lse, const int32_t* kv_len, int B,
                              int S, int Hq, int Hkv, int D, float scale, int causal, int dtype,
                              void* stream) {
    tkm::t_kernels = 0;
    if (!qkv || !o) return fail(TKM_ATTN_EINVAL, "qkv and o must be non-null");
    int rc = check_shape(B, S, Hq, Hkv, D, causal, dtype);
    if (rc) return rc;
    if (!aligned(qkv, 16) || !aligned(o, 16) || (lse && !aligned(lse, 4)) ||
        (kv_len && !aligned(kv_len, 4)))
        return fail(TKM_ATTN_EALIGN, "16-bit tensors must be 16-byte aligned, lse/kv_len 4-byte");
    if (!(scale > 0.f) || scale == INFINITY) return fail(TKM_ATTN_EINVAL, "scale must be positive and finite");
    tkm::FwdArgs a{qkv, o, lse, kv_len, B, S, Hq, Hkv, D, scale, causal, dtype, stream};
    return launch_status(tkm::launch_fwd(a), "forward");
}

TKM_ATTN_API size_t tkm_attn_bwd_workspace_bytes(int B, int S, int Hq) {
    if (B < 1 || S < 1 || Hq < 1) return 0;
    return tkm_ws_pairs_offset(B, S, Hq) + (size_t)B * Hq * (((size_t)S + 31) & ~(size_t)31) * 8;
}

TKM_ATTN_API int tkm_attn_bwd(const void* qkv, const void* o, const void* dout, const float* lse,
                              void* dqkv, const int32_t* kv_len, int B, int S, int Hq, int Hkv,
                              int D, float scale, int causal, int dtype, void* workspace,
                              size_t workspace_bytes, void* stream) {
    tkm::t_kernels = 0;
    tkm::BwdArgs a;
    int rc = prepare_bwd(a, qkv, o, dout, lse, dqkv, kv_len, B, S, Hq, Hkv, D, scale, causal,
                         dtype, workspace, workspace_bytes, stream);
    if (rc) return rc;
    for (int stage : {TKM_ATTN_BWD_DQ_DELTA, TKM_ATTN_BWD_DKDV}) {
        rc = run_bwd_stage(stage, a);
        if (rc) return rc;
    }
    return TKM_ATTN_OK;
}

TKM_ATTN_API int tkm_attn_bwd_noalloc(const void* qkv, const void* o, const void* dout,
                                      const float* lse, void* dqkv, const int32_t* kv_len, int B,
                                      int S, int Hq, int Hkv, int D, float scale, int causal,
                                      int dtype, void* stream) {
    tkm::t_kernels = 0;
    const size_t need = tkm_attn_bwd_workspace_bytes(B, S, Hq);
    if (need > (size_t)TKM_ATTN_NOALLOC_SCRATCH_BYTES)
        return fail(TKM_ATTN_EWORKSPACE,
                    "tkm_attn_bwd_noalloc: B=%d S=%d Hq=%d needs %zu bytes of scratch, the static "
                    "scratch holds %d (use tkm_attn_bwd with a workspace)",
                    B, S, Hq, need, (int)TKM_ATTN_NOALLOC_SCRATCH_BYTES);
    // Everything that needs no device is checked before the device is touched.
    int rc = check_bwd_args(qkv, o, dout, lse, dqkv, kv_len, B, S, Hq, Hkv, D, scale, causal, dtype);
    if (rc) return rc;
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(TKM_ATTN_EDEVICE, "hipGetDevice: %s", hipGetErrorString(e));
    rc = scratch_setup(dev);  // first call on this device only (tkm_attn_init does it too)
    if (rc) return rc;
    void* ws = g_scratch_ptr[dev];
    tkm::BwdArgs a;
    rc = prepare_bwd(a, qkv, o, dout, lse, dqkv, kv_len, B, S, Hq, Hkv, D, scale, causal, dtype,
                     ws, need, stream);
    if (rc) return rc;
    for (int stage : {TKM_ATTN_BWD_DQ_DELTA, TKM_ATTN_BWD_DKDV}) {
        rc = run_bwd_stage(stage, a);
        if (rc) return rc;
    }
    return TKM_ATTN_OK;
}

TKM_ATTN_API int tkm_attn_bwd_stage(int stage, const void* qkv, const void* o, const void* dout,
                                    const float* lse, void* dqkv, const int32_t* kv_len, int B,
                                    int S, int Hq, int Hkv, int D, float scale, int causal,
                                    int dtype, void* workspace, size_t workspace_bytes,
                                    void* stream) {
    tkm::t_kernels = 0;
    if (stage < TKM_ATTN_BWD_DELTA || stage > TKM_ATTN_BWD_DQ_DELTA)
        return fail(TKM_ATTN_EINVAL, "unknown backward stage %d", stage);
    tkm::BwdArgs a;
    int rc = prepare_bwd(a, qkv, o, dout, lse, dqkv, kv_len, B, S, Hq, Hkv, D, scale, causal,
                         dtype, workspace, workspace_bytes, stream);
    if (rc) return rc;
    return run_bwd_stage(stage, a);
}

TKM_ATTN_API const char* tkm_attn_status_string(int status) {
    switch (status) {
        case TKM_ATTN_OK: return "ok";
        case TKM_ATTN_EINVAL: return "invalid argument";
        case TKM_ATTN_EUNSUPPORTED: return "unsupported configuration";
        case TKM_ATTN_EALIGN: return "misaligned pointer";
        case TKM_ATTN_EWORKSPACE: return "workspace missing or too small";
        case TKM_ATTN_ELAUNCH: return "kernel launch failed";
        case TKM_ATTN_ECOMPILE: return "run-time compilation failed";
        case TKM_ATTN_EDEVICE: return "device, module or graph error";
        default: return "unknown status";
    }
}

TKM_ATTN_API int tkm_attn_init(void) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(TKM_ATTN_EDEVICE, "hipGetDevice: %s", hipGetErrorString(e));
    if (tkm::asm_init_current_device() != 0)
        return fail(TKM_ATTN_EDEVICE, "gfx950 assembly kernels failed to load on device %d (%s)",
                    dev, tkm::asm_load_error());
    return scratch_setup(dev);
}

TKM_ATTN_API int tkm_attn_asm_available(void) {
    return tkm::asm_available_current_device() ? 1 : 0;
}

TKM_ATTN_API unsigned tkm_attn_last_kernels(void) { return tkm::t_kernels; }

TKM_ATTN_API int tkm_attn_version(void) { return 200; }

}  // extern "C"
