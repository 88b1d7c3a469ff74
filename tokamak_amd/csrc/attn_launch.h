// attn_launch.h -- internal launch records passed from the C ABI layer to the kernels.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace tkm {

struct FwdArgs {
    const void* qkv;
    void* o;
    float* lse;
    const int32_t* kv_len;
    int B, S, Hq, Hkv, D;
    float scale;
    int causal, dtype;
    void* stream;
};

struct BwdArgs {
    const void* qkv;
    const void* o;
    const void* dout;
    const float* lse;
    void* dqkv;
    const int32_t* kv_len;
    float* delta;  // workspace: D per row, B*Hq*S floats
    float* ld;     // workspace: per (b, h) and row pair m, m+1 (rows padded to 32):
                   // -LSE*log2(e) of m, m+1, then -D of m, m+1
    int B, S, Hq, Hkv, D;
    float scale;
    int causal, dtype;
    void* stream;
};

// Kernels a call launched (tkm_attn_last_kernels); values of the TKM_ATTN_K_* bits of
// include/tkm_attn.h.
enum KernelBit : unsigned {
    kFwdAsm = 1u, kFwdHip = 2u, kDqAsm = 4u, kDqHip = 8u, kDkdvAsm = 16u, kDkdvHip = 32u,
    kDeltaHip = 64u
};
void note_kernels(unsigned bits);  // ORs bits into the calling thread's record

// Assembly code objects: load on the current device (0, or -2 with asm_load_error()),
// and whether the assembly path exists there (gfx950, loaded).
int asm_init_current_device();
bool asm_available_current_device();
const char* asm_load_error();

// Launchers return 0 (launched), -1 (HIP launch error) or -2 (the assembly code objects
// failed to load on a gfx950 device).
int launch_fwd(const FwdArgs& a);
int launch_fwd_asm(const FwdArgs& a);  // also 1 = configuration not handled there
int launch_bwd_delta(const BwdArgs& a);
int launch_bwd_dkdv(const BwdArgs& a);
int launch_bwd_dkdv_asm(const BwdArgs& a);  // 1 = configuration not handled there
int launch_bwd_dq_asm(const BwdArgs& a, bool compute_d);  // 1 = not handled there
int launch_bwd_dq(const BwdArgs& a);
int launch_bwd_dq_delta(const BwdArgs& a);  // dQ, and D written for launch_bwd_dkdv

}  // namespace tkm
