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

int launch_fwd(const FwdArgs& a);
int launch_fwd_asm(const FwdArgs& a);  // 1 = configuration not handled there
int launch_bwd_delta(const BwdArgs& a);
int launch_bwd_dkdv(const BwdArgs& a);
int launch_bwd_dkdv_asm(const BwdArgs& a);  // 1 = configuration not handled there
int launch_bwd_dq_asm(const BwdArgs& a, bool compute_d);  // 1 = not handled there
int launch_bwd_dq(const BwdArgs& a);
int launch_bwd_dq_delta(const BwdArgs& a);  // dQ, and D written for launch_bwd_dkdv

}  // namespace tkm
