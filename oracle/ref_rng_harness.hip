// Test infrastructure (the oracle's pins): runs the reference's own Drop generators on the GPU.
// _ref/ref_rng.inc is the reference's generator code (src/tkm_gpu.cu:751-794), extracted by
// extract_ref_rng.py in the build container; this file only calls it.  Built by `make rng`
// into oracle/_ref/libref_rng.so; tests/golden/make_rng_vectors.py writes the vectors that
// tests/test_oracle.py holds the oracle's restatement (plasma_ref.c) to.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ref_rng.inc"

template <typename R>
__device__ void draw(uint32_t seed, uint32_t idx, int draws, uint32_t* out, float* uni) {
    R r;
    rng_init(&r, seed, idx);
    for (int d = 0; d < draws; ++d) out[d] = rng_u32(&r);
    R u;
    rng_init(&u, seed, idx);
    for (int d = 0; d < draws; ++d) uni[d] = rng_uniform(&u);
}

// Stream i: generator `type` (the reference's TkmRngType: 1 xorshift32, 2 Wang hash + xorshift32,
// 3 PCG32, 4 the counter generator) from rng_init(seed[i], idx[i]); `draws` outputs of rng_u32
// and, from a second stream with the same start, of rng_uniform.
extern "C" __global__ void ref_rng_kernel(int type, const uint32_t* seeds, const uint32_t* idxs, int n, int draws,
                                          uint32_t* out, float* uni) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t* o = out + (size_t)i * draws;
    float* u = uni + (size_t)i * draws;
    switch (type) {
        case 1: draw<RngXorshift32>(seeds[i], idxs[i], draws, o, u); break;
        case 2: draw<RngWangXorshift32>(seeds[i], idxs[i], draws, o, u); break;
        case 3: draw<RngPcg32>(seeds[i], idxs[i], draws, o, u); break;
        default: draw<RngPhilox>(seeds[i], idxs[i], draws, o, u); break;
    }
}

// Host side: copies in, runs, copies out.  0 on success.
extern "C" int ref_rng_run(int type, const uint32_t* seeds, const uint32_t* idxs, int n, int draws, uint32_t* out,
                           float* uni) {
    if (n <= 0 || draws <= 0 || type < 1 || type > 4) return -1;
    uint32_t *d_s = nullptr, *d_i = nullptr, *d_o = nullptr;
    float* d_u = nullptr;
    const size_t m = (size_t)n * draws;
    int rc = -1;
    if (hipMalloc(&d_s, n * 4) == hipSuccess && hipMalloc(&d_i, n * 4) == hipSuccess &&
        hipMalloc(&d_o, m * 4) == hipSuccess && hipMalloc(&d_u, m * 4) == hipSuccess &&
        hipMemcpy(d_s, seeds, n * 4, hipMemcpyHostToDevice) == hipSuccess &&
        hipMemcpy(d_i, idxs, n * 4, hipMemcpyHostToDevice) == hipSuccess) {
        hipLaunchKernelGGL(ref_rng_kernel, dim3((n + 63) / 64), dim3(64), 0, 0, type, d_s, d_i, n, draws, d_o, d_u);
        if (hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess &&
            hipMemcpy(out, d_o, m * 4, hipMemcpyDeviceToHost) == hipSuccess &&
            hipMemcpy(uni, d_u, m * 4, hipMemcpyDeviceToHost) == hipSuccess)
            rc = 0;
    }
    (void)hipFree(d_s);
    (void)hipFree(d_i);
    (void)hipFree(d_o);
    (void)hipFree(d_u);
    return rc;
}
