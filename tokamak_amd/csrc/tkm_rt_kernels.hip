// tkm_rt_kernels.hip -- the runtime's own small kernels (gfx950), called by tkm_hip.c through
// the C launchers at the end of this file:
//   input staging        fp32 host rows -> 16-bit arena rows   (reference k_f32_to_f16, tkm_gpu.cu:58-61)
//   fill                 32-bit fill of a buffer (the gradient arena's per-step clear; no
//                        hipMemsetAsync, so the step graph holds no memset node)
//   softmax + loss       per-row softmax with CE / focal / MSE loss and its gradient
//                        (k_softmax_loss_fwd_bwd_h, tkm_gpu.cu:632-682), one wave per row, and
//                        a fixed-order reduction of the per-row losses (no float atomics)
//   softmax fwd / bwd    (k_softmax_fwd_h / k_softmax_bwd_h, tkm_gpu.cu:600-630)
//   SGD                  momentum SGD over every learnable tensor (k_tkm_multi_tensor_sgd,
//                        tkm_gpu.cu:684-720), with the fp32 master and its 16-bit copy
//   perturb, gather      the gradient-check probe (tkm_gpu.cu:121-126) and the resident
//                        dataset's batch gather (k_resident_gather, tkm_gpu.cu:70-102)
// 16-bit tensors are fp16 (the reference's type) or bf16 (dtype 1), converted with RNE.
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <math.h>
#include <stdint.h>

#include "tkm_rt_kernels.h"

namespace {

__device__ __forceinline__ float ld16(const uint16_t* p, size_t i, int dt) {
    const uint16_t b = p[i];
    if (dt == 1) return __uint_as_float((uint32_t)b << 16);
    return __half2float(__ushort_as_half(b));
}

__device__ __forceinline__ uint16_t to16(float v, int dt) {
    if (dt == 1) {
        const uint32_t u = __float_as_uint(v);
        if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // NaN stays NaN
        return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
    return __half_as_ushort(__float2half_rn(v));
}

__global__ void k_f32_to_16(const float* __restrict__ src, uint16_t* __restrict__ dst, size_t n, int dt) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = to16(src[i], dt);
}

__global__ void k_16_to_f32(const uint16_t* __restrict__ src, float* __restrict__ dst, size_t n, int dt) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = ld16(src, i, dt);
}

__global__ void k_fill_u32x4(uint4* __restrict__ dst, size_t n4, uint32_t v) {
    const uint4 q = make_uint4(v, v, v, v);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = q;
}

__global__ void k_fill_u32(uint32_t* __restrict__ dst, size_t n, uint32_t v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// One wave per row.  The argmax is the first maximal column, as the reference's strict '>'
// scan finds it; the sums run over the wave's lanes in a fixed order (deterministic).
__global__ __launch_bounds__(256) void k_softmax_loss(const uint16_t* __restrict__ logits, int dt,
                                                      const void* __restrict__ labels, int label_i32,
                                                      uint16_t* __restrict__ dlogits, float* __restrict__ row_loss,
                                                      int* __restrict__ row_correct, int rows, int cols,
                                                      int is_eval, int valid_rows, int loss_kind, float gamma) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const size_t base = (size_t)r * cols;
    float mx = -1e30f;
    int pred = 0x7fffffff;
    for (int c = lane; c < cols; c += 64) {
        const float v = ld16(logits, base + c, dt);
        if (v > mx) { mx = v; pred = c; }
    }
    // combine (max, first index) over the wave
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float om = __shfl_xor(mx, o, 64);
        const int op = __shfl_xor(pred, o, 64);
        if (om > mx || (om == mx && op < pred)) { mx = om; pred = op; }
    }
    if (pred == 0x7fffffff) pred = 0;
    float sum = 0.f;
    for (int c = lane; c < cols; c += 64) sum += expf(ld16(logits, base + c, dt) - mx);
    sum = wave_sum(sum);
    int lbl = 0;
    if (labels) lbl = label_i32 ? ((const int32_t*)labels)[r] : (int)((const uint8_t*)labels)[r];
    if (lbl < 0 || lbl >= cols) lbl = 0;
    if (lane == 0) row_correct[r] = ((!is_eval || r < valid_rows) && pred == lbl) ? 1 : 0;
    if (is_eval) {
        if (lane == 0) row_loss[r] = 0.f;
        return;
    }
    const float inv_rows = 1.0f / (float)rows;
    float tp = expf(ld16(logits, base + lbl, dt) - mx) / sum;
    tp = fmaxf(tp, 1e-7f);
    const float fw = powf(1.0f - tp, gamma);
    const float fscale = loss_kind == 1 ? fw - gamma * tp * powf(1.0f - tp, gamma - 1.0f) * logf(tp) : 1.0f;
    float brier = 0.f, mse = 0.f;
    if (loss_kind == 2) {
        for (int c = lane; c < cols; c += 64) {
            const float p = expf(ld16(logits, base + c, dt) - mx) / sum;
            const float t = c == lbl ? 1.0f : 0.0f;
            brier += p * (p - t);
            mse += (p - t) * (p - t) / (float)cols;
        }
        brier = wave_sum(brier);
        mse = wave_sum(mse);
    }
    for (int c = lane; c < cols; c += 64) {
        const float p = expf(ld16(logits, base + c, dt) - mx) / sum;
        const float t = c == lbl ? 1.0f : 0.0f;
        float g;
        if (loss_kind == 0) g = p - t;
        else if (loss_kind == 1) g = fscale * (p - t);
        else g = (2.0f / (float)cols) * p * ((p - t) - brier);
        dlogits[base + c] = to16(g * inv_rows, dt);
    }
    if (lane == 0) {
        float l;
        if (loss_kind == 0) l = -logf(tp);
        else if (loss_kind == 1) l = -fw * logf(tp);
        else l = mse;
        row_loss[r] = l * inv_rows;
    }
}

// The same per-row softmax and loss for rows of a multiple of 8 columns, at most 8192: the
// wave reads its row once into registers (16-byte loads, lane l holding columns
// (64k + l)*8 .. +7 of chunk k) and runs max, sum and gradient from them, writing dlogits as
// 16-byte stores.  Per element the arithmetic is the scalar kernel's; the sums run over each
// lane's elements in column order, then over the wave.
template <int NCH>
__global__ __launch_bounds__(256) void k_softmax_loss_v(const uint16_t* __restrict__ logits, int dt,
                                                        const void* __restrict__ labels, int label_i32,
                                                        uint16_t* __restrict__ dlogits, float* __restrict__ row_loss,
                                                        int* __restrict__ row_correct, int rows, int cols,
                                                        int is_eval, int valid_rows, int loss_kind, float gamma) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const size_t base = (size_t)r * cols;
    const int nchunk = cols / 8;
    uint4 x[NCH];
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int ch = k * 64 + lane;
        x[k] = ch < nchunk ? *(const uint4*)(logits + base + (size_t)ch * 8) : make_uint4(0u, 0u, 0u, 0u);
    }
    auto val = [&](const uint4& q, int j) __attribute__((always_inline)) {
        const int wi = j >> 1;
        const uint32_t w = wi == 0 ? q.x : (wi == 1 ? q.y : (wi == 2 ? q.z : q.w));
        const uint16_t b = (uint16_t)((j & 1) ? (w >> 16) : (w & 0xffffu));
        return dt == 1 ? __uint_as_float((uint32_t)b << 16) : __half2float(__ushort_as_half(b));
    };
    float mx = -1e30f;
    int pred = 0x7fffffff;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int ch = k * 64 + lane;
        if (ch < nchunk) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = val(x[k], j);
                if (v > mx) { mx = v; pred = ch * 8 + j; }
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float om = __shfl_xor(mx, o, 64);
        const int op = __shfl_xor(pred, o, 64);
        if (om > mx || (om == mx && op < pred)) { mx = om; pred = op; }
    }
    if (pred == 0x7fffffff) pred = 0;
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < NCH; ++k)
        if (k * 64 + lane < nchunk) {
#pragma unroll
            for (int j = 0; j < 8; ++j) sum += expf(val(x[k], j) - mx);
        }
    sum = wave_sum(sum);
    int lbl = 0;
    if (labels) lbl = label_i32 ? ((const int32_t*)labels)[r] : (int)((const uint8_t*)labels)[r];
    if (lbl < 0 || lbl >= cols) lbl = 0;
    if (lane == 0) row_correct[r] = ((!is_eval || r < valid_rows) && pred == lbl) ? 1 : 0;
    if (is_eval) {
        if (lane == 0) row_loss[r] = 0.f;
        return;
    }
    const float inv_rows = 1.0f / (float)rows;
    float tp = expf(ld16(logits, base + lbl, dt) - mx) / sum;
    tp = fmaxf(tp, 1e-7f);
    const float fw = powf(1.0f - tp, gamma);
    const float fscale = loss_kind == 1 ? fw - gamma * tp * powf(1.0f - tp, gamma - 1.0f) * logf(tp) : 1.0f;
    float brier = 0.f, mse = 0.f;
    if (loss_kind == 2) {
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int ch = k * 64 + lane;
            if (ch < nchunk) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p = expf(val(x[k], j) - mx) / sum;
                    const float t = ch * 8 + j == lbl ? 1.0f : 0.0f;
                    brier += p * (p - t);
                    mse += (p - t) * (p - t) / (float)cols;
                }
            }
        }
        brier = wave_sum(brier);
        mse = wave_sum(mse);
    }
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int ch = k * 64 + lane;
        if (ch < nchunk) {
            uint32_t w[4];
#pragma unroll
            for (int j2 = 0; j2 < 4; ++j2) {
                uint16_t h2[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int j = 2 * j2 + e;
                    const float p = expf(val(x[k], j) - mx) / sum;
                    const float t = ch * 8 + j == lbl ? 1.0f : 0.0f;
                    float g;
                    if (loss_kind == 0) g = p - t;
                    else if (loss_kind == 1) g = fscale * (p - t);
                    else g = (2.0f / (float)cols) * p * ((p - t) - brier);
                    h2[e] = to16(g * inv_rows, dt);
                }
                w[j2] = (uint32_t)h2[0] | ((uint32_t)h2[1] << 16);
            }
            *(uint4*)(dlogits + base + (size_t)ch * 8) = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
    if (lane == 0) {
        float l;
        if (loss_kind == 0) l = -logf(tp);
        else if (loss_kind == 1) l = -fw * logf(tp);
        else l = mse;
        row_loss[r] = l * inv_rows;
    }
}

// Sum of the per-row losses and correct flags in row order (one block of 1024 threads: strided
// partial sums, then a fixed tree); out[0] += loss, *correct += count when accumulate, else =.
__global__ __launch_bounds__(1024) void k_loss_reduce(const float* __restrict__ row_loss,
                                                      const int* __restrict__ row_correct, int rows,
                                                      float* __restrict__ loss_out, int* __restrict__ correct_out,
                                                      int acc_loss, int acc_correct) {
    __shared__ float sl[1024];
    __shared__ int sc[1024];
    float l = 0.f;
    int c = 0;
    for (int r = threadIdx.x; r < rows; r += 1024) {
        l += row_loss[r];
        c += row_correct[r];
    }
    sl[threadIdx.x] = l;
    sc[threadIdx.x] = c;
    __syncthreads();
    for (int s = 512; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            sl[threadIdx.x] += sl[threadIdx.x + s];
            sc[threadIdx.x] += sc[threadIdx.x + s];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        if (loss_out) *loss_out = acc_loss ? *loss_out + sl[0] : sl[0];
        if (correct_out) *correct_out = acc_correct ? *correct_out + sc[0] : sc[0];
    }
}

__global__ __launch_bounds__(256) void k_softmax_fwd(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                     int rows, int cols, int dt) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const size_t base = (size_t)r * cols;
    float mx = -1e30f;
    for (int c = lane; c < cols; c += 64) mx = fmaxf(mx, ld16(x, base + c, dt));
    mx = wave_max(mx);
    float sum = 0.f;
    for (int c = lane; c < cols; c += 64) sum += expf(ld16(x, base + c, dt) - mx);
    sum = wave_sum(sum);
    for (int c = lane; c < cols; c += 64) y[base + c] = to16(expf(ld16(x, base + c, dt) - mx) / sum, dt);
}

// din += p * (dp - <p, dp>)   (the reference accumulates into dlogits)
__global__ __launch_bounds__(256) void k_softmax_bwd(const uint16_t* __restrict__ p, const uint16_t* __restrict__ dp,
                                                     uint16_t* __restrict__ din, int rows, int cols, int dt) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const size_t base = (size_t)r * cols;
    float dot = 0.f;
    for (int c = lane; c < cols; c += 64) dot += ld16(p, base + c, dt) * ld16(dp, base + c, dt);
    dot = wave_sum(dot);
    for (int c = lane; c < cols; c += 64) {
        const float pv = ld16(p, base + c, dt);
        din[base + c] = to16(ld16(din, base + c, dt) + pv * (ld16(dp, base + c, dt) - dot), dt);
    }
}

// Momentum SGD with the reference's update (tkm_gpu.cu:696-720): decoupled-from-nothing weight
// decay on tensors that have a 16-bit copy (GEMM weights), then
//   v = momentum * v + g,  p -= lr * (momentum * v + g)   (Nesterov form),  w16 = round(p).
// One block updates TKM_SGD_CHUNK consecutive elements of one tensor, 8 per thread with
// 16-byte accesses (every tensor starts 256-byte aligned); the block finds its tensor by a
// binary search over the tensors' first blocks.  Block 0 advances the step seed of the
// stochastic ops.
__device__ __forceinline__ void sgd_one(float& p, float& v, float g, float lr, float momentum, float wd, bool decay) {
    if (decay) g = fmaf(wd, p, g);
    v = fmaf(momentum, v, g);
    p = fmaf(-lr, fmaf(momentum, v, g), p);
}

__global__ __launch_bounds__(256) void k_sgd(const TkmSgdTensor* __restrict__ t, int nt,
                                             const float* __restrict__ d_lr, float momentum, float wd,
                                             uint32_t* __restrict__ d_seed, int dt) {
    const long long blk = blockIdx.x;
    if (blk == 0 && threadIdx.x == 0 && d_seed) *d_seed += 0x9E3779B9u;
    int lo = 0, hi = nt - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (t[mid].block0 <= blk) lo = mid; else hi = mid - 1;
    }
    const TkmSgdTensor tt = t[lo];
    const long long i0 = (blk - tt.block0) * TKM_SGD_CHUNK + (long long)threadIdx.x * 8;
    if (i0 >= tt.size) return;
    const float lr = *d_lr;
    const bool decay = tt.w16 != nullptr;
    if (i0 + 8 <= tt.size) {
        float4* mp = (float4*)(tt.master + i0);
        float4* vp = (float4*)(tt.vel + i0);
        const float4* gp = (const float4*)(tt.grad + i0);
        float4 p0 = mp[0], p1 = mp[1], v0 = vp[0], v1 = vp[1];
        const float4 g0 = gp[0], g1 = gp[1];
        sgd_one(p0.x, v0.x, g0.x, lr, momentum, wd, decay);
        sgd_one(p0.y, v0.y, g0.y, lr, momentum, wd, decay);
        sgd_one(p0.z, v0.z, g0.z, lr, momentum, wd, decay);
        sgd_one(p0.w, v0.w, g0.w, lr, momentum, wd, decay);
        sgd_one(p1.x, v1.x, g1.x, lr, momentum, wd, decay);
        sgd_one(p1.y, v1.y, g1.y, lr, momentum, wd, decay);
        sgd_one(p1.z, v1.z, g1.z, lr, momentum, wd, decay);
        sgd_one(p1.w, v1.w, g1.w, lr, momentum, wd, decay);
        mp[0] = p0;
        mp[1] = p1;
        vp[0] = v0;
        vp[1] = v1;
        if (decay) {
            const uint4 w = make_uint4((uint32_t)to16(p0.x, dt) | ((uint32_t)to16(p0.y, dt) << 16),
                                       (uint32_t)to16(p0.z, dt) | ((uint32_t)to16(p0.w, dt) << 16),
                                       (uint32_t)to16(p1.x, dt) | ((uint32_t)to16(p1.y, dt) << 16),
                                       (uint32_t)to16(p1.z, dt) | ((uint32_t)to16(p1.w, dt) << 16));
            *(uint4*)((uint16_t*)tt.w16 + i0) = w;
        }
        return;
    }
    for (long long i = i0; i < tt.size; ++i) {
        float p = tt.master[i], v = tt.vel[i];
        sgd_one(p, v, tt.grad[i], lr, momentum, wd, decay);
        tt.vel[i] = v;
        tt.master[i] = p;
        if (decay) ((uint16_t*)tt.w16)[i] = to16(p, dt);
    }
}

// Parameter gradients of every group from their band partials, in one launch at the end of
// the backward: per 64 columns, 16 waves sum bands w, w+16, ... and wave 0 adds the 16 sums in
// order, as the generated per-group reduce kernels do.
__global__ __launch_bounds__(1024) void k_reduce_parts(const TkmReduceChunk* __restrict__ t) {
    const TkmReduceChunk e = t[blockIdx.x];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float acc = 0.f;
    if (lane < e.ncols) {
#pragma unroll 4
        for (int b = wave; b < e.bands; b += 16) acc += e.part[(size_t)b * e.pw + e.col0 + lane];
    }
    __shared__ float red[16][64];
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0 || lane >= e.ncols) return;
    float sum = red[0][lane];
    for (int q = 1; q < 16; ++q) sum += red[q][lane];
    e.dst[lane] = sum;
}

__global__ void k_perturb(uint16_t* __restrict__ p, long long i, float delta, int dt) {
    p[i] = to16(ld16(p, (size_t)i, dt) + delta, dt);
}

__global__ void k_add_f32(float* __restrict__ acc, const float* __restrict__ v) { *acc += *v; }

// Batch b of a resident dataset: rows of samples order[b*B + s] -> the input rows and labels.
__global__ void k_gather(const uint16_t* __restrict__ images, const uint8_t* __restrict__ labels,
                         const uint32_t* __restrict__ order, long long first, int B, size_t elems,
                         uint16_t* __restrict__ dst, uint8_t* __restrict__ dst_labels) {
    const int s = blockIdx.y;
    const size_t src = (size_t)order[first + s];
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < elems; i += (size_t)gridDim.x * blockDim.x)
        dst[(size_t)s * elems + i] = images[src * elems + i];
    if (blockIdx.x == 0 && threadIdx.x == 0) dst_labels[s] = labels[src];
}

unsigned grid_for(size_t n, unsigned block) {
    size_t g = (n + block - 1) / block;
    if (g > 65536) g = 65536;
    return g < 1 ? 1u : (unsigned)g;
}

int status(void) { return hipGetLastError() == hipSuccess ? 0 : -1; }

}  // namespace

extern "C" {

int tkm_rt_f32_to_16(const float* src, void* dst, size_t n, int dtype, void* stream) {
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_f32_to_16, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t)stream, src,
                       (uint16_t*)dst, n, dtype);
    return status();
}

int tkm_rt_16_to_f32(const void* src, float* dst, size_t n, int dtype, void* stream) {
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_16_to_f32, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)src, dst, n, dtype);
    return status();
}

int tkm_rt_fill_u32(void* dst, size_t bytes, uint32_t value, void* stream) {
    if (bytes == 0) return 0;
    if (((uintptr_t)dst & 15u) == 0 && bytes % 16 == 0) {
        hipLaunchKernelGGL(k_fill_u32x4, dim3(grid_for(bytes / 16, 256)), dim3(256), 0, (hipStream_t)stream,
                           (uint4*)dst, bytes / 16, value);
    } else {
        hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(bytes / 4, 256)), dim3(256), 0, (hipStream_t)stream,
                           (uint32_t*)dst, bytes / 4, value);
    }
    return status();
}

int tkm_rt_softmax_loss(const void* logits, int dtype, const void* labels, int label_i32, void* dlogits,
                        float* row_loss, int* row_correct, int rows, int cols, int is_eval, int valid_rows,
                        int loss_kind, float gamma, float* loss_out, int* correct_out, int acc_loss,
                        int acc_correct, void* stream) {
    if (rows <= 0) return 0;
    const bool vec = cols % 8 == 0 && cols <= 8192 && ((uintptr_t)logits & 15u) == 0 &&
                     (is_eval || ((uintptr_t)dlogits & 15u) == 0);
    if (vec && cols <= 2048)
        hipLaunchKernelGGL(k_softmax_loss_v<4>, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t*)logits, dtype, labels, label_i32, (uint16_t*)dlogits, row_loss,
                           row_correct, rows, cols, is_eval, valid_rows, loss_kind, gamma);
    else if (vec)
        hipLaunchKernelGGL(k_softmax_loss_v<16>, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t*)logits, dtype, labels, label_i32, (uint16_t*)dlogits, row_loss,
                           row_correct, rows, cols, is_eval, valid_rows, loss_kind, gamma);
    else
        hipLaunchKernelGGL(k_softmax_loss, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t*)logits, dtype, labels, label_i32, (uint16_t*)dlogits, row_loss,
                           row_correct, rows, cols, is_eval, valid_rows, loss_kind, gamma);
    if (status()) return -1;
    hipLaunchKernelGGL(k_loss_reduce, dim3(1), dim3(1024), 0, (hipStream_t)stream, row_loss, row_correct, rows,
                       loss_out, correct_out, acc_loss, acc_correct);
    return status();
}

int tkm_rt_softmax_fwd(const void* x, void* y, int rows, int cols, int dtype, void* stream) {
    if (rows <= 0) return 0;
    hipLaunchKernelGGL(k_softmax_fwd, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)x, (uint16_t*)y, rows, cols, dtype);
    return status();
}

int tkm_rt_softmax_bwd(const void* p, const void* dp, void* din, int rows, int cols, int dtype, void* stream) {
    if (rows <= 0) return 0;
    hipLaunchKernelGGL(k_softmax_bwd, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)p, (const uint16_t*)dp, (uint16_t*)din, rows, cols, dtype);
    return status();
}

int tkm_rt_sgd(const TkmSgdTensor* tensors, int nt, long long n_blocks, const float* d_lr, float momentum, float wd,
               uint32_t* d_seed, int dtype, void* stream) {
    if (nt <= 0 || n_blocks <= 0) return 0;
    hipLaunchKernelGGL(k_sgd, dim3((unsigned)n_blocks), dim3(256), 0, (hipStream_t)stream, tensors, nt, d_lr,
                       momentum, wd, d_seed, dtype);
    return status();
}

int tkm_rt_reduce_parts(const TkmReduceChunk* chunks, int n, void* stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_reduce_parts, dim3((unsigned)n), dim3(1024), 0, (hipStream_t)stream, chunks);
    return status();
}

int tkm_rt_perturb(void* p, long long i, float delta, int dtype, void* stream) {
    hipLaunchKernelGGL(k_perturb, dim3(1), dim3(1), 0, (hipStream_t)stream, (uint16_t*)p, i, delta, dtype);
    return status();
}

int tkm_rt_add_f32(float* acc, const float* v, void* stream) {
    hipLaunchKernelGGL(k_add_f32, dim3(1), dim3(1), 0, (hipStream_t)stream, acc, v);
    return status();
}

int tkm_rt_gather(const void* images, const uint8_t* labels, const uint32_t* order, long long first, int B,
                  size_t elems, void* dst, uint8_t* dst_labels, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL(k_gather, dim3(grid_for(elems, 256) > 64 ? 64 : grid_for(elems, 256), (unsigned)B),
                       dim3(256), 0, (hipStream_t)stream, (const uint16_t*)images, labels, order, first, B, elems,
                       (uint16_t*)dst, dst_labels);
    return status();
}

}  // extern "C"
