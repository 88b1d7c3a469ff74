// attn_fwd.hip -- FlashAttention forward for CDNA4 (gfx950), fp16/bf16 in, fp32 accumulate.
//
// Replaces k_gqa_flash_attn_tc_fwd<HEAD_DIM> (reference src/tkm_gpu.cu:302-438) and its
// dispatch (src/tkm_gpu.cu:1252-1265); same inputs, outputs and conventions:
//   qkv [B][S][(Hq+2Hkv)*D], O [B][S][Hq*D], LSE [B][Hq][S] natural log of the scaled
//   scores, q-head h reads kv-head h/(Hq/Hkv), key j visible iff j < kv_len[b] and
//   (!causal || j <= i).
//
// Work decomposition: one workgroup = 4 waves = one (batch, q-head, block of 128 query
// rows); two workgroups share a CU (2 waves per SIMD), so one wave's softmax overlaps the
// other's MFMAs.  Each wave keeps its 32 query rows of Q in registers and walks the key
// range in tiles of 64 keys.  K and V tiles go HBM -> LDS by buffer DMA (no registers, rows
// past the valid range read as zero), double-buffered: the DMA of tile t+1 is in flight
// while tile t is consumed.  Tiles are stored row-major with an XOR chunk swizzle.
//
// Per tile and wave:
//   S^T = K Q^T        32 keys x 32 queries per MFMA block; lane = query row, so the row
//                      max is an in-register max plus one swap between lane halves.
//   P^T = exp2(S^T * scale*log2e - m), m = running row max in the same units; the row sum
//                      is accumulated per lane (fp32 dot of the rounded P) and the halves
//                      are combined once at the end.  m (and O) is only rescaled when the
//                      max grows by more than 8, so P <= 256 stays exact in fp16/bf16.
//   O^T += V^T P^T     the P^T accumulator, rounded to 16 bits, is the B operand in place;
//                      V^T comes from the row-major V tile through ds_read_b64_tr_b16.
// Causal: tiles above the diagonal are neither loaded nor computed, only tiles crossing the
// diagonal (or the kv_len / S edge) are masked, heaviest query blocks are launched first.
#include "attn_common.h"
#include "attn_launch.h"

namespace tkm {

template <int D, int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fa_fwd_kernel(const uint16_t* __restrict__ qkv, uint16_t* __restrict__ out,
                   float* __restrict__ lse, const int32_t* __restrict__ kv_len, int B, int S,
                   int Hq, int Hkv, float sl2, int causal, int n_qblk) {
    constexpr int BM = 128, BN = 64;
    constexpr int KS = D / 16;    // k-steps over the head dim (S^T)
    constexpr int NKB = BN / 32;  // 32-key blocks per tile
    constexpr int NDB = D / 32;   // 32-wide head-dim blocks of O
    constexpr int PKS = BN / 16;  // k-steps over keys (PV)
    constexpr int ROWB = D * 2;   // bytes per tile row in LDS
    constexpr int CPR = D / 8;    // 16-byte chunks per row
    constexpr int TILEB = BN * ROWB;
    constexpr int RPI = 64 / CPR;       // rows per DMA instruction (64 lanes x 16 bytes)
    constexpr int NI = BN / RPI / 4;    // DMA instructions per wave, per tile and tensor
    __shared__ __attribute__((aligned(1024))) char smem[2][2][TILEB];  // [buffer][K, V]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31, hi = lane >> 5;
    const int nh = B * Hq;
    const int bid = blockIdx.x;
    const int qblk = causal ? (n_qblk - 1 - bid / nh) : (bid / nh);
    const int bh = bid % nh, b = bh / Hq, h = bh % Hq;
    const int kvh = h / (Hq / Hkv);
    const size_t ld = (size_t)(Hq + 2 * Hkv) * D;
    const uint32_t ldb = (uint32_t)(ld * 2);
    const uint16_t* bqkv = qkv + (size_t)b * S * ld;
    const char* Kb = (const char*)(bqkv + (size_t)(Hq + kvh) * D);
    const char* Vb = (const char*)(bqkv + (size_t)(Hq + Hkv + kvh) * D);
    int kvl = S;
    if (kv_len) {
        kvl = kv_len[b];
        kvl = kvl < 0 ? 0 : (kvl > S ? S : kvl);
    }

    const int q0 = qblk * BM + wave * 32;  // first query row of this wave
    const int q = q0 + l32;
    u32x4 qf[KS];
    {
        const uint16_t* qp = bqkv + (size_t)q * ld + (size_t)h * D + hi * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            qf[ks] = q < S ? ld_global16(qp + ks * 16) : u32x4{0u, 0u, 0u, 0u};
    }

    int kv_end = kvl;
    if (causal) kv_end = min(kv_end, qblk * BM + BM);
    const int ntiles = (kv_end + BN - 1) / BN;

    // DMA geometry of this lane: row dma_r of each RPI-row group, LDS slot dma_p.
    const int dma_r = lane / CPR, dma_p = lane % CPR;
    auto issue = [&](int t, int buf) {
        const int k0 = t * BN;
        const uint32_t bytes = (uint32_t)min(BN, kv_end - k0) * ldb;
        const auto rk = make_rsrc(Kb + (size_t)k0 * ldb, bytes);
        const auto rv = make_rsrc(Vb + (size_t)k0 * ldb, bytes);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int r0 = (wave * NI + i) * RPI, r = r0 + dma_r;
            const uint32_t voff = (uint32_t)r * ldb + (uint32_t)((dma_p ^ swz<D>(r)) << 4);
            dma16(rk, &smem[buf][0][r0 * ROWB], voff);
            dma16(rv, &smem[buf][1][r0 * ROWB], voff);
        }
    };

    // LDS read geometry.  K (A operand of S^T): row kb*32 + l32, chunk ks*2 + hi.
    const int fk = swz<D>(l32);
    // V^T (A operand of PV) via transposed reads: row-in-block trow, column tcol of the
    // 32-wide head-dim block.
    const int trow = (lane & 15) >> 2;
    const int tcol = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;

    f32x16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = f32x16{};
    float m = -INFINITY, lsum = 0.f;

    if (ntiles > 0) issue(0, 0);
    wait_dma();
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const int k0 = t * BN;
        if (t + 1 < ntiles) issue(t + 1, buf ^ 1);
        const bool active = !causal || (k0 <= q0 + 31);
        if (active) {
            const char* kt = smem[buf][0];
            const char* vt = smem[buf][1];
            f32x16 s[NKB];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) s[kb] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    const u32x4 a = ld_lds16((const uint16_t*)(kt + (kb * 32 + l32) * ROWB +
                                                               (((ks * 2 + hi) ^ fk) << 4)));
                    s[kb] = mfma32<DT>(a, qf[ks], s[kb]);
                }
            }

            // online softmax (lane = query row q; registers = keys)
            const bool need_mask = (causal && k0 + BN - 1 > q0) || (k0 + BN > kvl);
            if (need_mask) {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = k0 + kb * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
                        if (key >= kvl || (causal && key > q)) s[kb][r] = -INFINITY;
                    }
            }
            float mx = s[0][0];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = (kb == 0 ? 1 : 0); r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
            mx = half_max(mx) * sl2;  // scale > 0: max commutes with the scaling
            const float mnew = fmaxf(m, mx);
            if (__any(mnew > m + 8.0f)) {
                const float alpha = (mnew == -INFINITY) ? 1.0f : fast_exp2(m - mnew);
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
                lsum *= alpha;
                m = mnew;
            }
            const float msub = (m == -INFINITY) ? 0.0f : m;
            u32x4 pf[PKS], pl[Split<DT>::on ? PKS : 1];
#pragma unroll
            for (int ks = 0; ks < PKS; ++ks) {
                const int kb = ks >> 1, r0 = (ks & 1) * 8;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const float p0 = fast_exp2(__builtin_fmaf(s[kb][r0 + 2 * w], sl2, -msub));
                    const float p1 = fast_exp2(__builtin_fmaf(s[kb][r0 + 2 * w + 1], sl2, -msub));
                    if constexpr (Split<DT>::on) {
                        const u32x2 hl = pack_split_bf16(p0, p1);
                        pf[ks][w] = hl[0];
                        pl[ks][w] = hl[1];
                        lsum = dot2_ones<DT>(hl[1], dot2_ones<DT>(hl[0], lsum));
                    } else {
                        const uint32_t pw = pack2<DT>(p0, p1);
                        pf[ks][w] = pw;
                        lsum = dot2_ones<DT>(pw, lsum);
                    }
                }
            }

            // O^T += V^T P^T
#pragma unroll
            for (int ks = 0; ks < PKS; ++ks) {
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    u32x2 v[2];
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
                        const int key = ks * 16 + tt * 8 + hi * 4 + trow;
                        const int d = db * 32 + tcol;
                        v[tt] = ld_lds_tr(vt + key * ROWB + ((((d >> 3) ^ swz<D>(key))) << 4) + (d & 7) * 2);
                    }
                    const u32x4 a = {v[0][0], v[0][1], v[1][0], v[1][1]};
                    o[db] = mfma32<DT>(a, pf[ks], o[db]);
                    if constexpr (Split<DT>::on) o[db] = mfma32<DT>(a, pl[ks], o[db]);
                }
            }
        }
        wait_dma();
        __syncthreads();
    }

    const float l = half_sum(lsum);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    if (q < S) {
        uint16_t* orow = out + ((size_t)b * S + q) * ((size_t)Hq * D) + (size_t)h * D;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                u32x2 w = {pack2<DT>(o[db][g4 * 4 + 0] * inv, o[db][g4 * 4 + 1] * inv),
                           pack2<DT>(o[db][g4 * 4 + 2] * inv, o[db][g4 * 4 + 3] * inv)};
                *reinterpret_cast<u32x2*>(orow + db * 32 + g4 * 8 + hi * 4) = w;
            }
        if (lse && hi == 0)
            lse[((size_t)b * Hq + h) * S + q] =
                l > 0.f ? (m + __log2f(l)) * 0.69314718055994530942f : -INFINITY;
    }
}

template <int D, int DT>
static int launch_fwd_t(const FwdArgs& a) {
    constexpr int BM = 128;
    const int n_qblk = (a.S + BM - 1) / BM;
    dim3 grid((unsigned)(a.B * a.Hq * n_qblk)), block(256);
    hipLaunchKernelGGL((fa_fwd_kernel<D, DT>), grid, block, 0, (hipStream_t)a.stream,
                       (const uint16_t*)a.qkv, (uint16_t*)a.o, a.lse, a.kv_len, a.B, a.S, a.Hq,
                       a.Hkv, a.scale * 1.4426950408889634f, a.causal, n_qblk);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_fwd(const FwdArgs& a) {
    if (a.D == 128) return a.dtype == DT_F16 ? launch_fwd_t<128, DT_F16>(a) : launch_fwd_t<128, DT_BF16>(a);
    return a.dtype == DT_F16 ? launch_fwd_t<64, DT_F16>(a) : launch_fwd_t<64, DT_BF16>(a);
}

}  // namespace tkm
