// attn_fwd.hip -- FlashAttention forward for CDNA4 (gfx950), fp16/bf16 in, fp32 accumulate.
//
// Replaces k_gqa_flash_attn_tc_fwd<HEAD_DIM> (reference src/tkm_gpu.cu:302-438) and its
// dispatch (src/tkm_gpu.cu:1252-1265); same inputs, outputs and conventions:
//   qkv [B][S][(Hq+2Hkv)*D], O [B][S][Hq*D], LSE [B][Hq][S] natural log of the scaled
//   scores, q-head h reads kv-head h/(Hq/Hkv), key j visible iff j < kv_len[b] and
//   (!causal || j <= i).
//
// Work decomposition: one workgroup = 4 waves = one (batch, q-head, block of 4*32*QB
// query rows).  Each wave keeps its 32*QB query rows of Q in registers and walks the
// key range in tiles of BN keys that the workgroup stages through LDS (K row-major,
// V transposed), double-buffered: tile t+1 is fetched from HBM into registers while
// tile t is consumed by the MFMAs, then written to the other LDS buffer.
//
// Per tile and wave:
//   S^T = K Q^T     (32 keys x 32 queries per MFMA block; lane = query row)
//   online softmax in the exp2 domain with scale*log2(e) folded into one multiply;
//   row max = in-register max + one exchange between lane halves; the row sum is kept
//   per lane and combined once at the end; the running max is only moved (and O
//   rescaled) when it grows by more than 2^8, so P <= 256 stays exact in fp16/bf16.
//   O^T += V^T P^T  (P^T is the S^T accumulator rounded to 16 bits, used in place)
// Causal: tiles above the diagonal are never loaded or computed; only tiles crossing
// the diagonal (or the kv_len / S edge) are masked; heaviest query blocks launch first.
#include "attn_common.h"
#include "attn_launch.h"

namespace tkm {

template <int D, int DT, int BN, int QB>
__global__ __launch_bounds__(256) void fa_fwd_kernel(const uint16_t* __restrict__ qkv,
                                                     uint16_t* __restrict__ out,
                                                     float* __restrict__ lse,
                                                     const int32_t* __restrict__ kv_len, int B,
                                                     int S, int Hq, int Hkv, float scale_log2,
                                                     int causal, int n_qblk) {
    constexpr int NT = 256, NW = 4;
    constexpr int BM = NW * QB * 32;
    constexpr int KS = D / 16;   // k-steps over the head dim (S^T)
    constexpr int NKB = BN / 32; // 32-key blocks per tile
    constexpr int NDB = D / 32;  // 32-wide head-dim blocks of O
    constexpr int PKS = BN / 16; // k-steps over keys (PV)
    constexpr int LDK = D + 8;   // padded K row (16-bit elements)
    constexpr int LDV = BN + 8;  // padded V^T row
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][BN * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][D * LDV];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hi = lane >> 5;
    const int nh = B * Hq;
    const int bid = blockIdx.x;
    const int qblk = causal ? (n_qblk - 1 - bid / nh) : (bid / nh);
    const int bh = bid % nh, b = bh / Hq, h = bh % Hq;
    const int kvh = h / (Hq / Hkv);
    const size_t ld = (size_t)(Hq + 2 * Hkv) * D;
    const uint16_t* bqkv = qkv + (size_t)b * S * ld;
    const uint16_t* Qp = bqkv + (size_t)h * D;
    const uint16_t* Kp = bqkv + (size_t)(Hq + kvh) * D;
    const uint16_t* Vp = bqkv + (size_t)(Hq + Hkv + kvh) * D;
    int kvl = S;
    if (kv_len) {
        kvl = kv_len[b];
        kvl = kvl < 0 ? 0 : (kvl > S ? S : kvl);
    }

    const int q0 = qblk * BM + wave * QB * 32;  // first query row of this wave
    u32x4 qf[QB][KS];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int row = q0 + qb * 32 + l32;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            qf[qb][ks] = row < S ? ld_global16(Qp + (size_t)row * ld + ks * 16 + hi * 8)
                                 : u32x4{0u, 0u, 0u, 0u};
    }

    int kv_end = kvl;
    if (causal) kv_end = min(kv_end, qblk * BM + BM);
    const int ntiles = (kv_end + BN - 1) / BN;

    f32x16 o[NDB][QB];
    float m[QB], lsum[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        m[qb] = -INFINITY;
        lsum[qb] = 0.f;
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[db][qb] = f32x16{};
    }

    TileIO<BN, D, NT> kio, vio;
    if (ntiles > 0) {
        kio.load(Kp, ld, 0, kv_end, tid);
        vio.load(Vp, ld, 0, kv_end, tid);
        kio.template store_rows<LDK>(sK[0], tid);
        vio.template store_cols<LDV>(sV[0], tid);
    }
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const int k0 = t * BN;
        if (t + 1 < ntiles) {
            kio.load(Kp, ld, k0 + BN, kv_end, tid);
            vio.load(Vp, ld, k0 + BN, kv_end, tid);
        }
        const bool active = !causal || (k0 <= q0 + QB * 32 - 1);
        if (active) {
            const bool need_mask = (causal && k0 + BN - 1 > q0) || (k0 + BN > kvl);
            f32x16 s[NKB][QB];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) s[kb][qb] = f32x16{};
            const uint16_t* sk = sK[buf];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    u32x4 a = ld_lds16(sk + (kb * 32 + l32) * LDK + ks * 16 + hi * 8);
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb) s[kb][qb] = mfma32<DT>(a, qf[qb][ks], s[kb][qb]);
                }
            }

            u32x4 pf[QB][PKS];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const int q = q0 + qb * 32 + l32;
                float mx = -INFINITY;
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        float x = s[kb][qb][r] * scale_log2;
                        if (need_mask) {
                            const int key = k0 + kb * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
                            if (key >= kvl || (causal && key > q)) x = -INFINITY;
                        }
                        s[kb][qb][r] = x;
                        mx = fmaxf(mx, x);
                    }
                }
                mx = fmaxf(mx, xor32(mx));
                const float mnew = fmaxf(m[qb], mx);
                if (__any(mnew > m[qb] + 8.0f)) {
                    const float alpha = (mnew == -INFINITY) ? 1.0f : fast_exp2(m[qb] - mnew);
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
#pragma unroll
                        for (int r = 0; r < 16; ++r) o[db][qb][r] *= alpha;
                    lsum[qb] *= alpha;
                    m[qb] = mnew;
                }
                const float msub = (m[qb] == -INFINITY) ? 0.0f : m[qb];
#pragma unroll
                for (int ks = 0; ks < PKS; ++ks) {
                    const int kb = ks >> 1, r0 = (ks & 1) * 8;
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        const uint32_t pw = pack2<DT>(fast_exp2(s[kb][qb][r0 + 2 * w] - msub),
                                                      fast_exp2(s[kb][qb][r0 + 2 * w + 1] - msub));
                        pf[qb][ks][w] = pw;
                        lsum[qb] = dot2_ones<DT>(pw, lsum[qb]);
                    }
                }
            }

            const uint16_t* sv = sV[buf];
#pragma unroll
            for (int ks = 0; ks < PKS; ++ks) {
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    u32x4 a = ld_lds16(sv + (db * 32 + l32) * LDV + ks * 16 + hi * 8);
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb) o[db][qb] = mfma32<DT>(a, pf[qb][ks], o[db][qb]);
                }
            }
        }
        if (t + 1 < ntiles) {
            kio.template store_rows<LDK>(sK[buf ^ 1], tid);
            vio.template store_cols<LDV>(sV[buf ^ 1], tid);
        }
        __syncthreads();
    }

    const size_t ldo = (size_t)Hq * D;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const float l = lsum[qb] + xor32(lsum[qb]);
        const float inv = l > 0.f ? 1.0f / l : 0.f;
        const int q = q0 + qb * 32 + l32;
        if (q < S) {
            uint16_t* orow = out + ((size_t)b * S + q) * ldo + (size_t)h * D;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const f32x16& acc = o[db][qb];
                    u32x2 w = {pack2<DT>(acc[g4 * 4 + 0] * inv, acc[g4 * 4 + 1] * inv),
                               pack2<DT>(acc[g4 * 4 + 2] * inv, acc[g4 * 4 + 3] * inv)};
                    *reinterpret_cast<u32x2*>(orow + db * 32 + g4 * 8 + hi * 4) = w;
                }
            if (lse && hi == 0)
                lse[((size_t)b * Hq + h) * S + q] =
                    l > 0.f ? (m[qb] + __log2f(l)) * 0.69314718055994530942f : -INFINITY;
        }
    }
}

template <int D, int DT>
static int launch_fwd_t(const FwdArgs& a) {
    constexpr int BN = 64, QB = 1, BM = 4 * QB * 32;
    const int n_qblk = (a.S + BM - 1) / BM;
    dim3 grid((unsigned)(a.B * a.Hq * n_qblk)), block(256);
    hipLaunchKernelGGL((fa_fwd_kernel<D, DT, BN, QB>), grid, block, 0, (hipStream_t)a.stream,
                       (const uint16_t*)a.qkv, (uint16_t*)a.o, a.lse, a.kv_len, a.B, a.S, a.Hq,
                       a.Hkv, a.scale * 1.4426950408889634f, a.causal, n_qblk);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_fwd(const FwdArgs& a) {
    if (a.D == 128) return a.dtype == DT_F16 ? launch_fwd_t<128, DT_F16>(a) : launch_fwd_t<128, DT_BF16>(a);
    return a.dtype == DT_F16 ? launch_fwd_t<64, DT_F16>(a) : launch_fwd_t<64, DT_BF16>(a);
}

}  // namespace tkm
