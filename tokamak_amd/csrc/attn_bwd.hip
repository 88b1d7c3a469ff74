// attn_bwd.hip -- FlashAttention backward for CDNA4 (gfx950), fp16/bf16 in, fp32 accumulate.
//
// Replaces k_gqa_flash_attn_tc_bwd<HEAD_DIM> (reference src/tkm_gpu.cu:440-598) and its
// dispatch (src/tkm_gpu.cu:1389-1404).  The reference computes dQ only (dK/dV are written
// as copies of dQ/dO at tkm_gpu.cu:588-596); this path computes the true gradient:
//   D_i  = <O_i, dO_i>                              (fa_bwd_delta_kernel)
//   P_ij = exp(s_ij - LSE_i),  dS_ij = P_ij (<dO_i, v_j> - D_i)
//   dK_j = scale sum_i dS_ij q_i,  dV_j = sum_i P_ij dO_i   (fa_bwd_dkdv_kernel)
//   dQ_i = scale sum_j dS_ij k_j                            (fa_bwd_dq_kernel)
// in three launches.  dK/dV are accumulated in registers by the one workgroup that owns
// a key block (looping over every query block and every q-head of the kv group) and
// written once, so the backward uses no atomics and is deterministic.  dQ is produced by
// a separate pass that owns a query block and loops over key blocks.  All three write
// (never accumulate into) dqkv, which has the qkv layout.
#include "attn_common.h"
#include "attn_launch.h"

namespace tkm {

// ---------------------------------------------------------------- D = rowsum(O * dO)
// One thread per 8 head-dim elements; D/8 consecutive lanes reduce one (row, head).
template <int D, int DT>
__global__ __launch_bounds__(256) void fa_bwd_delta_kernel(const uint16_t* __restrict__ o,
                                                           const uint16_t* __restrict__ dout,
                                                           float* __restrict__ delta, int B, int S,
                                                           int Hq) {
    constexpr int DC = D / 8;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t total = (size_t)B * S * Hq * DC;
    float acc = 0.f;
    if (idx < total) {
        const u32x4 x = ld_global16(o + idx * 8), y = ld_global16(dout + idx * 8);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            acc += to_f32<DT>((uint16_t)(x[w] & 0xffffu)) * to_f32<DT>((uint16_t)(y[w] & 0xffffu));
            acc += to_f32<DT>((uint16_t)(x[w] >> 16)) * to_f32<DT>((uint16_t)(y[w] >> 16));
        }
    }
#pragma unroll
    for (int off = DC / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (idx < total && (idx % DC) == 0) {
        const size_t rh = idx / DC;  // (b*S + i)*Hq + h
        const int h = (int)(rh % Hq);
        const size_t row = rh / Hq;
        const int i = (int)(row % S), b = (int)(row / S);
        delta[((size_t)b * Hq + h) * S + i] = acc;
    }
}

// ---------------------------------------------------------------- dK, dV
// Workgroup = 4 waves = one (batch, kv-head, block of 128 keys); each wave owns 32 keys,
// keeps K and V of those keys in registers (B operands) and dK/dV in accumulators.
// Query tiles of BM rows (Q, dO: row-major for S and dP, transposed for dK and dV; LSE
// and D) are staged through LDS, double-buffered.  Per tile and wave:
//   S = Q K^T, dP = dO V^T       (C[m = query][n = key]; lane = key)
//   P = exp2(S*scale*log2e - LSE*log2e), dS = P (dP - D)
//   dV += P^T dO, dK += dS^T Q  (P, dS accumulators are the A operands in place)
template <int D, int DT, int BM>
__global__ __launch_bounds__(256) void fa_bwd_dkdv_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, uint16_t* __restrict__ dqkv,
    const int32_t* __restrict__ kv_len, int B, int S, int Hq, int Hkv, float scale,
    float scale_log2, int causal) {
    constexpr int NT = 256, BN = 128;
    constexpr int KS = D / 16;    // k-steps over the head dim (S, dP)
    constexpr int QBT = BM / 32;  // 32-query blocks per tile
    constexpr int NDB = D / 32;   // 32-wide head-dim blocks of dK, dV
    constexpr int PKS = BM / 16;  // k-steps over queries (dK, dV)
    constexpr int LDQ = D + 8;    // padded row-major row
    constexpr int LDT = BM + 8;   // padded transposed row
    __shared__ __attribute__((aligned(16))) uint16_t sQ[2][BM * LDQ];
    __shared__ __attribute__((aligned(16))) uint16_t sdO[2][BM * LDQ];
    __shared__ __attribute__((aligned(16))) uint16_t sQt[2][D * LDT];
    __shared__ __attribute__((aligned(16))) uint16_t sdOt[2][D * LDT];
    __shared__ __attribute__((aligned(16))) float sL[2][BM];
    __shared__ __attribute__((aligned(16))) float sD[2][BM];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hi = lane >> 5;
    const int nh = B * Hkv;
    const int kblk = blockIdx.x / nh;  // ascending key block = most query tiles first (causal)
    const int bh = blockIdx.x % nh, b = bh / Hkv, kvh = bh % Hkv;
    const int g = Hq / Hkv;
    const size_t ld = (size_t)(Hq + 2 * Hkv) * D, ldo = (size_t)Hq * D;
    const uint16_t* bqkv = qkv + (size_t)b * S * ld;
    uint16_t* bd = dqkv + (size_t)b * S * ld;
    int kvl = S;
    if (kv_len) {
        kvl = kv_len[b];
        kvl = kvl < 0 ? 0 : (kvl > S ? S : kvl);
    }
    const int kb0 = kblk * BN, kw0 = kb0 + wave * 32;
    const int key = kw0 + l32;  // this lane's key (column of S)

    f32x16 dk[NDB], dv[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) dk[db] = dv[db] = f32x16{};

    if (kb0 < kvl) {
        u32x4 kf[KS], vf[KS];
        {
            const uint16_t* kp = bqkv + (size_t)key * ld + (size_t)(Hq + kvh) * D + hi * 8;
            const uint16_t* vp = bqkv + (size_t)key * ld + (size_t)(Hq + Hkv + kvh) * D + hi * 8;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                kf[ks] = key < kvl ? ld_global16(kp + ks * 16) : u32x4{0u, 0u, 0u, 0u};
                vf[ks] = key < kvl ? ld_global16(vp + ks * 16) : u32x4{0u, 0u, 0u, 0u};
            }
        }
        const int qt_begin = causal ? kb0 / BM : 0;
        const int n_qt = (S + BM - 1) / BM;
        const int nq = n_qt - qt_begin;
        const int iters = g * nq;

        TileIO<BM, D, NT> qio, dio;
        auto fetch = [&](int it) {
            const int h = kvh * g + it / nq, qr0 = (qt_begin + it % nq) * BM;
            qio.load(bqkv + (size_t)h * D, ld, qr0, S, tid);
            dio.load(dout + (size_t)b * S * ldo + (size_t)h * D, ldo, qr0, S, tid);
        };
        auto stash = [&](int it, int buf) {
            const int h = kvh * g + it / nq, qr0 = (qt_begin + it % nq) * BM;
            qio.template store_rows<LDQ>(sQ[buf], tid);
            qio.template store_cols<LDT>(sQt[buf], tid);
            dio.template store_rows<LDQ>(sdO[buf], tid);
            dio.template store_cols<LDT>(sdOt[buf], tid);
            if (tid < BM) {
                const int row = qr0 + tid;
                const size_t li = ((size_t)b * Hq + h) * S + row;
                sL[buf][tid] = row < S ? lse[li] * 1.4426950408889634f : INFINITY;
                sD[buf][tid] = row < S ? delta[li] : 0.f;
            }
        };
        fetch(0);
        stash(0, 0);
        __syncthreads();

        for (int it = 0; it < iters; ++it) {
            const int buf = it & 1;
            const int qr0 = (qt_begin + it % nq) * BM;
            if (it + 1 < iters) fetch(it + 1);
            const bool active = !causal || (qr0 + BM - 1 >= kw0);
            if (active) {
                const bool need_mask = (causal && qr0 < kw0 + 31) || (kw0 + 32 > kvl);
                f32x16 s[QBT], dp[QBT];
#pragma unroll
                for (int qb = 0; qb < QBT; ++qb) s[qb] = dp[qb] = f32x16{};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                    for (int qb = 0; qb < QBT; ++qb) {
                        const int off = (qb * 32 + l32) * LDQ + ks * 16 + hi * 8;
                        s[qb] = mfma32<DT>(ld_lds16(sQ[buf] + off), kf[ks], s[qb]);
                        dp[qb] = mfma32<DT>(ld_lds16(sdO[buf] + off), vf[ks], dp[qb]);
                    }
                }
                u32x4 pf[PKS], sf[PKS];
#pragma unroll
                for (int qb = 0; qb < QBT; ++qb) {
#pragma unroll
                    for (int g4 = 0; g4 < 4; ++g4) {
                        const f32x4 L = *reinterpret_cast<const f32x4*>(&sL[buf][qb * 32 + g4 * 8 + hi * 4]);
                        const f32x4 Dl = *reinterpret_cast<const f32x4*>(&sD[buf][qb * 32 + g4 * 8 + hi * 4]);
                        float p[4], ds[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int r = g4 * 4 + i;
                            float pv = fast_exp2(s[qb][r] * scale_log2 - L[i]);
                            if (need_mask) {
                                const int qrow = qr0 + qb * 32 + g4 * 8 + hi * 4 + i;
                                if (key >= kvl || (causal && key > qrow)) pv = 0.f;
                            }
                            p[i] = pv;
                            ds[i] = pv * (dp[qb][r] - Dl[i]);
                        }
                        // registers r = g4*4..g4*4+3 are k-slots (g4&1)*4.. of step qb*2 + g4/2
                        const int ks = qb * 2 + (g4 >> 1), w = (g4 & 1) * 2;
                        pf[ks][w] = pack2<DT>(p[0], p[1]);
                        pf[ks][w + 1] = pack2<DT>(p[2], p[3]);
                        sf[ks][w] = pack2<DT>(ds[0], ds[1]);
                        sf[ks][w + 1] = pack2<DT>(ds[2], ds[3]);
                    }
                }
#pragma unroll
                for (int ks = 0; ks < PKS; ++ks) {
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        const int off = (db * 32 + l32) * LDT + ks * 16 + hi * 8;
                        dv[db] = mfma32<DT>(pf[ks], ld_lds16(sdOt[buf] + off), dv[db]);
                        dk[db] = mfma32<DT>(sf[ks], ld_lds16(sQt[buf] + off), dk[db]);
                    }
                }
            }
            if (it + 1 < iters) stash(it + 1, buf ^ 1);
            __syncthreads();
        }
    }

    // dK (scaled), dV: C[m = key][n = d]; lane holds d = db*32 + l32, keys (r/4)*8 + hi*4 + r%4.
    uint16_t* dkp = bd + (size_t)(Hq + kvh) * D;
    uint16_t* dvp = bd + (size_t)(Hq + Hkv + kvh) * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int kr = kw0 + (r >> 2) * 8 + hi * 4 + (r & 3);
            if (kr < S) {
                const int d = db * 32 + l32;
                const uint32_t wk = pack2<DT>(dk[db][r] * scale, 0.f);
                const uint32_t wv = pack2<DT>(dv[db][r], 0.f);
                dkp[(size_t)kr * ld + d] = (uint16_t)(wk & 0xffffu);
                dvp[(size_t)kr * ld + d] = (uint16_t)(wv & 0xffffu);
            }
        }
    }
}

// ---------------------------------------------------------------- dQ
// Workgroup = 4 waves = one (batch, q-head, block of 128 queries); each wave owns 32
// queries with Q and dO in registers (B operands) and walks key tiles of BN keys staged
// in LDS (K and V row-major, K transposed).  Per tile and wave:
//   S^T = K Q^T, dP^T = V dO^T  (lane = query row: LSE and D are per-lane scalars)
//   dS^T = P^T (dP^T - D),  dQ^T += K^T dS^T
template <int D, int DT, int BN>
__global__ __launch_bounds__(256) void fa_bwd_dq_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, uint16_t* __restrict__ dqkv,
    const int32_t* __restrict__ kv_len, int B, int S, int Hq, int Hkv, float scale,
    float scale_log2, int causal, int n_qblk) {
    constexpr int NT = 256, BM = 128;
    constexpr int KS = D / 16;
    constexpr int NKB = BN / 32;
    constexpr int NDB = D / 32;
    constexpr int PKS = BN / 16;
    constexpr int LDK = D + 8;
    constexpr int LDT = BN + 8;
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][BN * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][BN * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t sKt[2][D * LDT];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hi = lane >> 5;
    const int nh = B * Hq;
    const int bid = blockIdx.x;
    const int qblk = causal ? (n_qblk - 1 - bid / nh) : (bid / nh);
    const int bh = bid % nh, b = bh / Hq, h = bh % Hq;
    const int kvh = h / (Hq / Hkv);
    const size_t ld = (size_t)(Hq + 2 * Hkv) * D, ldo = (size_t)Hq * D;
    const uint16_t* bqkv = qkv + (size_t)b * S * ld;
    const uint16_t* Kp = bqkv + (size_t)(Hq + kvh) * D;
    const uint16_t* Vp = bqkv + (size_t)(Hq + Hkv + kvh) * D;
    int kvl = S;
    if (kv_len) {
        kvl = kv_len[b];
        kvl = kvl < 0 ? 0 : (kvl > S ? S : kvl);
    }
    const int q0 = qblk * BM + wave * 32;
    const int q = q0 + l32;
    u32x4 qf[KS], of[KS];
    float L2 = INFINITY, Dl = 0.f;
    if (q < S) {
        const uint16_t* qp = bqkv + (size_t)q * ld + (size_t)h * D + hi * 8;
        const uint16_t* op = dout + ((size_t)b * S + q) * ldo + (size_t)h * D + hi * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            qf[ks] = ld_global16(qp + ks * 16);
            of[ks] = ld_global16(op + ks * 16);
        }
        const size_t li = ((size_t)b * Hq + h) * S + q;
        L2 = lse[li] * 1.4426950408889634f;
        Dl = delta[li];
    } else {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[ks] = of[ks] = u32x4{0u, 0u, 0u, 0u};
    }

    int kv_end = kvl;
    if (causal) kv_end = min(kv_end, qblk * BM + BM);
    const int ntiles = (kv_end + BN - 1) / BN;

    f32x16 dq[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) dq[db] = f32x16{};

    TileIO<BN, D, NT> kio, vio;
    if (ntiles > 0) {
        kio.load(Kp, ld, 0, kv_end, tid);
        vio.load(Vp, ld, 0, kv_end, tid);
        kio.template store_rows<LDK>(sK[0], tid);
        kio.template store_cols<LDT>(sKt[0], tid);
        vio.template store_rows<LDK>(sV[0], tid);
    }
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const int k0 = t * BN;
        if (t + 1 < ntiles) {
            kio.load(Kp, ld, k0 + BN, kv_end, tid);
            vio.load(Vp, ld, k0 + BN, kv_end, tid);
        }
        const bool active = !causal || (k0 <= q0 + 31);
        if (active) {
            const bool need_mask = (causal && k0 + BN - 1 > q0) || (k0 + BN > kvl);
            f32x16 s[NKB], dp[NKB];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) s[kb] = dp[kb] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    const int off = (kb * 32 + l32) * LDK + ks * 16 + hi * 8;
                    s[kb] = mfma32<DT>(ld_lds16(sK[buf] + off), qf[ks], s[kb]);
                    dp[kb] = mfma32<DT>(ld_lds16(sV[buf] + off), of[ks], dp[kb]);
                }
            }
            u32x4 sf[PKS];
#pragma unroll
            for (int ks = 0; ks < PKS; ++ks) {
                const int kb = ks >> 1, r0 = (ks & 1) * 8;
                float ds[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int r = r0 + i;
                    float pv = fast_exp2(s[kb][r] * scale_log2 - L2);
                    if (need_mask) {
                        const int kr = k0 + kb * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
                        if (kr >= kvl || (causal && kr > q)) pv = 0.f;
                    }
                    ds[i] = pv * (dp[kb][r] - Dl);
                }
#pragma unroll
                for (int w = 0; w < 4; ++w) sf[ks][w] = pack2<DT>(ds[2 * w], ds[2 * w + 1]);
            }
#pragma unroll
            for (int ks = 0; ks < PKS; ++ks) {
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    const u32x4 a = ld_lds16(sKt[buf] + (db * 32 + l32) * LDT + ks * 16 + hi * 8);
                    dq[db] = mfma32<DT>(a, sf[ks], dq[db]);
                }
            }
        }
        if (t + 1 < ntiles) {
            kio.template store_rows<LDK>(sK[buf ^ 1], tid);
            kio.template store_cols<LDT>(sKt[buf ^ 1], tid);
            vio.template store_rows<LDK>(sV[buf ^ 1], tid);
        }
        __syncthreads();
    }

    if (q < S) {
        uint16_t* qrow = dqkv + ((size_t)b * S + q) * ld + (size_t)h * D;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const f32x16& acc = dq[db];
                u32x2 w = {pack2<DT>(acc[g4 * 4 + 0] * scale, acc[g4 * 4 + 1] * scale),
                           pack2<DT>(acc[g4 * 4 + 2] * scale, acc[g4 * 4 + 3] * scale)};
                *reinterpret_cast<u32x2*>(qrow + db * 32 + g4 * 8 + hi * 4) = w;
            }
    }
}

// ---------------------------------------------------------------- launchers
template <int D, int DT>
static int launch_delta_t(const BwdArgs& a) {
    const size_t total = (size_t)a.B * a.S * a.Hq * (D / 8);
    dim3 grid((unsigned)((total + 255) / 256)), block(256);
    hipLaunchKernelGGL((fa_bwd_delta_kernel<D, DT>), grid, block, 0, (hipStream_t)a.stream,
                       (const uint16_t*)a.o, (const uint16_t*)a.dout, a.delta, a.B, a.S, a.Hq);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int D, int DT>
static int launch_dkdv_t(const BwdArgs& a) {
    constexpr int BM = 64, BN = 128;
    const int n_kblk = (a.S + BN - 1) / BN;
    dim3 grid((unsigned)(a.B * a.Hkv * n_kblk)), block(256);
    hipLaunchKernelGGL((fa_bwd_dkdv_kernel<D, DT, BM>), grid, block, 0, (hipStream_t)a.stream,
                       (const uint16_t*)a.qkv, (const uint16_t*)a.dout, a.lse, (const float*)a.delta,
                       (uint16_t*)a.dqkv, a.kv_len, a.B, a.S, a.Hq, a.Hkv, a.scale,
                       a.scale * 1.4426950408889634f, a.causal);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int D, int DT>
static int launch_dq_t(const BwdArgs& a) {
    constexpr int BN = 64, BM = 128;
    const int n_qblk = (a.S + BM - 1) / BM;
    dim3 grid((unsigned)(a.B * a.Hq * n_qblk)), block(256);
    hipLaunchKernelGGL((fa_bwd_dq_kernel<D, DT, BN>), grid, block, 0, (hipStream_t)a.stream,
                       (const uint16_t*)a.qkv, (const uint16_t*)a.dout, a.lse, (const float*)a.delta,
                       (uint16_t*)a.dqkv, a.kv_len, a.B, a.S, a.Hq, a.Hkv, a.scale,
                       a.scale * 1.4426950408889634f, a.causal, n_qblk);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

#define TKM_DISPATCH(FN, a)                                                                 \
    ((a).D == 128 ? ((a).dtype == DT_F16 ? FN<128, DT_F16>(a) : FN<128, DT_BF16>(a))        \
                  : ((a).dtype == DT_F16 ? FN<64, DT_F16>(a) : FN<64, DT_BF16>(a)))

int launch_bwd_delta(const BwdArgs& a) { return TKM_DISPATCH(launch_delta_t, a); }
int launch_bwd_dkdv(const BwdArgs& a) { return TKM_DISPATCH(launch_dkdv_t, a); }
int launch_bwd_dq(const BwdArgs& a) { return TKM_DISPATCH(launch_dq_t, a); }

}  // namespace tkm
