// attn_bwd.hip -- FlashAttention backward for CDNA4 (gfx950), fp16/bf16 in, fp32 accumulate.
//
// Replaces k_gqa_flash_attn_tc_bwd<HEAD_DIM> (reference src/tkm_gpu.cu:440-598) and its
// dispatch (src/tkm_gpu.cu:1389-1404).  The reference computes dQ only (dK/dV are written
// as copies of dQ/dO at tkm_gpu.cu:588-596); this path computes the true gradient:
//   D_i  = <O_i, dO_i>                              (fa_bwd_delta_kernel)
//   P_ij = exp(s_ij - LSE_i),  dS_ij = P_ij (<dO_i, v_j> - D_i)
//   dK_j = scale sum_i dS_ij q_i,  dV_j = sum_i P_ij dO_i   (fa_bwd_dkdv_kernel)
//   dQ_i = scale sum_j dS_ij k_j                            (fa_bwd_dq_kernel)
// in three launches, or two: fa_bwd_dq_kernel<WD = true> computes D for its own rows from
// the O and dO rows it loads anyway, uses it and writes it for fa_bwd_dkdv_kernel, which
// then runs second.  dK/dV are accumulated in registers by the one workgroup that owns
// a key block (looping over every query block and every q-head of the kv group) and
// written once, so the backward uses no atomics and is deterministic.  dQ is produced by
// a separate pass that owns a query block and loops over key blocks.  All three write
// (never accumulate into) dqkv, which has the qkv layout.  Tile movement, LDS layout and
// operand conventions are those of the forward (attn_common.h).
#include "attn_common.h"
#include "attn_launch.h"

namespace tkm {

// ---------------------------------------------------------------- D = rowsum(O * dO)
// One workgroup per (batch, head, tile of 32 rows).  D/8 lanes per row each load 16 bytes of
// O and dO and reduce by shuffles; the tile's 32 sums meet in LDS and leave as one 128-byte
// run of delta and one 256-byte row-value tile (zeros for the padding rows S..SP-1), so
// every write is a whole contiguous run.

// Row values of the workspace: per (batch, head) the rows are padded to SP (a multiple of 32)
// and stored in tiles of 32 rows, 256 bytes each: -LSE*log2(e) of the tile's rows, then -D of
// the same rows.  Index of row i's -LSE*log2(e) (its -D is 32 floats further).
__device__ __forceinline__ size_t row_tile_index(size_t bh, int SP, int i) {
    return bh * SP * 2 + (size_t)(i >> 5) * 64 + (i & 31);
}

template <int D, int DT>
__global__ __launch_bounds__(256) void fa_bwd_delta_kernel(const uint16_t* __restrict__ o,
                                                           const uint16_t* __restrict__ dout,
                                                           const float* __restrict__ lse,
                                                           float* __restrict__ delta,
                                                           float* __restrict__ quads, int B,
                                                           int S, int Hq) {
    constexpr int DC = D / 8;          // lanes per row
    constexpr int RPP = 256 / DC;      // rows per pass
    static_assert(32 % RPP == 0 && DC <= 64, "delta tiling");
    __shared__ float sums[32];
    const int SP = (S + 31) & ~31, ntile = SP / 32;
    const int tile = (int)(blockIdx.x % ntile);
    const size_t bh = blockIdx.x / ntile;
    const int b = (int)(bh / Hq), h = (int)(bh % Hq);
    const int g = threadIdx.x / DC, c = threadIdx.x % DC;
#pragma unroll
    for (int p = 0; p < 32 / RPP; ++p) {
        const int r = p * RPP + g, i = tile * 32 + r;
        float acc = 0.f;
        if (i < S) {
            const size_t off = (((size_t)b * S + i) * Hq + h) * D + c * 8;
            const u32x4 x = ld_global16(o + off), y = ld_global16(dout + off);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                acc += to_f32<DT>((uint16_t)(x[w] & 0xffffu)) * to_f32<DT>((uint16_t)(y[w] & 0xffffu));
                acc += to_f32<DT>((uint16_t)(x[w] >> 16)) * to_f32<DT>((uint16_t)(y[w] >> 16));
            }
        }
#pragma unroll
        for (int off = DC / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
        if (c == 0) sums[r] = acc;
    }
    __syncthreads();
    const int t = threadIdx.x;
    if (t < 32) {
        const int i = tile * 32 + t;
        if (i < S) delta[bh * S + i] = sums[t];
    } else if (t < 96) {
        const int k = t - 32, r = k & 31, i = tile * 32 + r;   // k < 32: -LSE*log2e, else -D
        float v = 0.f;
        if (i < S) v = k < 32 ? -lse[bh * S + i] * 1.4426950408889634f : -sums[r];
        quads[row_tile_index(bh, SP, i) + (k & 32)] = v;
    }
}

// ---------------------------------------------------------------- dK, dV
// Workgroup = 4 waves = one (batch, kv-head, block of 128 keys); each wave owns 32 keys,
// keeps K and V of those keys in registers (B operands of S and dP) and dK^T, dV^T in
// accumulators.  It walks every query tile of 32 rows of every q-head of its kv group
// (causal: only tiles at or below its keys); Q and dO tiles plus their LSE and D values go
// HBM -> LDS by buffer DMA, double-buffered, tiles stored with the same swizzle as the
// forward.  Per tile and wave:
//   S = Q K^T, dP = dO V^T         C[m = query][n = key]: lane = key, registers = queries
//   P = exp2(S*scale*log2e - LSE*log2e), dS = P (dP - D)
//   dV^T += dO^T P,  dK^T += Q^T dS the P / dS accumulators are the B operands in place,
//                                  dO^T and Q^T come from transposed LDS reads
// dK (times scale) and dV are written once; no atomics.
// KSPLIT = 2 (small grids): two groups of NW waves over the same keys; group g walks every
// other query tile of the key block's list through its own buffers (its waves load the same
// K; group 0 moves the V rows both read), and group 1 adds its dK and dV accumulators into
// group 0's through LDS before group 0 writes them.  NW = 4: blocks of 128 keys (one
// workgroup of 8 waves per CU).  NW = 2 (causal): blocks of 64 keys, two workgroups of 4 waves
// per CU, numbered so that the workgroups the dispatcher puts on one CU (blocks i and
// i + grid/2) pair a heavy (early) key block with a light one.
template <int D, int DT, int KSPLIT, int NW = 4>
__global__ __launch_bounds__(64 * NW * KSPLIT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fa_bwd_dkdv_kernel(const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ dout,
                        const float* __restrict__ lse, const float* __restrict__ delta,
                        uint16_t* __restrict__ dqkv, const int32_t* __restrict__ kv_len, int B,
                        int S, int Hq, int Hkv, float scale, float sl2, int causal) {
    constexpr int BN = 32 * NW, BM = 32;
    constexpr int KS = D / 16;    // k-steps over the head dim (S, dP)
    constexpr int NDB = D / 32;   // 32-wide head-dim blocks of dK, dV
    constexpr int PKS = BM / 16;  // k-steps over queries (dK, dV)
    constexpr int ROWB = D * 2, CPR = D / 8, TILEB = BM * ROWB;
    constexpr int RPI = 64 / CPR;     // rows per DMA instruction
    constexpr int NI = BM / RPI / NW;  // DMA instructions per wave, per tile and tensor
    __shared__ __attribute__((aligned(1024))) char smem[KSPLIT][2][2][TILEB];  // [group][buffer][Q, dO]
    __shared__ __attribute__((aligned(1024))) char sV[NW][32 * ROWB];  // V rows of each wave
    __shared__ __attribute__((aligned(16))) float sLD[KSPLIT][2][2][64];       // [group][buffer][LSE, D]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int grp = wv / NW, wave = wv % NW;                   // key-split group, wave in it
    const int l32 = lane & 31, hi = lane >> 5;
    const int nh = B * Hkv;
    // ascending key block = most query tiles first (causal); NW = 2: the heavy half ascending,
    // then the light half from the last block down
    const int n_kblk = (S + BN - 1) / BN, kq = blockIdx.x / nh, n_heavy = (n_kblk + 1) / 2;
    const int kblk = (NW == 2 && causal && kq >= n_heavy) ? n_kblk - 1 - (kq - n_heavy) : kq;
    const int bh = blockIdx.x % nh, b = bh / Hkv, kvh = bh % Hkv;
    const int g = Hq / Hkv;
    const size_t ld = (size_t)(Hq + 2 * Hkv) * D, ldo = (size_t)Hq * D;
    const uint32_t ldb = (uint32_t)(ld * 2), ldob = (uint32_t)(ldo * 2);
    const uint16_t* bqkv = qkv + (size_t)b * S * ld;
    uint16_t* bd = dqkv + (size_t)b * S * ld;
    int kvl = S;
    if (kv_len) {
        kvl = kv_len[b];
        kvl = kvl < 0 ? 0 : (kvl > S ? S : kvl);
    }
    const int kb0 = kblk * BN, kw0 = kb0 + wave * 32;
    const int key = kw0 + l32;  // this lane's key (column of S)

    f32x16 dk[NDB], dv[NDB];  // dK^T, dV^T: C[m = d][n = key]
#pragma unroll
    for (int db = 0; db < NDB; ++db) dk[db] = dv[db] = f32x16{};

    if (kb0 < kvl) {
        // K of this lane's key in registers; V rows of the wave's 32 keys in LDS (register
        // budget of 2 waves per SIMD), both B operands indexed [key][head dim].
        u32x4 kf[KS];
        {
            const uint16_t* kp = bqkv + (size_t)key * ld + (size_t)(Hq + kvh) * D + hi * 8;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                kf[ks] = key < kvl ? ld_global16(kp + ks * 16) : u32x4{0u, 0u, 0u, 0u};
            const int vrows = max(0, min(32, kvl - kw0));
            const auto rv = make_rsrc(bqkv + (size_t)kw0 * ld + (size_t)(Hq + Hkv + kvh) * D,
                                      rows_bytes(vrows, ldb, D * 2));
            if (grp == 0) {
#pragma unroll
                for (int i = 0; i < 32 / RPI; ++i) {
                    const int r = i * RPI + lane / CPR;
                    dma16(rv, &sV[wave][i * RPI * ROWB],
                          (uint32_t)r * ldb + (uint32_t)(((lane % CPR) ^ swz<D>(r)) << 4));
                }
            }
        }
        const int qt_begin = causal ? kb0 / BM : 0;
        const int nq = (S + BM - 1) / BM - qt_begin;
        const int iters = g * nq;
        // group g takes iterations g, g + KSPLIT, ...; every group runs nit (barriers matched)
        const int nit = (iters + KSPLIT - 1) / KSPLIT;

        const int dma_r = lane / CPR, dma_p = lane % CPR;
        auto issue = [&](int it, int buf) __attribute__((always_inline)) {
            const int h = kvh * g + it / nq, qr0 = (qt_begin + it % nq) * BM;
            const uint32_t rows = (uint32_t)min(BM, S - qr0);
            const auto rq = make_rsrc(bqkv + (size_t)qr0 * ld + (size_t)h * D, rows_bytes(rows, ldb, D * 2));
            const auto ro = make_rsrc(dout + ((size_t)b * S + qr0) * ldo + (size_t)h * D,
                                      rows_bytes(rows, ldob, D * 2));
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int r0 = (wave * NI + i) * RPI, r = r0 + dma_r;
                const uint32_t sw = (uint32_t)((dma_p ^ swz<D>(r)) << 4);
                dma16(rq, &smem[grp][buf][0][r0 * ROWB], (uint32_t)r * ldb + sw);
                dma16(ro, &smem[grp][buf][1][r0 * ROWB], (uint32_t)r * ldob + sw);
            }
            if (wave == 0) {
                const size_t li = ((size_t)b * Hq + h) * S + qr0;
                dma4(make_rsrc(lse + li, rows * 4), &sLD[grp][buf][0][0], (uint32_t)l32 * 4);
                dma4(make_rsrc(delta + li, rows * 4), &sLD[grp][buf][1][0], (uint32_t)l32 * 4);
            }
        };

        const int fq = swz<D>(l32);  // row l32 of a tile: S/dP A-operand reads
        const int trow = (lane & 15) >> 2;
        const int tcol = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;

        if (grp < iters) issue(grp, 0);
        wait_dma();
        __syncthreads();

        for (int j = 0; j < nit; ++j) {
            const int it = grp + j * KSPLIT;
            const int buf = j & 1;
            const int qr0 = (qt_begin + it % nq) * BM;
            if (it + KSPLIT < iters) issue(it + KSPLIT, buf ^ 1);
            const bool active = it < iters && (!causal || (qr0 + BM - 1 >= kw0));
            if (active) {
                const char* qt = smem[grp][buf][0];
                const char* ot = smem[grp][buf][1];
                f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int off = l32 * ROWB + (((ks * 2 + hi) ^ fq) << 4);
                    const u32x4 vfk = ld_lds16((const uint16_t*)(sV[wave] + off));
                    s = mfma32<DT>(ld_lds16((const uint16_t*)(qt + off)), kf[ks], s);
                    dp = mfma32<DT>(ld_lds16((const uint16_t*)(ot + off)), vfk, dp);
                }
                // Branch-free mask: query row qr0 + hi*4 + c (c = g4*8 + i) is hidden from this
                // lane's key iff c < tk (causal, or every row for keys past kv_len), so the tile
                // stays one basic block and the softmax VALU work can overlap MFMAs.  Rows past S
                // need no mask: their Q, dO, LSE and D are zero-filled (P = 1, dS = 0, both
                // multiplying zero rows).
                const int tk = key >= kvl ? BM : (causal ? key - qr0 - hi * 4 : -BM);
                u32x4 pf[PKS], sf[PKS];
                u32x4 pl[Split<DT>::on ? PKS : 1], sl[Split<DT>::on ? PKS : 1];
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const f32x4 L = *reinterpret_cast<const f32x4*>(&sLD[grp][buf][0][g4 * 8 + hi * 4]);
                    const f32x4 Dl = *reinterpret_cast<const f32x4*>(&sLD[grp][buf][1][g4 * 8 + hi * 4]);
                    float p[4], ds[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int r = g4 * 4 + i;
                        float pv = fast_exp2(__builtin_fmaf(s[r], sl2, -L[i] * 1.4426950408889634f));
                        pv = (g4 * 8 + i < tk) ? 0.f : pv;
                        p[i] = pv;
                        ds[i] = pv * (dp[r] - Dl[i]);
                    }
                    // registers g4*4..+3 are k-slots (g4&1)*4..+3 of query step g4/2
                    const int ks = g4 >> 1, w = (g4 & 1) * 2;
                    if constexpr (Split<DT>::on) {
                        const u32x2 p01 = pack_split_bf16(p[0], p[1]), p23 = pack_split_bf16(p[2], p[3]);
                        const u32x2 s01 = pack_split_bf16(ds[0], ds[1]), s23 = pack_split_bf16(ds[2], ds[3]);
                        pf[ks][w] = p01[0];
                        pl[ks][w] = p01[1];
                        pf[ks][w + 1] = p23[0];
                        pl[ks][w + 1] = p23[1];
                        sf[ks][w] = s01[0];
                        sl[ks][w] = s01[1];
                        sf[ks][w + 1] = s23[0];
                        sl[ks][w + 1] = s23[1];
                    } else {
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
                        u32x2 vo[2], vq[2];
#pragma unroll
                        for (int tt = 0; tt < 2; ++tt) {
                            const int row = ks * 16 + tt * 8 + hi * 4 + trow;
                            const int d = db * 32 + tcol;
                            const int off = row * ROWB + (((d >> 3) ^ swz<D>(row)) << 4) + (d & 7) * 2;
                            vo[tt] = ld_lds_tr(ot + off);
                            vq[tt] = ld_lds_tr(qt + off);
                        }
                        const u32x4 ao = {vo[0][0], vo[0][1], vo[1][0], vo[1][1]};
                        const u32x4 aq = {vq[0][0], vq[0][1], vq[1][0], vq[1][1]};
                        dv[db] = mfma32<DT>(ao, pf[ks], dv[db]);
                        dk[db] = mfma32<DT>(aq, sf[ks], dk[db]);
                        if constexpr (Split<DT>::on) {
                            dv[db] = mfma32<DT>(ao, pl[ks], dv[db]);
                            dk[db] = mfma32<DT>(aq, sl[ks], dk[db]);
                        }
                    }
                }
            }
            wait_dma();
            __syncthreads();
        }
    }

    if constexpr (KSPLIT == 2) {
        // Group 1's dK^T then dV^T accumulators into group 0's, through the Q/dO buffers (free
        // once the last iteration ended with every DMA done and a barrier): element r of block
        // db of wave w's lane at float ((db*16 + r)*NW + w)*64 + lane.
        float* xs = reinterpret_cast<float*>(&smem[0][0][0][0]);
        static_assert(NDB * 16 * NW * 64 * 4 <= (int)sizeof(smem), "one accumulator set fits the buffers");
        auto at = [&](int db, int r) -> float& { return xs[((db * 16 + r) * NW + wave) * 64 + lane]; };
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
            f32x16(&acc)[NDB] = pass ? dv : dk;
            if (grp == 1) {
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) at(db, r) = acc[db][r];
            }
            __syncthreads();
            if (grp == 0) {
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[db][r] += at(db, r);
            }
            __syncthreads();
        }
        if (grp == 1) return;
    }

    // dK^T (scaled), dV^T: lane holds key = kw0 + l32, d = db*32 + g4*8 + hi*4 + 0..3.
    // Keys at or past kv_len had P = dS = 0 in every tile: their gradients are zero.
    if (key < S) {
        uint16_t* dkp = bd + (size_t)key * ld + (size_t)(Hq + kvh) * D;
        uint16_t* dvp = bd + (size_t)key * ld + (size_t)(Hq + Hkv + kvh) * D;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = db * 32 + g4 * 8 + hi * 4;
                u32x2 wk = {pack2<DT>(dk[db][g4 * 4 + 0] * scale, dk[db][g4 * 4 + 1] * scale),
                            pack2<DT>(dk[db][g4 * 4 + 2] * scale, dk[db][g4 * 4 + 3] * scale)};
                u32x2 wv = {pack2<DT>(dv[db][g4 * 4 + 0], dv[db][g4 * 4 + 1]),
                            pack2<DT>(dv[db][g4 * 4 + 2], dv[db][g4 * 4 + 3])};
                *reinterpret_cast<u32x2*>(dkp + d) = wk;
                *reinterpret_cast<u32x2*>(dvp + d) = wv;
            }
    }
}

// ---------------------------------------------------------------- dQ
// Workgroup = 4 waves = one (batch, q-head, block of 128 queries); each wave owns 32
// queries with Q and dO in registers (B operands) and walks key tiles of 64 keys; K and V
// tiles go HBM -> LDS by buffer DMA, double-buffered, as in the forward.  Per tile and wave:
//   S^T = K Q^T, dP^T = V dO^T  (lane = query row: LSE and D are per-lane scalars)
//   dS^T = P^T (dP^T - D),  dQ^T += K^T dS^T  (K^T from transposed LDS reads)
// WD: D of the wave's rows is computed here (fp32 sum of O * dO over the lane pair that holds
// the row) and written to delta instead of read from it.
// KSPLIT = 2, NW = 2 (causal D = 64, small grids): blocks of 64 queries, two groups of two
// waves over the same rows, group g walking its half of the key tiles through its own
// buffers (both form D from the O rows; group 0 writes it); group 1 adds its dQ accumulators
// into group 0's through LDS.  Two workgroups per CU, numbered so that blocks i and
// i + grid/2 pair a heavy (late) query block with a light one.
template <int D, int DT, bool WD, int KSPLIT = 1, int NW = 4>
__global__ __launch_bounds__(64 * NW * KSPLIT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fa_bwd_dq_kernel(const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ o,
                      const uint16_t* __restrict__ dout, const float* __restrict__ lse,
                      float* __restrict__ delta, float* __restrict__ quads,
                      uint16_t* __restrict__ dqkv,
                      const int32_t* __restrict__ kv_len, int B, int S, int Hq, int Hkv,
                      float scale, float sl2, int causal, int n_qblk) {
    constexpr int BM = 32 * NW, BN = 64;
    constexpr int KS = D / 16, NKB = BN / 32, NDB = D / 32, PKS = BN / 16;
    constexpr int ROWB = D * 2, CPR = D / 8, TILEB = BN * ROWB;
    constexpr int RPI = 64 / CPR, NI = BN / RPI / NW;
    __shared__ __attribute__((aligned(1024))) char smem[KSPLIT][2][2][TILEB];  // [group][buffer][K, V]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int grp = wv / NW, wave = wv % NW;                   // key-split group, wave in it
    const int l32 = lane & 31, hi = lane >> 5;
    const int nh = B * Hq;
    const int bid = blockIdx.x;
    const int kq = bid / nh, n_heavy = (n_qblk + 1) / 2;
    const int qblk = !causal ? kq
                   : (NW == 2 ? (kq < n_heavy ? n_qblk - 1 - kq : kq - n_heavy) : n_qblk - 1 - kq);
    const int bh = bid % nh, b = bh / Hq, h = bh % Hq;
    const int kvh = h / (Hq / Hkv);
    const size_t ld = (size_t)(Hq + 2 * Hkv) * D, ldo = (size_t)Hq * D;
    const uint32_t ldb = (uint32_t)(ld * 2);
    const uint16_t* bqkv = qkv + (size_t)b * S * ld;
    const char* Kb = (const char*)(bqkv + (size_t)(Hq + kvh) * D);
    const char* Vb = (const char*)(bqkv + (size_t)(Hq + Hkv + kvh) * D);
    int kvl = S;
    if (kv_len) {
        kvl = kv_len[b];
        kvl = kvl < 0 ? 0 : (kvl > S ? S : kvl);
    }
    const int q0 = qblk * BM + wave * 32;
    const int q = q0 + l32;
    u32x4 qf[KS], of[KS];
    float nl2 = 0.f, Dl = 0.f;  // -LSE*log2(e) and D of this lane's query row
    const size_t li = ((size_t)b * Hq + h) * S + q;
    if (q < S) {
        const uint16_t* qp = bqkv + (size_t)q * ld + (size_t)h * D + hi * 8;
        const uint16_t* op = dout + ((size_t)b * S + q) * ldo + (size_t)h * D + hi * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            qf[ks] = ld_global16(qp + ks * 16);
            of[ks] = ld_global16(op + ks * 16);
        }
        nl2 = -lse[li] * 1.4426950408889634f;
        if constexpr (!WD) Dl = delta[li];
    } else {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[ks] = of[ks] = u32x4{0u, 0u, 0u, 0u};
    }
    if constexpr (WD) {
        // This lane holds head-dim elements ks*16 + hi*8 + 0..7 of dO; lane l ^ 32 the rest.
        float acc = 0.f;
        if (q < S) {
            const uint16_t* orow = o + ((size_t)b * S + q) * ldo + (size_t)h * D + hi * 8;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const u32x4 x = ld_global16(orow + ks * 16);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    acc += to_f32<DT>((uint16_t)(x[w] & 0xffffu)) * to_f32<DT>((uint16_t)(of[ks][w] & 0xffffu));
                    acc += to_f32<DT>((uint16_t)(x[w] >> 16)) * to_f32<DT>((uint16_t)(of[ks][w] >> 16));
                }
            }
        }
        Dl = acc + xor32(acc);
        if (q < S && hi == 0 && grp == 0) delta[li] = Dl;
        const int SP = (S + 31) & ~31;
        if (q < SP && hi == 0 && grp == 0) {  // rows S..SP-1: zeros (nl2 = Dl = 0 there)
            float* qd = quads + row_tile_index((size_t)b * Hq + h, SP, q);
            qd[0] = nl2;
            qd[32] = -Dl;
        }
    }

    int kv_end = kvl;
    if (causal) kv_end = min(kv_end, qblk * BM + BM);
    const int ntiles = (kv_end + BN - 1) / BN;
    // this group's tiles [tb, te); every group runs nit iterations (barriers stay matched)
    const int nit = KSPLIT == 2 ? (ntiles + 1) / 2 : ntiles;
    const int tb = grp == 0 ? 0 : nit, te = grp == 0 ? nit : ntiles;

    const int dma_r = lane / CPR, dma_p = lane % CPR;
    auto issue = [&](int t, int buf) __attribute__((always_inline)) {
        const int k0 = t * BN;
        const uint32_t bytes = rows_bytes(min(BN, kv_end - k0), ldb, D * 2);
        const auto rk = make_rsrc(Kb + (size_t)k0 * ldb, bytes);
        const auto rv = make_rsrc(Vb + (size_t)k0 * ldb, bytes);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int r0 = (wave * NI + i) * RPI, r = r0 + dma_r;
            const uint32_t voff = (uint32_t)r * ldb + (uint32_t)((dma_p ^ swz<D>(r)) << 4);
            dma16(rk, &smem[grp][buf][0][r0 * ROWB], voff);
            dma16(rv, &smem[grp][buf][1][r0 * ROWB], voff);
        }
    };
    const int fk = swz<D>(l32);
    const int trow = (lane & 15) >> 2;
    const int tcol = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;

    f32x16 dq[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) dq[db] = f32x16{};

    if (tb < te) issue(tb, 0);
    wait_dma();
    __syncthreads();

    for (int i = 0; i < nit; ++i) {
        const int t = tb + i;
        const int buf = i & 1;
        const int k0 = t * BN;
        if (t + 1 < te) issue(t + 1, buf ^ 1);
        const bool active = t < te && (!causal || (k0 <= q0 + 31));
        if (active) {
            const char* kt = smem[grp][buf][0];
            const char* vt = smem[grp][buf][1];
            f32x16 s[NKB], dp[NKB];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) s[kb] = dp[kb] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    const int off = (kb * 32 + l32) * ROWB + (((ks * 2 + hi) ^ fk) << 4);
                    s[kb] = mfma32<DT>(ld_lds16((const uint16_t*)(kt + off)), qf[ks], s[kb]);
                    dp[kb] = mfma32<DT>(ld_lds16((const uint16_t*)(vt + off)), of[ks], dp[kb]);
                }
            }
            // Branch-free mask: key k0 + hi*4 + c (c = kb*32 + (r/4)*8 + r%4) is hidden from
            // this lane's query iff c > tq (causal, or the key is past kv_len), so the tile stays
            // one basic block.  Masked entries get P = dS = 0 exactly: no inf * 0 from the
            // zero-filled K and V rows past kv_len when a row's LSE is very negative.
            const int tq = min(causal ? q - k0 - hi * 4 : BN, kvl - 1 - k0 - hi * 4);
            u32x4 sf[PKS], sl[Split<DT>::on ? PKS : 1];
#pragma unroll
            for (int ks = 0; ks < PKS; ++ks) {
                const int kb = ks >> 1, r0 = (ks & 1) * 8;
                float ds[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int r = r0 + i;
                    float pv = fast_exp2(__builtin_fmaf(s[kb][r], sl2, nl2));
                    pv = (kb * 32 + (r >> 2) * 8 + (r & 3) > tq) ? 0.f : pv;
                    ds[i] = pv * (dp[kb][r] - Dl);
                }
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    if constexpr (Split<DT>::on) {
                        const u32x2 hl = pack_split_bf16(ds[2 * w], ds[2 * w + 1]);
                        sf[ks][w] = hl[0];
                        sl[ks][w] = hl[1];
                    } else {
                        sf[ks][w] = pack2<DT>(ds[2 * w], ds[2 * w + 1]);
                    }
                }
            }
#pragma unroll
            for (int ks = 0; ks < PKS; ++ks) {
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    u32x2 v[2];
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
                        const int row = ks * 16 + tt * 8 + hi * 4 + trow;
                        const int d = db * 32 + tcol;
                        v[tt] = ld_lds_tr(kt + row * ROWB + (((d >> 3) ^ swz<D>(row)) << 4) + (d & 7) * 2);
                    }
                    const u32x4 a = {v[0][0], v[0][1], v[1][0], v[1][1]};
                    dq[db] = mfma32<DT>(a, sf[ks], dq[db]);
                    if constexpr (Split<DT>::on) dq[db] = mfma32<DT>(a, sl[ks], dq[db]);
                }
            }
        }
        wait_dma();
        __syncthreads();
    }

    if constexpr (KSPLIT == 2) {
        // Group 1's dQ^T accumulators into group 0's through the K/V buffers (free after the
        // loop's last barrier): element r of block db of wave w's lane at float
        // ((db*16 + r)*NW + w)*64 + lane.
        float* xs = reinterpret_cast<float*>(&smem[0][0][0][0]);
        static_assert(NDB * 16 * NW * 64 * 4 <= (int)sizeof(smem), "one accumulator set fits the buffers");
        auto at = [&](int db, int r) -> float& { return xs[((db * 16 + r) * NW + wave) * 64 + lane]; };
        if (grp == 1) {
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) at(db, r) = dq[db][r];
        }
        __syncthreads();
        if (grp == 0) {
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) dq[db][r] += at(db, r);
        }
        __syncthreads();
    }

    // dQ (times scale) leaves through LDS: a lane holds query q, d = db*32 + g4*8 + hi*4 + 0..3;
    // the wave's rows go to LDS row-major (rows padded by 16 bytes against bank conflicts, the
    // K/V tiles are free after the loop's last barrier) and come back 16 bytes per lane, so
    // each store writes whole rows instead of 8 bytes in each of 32 rows.
    constexpr int SROW = ROWB + 16, RPP = 64 / CPR;  // staging row bytes; rows per pass
    char* stg = &smem[0][0][0][0] + wave * 32 * SROW;
    if (grp == 0) {  // (KSPLIT = 2: group 1's sums are in group 0's accumulators)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                u32x2 w = {pack2<DT>(dq[db][g4 * 4 + 0] * scale, dq[db][g4 * 4 + 1] * scale),
                           pack2<DT>(dq[db][g4 * 4 + 2] * scale, dq[db][g4 * 4 + 3] * scale)};
                *reinterpret_cast<u32x2*>(stg + l32 * SROW + (db * 4 + g4) * 16 + hi * 8) = w;
            }
    }
    __syncthreads();
    if (grp == 0) {
#pragma unroll
        for (int i = 0; i < 32 / RPP; ++i) {
            const int row = i * RPP + lane / CPR, chunk = lane % CPR;
            const u32x4 v = *reinterpret_cast<const u32x4*>(stg + row * SROW + chunk * 16);
            if (q0 + row < S)
                *reinterpret_cast<u32x4*>(dqkv + ((size_t)b * S + q0 + row) * ld + (size_t)h * D + chunk * 8) = v;
        }
    }
}

// ---------------------------------------------------------------- launchers
template <int D, int DT>
static int launch_delta_t(const BwdArgs& a) {
    dim3 grid((unsigned)((size_t)a.B * a.Hq * ((a.S + 31) / 32))), block(256);
    hipLaunchKernelGGL((fa_bwd_delta_kernel<D, DT>), grid, block, 0, (hipStream_t)a.stream,
                       (const uint16_t*)a.o, (const uint16_t*)a.dout, a.lse, a.delta, a.ld,
                       a.B, a.S, a.Hq);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

static int compute_units_bwd() {
    static int cached[64];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cached[dev] <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cached[dev] = n;
    }
    return cached[dev];
}

template <int D, int DT>
static int launch_dkdv_t(const BwdArgs& a) {
    constexpr int BN = 128;
    const int n_kblk = (a.S + BN - 1) / BN;
    const long long n_wg = (long long)a.B * a.Hkv * n_kblk;
    dim3 grid((unsigned)n_wg);
    // At most one workgroup of 128 keys per CU: split each key block's query tiles over two
    // groups of waves.  Causal D = 64: blocks of 64 keys instead, two workgroups per CU
    // (2 x 48 KB of LDS) pairing heavy and light key blocks.
    if constexpr (D == 64) {
        if (n_wg <= compute_units_bwd() && a.causal) {
            dim3 grid64((unsigned)((long long)a.B * a.Hkv * ((a.S + 63) / 64)));
            hipLaunchKernelGGL((fa_bwd_dkdv_kernel<D, DT, 2, 2>), grid64, dim3(256), 0, (hipStream_t)a.stream,
                               (const uint16_t*)a.qkv, (const uint16_t*)a.dout, a.lse, (const float*)a.delta,
                               (uint16_t*)a.dqkv, a.kv_len, a.B, a.S, a.Hq, a.Hkv, a.scale,
                               a.scale * 1.4426950408889634f, a.causal);
            return hipGetLastError() == hipSuccess ? 0 : -1;
        }
    }
    if (n_wg <= compute_units_bwd())
        hipLaunchKernelGGL((fa_bwd_dkdv_kernel<D, DT, 2>), grid, dim3(512), 0, (hipStream_t)a.stream,
                           (const uint16_t*)a.qkv, (const uint16_t*)a.dout, a.lse, (const float*)a.delta,
                           (uint16_t*)a.dqkv, a.kv_len, a.B, a.S, a.Hq, a.Hkv, a.scale,
                           a.scale * 1.4426950408889634f, a.causal);
    else
        hipLaunchKernelGGL((fa_bwd_dkdv_kernel<D, DT, 1>), grid, dim3(256), 0, (hipStream_t)a.stream,
                           (const uint16_t*)a.qkv, (const uint16_t*)a.dout, a.lse, (const float*)a.delta,
                           (uint16_t*)a.dqkv, a.kv_len, a.B, a.S, a.Hq, a.Hkv, a.scale,
                           a.scale * 1.4426950408889634f, a.causal);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int D, int DT, bool WD>
static int launch_dq_t(const BwdArgs& a) {
    constexpr int BM = 128;
    const int n_qblk = (a.S + BM - 1) / BM;
    // Causal D = 64 with at most one 128-row block per CU: 64-row blocks over two groups of
    // two waves (each walks half the key tiles), two workgroups per CU pairing heavy and light.
    if constexpr (D == 64) {
        if (a.causal && (long long)a.B * a.Hq * n_qblk <= compute_units_bwd()) {
            const int n_qblk64 = (a.S + 63) / 64;
            hipLaunchKernelGGL((fa_bwd_dq_kernel<D, DT, WD, 2, 2>), dim3((unsigned)(a.B * a.Hq * n_qblk64)),
                               dim3(256), 0, (hipStream_t)a.stream,
                               (const uint16_t*)a.qkv, (const uint16_t*)a.o, (const uint16_t*)a.dout, a.lse,
                               a.delta, a.ld, (uint16_t*)a.dqkv, a.kv_len, a.B, a.S, a.Hq, a.Hkv, a.scale,
                               a.scale * 1.4426950408889634f, a.causal, n_qblk64);
            return hipGetLastError() == hipSuccess ? 0 : -1;
        }
    }
    dim3 grid((unsigned)(a.B * a.Hq * n_qblk)), block(256);
    hipLaunchKernelGGL((fa_bwd_dq_kernel<D, DT, WD>), grid, block, 0, (hipStream_t)a.stream,
                       (const uint16_t*)a.qkv, (const uint16_t*)a.o, (const uint16_t*)a.dout, a.lse,
                       a.delta, a.ld, (uint16_t*)a.dqkv, a.kv_len, a.B, a.S, a.Hq, a.Hkv, a.scale,
                       a.scale * 1.4426950408889634f, a.causal, n_qblk);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
template <int D, int DT>
static int launch_dq_read_t(const BwdArgs& a) { return launch_dq_t<D, DT, false>(a); }
template <int D, int DT>
static int launch_dq_write_t(const BwdArgs& a) { return launch_dq_t<D, DT, true>(a); }

#define TKM_DISPATCH(FN, a)                                                                 \
    ((a).D == 128 ? ((a).dtype == DT_F16 ? FN<128, DT_F16>(a) : FN<128, DT_BF16>(a))        \
                  : ((a).dtype == DT_F16 ? FN<64, DT_F16>(a) : FN<64, DT_BF16>(a)))

// Each stage tries its assembly kernel first (D = 128 fp16); 1 from it means "not handled
// there" and selects the HIP kernel, any other status is final.
static int settle(int r, unsigned asm_bit) {
    if (r == 0) note_kernels(asm_bit);
    return r;
}

int launch_bwd_delta(const BwdArgs& a) {
    note_kernels(kDeltaHip);
    return TKM_DISPATCH(launch_delta_t, a);
}
int launch_bwd_dkdv(const BwdArgs& a) {
    const int r = launch_bwd_dkdv_asm(a);
    if (r != 1) return settle(r, kDkdvAsm);
    note_kernels(kDkdvHip);
    return TKM_DISPATCH(launch_dkdv_t, a);
}
int launch_bwd_dq(const BwdArgs& a) {
    const int r = launch_bwd_dq_asm(a, false);
    if (r != 1) return settle(r, kDqAsm);
    note_kernels(kDqHip);
    return TKM_DISPATCH(launch_dq_read_t, a);
}
int launch_bwd_dq_delta(const BwdArgs& a) {
    const int r = launch_bwd_dq_asm(a, true);
    if (r != 1) return settle(r, kDqAsm);
    note_kernels(kDqHip);
    return TKM_DISPATCH(launch_dq_write_t, a);
}

}  // namespace tkm
