// attn_fwd.hip -- FlashAttention forward for CDNA4 (gfx950), fp16/bf16 in, fp32 accumulate.
//
// Replaces k_gqa_flash_attn_tc_fwd<HEAD_DIM> (reference src/tkm_gpu.cu:302-438) and its
// dispatch (src/tkm_gpu.cu:1252-1265); same inputs, outputs and conventions:
//   qkv [B][S][(Hq+2Hkv)*D], O [B][S][Hq*D], LSE [B][Hq][S] natural log of the scaled
//   scores, q-head h reads kv-head h/(Hq/Hkv), key j visible iff j < kv_len[b] and
//   (!causal || j <= i).
//
// Work decomposition: one workgroup = 4 waves = one (batch, q-head, block of 128 query
// rows); two workgroups share a CU (2 waves per SIMD).  Small grids split a block's key tiles
// over two groups of waves, and causal D = 64 takes blocks of 64 rows paired heavy with light
// on a CU (fa_fwd_kernel's KSPLIT and NW below).  Each wave keeps its 32 query rows
// of Q in registers and walks the key range in tiles of 64 keys that the workgroup moves
// HBM -> LDS by buffer DMA (rows past the valid range read as zero), stored row-major with
// an XOR chunk swizzle.
//
// Per tile and wave:
//   S^T = K Q^T        32 keys x 32 queries per MFMA block; lane = query row.
//   P^T = exp2(S^T * scale*log2e - m) with m the row offset (log2 units, below); the row sum
//                      is an fp32 dot of the rounded P per lane, lane halves combined at the
//                      end.
//   O^T += V^T P^T     the P^T accumulator, rounded to 16 bits, is the B operand in place;
//                      V^T comes from the row-major V tile through ds_read_b64_tr_b16.
//
// Tiles are double-buffered: the DMA of tile t+1 is in flight while tile t is consumed;
// the loop is unrolled by two so every LDS address is a per-lane constant plus an
// immediate.  The two waves of a SIMD (different workgroups) overlap each other's softmax
// with MFMAs.
//
// Scores are the unscaled 16-bit products summed in fp32; scale*log2e and -m are applied in
// fp32 with one FMA per score, P = exp2(fma(s, c, -m)), as the reference's kernel scales in
// fp32 (a scale folded into Q and rounded to 16 bits would move a score s by up to
// |s|*2^-12, which trained attention logits turn into errors past the bars).  m starts as
// the row max of the first tile and moves only when it must (a lazy online softmax): when a
// later tile's packed P sum reaches fp16's largest value (a P past the fp16 range gives an
// infinite sum), the wave raises m of its rows to max(m, the tile's row max), multiplies O and
// the row sums by 2^(m_old - m_new) and repeats the tile's exp2 before its PV product.
// Causal: tiles above the diagonal are neither loaded nor computed, tiles crossing the
// diagonal (or the kv_len / S edge) are masked, heaviest query blocks are launched first.
#include <type_traits>

#include "attn_common.h"
#include "attn_launch.h"


namespace tkm {

// A lane's packed P sum over a tile at or above this moves m (see softmax_next): fp16's
// largest finite value, so no P that reaches a PV product exceeds it, in either type.
constexpr float P_SUM_MAX = 65504.0f;

// KSPLIT = 2 (small grids): two groups of NW waves over the same query rows; group g walks its
// own half of the block's key tiles through its own buffers, with its own m, and group 1 hands
// (m, l, O) to group 0 through LDS at the end, which merges them (rescaling each side by
// 2^(m_side - m)) and writes O and LSE.  The heaviest causal block then walks half its tiles.
// NW = 4: blocks of 128 rows (one workgroup of 8 waves per CU).  NW = 2 (causal): blocks of 64
// rows, two workgroups of 4 waves per CU, numbered so that the workgroups the dispatcher puts
// on one CU (blocks i and i + grid/2) pair a heavy block with a light one.
template <int D, int DT, int QB, int KSPLIT, int NW = 4>
__global__ __launch_bounds__(64 * NW * KSPLIT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fa_fwd_kernel(const uint16_t* __restrict__ qkv, uint16_t* __restrict__ out,
                   float* __restrict__ lse, const int32_t* __restrict__ kv_len, int B, int S,
                   int Hq, int Hkv, float sl2, int causal, int n_qblk) {
    constexpr bool SPL = Split<DT>::on;   // bf16: P as hi + lo
    constexpr int WR = 32 * QB;           // query rows per wave
    constexpr int BM = NW * WR, BN = 64;
    constexpr int KS = D / 16;    // k-steps over the head dim (S^T)
    constexpr int NKB = BN / 32;  // 32-key blocks per tile
    constexpr int NDB = D / 32;   // 32-wide head-dim blocks of O
    constexpr int PKS = BN / 16;  // k-steps over keys (PV)
    constexpr int ROWB = D * 2;   // bytes per tile row in LDS
    constexpr int CPR = D / 8;    // 16-byte chunks per row
    constexpr int TILEB = BN * ROWB;
    constexpr int RPI = 64 / CPR;     // rows per DMA instruction (64 lanes x 16 bytes)
    constexpr int NI = BN / RPI / NW;  // DMA instructions per wave, per tile and tensor
    constexpr int NL = SPL ? PKS : 1;
    __shared__ __attribute__((aligned(1024))) char smem[KSPLIT][2][2][TILEB];  // [group][K, V][buffer]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int grp = wave / NW, gw = wave % NW;                   // key-split group, wave in it
    const int l32 = lane & 31, hi = lane >> 5;
    const int nh = B * Hq;
    const int bid = blockIdx.x;
    // causal: heaviest blocks first, or (NW = 2) the heavy half descending, then the light half
    // ascending, so that blocks i and i + grid/2 carry about the same number of tiles together
    const int kq = bid / nh, n_heavy = (n_qblk + 1) / 2;
    const int qblk = !causal ? kq
                   : (NW == 2 ? (kq < n_heavy ? n_qblk - 1 - kq : kq - n_heavy) : n_qblk - 1 - kq);
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

    const int q0 = qblk * BM + gw * WR;  // first query row of this wave
    u32x4 qf[QB][KS];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int q = q0 + qb * 32 + l32;
        const uint16_t* qp = bqkv + (size_t)q * ld + (size_t)h * D + hi * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            qf[qb][ks] = q < S ? ld_global16(qp + ks * 16) : u32x4{0u, 0u, 0u, 0u};
        }
    }

    int kv_end = kvl;
    if (causal) kv_end = min(kv_end, qblk * BM + BM);
    const int ntiles = (kv_end + BN - 1) / BN;
    // tiles [0, n_plain) need no mask for any row of this wave
    const int n_plain = min(kvl / BN, causal ? (q0 + 1) / BN : ntiles);
    // tiles [0, n_act) hold at least one key visible to this wave
    const int n_act = causal ? min(ntiles, (q0 + WR - 1) / BN + 1) : ntiles;
    // this group's tiles [tb, te); every group runs nit iterations (barriers stay matched)
    const int nit = KSPLIT == 2 ? (ntiles + 1) / 2 : ntiles;
    const int tb = grp == 0 ? 0 : nit, te = grp == 0 ? nit : ntiles;

    // DMA of one tile (tensor 0 = K, 1 = V) into buffer buf: wave w moves rows
    // [w*NI*RPI, (w+1)*NI*RPI) of the BN-row tile.
    const int dma_r = lane / CPR, dma_p = lane % CPR;
    auto issue = [&](int t, int tensor, int buf) __attribute__((always_inline)) {
        const int k0 = t * BN;
        const auto r = make_rsrc((tensor ? Vb : Kb) + (size_t)k0 * ldb,
                                 rows_bytes(min(BN, kv_end - k0), ldb, D * 2));
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int r0 = (gw * NI + i) * RPI, row = r0 + dma_r;
            dma16(r, &smem[grp][tensor][buf][r0 * ROWB],
                  (uint32_t)row * ldb + (uint32_t)((dma_p ^ swz<D>(row)) << 4));
        }
    };

    // Per-lane LDS offsets.  K (A operand of S^T): row kb*32 + l32, chunk ks*2 + hi.
    int koff[KS];
    const int fk = swz<D>(l32);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) koff[ks] = l32 * ROWB + (((ks * 2 + hi) ^ fk) << 4);
    // V^T (A operand of PV) by transposed reads: rows ks*16 + tt*8 + hi*4 + trow, columns
    // db*32 + tcol; the swizzle depends on the row only through tt (ks*16 keeps row & 15).
    int voff[2][NDB];
    {
        const int trow = (lane & 15) >> 2;
        const int tcol = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int row = tt * 8 + hi * 4 + trow;
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const int d = db * 32 + tcol;
                voff[tt][db] = row * ROWB + (((d >> 3) ^ swz<D>(row)) << 4) + (d & 7) * 2;
            }
        }
    }

    f32x16 o[NDB][QB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) o[db][qb] = f32x16{};
    float m[QB], lsum[QB];      // m: running max (log2 units) once tile 0 is done
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        m[qb] = 0.f;
        lsum[qb] = 0.f;
    }
    f32x16 sr[1][NKB][QB];  // scores of the current tile
    u32x4 pr[1][QB][PKS];   // its P (hi part for bf16)
    u32x4 plr[1][QB][NL];   // bf16: lo part

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // S(tile) into register set J: S^T = K Q^T (unscaled).
    auto stage_s = [&](const char* kt, auto Jc) __attribute__((always_inline)) {
        constexpr int J = decltype(Jc)::value;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                const u32x4 a = ld_lds16((const uint16_t*)(kt + kb * 32 * ROWB + koff[ks]));
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
                    sr[J][kb][qb] = mfma32<DT>(a, qf[qb][ks], ks == 0 ? f32x16{} : sr[J][kb][qb]);
            }
    };
    auto stage_mask = [&](int t, auto Jc) __attribute__((always_inline)) {
        constexpr int J = decltype(Jc)::value;
        const int k0 = t * BN;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const int q = q0 + qb * 32 + l32;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = k0 + kb * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
                    if (key >= kvl || (causal && key > q)) sr[J][kb][qb][r] = -INFINITY;
                }
        }
    };
    // exp2 of the scores in set J (relative to mm[qb]), packed to 16 bits into P set J;
    // lt[qb] = the lane's fp32 sum of the packed values.
    auto stage_exp = [&](auto Jc, const float (&mm)[QB], float (&lt)[QB]) __attribute__((always_inline)) {
        constexpr int J = decltype(Jc)::value;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            lt[qb] = 0.f;
#pragma unroll
            for (int ks = 0; ks < PKS; ++ks) {
                const int kb = ks >> 1, r0 = (ks & 1) * 8;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    float x0 = sr[J][kb][qb][r0 + 2 * w], x1 = sr[J][kb][qb][r0 + 2 * w + 1];
                    x0 = __builtin_fmaf(x0, sl2, -mm[qb]);
                    x1 = __builtin_fmaf(x1, sl2, -mm[qb]);
                    const float p0 = fast_exp2(x0), p1 = fast_exp2(x1);
                    if constexpr (SPL) {
                        const u32x2 hl = pack_split_bf16(p0, p1);
                        pr[J][qb][ks][w] = hl[0];
                        plr[J][qb][ks][w] = hl[1];
                        lt[qb] = dot2_ones<DT>(hl[1], dot2_ones<DT>(hl[0], lt[qb]));
                    } else {
                        const uint32_t pw = pack2<DT>(p0, p1);
                        pr[J][qb][ks][w] = pw;
                        lt[qb] = dot2_ones<DT>(pw, lt[qb]);
                    }
                }
            }
        }
    };
    // O^T += V^T P^T with P set J.
    auto stage_pv = [&](const char* vt, auto Jc) __attribute__((always_inline)) {
        constexpr int J = decltype(Jc)::value;
#pragma unroll
        for (int ks = 0; ks < PKS; ++ks)
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const u32x2 v0 = ld_lds_tr(vt + ks * 16 * ROWB + voff[0][db]);
                const u32x2 v1 = ld_lds_tr(vt + ks * 16 * ROWB + voff[1][db]);
                const u32x4 a = {v0[0], v0[1], v1[0], v1[1]};
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    o[db][qb] = mfma32<DT>(a, pr[J][qb][ks], o[db][qb]);
                    if constexpr (SPL) o[db][qb] = mfma32<DT>(a, plr[J][qb][ks], o[db][qb]);
                }
            }
    };
    auto row_max = [&](auto Jc, float (&mx)[QB]) __attribute__((always_inline)) {
        constexpr int J = decltype(Jc)::value;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            float v = sr[J][0][qb][0];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = (kb == 0 ? 1 : 0); r < 16; ++r) v = fmaxf(v, sr[J][kb][qb][r]);
            mx[qb] = half_max(v);
        }
    };
    // The group's first tile: m (log2 units) from its row max.
    auto softmax_first = [&](auto Jc) __attribute__((always_inline)) {
        float mx[QB];
        row_max(Jc, mx);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const float v = mx[qb] * sl2;
            m[qb] = (v == -INFINITY) ? 0.f : v;
        }
        stage_exp(Jc, m, lsum);
    };
    // Later tiles, against m.  A lane whose packed row sum of the tile reaches P_SUM_MAX (some
    // P near or past fp16's range, where the fp16 pack gives an infinite sum) makes the wave
    // raise m of its rows to max(m, the tile's row max), rescale O and the row sums by
    // 2^(m_old - m_new) (exactly 1 for rows whose m stays) and repeat the tile's exp2 and
    // packing, all before the tile's PV.  The bound holds for bf16 too: bf16 P would not
    // overflow until 2^128, but O = sum P V would overflow first.  Inputs whose scores stay
    // near the first tile's never take that path.
    auto softmax_next = [&](auto Jc) __attribute__((always_inline)) {
        float lt[QB];
        stage_exp(Jc, m, lt);
        bool bad = false;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) bad |= !(lt[qb] < P_SUM_MAX);
        if (__builtin_expect(__any(bad), 0)) {
            float mx[QB];
            row_max(Jc, mx);
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const float mn = fmaxf(m[qb], mx[qb] * sl2);
                const float a = fast_exp2(m[qb] - mn);
                lsum[qb] *= a;
#pragma unroll
                for (int db = 0; db < NDB; ++db) o[db][qb] *= a;
                m[qb] = mn;
            }
            stage_exp(Jc, m, lt);
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) lsum[qb] += lt[qb];
    };

    // Tile loop.  Tile t: S(t), softmax, PV(t), with the DMA of K(t+1) and V(t+1) in flight
    // into the other buffers (K(j), V(j) live in buffers j&1).  The loop is unrolled by two
    // so buffer indices are constants.  The two waves sharing a SIMD (different workgroups)
    // overlap each other's phases.
    auto iteration = [&](auto Pc, int i) __attribute__((always_inline)) {
        constexpr int P = decltype(Pc)::value;  // = i & 1
        const int t = tb + i;
        if (t + 1 < te) {
            issue(t + 1, 0, P ^ 1);
            issue(t + 1, 1, P ^ 1);
        }
        if (t < te && t < n_act) {
            stage_s(smem[grp][0][P], I0{});
            if (t >= n_plain) stage_mask(t, I0{});
            if (t == tb) softmax_first(I0{});
            else softmax_next(I0{});
            stage_pv(smem[grp][1][P], I0{});
        }
        wait_dma();
        __syncthreads();
    };
    if (tb < te) {
        issue(tb, 0, 0);
        issue(tb, 1, 0);
    }
    wait_dma();
    __syncthreads();
    for (int i = 0; i < nit; i += 2) {
        iteration(I0{}, i);
        if (i + 1 < nit) iteration(I1{}, i + 1);
    }

    if constexpr (KSPLIT == 2) {
        // Group 1's m, partial row sums and O^T accumulators to group 0 (the buffers are free:
        // the last iteration ended with every DMA done and a barrier).  Element j of the
        // state of wave gw's lane sits at float (j*NW + gw)*64 + lane.
        constexpr int NV = QB * (2 + NDB * 16);
        float* xs = reinterpret_cast<float*>(&smem[0][0][0][0]);
        static_assert(NV * NW * 64 * 4 <= (int)sizeof(smem), "merge state fits the tile buffers");
        auto at = [&](int j) -> float& { return xs[(j * NW + gw) * 64 + lane]; };
        if (grp == 1) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                at(qb * (2 + NDB * 16)) = m[qb];
                at(qb * (2 + NDB * 16) + 1) = lsum[qb];
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) at(qb * (2 + NDB * 16) + 2 + db * 16 + r) = o[db][qb][r];
            }
        }
        __syncthreads();
        if (grp == 1) return;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const int base = qb * (2 + NDB * 16);
            const float m1 = at(base), l1 = at(base + 1);
            // a side without a visible key of the row (its row sum 0) takes no part
            const float L0 = half_sum(lsum[qb]), L1 = half_sum(l1);
            if (L1 > 0.f) {
                const float mn = L0 > 0.f ? fmaxf(m[qb], m1) : m1;
                const float a0 = L0 > 0.f ? fast_exp2(m[qb] - mn) : 0.f;
                const float a1 = fast_exp2(m1 - mn);
                lsum[qb] = lsum[qb] * a0 + l1 * a1;
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        o[db][qb][r] = o[db][qb][r] * a0 + at(base + 2 + db * 16 + r) * a1;
                m[qb] = mn;
            }
        }
    }

#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const float l = half_sum(lsum[qb]);
        const float inv = l > 0.f ? 1.0f / l : 0.f;
        const int q = q0 + qb * 32 + l32;
        if (q < S) {
            uint16_t* orow = out + ((size_t)b * S + q) * ((size_t)Hq * D) + (size_t)h * D;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    u32x2 w = {pack2<DT>(o[db][qb][g4 * 4 + 0] * inv, o[db][qb][g4 * 4 + 1] * inv),
                               pack2<DT>(o[db][qb][g4 * 4 + 2] * inv, o[db][qb][g4 * 4 + 3] * inv)};
                    *reinterpret_cast<u32x2*>(orow + db * 32 + g4 * 8 + hi * 4) = w;
                }
            if (lse && hi == 0)
                lse[((size_t)b * Hq + h) * S + q] =
                    l > 0.f ? (m[qb] + __log2f(l)) * 0.69314718055994530942f : -INFINITY;
        }
    }
}

// Compute units of the current device (cached per device; 0 if it cannot be read).
static int compute_units() {
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
static int launch_fwd_t(const FwdArgs& a) {
    constexpr int QB = 1;  // 32-row blocks per wave
    constexpr int BM = 128 * QB;
    const int n_qblk = (a.S + BM - 1) / BM;
    const long long n_wg = (long long)a.B * a.Hq * n_qblk;
    dim3 grid((unsigned)n_wg);
    // At most one workgroup of 128 rows per CU: split each block's keys over two groups of
    // waves (the critical causal block walks half its tiles, and every SIMD holds two waves).
    // Causal D = 64: blocks of 64 rows instead, two workgroups per CU (2 x 64 KB of LDS)
    // pairing heavy and light blocks, so that no CU holds more than about the mean number of
    // tiles.  (At D = 128 two such workgroups would need 256 KB of LDS.)
    if constexpr (D == 64) {
        if (n_wg <= compute_units() && a.causal) {
            const int n_qblk64 = (a.S + 63) / 64;
            dim3 grid64((unsigned)((long long)a.B * a.Hq * n_qblk64));
            hipLaunchKernelGGL((fa_fwd_kernel<D, DT, QB, 2, 2>), grid64, dim3(256), 0, (hipStream_t)a.stream,
                               (const uint16_t*)a.qkv, (uint16_t*)a.o, a.lse, a.kv_len, a.B, a.S, a.Hq,
                               a.Hkv, a.scale * 1.4426950408889634f, a.causal, n_qblk64);
            return hipGetLastError() == hipSuccess ? 0 : -1;
        }
    }
    if (n_wg <= compute_units()) {
        hipLaunchKernelGGL((fa_fwd_kernel<D, DT, QB, 2>), grid, dim3(512), 0, (hipStream_t)a.stream,
                           (const uint16_t*)a.qkv, (uint16_t*)a.o, a.lse, a.kv_len, a.B, a.S, a.Hq,
                           a.Hkv, a.scale * 1.4426950408889634f, a.causal, n_qblk);
    } else {
        hipLaunchKernelGGL((fa_fwd_kernel<D, DT, QB, 1>), grid, dim3(256), 0, (hipStream_t)a.stream,
                           (const uint16_t*)a.qkv, (uint16_t*)a.o, a.lse, a.kv_len, a.B, a.S, a.Hq,
                           a.Hkv, a.scale * 1.4426950408889634f, a.causal, n_qblk);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_fwd(const FwdArgs& a) {
    const int rc = launch_fwd_asm(a);  // D = 128 fp16 and bf16: hand-scheduled assembly kernels
    if (rc != 1) {
        if (rc == 0) note_kernels(kFwdAsm);
        return rc;
    }
    note_kernels(kFwdHip);
    if (a.D == 128) return a.dtype == DT_F16 ? launch_fwd_t<128, DT_F16>(a) : launch_fwd_t<128, DT_BF16>(a);
    return a.dtype == DT_F16 ? launch_fwd_t<64, DT_F16>(a) : launch_fwd_t<64, DT_BF16>(a);
}

}  // namespace tkm
