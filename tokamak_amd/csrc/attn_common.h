// attn_common.h -- device helpers shared by the CDNA4 (gfx950) attention kernels.
//
// MFMA operand layouts used throughout (v_mfma_f32_32x32x16_{f16,bf16}, wave64):
//   lane l, l32 = l & 31, hi = l >> 5
//   A (32 x 16) : lane holds A[m = l32][k = hi*8 + i],  i = 0..7   (one 128-bit VGPR quad)
//   B (16 x 32) : lane holds B[k = hi*8 + i][n = l32],  i = 0..7
//   C (32 x 32) : lane holds C[m = (r/4)*8 + hi*4 + (r%4)][n = l32], r = 0..15 (fp32)
// An accumulator C[m][n] therefore feeds the next MFMA as a B operand (or, for
// C[m=q][n=key], as an A operand of the transposed product) without any lane
// exchange, provided the k index of that product is permuted the same way in
// the other operand: k-slot (hi*8 + i) of a 16-wide k step ks stands for row
//   kslot_row(ks, hi, i) = ks*16 + (i/4)*8 + hi*4 + (i%4)
// of the accumulator.  Operands read from LDS that are indexed by such a
// permuted k (V^T in the forward, Q^T/dO^T/K^T in the backward) are stored
// with each 16-row group reordered by perm16 so one 128-bit read per lane
// fetches the 8 slots in order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tkm {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum { DT_F16 = 0, DT_BF16 = 1 };

// Position of row k (0..15) inside its 16-row group in LDS: swaps bits 2 and 3,
// so that rows {0-3, 8-11} (k-slots of lanes 0-31) come first, then {4-7, 12-15}.
__device__ __forceinline__ int perm16(int k) {
    return (k & 3) | (((k >> 3) & 1) << 2) | (((k >> 2) & 1) << 3);
}
// Row of a 16-aligned block given its in-group index k; quads move as a unit.
__device__ __forceinline__ int perm_row(int r) { return (r & ~15) | perm16(r & 15); }

template <int DT>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (DT == DT_F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Two fp32 -> packed 16-bit (round to nearest even).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
    if constexpr (DT == DT_F16) {
        f16x2 h = {(_Float16)x, (_Float16)y};
        return __builtin_bit_cast(uint32_t, h);
    } else {
        bf16x2 h = {(__bf16)x, (__bf16)y};
        return __builtin_bit_cast(uint32_t, h);
    }
}

// Sum of the two 16-bit values in w, accumulated in fp32.
template <int DT>
__device__ __forceinline__ float dot2_ones(uint32_t w, float acc) {
    if constexpr (DT == DT_F16) {
        const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one, acc, false);
    } else {
        const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one, acc, false);
    }
}

// bf16 keeps 8 significant bits, too few for the probabilities P and dS that feed the
// second GEMM of each pair at the stated tolerance.  In bf16 mode they are therefore split
// into hi = bf16(x) and lo = bf16(x - hi) and both halves go through the MFMA (same A
// operand), which carries ~16 significant bits; fp16 (11 bits) needs no split.
template <int DT>
struct Split {
    static constexpr bool on = DT == DT_BF16;
    static constexpr int n = on ? 1 : 0;
};
// Returns {hi, lo}, each two packed bf16 values.
__device__ __forceinline__ u32x2 pack_split_bf16(float x, float y) {
    const uint32_t hi = pack2<DT_BF16>(x, y);
    const float xh = __uint_as_float(hi << 16), yh = __uint_as_float(hi & 0xffff0000u);
    return u32x2{hi, pack2<DT_BF16>(x - xh, y - yh)};
}

// Reinterpret one 32-bit word as two fp16.  The word is taken by value on purpose: with
// this toolchain, __builtin_bit_cast applied directly to an ext-vector element lvalue
// (v[i]) reads element 0's storage, so element words must be copied out first.
__device__ __forceinline__ f16x2 as_f16x2(uint32_t w) { return __builtin_bit_cast(f16x2, w); }

template <int DT>
__device__ __forceinline__ float to_f32(uint16_t bits) {
    if constexpr (DT == DT_F16) return (float)__builtin_bit_cast(_Float16, bits);
    else return __builtin_bit_cast(float, (uint32_t)bits << 16);
}

// Low / high 16-bit halves of two words, interleaved: (lo(a), lo(b)) and (hi(a), hi(b)).
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
    return (a & 0xffffu) | (b << 16);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
    return (a >> 16) | (b & 0xffff0000u);
}

__device__ __forceinline__ u32x4 ld_global16(const uint16_t* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x4 ld_lds16(const uint16_t* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st_lds16(uint16_t* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void st_lds8(uint16_t* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// Reductions across the two lane halves (l, l ^ 32) with v_permlane32_swap: the swap
// leaves x[l] and x[l ^ 32] in the two results, in an order that does not matter here.
__device__ __forceinline__ float half_max(float x) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float half_sum(float x) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// ---------------------------------------------------------------------------
// Instruction-schedule shaping (LLVM sched_group_barrier masks).  A stage that reads N LDS
// operands and issues M MFMAs per read is ordered as: LEAD reads, then (M MFMAs, 1 read)
// repeated, then the remaining MFMAs, so only LEAD reads are in flight ahead of the MFMAs
// that consume them (bounds register pressure; without it the compiler hoists every read).
enum : unsigned { SG_MFMA = 0x008, SG_VALU = 0x002, SG_DS_READ = 0x100, SG_TRANS = 0x400 };
template <int N, int M, int LEAD, int READS_PER_STEP = 1>
__device__ __forceinline__ void sched_reads_mfma() {
    __builtin_amdgcn_sched_group_barrier(SG_DS_READ, LEAD * READS_PER_STEP, 0);
#pragma unroll
    for (int i = 0; i < N - LEAD; ++i) {
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, M, 0);
        __builtin_amdgcn_sched_group_barrier(SG_DS_READ, READS_PER_STEP, 0);
    }
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, M * LEAD, 0);
}

// Steady-state block of a software-pipelined attention loop: NM MFMAs, ND LDS operand reads
// and NE exp2 (plus ~2 other VALU each).  Order: a batch of reads first, then per MFMA one
// exp, two VALU and one or two reads, so the transcendentals sit between MFMAs of the same
// wave (on gfx950 they overlap with MFMA only within a wave) and reads run ahead of use.
template <int NM, int ND, int NE>
__device__ __forceinline__ void sched_steady() {
    constexpr int LEAD = 8;
    constexpr int REST = ND - LEAD;
    __builtin_amdgcn_sched_group_barrier(SG_DS_READ, LEAD, 0);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
        if (i < NE) __builtin_amdgcn_sched_group_barrier(SG_TRANS, (NE + NM - 1) / NM, 0);
        __builtin_amdgcn_sched_group_barrier(SG_VALU, 2, 0);
        if (i < REST) __builtin_amdgcn_sched_group_barrier(SG_DS_READ, (REST + NM - 1) / NM, 0);
    }
}

// ---------------------------------------------------------------------------
// Buffer resources and HBM -> LDS DMA.
// A raw buffer resource covering `bytes` bytes from `base`: loads at offsets beyond it
// return zero, which is how partial tiles (rows >= S or >= kv_len) are zero-filled.
// Both arguments must be wave-uniform; readfirstlane makes that explicit so the descriptor
// lives in SGPRs (a VGPR descriptor would need a waterfall loop around every load).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                             __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000);
}
// Bytes a descriptor over `rows` rows of `pitch` bytes needs when lanes touch only the first
// `width` bytes of each row: it ends at the last row's last touched byte, never at the row's
// pitch, so no request through it can reach past the tensor that holds those rows.
__device__ __forceinline__ uint32_t rows_bytes(int rows, uint32_t pitch, uint32_t width) {
    return rows > 0 ? (uint32_t)(rows - 1) * pitch + width : 0u;
}
typedef __attribute__((address_space(3))) void* lds_ptr_t;
// 16 bytes per lane from rsrc+voffset into LDS at lds + 16*lane (lds is wave-uniform).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, const void* lds, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, voffset, 0, 0, 0);
}
// Wait until every memory operation of this wave, LDS DMA included, has completed.
// 4 bytes per lane from rsrc+voffset into LDS at lds + 4*lane.
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, const void* lds, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 4, voffset, 0, 0, 0);
}
__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0); }

typedef short s16x4 __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element i%4 of the
// 8-byte words read by lanes 4e + i/4 (e = 0..3).  With lane j of the group pointing at
// row j/4, columns 4*(j%4)..+3 of a 4 x 16 block of 16-bit values, lane i gets column i.
__device__ __forceinline__ u32x2 ld_lds_tr(const char* p) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
    return __builtin_bit_cast(u32x2, v);
}

// Tiles in LDS are stored row-major without padding, one row = D 16-bit values = D/8
// 16-byte chunks; chunk c of row r is stored at slot c ^ swz<D>(r).  The swizzle makes
// both access patterns conflict-free on the 64 x 4-byte LDS banks:
//   128-bit reads of one chunk from 16 consecutive rows (MFMA operands along the row),
//   transposed 64-bit reads of 4 consecutive rows x 4 consecutive chunks.
template <int D>
__device__ __forceinline__ int swz(int r) {
    if constexpr (D == 128) return ((r & 3) << 2) | ((r >> 2) & 3);
    else return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
}

// ---------------------------------------------------------------------------
// Tile movement HBM -> registers -> LDS.
// A tile is ROWS consecutive sequence rows x D contiguous 16-bit values of one
// head (row stride ld elements).  Thread t owns "quad chunks": 4 consecutive
// rows x 8 columns (four 16-byte global loads), so a row-major LDS copy takes
// 4 128-bit stores and a transposed copy takes 8 64-bit stores.
template <int ROWS, int D, int NT>
struct TileIO {
    static constexpr int DC = D / 8;                 // 16-byte chunks per row
    static constexpr int NCH = (ROWS / 4) * DC;      // quad chunks per tile
    static constexpr int PER = (NCH + NT - 1) / NT;  // per thread
    u32x4 r[PER][4];

    // rows at or beyond row_end are zero-filled (never read).
    __device__ __forceinline__ void load(const uint16_t* base, size_t ld, int row0, int row_end, int tid) {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            int c = tid + p * NT;
            if (NCH % NT == 0 || c < NCH) {
                int rg = c / DC, dc = c % DC;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    int row = row0 + rg * 4 + j;
                    if (row < row_end)
                        r[p][j] = ld_global16(base + (size_t)row * ld + dc * 8);
                    else
                        r[p][j] = u32x4{0u, 0u, 0u, 0u};
                }
            }
        }
    }
    // row-major copy: lds[row * LDR + col]
    template <int LDR>
    __device__ __forceinline__ void store_rows(uint16_t* lds, int tid) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            int c = tid + p * NT;
            if (NCH % NT == 0 || c < NCH) {
                int rg = c / DC, dc = c % DC;
#pragma unroll
                for (int j = 0; j < 4; ++j) st_lds16(lds + (rg * 4 + j) * LDR + dc * 8, r[p][j]);
            }
        }
    }
    // transposed copy with perm16 row order: lds[col * LDT + perm_row(row)]
    template <int LDT>
    __device__ __forceinline__ void store_cols(uint16_t* lds, int tid) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            int c = tid + p * NT;
            if (NCH % NT == 0 || c < NCH) {
                int rg = c / DC, dc = c % DC;
                int prow = perm_row(rg * 4);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    // column dc*8 + 2w (low halves) and dc*8 + 2w + 1 (high halves)
                    u32x2 lo = {pack_lo(r[p][0][w], r[p][1][w]), pack_lo(r[p][2][w], r[p][3][w])};
                    u32x2 hi = {pack_hi(r[p][0][w], r[p][1][w]), pack_hi(r[p][2][w], r[p][3][w])};
                    st_lds8(lds + (dc * 8 + 2 * w) * LDT + prow, lo);
                    st_lds8(lds + (dc * 8 + 2 * w + 1) * LDT + prow, hi);
                }
            }
        }
    }
};

}  // namespace tkm
