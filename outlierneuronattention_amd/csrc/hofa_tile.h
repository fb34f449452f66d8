// LDS tile staging and operand reads shared by the attention kernels (gfx950).
//
// Tiles of 64 rows x W 16-bit elements live in LDS row-major, their 16-byte
// granules swizzled per row (TileL); they are filled either by LDS DMA
// (TileDma: buffer loads that write LDS directly, 16-bit inputs) or through
// registers (TileStage: f32 inputs, split into bf16 hi/lo).  Operands whose k
// index runs along the tile rows are read with the transposing LDS load
// ds_read_b64_tr_b16 (tr_operand).  The staging helpers assume 256-thread
// blocks.
#pragma once

#include "hofa_mfma.h"

namespace hofa {
namespace tile {

constexpr int NT = 256;  // threads per block of the kernels that stage tiles

// A 64-row tile of width W (16-bit elements) in LDS: row pitch and the 16-byte
// granule swizzle (granule g of row r lives at g ^ swz(r)).  W = 16 rows are
// padded to 24 elements instead.  With 64 four-byte banks, 16-lane row reads
// of one granule column, the 8-row x 64-byte footprint of a transposing read
// and row-wise staging stores all touch distinct banks.
template <int W>
struct TileL {
    static constexpr int PITCH = W == 16 ? 24 : W;
    static constexpr int ELEMS = 64 * PITCH;
    __device__ static constexpr int swz(int r) {
        if constexpr (W == 16) return 0;
        else if constexpr (W == 32) return (r >> 2) & 3;
        else if constexpr (W == 64) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
        else return ((r & 3) << 2) | ((r >> 2) & 3);
    }
    // element offset of (row r, column c); c keeps its place inside its granule
    __device__ static int off(int r, int c) { return r * PITCH + ((((c >> 3) ^ swz(r))) << 3) + (c & 7); }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint2 lds_tr16(const uint16_t *p) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)p);
    return __builtin_bit_cast(uint2, v);
}

// A operand of v_mfma_f32_32x32x16 whose row index i runs along tile columns
// [col0, col0 + 32) and whose k index runs along tile rows:
//   lane l = 16 g + s, i = l % 32, k = 8 (l / 32) + e  <->  tile row krow0 + 8 (e / 4) + 4 (l / 32) + e % 4,
// the order in which a C-layout accumulator's entries [8 k2, 8 k2 + 8) pack into
// an operand (pack8).  ds_read_b64_tr_b16 hands output lane 4a + b of each
// 16-lane group element b of the 8-byte reads of lanes a, a + 4, a + 8, a + 12,
// so source lane s reads tile row krow0 + 4 (l / 32) + s / 4 at column
// col0 + i0 + 4 (s % 4).  Tiles narrower than 32 columns (W = 16) fill rows
// 16..31 of the operand with a copy of rows 0..15.
template <int W>
__device__ __forceinline__ u32x4 tr_operand(const uint16_t *tile, int krow0, int col0, int lane) {
    const int g = lane >> 4, s = lane & 15;
    const int i0 = W >= 32 ? 16 * (g & 1) : 0;
    const int row = krow0 + 4 * (g >> 1) + (s >> 2);
    const int col = col0 + i0 + 4 * (s & 3);
    const uint2 a = lds_tr16(tile + TileL<W>::off(row, col));
    const uint2 b = lds_tr16(tile + TileL<W>::off(row + 8, col));
    return u32x4{a.x, a.y, b.x, b.y};
}

// As tr_operand with k in natural order, for operands that pair with rows
// loaded straight from memory: lane l, k = 8 (l / 32) + e  <->  tile row
// krow0 + 8 (l / 32) + e (source lane s reads row krow0 + 8 (l / 32) + s / 4,
// then 4 rows further).  Also conflict-free on TileL<64> and TileL<128>.
template <int W>
__device__ __forceinline__ u32x4 tr_operand_lin(const uint16_t *tile, int krow0, int col0, int lane) {
    const int g = lane >> 4, s = lane & 15;
    const int i0 = W >= 32 ? 16 * (g & 1) : 0;
    const int row = krow0 + 8 * (g >> 1) + (s >> 2);
    const int col = col0 + i0 + 4 * (s & 3);
    const uint2 a = lds_tr16(tile + TileL<W>::off(row, col));
    const uint2 b = lds_tr16(tile + TileL<W>::off(row + 4, col));
    return u32x4{a.x, a.y, b.x, b.y};
}

// The two LDS reads of tr_operand<W>(tile, krow0, col0, lane) are at
// tile + krow0 * PITCH + tr_lane_off<W>(col0, lane, j), j = 0, 1 (krow0 a
// multiple of 16): loops that read many operands of one tile keep these
// per-lane offsets in registers instead of recomputing the swizzle.
template <int W>
__device__ __forceinline__ int tr_lane_off(int col0, int lane, int j) {
    const int g = lane >> 4, s = lane & 15;
    const int i0 = W >= 32 ? 16 * (g & 1) : 0;
    return TileL<W>::off(4 * (g >> 1) + (s >> 2) + 8 * j, col0 + i0 + 4 * (s & 3));
}

// Rows [t0, t0+64) of a [T, W] input matrix, staged global -> registers
// (fetch, issued a tile ahead) -> LDS (put) as row-major 16-bit operands in the
// TileL<W> layout, rows past T zero; f32 inputs also keep their bf16 rounding
// remainders (same layout, second array).  256 threads, one 16-byte granule
// (8 elements) of one row each per piece.
template <int DT, int W, bool WANT_LO = true>
struct TileStage {
    using in_t = typename Stor<DT>::type;
    static constexpr int NG = W / 8;
    static constexpr int NPIECE = 64 * NG;
    static constexpr int NP = (NPIECE + NT - 1) / NT;
    static constexpr bool LO = DT == HOFA_F32 && WANT_LO;
    u32x4 x[NP], l[LO ? NP : 1];

    __device__ void fetch(const in_t *base, int64_t st, int t0, int T) {
        const __amdgpu_buffer_rsrc_t r = rows_rsrc(base, (uint32_t)(T * st * sizeof(in_t)));
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int pi = min((int)threadIdx.x + NT * i, NPIECE - 1);  // extra threads repeat the last piece
            const uint32_t off = (uint32_t)(((t0 + pi / NG) * st + 8 * (pi % NG)) * sizeof(in_t));
            if constexpr (LO) x[i] = bload_op8<DT>(r, off, &l[i]);
            else x[i] = bload_op8<DT>(r, off);
        }
    }
    __device__ void put(uint16_t *tile, uint16_t *lo) const {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int pi = threadIdx.x + NT * i;
            if (NPIECE % NT != 0 && pi >= NPIECE) continue;
            const int o = TileL<W>::off(pi / NG, 8 * (pi % NG));
            *(u32x4 *)&tile[o] = x[i];
            if constexpr (LO) *(u32x4 *)&lo[o] = l[i];
        }
    }
};

// The same tile staged by the DMA path of 16-bit inputs: buffer loads that
// write LDS directly (buffer_load_dwordx4 ... lds), each wave load filling
// 1 KB of the tile image, lane j the 16-byte granule at 16 j.  A lane fetches
// the source granule that the TileL<W> swizzle puts at its position; padding
// granules (W = 16) and rows past T read out of range and land as zeros.
// The loads count against vmcnt: the issuing wave waits for them before the
// barrier that hands the buffer to the block.  SRCW < W: source rows of SRCW
// elements (a multiple of 8) fill the first SRCW columns, the rest read zeros.
template <int W, int SRCW = W>
struct TileDma {
    static constexpr int GPR = TileL<W>::PITCH / 8;  // 16-byte granules per LDS row, padding included
    static constexpr int NLOAD = GPR;                 // 64 rows x GPR granules / 64 lanes
    static constexpr int NW = (NLOAD + 3) / 4;        // wave loads per wave (the last wave may have one less)
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t voff[NW];  // byte offset of this lane's granule within a tile at row 0 (0x80000000: none)
    uint32_t row_bytes;

    // Rows [0, T) of one head's matrix (row stride st elements) through this wave.
    template <class in_t>
    __device__ void init(const in_t *base, int64_t st, int T, int wave, int lane) {
        rsrc = rows_rsrc(base, (uint32_t)(T * st * sizeof(in_t)));
        row_bytes = (uint32_t)(st * sizeof(in_t));
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            const int p = 64 * (4 * j + wave) + lane;
            const int row = p / GPR, pg = p % GPR;
            const int sg = pg ^ TileL<W>::swz(row);  // source granule at this position
            voff[j] = pg >= W / 8 || sg >= SRCW / 8 ? 0x80000000u : (uint32_t)(row * st * sizeof(in_t) + 16 * sg);
        }
    }
    // Rows [t0, t0 + 64) into `tile` (row t0 + i at tile row i).
    __device__ void fetch(uint16_t *tile, int t0, int wave) const {
        const uint32_t base = (uint32_t)t0 * row_bytes;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            const int i = 4 * j + wave;
            if (NLOAD % 4 != 0 && i >= NLOAD) break;
            constexpr bool kPad = TileL<W>::PITCH != W || SRCW != W;  // some lanes fetch padding
            const uint32_t off = !kPad || voff[j] != 0x80000000u ? voff[j] + base : voff[j];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(tile + 512 * i),
                                                     16, off, 0, 0, 0);
        }
    }
};

// Wait for this wave's outstanding vector-memory loads (the LDS DMA of a tile).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Operand dword of two 16-bit values (hi, lo) with hi + lo = x to about twice
// the operand precision.
template <int DT>
__device__ __forceinline__ uint32_t split_pair(float x) {
    const uint32_t h = pack2<DT>(x, 0.f) & 0xffffu;
    const float r = x - op_to_f32<DT>(h);
    return h | (pack2<DT>(r, 0.f) << 16);
}

// 8 consecutive input elements times `scale` (in f32) as a 16-bit operand
// pair hi + lo (about twice the operand precision), zeros when !valid.
template <int DT>
__device__ __forceinline__ void load_scaled_op8(const typename Stor<DT>::type *p, float scale, bool valid, u32x4 &hi,
                                                u32x4 &lo) {
    float x[8];
    if (valid) {
        const u32x4 w0 = *(const u32x4 *)p;
        if constexpr (DT == HOFA_F32) {
            const u32x4 w1 = *(const u32x4 *)(p + 4);
            unpack16<DT>(w0, x);
            unpack16<DT>(w1, x + 4);
        } else {
            unpack16<DT>(w0, x);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= scale;
    split8<DT>(x, hi, lo);
}

// (1, 1) as a dword of 16-bit operands.
template <int DT>
constexpr uint32_t kOnes2 = kF16Ops<DT> ? 0x3C003C00u : 0x3F803F80u;

}  // namespace tile
}  // namespace hofa
