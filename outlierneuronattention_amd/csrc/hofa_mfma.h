// MFMA helpers for gfx950 (CDNA4), 64-wide waves.
//
// v_mfma_f32_32x32x16_{bf16,f16}: C[32x32] += A[32x16] * B[16x32]
//   A operand, lane l: row l%32, k = 8*(l/32) + e  (e = 0..7, one 16-byte register quad)
//   B operand, lane l: col l%32, k = 8*(l/32) + e
//   C/D,       lane l: col l%32, rows 8*(v/4) + 4*(l/32) + v%4  (v = 0..15)
// v_mfma_f32_16x16x32_{bf16,f16}: C[16x16] += A[16x32] * B[32x16]
//   A operand, lane l: row l%16, k = 8*(l/16) + e
//   B operand, lane l: col l%16, k = 8*(l/16) + e
//   C/D,       lane l: col l%16, rows 4*(l/16) + v  (v = 0..3)
// Both layouts were checked against a host matrix product on the device.
#pragma once

#include "hofa_common.h"

namespace hofa {

// 16-bit operand element type used with an input dtype: f16 inputs use the
// f16 matrix cores, bf16 and f32 inputs use bf16 operands.
template <int DT> constexpr bool kF16Ops = (DT == HOFA_F16);

template <int DT>
__device__ __forceinline__ f32x16 mfma32(const u32x4 &a, const u32x4 &b, const f32x16 &c) {
    if constexpr (kF16Ops<DT>) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    if constexpr (kF16Ops<DT>) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two floats -> one dword of 16-bit operands (lo in bits 0..15), round to
// nearest even; one packed conversion instruction.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    const f32x2 v = {lo, hi};
    if constexpr (kF16Ops<DT>) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
    } else {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    }
}

template <int DT>
__device__ __forceinline__ u32x4 pack8(const float *x) {
    return u32x4{pack2<DT>(x[0], x[1]), pack2<DT>(x[2], x[3]), pack2<DT>(x[4], x[5]), pack2<DT>(x[6], x[7])};
}

// Eight consecutive entries x[off .. off+7] of an accumulator -> operand quad.
template <int DT>
__device__ __forceinline__ u32x4 pack8(const f32x16 &x, int off) {
    return u32x4{pack2<DT>(x[off], x[off + 1]), pack2<DT>(x[off + 2], x[off + 3]), pack2<DT>(x[off + 4], x[off + 5]),
                 pack2<DT>(x[off + 6], x[off + 7])};
}

// Split 8 floats into operand quads hi + lo with hi = round(x), lo = round(x - hi):
// hi + lo carries about twice the operand mantissa into the matrix cores.
template <int DT>
__device__ __forceinline__ void split8(const float *x, u32x4 &hi, u32x4 &lo);

template <int DT>
__device__ __forceinline__ void split8v(const f32x16 &x, int off, u32x4 &hi, u32x4 &lo) {
    float t[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = x[off + e];
    split8<DT>(t, hi, lo);
}

// 16-bit operand -> float.
template <int DT>
__device__ __forceinline__ float op_to_f32(uint32_t bits16) {
    if constexpr (kF16Ops<DT>) {
        return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
    } else {
        return __uint_as_float(bits16 << 16);
    }
}

template <int DT>
__device__ __forceinline__ void split8(const float *x, u32x4 &hi, u32x4 &lo) {
    hi = pack8<DT>(x);
    float r[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        r[2 * e] = x[2 * e] - op_to_f32<DT>(hi[e] & 0xffffu);
        r[2 * e + 1] = x[2 * e + 1] - op_to_f32<DT>(hi[e] >> 16);
    }
    lo = pack8<DT>(r);
}

// Load 8 consecutive input elements as one operand quad (converting f32 input).
template <int DT>
__device__ __forceinline__ u32x4 load_op8(const typename Stor<DT>::type *p) {
    if constexpr (DT == HOFA_F32) {
        const f32x4 a = *(const f32x4 *)p, b = *(const f32x4 *)(p + 4);
        return u32x4{pack2<DT>(a[0], a[1]), pack2<DT>(a[2], a[3]), pack2<DT>(b[0], b[1]), pack2<DT>(b[2], b[3])};
    } else {
        return *(const u32x4 *)p;
    }
}

// f32 input only: the bf16 rounding remainder of 8 consecutive elements
// (x - bf16(x)), so hi + lo carries ~16 mantissa bits into the matrix cores.
__device__ __forceinline__ u32x4 load_lo8_f32(const float *p) {
    const f32x4 a = *(const f32x4 *)p, b = *(const f32x4 *)(p + 4);
    float r[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        r[e] = a[e] - (float)(__bf16)a[e];
        r[4 + e] = b[e] - (float)(__bf16)b[e];
    }
    return pack8<HOFA_BF16>(r);
}

// Range-checked loads through a buffer resource: an access at or past
// `bytes` returns zeros, so tile loads past the last row need no branch.
// `base` must be wave-uniform (derived from blockIdx and kernel arguments).
constexpr int kBufRaw = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, bytes, kBufRaw);
}

__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// 8 consecutive elements at byte offset `off` as a 16-bit operand quad; f32
// inputs are rounded to bf16 (hi) and, when lo is given, their remainders.
template <int DT>
__device__ __forceinline__ u32x4 bload_op8(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 *lo = nullptr) {
    if constexpr (DT == HOFA_F32) {
        const u32x4 a = bload16(r, off), b = bload16(r, off + 16);
        float x[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[e] = __uint_as_float(a[e]);
            x[4 + e] = __uint_as_float(b[e]);
        }
        u32x4 hi, l;
        split8<DT>(x, hi, l);
        if (lo) *lo = l;
        return hi;
    } else {
        return bload16(r, off);
    }
}

// Block-index remap for kernels whose blocks carry unequal causal work.
// Blocks are dispatched round-robin over 8 XCDs; all blocks of one head stay
// on one XCD (its L2 holds the head's keys and values), and each XCD takes the
// work rank (0 = most work) as the outer index over its heads, so every XCD
// dispatches all of its longest blocks before any shorter one.
__device__ __forceinline__ void xcd_rank_remap(int blk, int nrank, int nhead, int *head, int *rank) {
    constexpr int kXcd = 8;
    if (nhead % kXcd == 0) {
        const int xcd = blk % kXcd, slot = blk / kXcd, hpx = nhead / kXcd;
        *rank = slot / hpx;
        *head = (slot % hpx) * kXcd + xcd;
    } else {
        *rank = blk / nhead;
        *head = blk % nhead;
    }
}

}  // namespace hofa
