// Shared device/host helpers for the gfx950 HOFA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstdio>
#include <string>

#include "../../include/hofa.h"

namespace hofa {

// ---------------------------------------------------------------- errors
void set_error(const std::string &msg);

#define HOFA_REQUIRE(cond, code, ...)                                  \
    do {                                                               \
        if (!(cond)) {                                                 \
            char _buf[512];                                            \
            snprintf(_buf, sizeof(_buf), __VA_ARGS__);                 \
            ::hofa::set_error(_buf);                                   \
            return (code);                                             \
        }                                                              \
    } while (0)

int check_launch(const char *what);
int device_cu_count();

// ---------------------------------------------------------------- types
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <int DT> struct Stor;
template <> struct Stor<HOFA_F32> { using type = float; };
template <> struct Stor<HOFA_BF16> { using type = uint16_t; };
template <> struct Stor<HOFA_F16> { using type = uint16_t; };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

template <int DT>
__device__ __forceinline__ float to_f32(typename Stor<DT>::type x) {
    if constexpr (DT == HOFA_F32) {
        return x;
    } else if constexpr (DT == HOFA_BF16) {
        return bf16_bits_to_f32(x);
    } else {
        return (float)__builtin_bit_cast(_Float16, x);
    }
}

template <int DT>
__device__ __forceinline__ typename Stor<DT>::type from_f32(float x) {
    if constexpr (DT == HOFA_F32) {
        return x;
    } else if constexpr (DT == HOFA_BF16) {
        return __builtin_bit_cast(uint16_t, (__bf16)x);  // round to nearest even
    } else {
        return __builtin_bit_cast(uint16_t, (_Float16)x);
    }
}

// Elements per 16-byte vector.
template <int DT> struct Vec { static constexpr int epv = 16 / sizeof(typename Stor<DT>::type); };

// Unpack one 16-byte vector into Vec<DT>::epv floats.
template <int DT>
__device__ __forceinline__ void unpack16(const u32x4 &w, float *out) {
    if constexpr (DT == HOFA_F32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(w[i]);
    } else if constexpr (DT == HOFA_BF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = __uint_as_float(w[i] << 16);
            out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu));
            out[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
        }
    }
}

// Scalar load of an element whose type is only known at run time (small
// per-head tensors: gates, scales, decays).
__device__ __forceinline__ float load_any(const void *p, int dtype, int64_t idx) {
    if (dtype == HOFA_F32) return ((const float *)p)[idx];
    uint16_t b = ((const uint16_t *)p)[idx];
    if (dtype == HOFA_BF16) return bf16_bits_to_f32(b);
    return (float)__builtin_bit_cast(_Float16, b);
}

// Scalar store with the element type chosen at run time (round to nearest even).
__device__ __forceinline__ void store_any(void *p, int dtype, int64_t idx, float x) {
    if (dtype == HOFA_F32) {
        ((float *)p)[idx] = x;
    } else if (dtype == HOFA_BF16) {
        ((uint16_t *)p)[idx] = __builtin_bit_cast(uint16_t, (__bf16)x);
    } else {
        ((uint16_t *)p)[idx] = __builtin_bit_cast(uint16_t, (_Float16)x);
    }
}

// ---------------------------------------------------------------- wave ops
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

// Lane value moved by a DPP control (GFX9 encoding): lanes whose source is
// outside the pattern, or whose row is not in ROW_MASK, read 0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_move(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, false));
}

// Inclusive prefix sum over the 64 lanes of a wave on the VALU (no LDS
// round trip): Hillis-Steele inside each row of 16 lanes (row_shr 1, 2, 4,
// 8; lanes shifted in from outside the row add 0), then row_bcast:15 adds
// row 0's total to row 1 and row 2's to row 3 (rows 1 and 3 enabled), and
// row_bcast:31 adds the total of rows 0-1 to rows 2-3.
__device__ __forceinline__ float wave_incl_scan(float x) {
    x += dpp_move<0x111>(x);        // row_shr:1
    x += dpp_move<0x112>(x);        // row_shr:2
    x += dpp_move<0x114>(x);        // row_shr:4
    x += dpp_move<0x118>(x);        // row_shr:8
    x += dpp_move<0x142, 0xa>(x);   // row_bcast:15
    x += dpp_move<0x143, 0xc>(x);   // row_bcast:31
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace hofa
