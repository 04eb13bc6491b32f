// vmc_common.hpp -- shared device helpers for the gfx950 attention kernels.
//
// Wave64 only.  MFMA operand layouts used throughout (16x16 tiles, kpl = values
// per lane, 4 for the x16 shapes and 8 for the gfx950 x32 shapes):
//   A[i][k] : lane l holds row i = l % 16, k = kpl*(l / 16) .. + kpl-1
//   B[k][j] : lane l holds col j = l % 16, k = kpl*(l / 16) .. + kpl-1
//   D[i][j] : lane l holds col j = l % 16, rows i = 4*(l / 16) .. + 3
// (checked on the device by the MFMA layout self-test, vmc_selftest_mfma).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "vmc_attn.h"

namespace vmc {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- numerics
// float -> fp16 / bf16 bits, round-to-nearest-even (v_cvt_f16_f32 in the
// default rounding mode; bf16 by integer rounding so NaN stays quiet).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}
template <bool BF16>
__device__ __forceinline__ float half_to_f32(uint16_t b) {
    if constexpr (BF16) return bf16_bits_to_f32(b);
    else return f16_bits_to_f32(b);
}
template <bool BF16>
__device__ __forceinline__ uint16_t f32_to_half(float f) {
    if constexpr (BF16) return f32_to_bf16_bits(f);
    else return f32_to_f16_bits(f);
}

// ---------------------------------------------------------------- wave ops
__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ float shfl(float v, int src) { return __shfl(v, src, kWave); }

// sum / max over the four 16-lane groups that share l % 16
__device__ __forceinline__ float sum_over_groups(float v) {
    v += shfl_xor(v, 16);
    v += shfl_xor(v, 32);
    return v;
}
__device__ __forceinline__ float max_over_groups(float v) {
    v = fmaxf(v, shfl_xor(v, 16));
    v = fmaxf(v, shfl_xor(v, 32));
    return v;
}

// ---------------------------------------------------------------- MFMA
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x16(f16x4 a, f16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x16(s16x4 a, s16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- misc
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return (uint32_t)*reinterpret_cast<const uint16_t*>(p);
}

}  // namespace vmc

// host-side launch error check: returns VMC_EIO from the enclosing function
#define VMC_LAUNCH_CHECK()                                       \
    do {                                                         \
        hipError_t e_ = hipGetLastError();                       \
        if (e_ != hipSuccess) return VMC_EIO;                    \
    } while (0)
