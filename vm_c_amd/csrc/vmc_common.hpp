// vmc_common.hpp -- shared device helpers for the gfx950 attention kernels.
//
// Wave64 only.  MFMA operand layouts used throughout (16x16 tiles, kpl = values
// per lane, 4 for the x16 shapes and 8 for the gfx950 x32 shapes):
//   A[i][k] : lane l holds row i = l % 16, k = kpl*(l / 16) .. + kpl-1
//   B[k][j] : lane l holds col j = l % 16, k = kpl*(l / 16) .. + kpl-1
//   D[i][j] : lane l holds col j = l % 16, rows i = 4*(l / 16) .. + 3
// (checked on the device by the layout self-test, vmc_selftest).
#pragma once

#include <utility>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "vmc_attn.h"

namespace vmc {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
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

// ---------------------------------------------------------------- unrolling
// f(integral_constant<int, 0>{}) .. f(integral_constant<int, N - 1>{})
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// ---------------------------------------------------------------- wave ops
__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ float shfl(float v, int src) { return __shfl(v, src, kWave); }

// sum / max over the four 16-lane rows that share l % 16, with the gfx950
// row-swap instructions (no LDS traffic): v_permlane16_swap exchanges rows
// 1 <-> 0 and 3 <-> 2 between its two operands, v_permlane32_swap the two
// halves; combining both results of each swap reduces over the pair.
// The second operand is a copy the compiler cannot see through: given two
// provably equal operands it treats both results as equal and drops one.
__device__ __forceinline__ void swap_pair16(uint32_t& a, uint32_t& b) {
    asm volatile("" : "+v"(b));
    auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
__device__ __forceinline__ void swap_pair32(uint32_t& a, uint32_t& b) {
    asm volatile("" : "+v"(b));
    auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
__device__ __forceinline__ float sum_over_groups(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    swap_pair16(a, b);
    v = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
    a = __builtin_bit_cast(uint32_t, v);
    b = a;
    swap_pair32(a, b);
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float max_over_groups(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    swap_pair16(a, b);
    v = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    a = __builtin_bit_cast(uint32_t, v);
    b = a;
    swap_pair32(a, b);
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

// Wave-private LDS exchange: lanes of row 0 publish v[l % 16]; every lane
// reads back the four values v[4*(l/16) .. +3] (one 16-byte LDS read).
__device__ __forceinline__ f32x4 gather4_from_row0(float v, float* sc, int r16, int grp) {
    if (grp == 0) sc[r16] = v;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const f32x4 r = *reinterpret_cast<const f32x4*>(sc + 4 * grp);
    __builtin_amdgcn_wave_barrier();
    return r;
}

// Wave-private LDS exchange from the diagonal of a 16x16 D-layout tile: the
// lane holding row r16 of column r16 (grp == r16 / 4) publishes v for row
// r16; every lane reads back rows 4*grp .. +3 (one 16-byte LDS read).
__device__ __forceinline__ f32x4 gather4_from_diag(float v, float* sc, int r16, int grp) {
    if ((r16 >> 2) == grp) sc[r16] = v;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const f32x4 r = *reinterpret_cast<const f32x4*>(sc + 4 * grp);
    __builtin_amdgcn_wave_barrier();
    return r;
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
