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
// round to nearest even; a NaN keeps its sign and upper payload with the
// quiet bit set ((x >> 16) | 0x40).  v_cvt_pk_bf16_f32 does both in one
// instruction; f32_to_bf16_bits_int is the same rule in integer arithmetic
// (the device self-test compares the two).
__device__ __forceinline__ uint16_t f32_to_bf16_bits_int(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
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

// 16-lane row exchanges by DPP (one VALU op, no LDS).  row_xor<M>: the value
// of lane l ^ M of the same 16-lane row (M = 1, 2: quad_perm; 8: row_ror:8;
// 4: row_shl:4 / row_shr:4 selected by lane bit 2).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
template <int M>
__device__ __forceinline__ uint32_t row_xor_u32(uint32_t v, int lane) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8, "xor distance within a 16-lane row");
    if constexpr (M == 1) return dpp_u32<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    else if constexpr (M == 2) return dpp_u32<0x4E>(v);  // quad_perm [2, 3, 0, 1]
    else if constexpr (M == 8) return dpp_u32<0x128>(v);  // row_ror:8
    else {
        const uint32_t up = dpp_u32<0x104>(v);    // row_shl:4: lane l + 4
        const uint32_t down = dpp_u32<0x114>(v);  // row_shr:4: lane l - 4
        return (lane & 4) ? down : up;
    }
}
template <int M>
__device__ __forceinline__ float row_xor(float v, int lane) {
    return __builtin_bit_cast(float, row_xor_u32<M>(__builtin_bit_cast(uint32_t, v), lane));
}
template <int M>
__device__ __forceinline__ int row_xor(int v, int lane) {
    return (int)row_xor_u32<M>((uint32_t)v, lane);
}
// Sum over a 16-lane row, every lane gets the same value: the butterfly
// s += s[l ^ 1], s += s[l ^ 2], s += s[l ^ 4], s += s[l ^ 8].  The last two
// steps read the mirrored lane (7 - l within 8, 15 - l within 16): after the
// steps before, it holds the same value as lane l ^ 4 (l ^ 8), so the sums
// are the butterfly's, bit for bit.
__device__ __forceinline__ float row_sum16(float s) {
    s = s + __builtin_bit_cast(float, dpp_u32<0xB1>(__builtin_bit_cast(uint32_t, s)));
    s = s + __builtin_bit_cast(float, dpp_u32<0x4E>(__builtin_bit_cast(uint32_t, s)));
    s = s + __builtin_bit_cast(float, dpp_u32<0x141>(__builtin_bit_cast(uint32_t, s)));  // row_half_mirror
    s = s + __builtin_bit_cast(float, dpp_u32<0x140>(__builtin_bit_cast(uint32_t, s)));  // row_mirror
    return s;
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
