// kv_quant.hpp -- GGUF block encoders shared by the append and prefill
// kernels, and the block decoders shared by the decode and prefill kernels.
//
// encode_q8_0: ggml/src/ggml-quants.c:234-257 (quantize_row_q8_0_ref)
//   d = amax/127, id = d ? 1/d : 0, q = roundf(x*id), d stored as fp16.
// encode_q4_0: ggml/src/ggml-quants.c:71-104 (quantize_row_q4_0_ref)
//   max = signed value of the largest |x| (first wins), d = max/-8,
//   q = min(15, (int8_t)(x*id + 8.5f)) with x*id rounded before the add,
//   byte j = q[j] | q[j+16] << 4.
// Both write through 16-bit stores (entries are 2-byte aligned).
#pragma once

#include "vmc_common.hpp"

namespace vmc {

constexpr int kQK = 32;

// Materialise x in a VGPR.  Without it the compiler folds
// fp16(x * c) into v_fma_mix(x, c, +0), which turns a -0.0 product into +0.0
// (ggml stores d = -0.0 for an all-zero q4_0 block: 0.0f / -8).
__device__ __forceinline__ float opaque(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ void encode_q8_0(const float* x, uint8_t* dst) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < kQK; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = opaque(amax / 127.0f);
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
    d16[0] = f32_to_f16_bits(d);
#pragma unroll
    for (int j = 0; j < kQK; j += 2) {
        const int q0 = (int)roundf(x[j] * id);
        const int q1 = (int)roundf(x[j + 1] * id);
        d16[1 + j / 2] = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
    }
}

__device__ __forceinline__ void encode_q4_0(const float* x, uint8_t* dst) {
    float amax = 0.0f, mx = 0.0f;
#pragma unroll
    for (int j = 0; j < kQK; ++j) {
        const float a = fabsf(x[j]);
        if (amax < a) {
            amax = a;
            mx = x[j];
        }
    }
    const float d = opaque(mx / -8.0f);
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
    d16[0] = f32_to_f16_bits(d);
    uint32_t q[kQK / 2];
#pragma unroll
    for (int j = 0; j < kQK / 2; ++j) {
        const float x0 = __fmul_rn(x[j], id);
        const float x1 = __fmul_rn(x[j + kQK / 2], id);
        const int t0 = (int)(int8_t)(int)__fadd_rn(x0, 8.5f);
        const int t1 = (int)(int8_t)(int)__fadd_rn(x1, 8.5f);
        q[j] = (uint32_t)(t0 < 15 ? t0 : 15) | ((uint32_t)(t1 < 15 ? t1 : 15) << 4);
    }
#pragma unroll
    for (int j = 0; j < kQK / 2; j += 2) d16[1 + j / 2] = (uint16_t)(q[j] | (q[j + 1] << 8));
}

template <bool SRC_BF16>
__device__ __forceinline__ void load_block32(const uint16_t* src, float* x) {
    const u32x4* p = reinterpret_cast<const u32x4*>(src);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const u32x4 w = p[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[c * 8 + 2 * e] = half_to_f32<SRC_BF16>((uint16_t)(w[e] & 0xffffu));
            x[c * 8 + 2 * e + 1] = half_to_f32<SRC_BF16>((uint16_t)(w[e] >> 16));
        }
    }
}

// One 32-value block of a (token, head) row into its page entry, any format.
template <int FMT, bool SRC_BF16>
__device__ __forceinline__ void append_block32(const uint16_t* src, uint8_t* entry, int ib) {
    if constexpr (FMT == VMC_KV_F16 || FMT == VMC_KV_BF16) {
        constexpr bool DST_BF16 = FMT == VMC_KV_BF16;
        const u32x4* s = reinterpret_cast<const u32x4*>(src);
        u32x4* o = reinterpret_cast<u32x4*>(entry + ib * kQK * 2);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            u32x4 w = s[c];
            if constexpr (DST_BF16 != SRC_BF16) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float lo = half_to_f32<SRC_BF16>((uint16_t)(w[e] & 0xffffu));
                    const float hi = half_to_f32<SRC_BF16>((uint16_t)(w[e] >> 16));
                    w[e] = (uint32_t)f32_to_half<DST_BF16>(lo) |
                           ((uint32_t)f32_to_half<DST_BF16>(hi) << 16);
                }
            }
            o[c] = w;
        }
    } else {
        float x[kQK];
        load_block32<SRC_BF16>(src, x);
        if constexpr (FMT == VMC_KV_Q8_0) encode_q8_0(x, entry + ib * 34);
        else encode_q4_0(x, entry + ib * 18);
    }
}

__device__ __forceinline__ int64_t kv_entry_offset(int64_t slot, int h, int64_t bs, int Hkv,
                                                   int64_t E, int64_t stride, bool hnd) {
    const int64_t blk = slot / bs, off = slot % bs;
    return hnd ? blk * stride + (int64_t)h * bs * E + off * E
               : blk * stride + off * Hkv * E + (int64_t)h * E;
}

// Two GGUF values -> packed fp16 x * d, bit-identical to fp16(float(x) * d):
// x * d is exact in fp32 (8-bit x, 11-bit d), and v_pk_mul_f16 rounds the
// exact product once, as the conversion does.  x enters as fp16 exactly: the
// two bytes spread into the 16-bit halves, then 0x64 in the high byte makes
// 1024 + low byte; q8_0 flips the sign bit first (1024 + x + 128 - 1152 = x),
// q4_0 takes a nibble (1024 + u - 1032 = u - 8).
__device__ __forceinline__ uint32_t q8_pair_f16(uint32_t w16, f16x2 d2) {
    const uint32_t t = __builtin_amdgcn_perm(0u, w16, 0x0c010c00u) ^ 0x64806480u;
    const f16x2 x = __builtin_bit_cast(f16x2, t) - f16x2{(_Float16)1152.0f, (_Float16)1152.0f};
    return __builtin_bit_cast(uint32_t, x * d2);
}
__device__ __forceinline__ uint32_t q4_pair_f16(uint32_t w16, int sh, f16x2 d2) {
    const uint32_t t = ((__builtin_amdgcn_perm(0u, w16, 0x0c010c00u) >> sh) & 0x000f000fu) | 0x64006400u;
    const f16x2 x = __builtin_bit_cast(f16x2, t) - f16x2{(_Float16)1032.0f, (_Float16)1032.0f};
    return __builtin_bit_cast(uint32_t, x * d2);
}

// fp16 bits of one of the reference's fp8 key codes (low byte of b):
// e4m3 (1 + m/8) 2^(e-7) -> exponent field e + 8; e4b15 (1 + m/8) 2^(e-15)
// -> exponent field e, or for e = 0 the fp16 subnormal (8 + m) 2^-18; the
// zero code (either sign) -> signed zero.  Exact.
__device__ __forceinline__ uint16_t fp8_f16_bits(uint32_t b, int e4b15) {
    const uint32_t mag = b & 0x7fu, m = b & 7u;
    const uint32_t h = !e4b15 ? (mag ? (mag << 7) + 0x2000u : 0u)
                              : ((mag >> 3) ? (mag << 7) : (m ? 0x200u + (m << 6) : 0u));
    return (uint16_t)(h | ((b & 0x80u) << 8));
}

}  // namespace vmc
