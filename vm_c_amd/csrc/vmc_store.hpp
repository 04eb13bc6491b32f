// vmc_store.hpp -- device pieces of the quantize-on-append kernels: the
// 16-lane (token, head) vector layout, the TurboQuant store of one vector
// (src/cuda/turboquant_kernels.cu:247-351) and the per-32-group variant's
// rotation and block quantizer (format in vmc_attn.h).
#pragma once

#include "vmc_common.hpp"
#include "vmc_tq.hpp"

namespace vmc {

// One 16-lane group per (token, kv head) vector; lane j owns dims 8j .. 8j+7
// (16 contiguous bytes of K and of V), a wave holds 4 vectors.
constexpr int kDims = 8;
constexpr int kGroup = 16;

template <bool BF16>
__device__ __forceinline__ void load8(const uint16_t* src, float* x) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(src);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        x[2 * e] = half_to_f32<BF16>((uint16_t)(w[e] & 0xffffu));
        x[2 * e + 1] = half_to_f32<BF16>((uint16_t)(w[e] >> 16));
    }
}

// Walsh-Hadamard butterflies of half-width 8 .. 64 across the group's lanes
// (partner j ^ m for m = 1, 2, 4, 8): the lane with bit m clear keeps a + b,
// its partner a - b, as in the sequential order
__device__ __forceinline__ void wht_lanes(float* y, int j) {
    static_for<4>([&](auto mi) {
        constexpr int M = 1 << decltype(mi)::value;
#pragma unroll
        for (int e = 0; e < kDims; ++e) {
            const float o = row_xor<M>(y[e], j);
            y[e] = (j & M) ? o - y[e] : y[e] + o;
        }
    });
}

// codes of this lane's 8 dims -> its bytes of the packed slot (dst 2-byte
// aligned).  4-bit: even d in the low nibble (:291), lane j's 4 bytes at 4j.
// 3-bit: 8 codes -> 3 bytes little endian, code i at bits 3i (:294-309);
// lanes 2i, 2i+1 form 6 bytes at 6i, written by the even lane.
template <int BITS>
__device__ __forceinline__ void store_codes8(const int* q, uint8_t* dst, int j) {
    uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
    if constexpr (BITS == 4) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) w |= (uint32_t)(q[i] & 0xf) << (4 * i);
        d16[2 * j] = (uint16_t)(w & 0xffffu);
        d16[2 * j + 1] = (uint16_t)(w >> 16);
    } else {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) w |= (uint32_t)(q[i] & 7) << (3 * i);
        const uint32_t hi = row_xor_u32<1>(w, j);
        if ((j & 1) == 0) {
            const uint64_t w48 = (uint64_t)w | ((uint64_t)hi << 24);
            d16[3 * (j >> 1) + 0] = (uint16_t)(w48 & 0xffff);
            d16[3 * (j >> 1) + 1] = (uint16_t)((w48 >> 16) & 0xffff);
            d16[3 * (j >> 1) + 2] = (uint16_t)((w48 >> 32) & 0xffff);
        }
    }
}

// V part of a TurboQuant slot (tq_store_mse_kernel :314-350, the same in
// half_to_fp8_store_kernel :228-244): asymmetric min/max over the whole
// vector, codes at vp, fp16/bf16 scale and zero at vp + val_data (+2)
template <int VB, bool BF16>
__device__ __forceinline__ void tq_store_v(const float* vv, int j, uint8_t* vp, bool write, int val_data) {
    int q[kDims];
    float y[kDims];
#pragma unroll
    for (int e = 0; e < kDims; ++e) y[e] = vv[e];
    float vmin = y[0], vmax = y[0];
#pragma unroll
    for (int e = 1; e < kDims; ++e) {
        vmin = fminf(vmin, y[e]);
        vmax = fmaxf(vmax, y[e]);
    }
    static_for<4>([&](auto m) {
        constexpr int M = 1 << decltype(m)::value;
        vmin = fminf(vmin, row_xor<M>(vmin, j));
        vmax = fmaxf(vmax, row_xor<M>(vmax, j));
    });
    constexpr int VMAXQ = VB == 4 ? 15 : 7;
    float vscale = (vmax - vmin) / (float)VMAXQ;
    vscale = fmaxf(vscale, 1e-8f);
#pragma unroll
    for (int e = 0; e < kDims; ++e) {
        int qq = (int)roundf((y[e] - vmin) / vscale);
        q[e] = qq < 0 ? 0 : (qq > VMAXQ ? VMAXQ : qq);
    }
    if (write) {
        store_codes8<VB>(q, vp, j);
        if (j == 0) {
            *reinterpret_cast<uint16_t*>(vp + val_data) = f32_to_half<BF16>(vscale);
            *reinterpret_cast<uint16_t*>(vp + val_data + 2) = f32_to_half<BF16>(vmin);
        }
    }
}

// The TurboQuant store of one (token, head) vector held by a 16-lane group,
// lane j owning dims 8j .. 8j+7 of K (y, overwritten) and V (vv):
// tq_store_mse_kernel (src/cuda/turboquant_kernels.cu:247-351) after the
// norm / normalize / rotation of :145-175, :841-848.  sq: this group's 128
// floats of LDS.  Writes only if write (the shuffles run in every lane).
template <int D, int KB, int VB, bool BF16>
__device__ __forceinline__ void tq_store_vec(float* y, float* vv, int j, uint8_t* sp, bool write,
                                             float* sq, const TQTables& tab, int mse_bytes,
                                             int key_packed, int val_data) {
    int q[kDims];
    // ---- K: norm by the reference's sequential fmaf chain over d = 0..D-1
    // (every lane of the group runs the same chain from LDS)
#pragma unroll
    for (int e = 0; e < kDims; ++e) sq[kDims * j + e] = y[e];
    // the group's 16 lanes are in one wave: a wave-level fence orders the
    // writes before the reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float nsq = 0.0f;
#pragma unroll
    for (int d = 0; d < D; d += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(&sq[d]);
#pragma unroll
        for (int e = 0; e < 4; ++e) nsq = __builtin_fmaf(v[e], v[e], nsq);
    }
    const float norm = sqrtf(nsq);
    const float inv = 1.0f / (norm + 1e-8f);
#pragma unroll
    for (int e = 0; e < kDims; ++e) y[e] = __fmul_rn(y[e], inv);
    // Walsh-Hadamard, half-widths 1, 2, 4 inside the lane, 8 .. 64 across lanes
    // (partner j ^ (h/8)); each butterfly is the same (a+b, a-b) as the
    // sequential order
#pragma unroll
    for (int hw = 1; hw < kDims; hw <<= 1)
#pragma unroll
        for (int i = 0; i < kDims; i += 2 * hw)
#pragma unroll
            for (int k = i; k < i + hw; ++k) {
                const float a = y[k], b = y[k + hw];
                y[k] = a + b;
                y[k + hw] = a - b;
            }
    wht_lanes(y, j);
    constexpr int NC = 1 << KB;
#pragma unroll
    for (int e = 0; e < kDims; ++e) {
        const float v = __fmul_rn(y[e], tab.rot_c);
        int idx = 0;
#pragma unroll
        for (int c = 0; c < NC - 1; ++c) idx += (v >= tab.midpoints[c]) ? 1 : 0;
        q[e] = idx;
    }
    // slot is uniform over the group, so the pair shuffle of the 3-bit packing
    // only reads lanes that take the same branch
    if (write) {
        store_codes8<KB>(q, sp, j);
        if (j == 0) *reinterpret_cast<uint16_t*>(sp + mse_bytes) = f32_to_half<BF16>(norm);
    }

    tq_store_v<VB, BF16>(vv, j, sp + key_packed, write, val_data);
}

// ---- per-32-group variant (no reference counterpart; format in vmc_attn.h)
// Same 16-lane ownership; lanes 4g .. 4g+3 hold group g (32 values).
// y = H (s x) / sqrt(128) in place: the sign flip, the butterflies of the
// reference-order rotation above, one multiply by rot_c
__device__ __forceinline__ void g32_rotate(float* y, int j, uint32_t sbits, float rot_c) {
#pragma unroll
    for (int e = 0; e < kDims; ++e) y[e] = ((sbits >> e) & 1) ? -y[e] : y[e];
#pragma unroll
    for (int hw = 1; hw < kDims; hw <<= 1)
#pragma unroll
        for (int i = 0; i < kDims; i += 2 * hw)
#pragma unroll
            for (int k = i; k < i + hw; ++k) {
                const float a = y[k], b = y[k + hw];
                y[k] = a + b;
                y[k + hw] = a - b;
            }
    wht_lanes(y, j);
#pragma unroll
    for (int e = 0; e < kDims; ++e) y[e] = __fmul_rn(y[e], rot_c);
}

// one part (K or V) of the slot: four 32-value blocks at dst
template <int BITS>
__device__ __forceinline__ void g32_quantize(const float* y, int j, uint8_t* dst, bool write) {
    const int l = j & 3;  // lane within the group, values 8l .. 8l+7 of it
    int q[kDims];
    if constexpr (BITS == 4) {
        float mn = y[0], mx = y[0];
#pragma unroll
        for (int e = 1; e < kDims; ++e) {
            mn = fminf(mn, y[e]);
            mx = fmaxf(mx, y[e]);
        }
        mn = fminf(mn, row_xor<1>(mn, j));
        mx = fmaxf(mx, row_xor<1>(mx, j));
        mn = fminf(mn, row_xor<2>(mn, j));
        mx = fmaxf(mx, row_xor<2>(mx, j));
        const float d = (mx - mn) / 15.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
        for (int e = 0; e < kDims; ++e) {
            float t = y[e] - mn;
            t = t * id;
            t = t + 0.5f;
            const int c = (int)t;
            q[e] = c > 15 ? 15 : c;
        }
        // byte i of the 16 = value i (lanes 0, 1) | value i + 16 << 4 (lanes 2, 3)
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lo |= (uint32_t)q[e] << (8 * e);
            hi |= (uint32_t)q[e + 4] << (8 * e);
        }
        const uint32_t plo = row_xor_u32<2>(lo, j);
        const uint32_t phi = row_xor_u32<2>(hi, j);
        if (write) {
            uint8_t* blk = dst + 20 * (j >> 2);
            if (l == 0)
                *reinterpret_cast<uint32_t*>(blk) =
                    (uint32_t)f32_to_f16_bits(d) | ((uint32_t)f32_to_f16_bits(mn) << 16);
            if (l < 2) {
                uint32_t* qs = reinterpret_cast<uint32_t*>(blk + 4 + 8 * l);
                qs[0] = lo | (plo << 4);
                qs[1] = hi | (phi << 4);
            }
        }
    } else {
        // first value of largest magnitude: (|y|, index) with ties to the lower index
        float amax = 0.0f, v = 0.0f;
        int idx = 1 << 20;
#pragma unroll
        for (int e = 0; e < kDims; ++e) {
            const float a = fabsf(y[e]);
            if (a > amax) {
                amax = a;
                v = y[e];
                idx = 8 * l + e;
            }
        }
        static_for<2>([&](auto m) {
            constexpr int M = 1 << decltype(m)::value;
            const float a2 = row_xor<M>(amax, j);
            const float v2 = row_xor<M>(v, j);
            const int i2 = row_xor<M>(idx, j);
            if (a2 > amax || (a2 == amax && i2 < idx)) {
                amax = a2;
                v = v2;
                idx = i2;
            }
        });
        const float d = v / -4.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < kDims; ++e) {
            float t = y[e] * id;
            t = t + 4.5f;
            const int c = (int)t;
            w |= (uint32_t)(c > 7 ? 7 : c) << (3 * e);
        }
        // lanes 2i, 2i+1 of the group: 6 bytes at 2 + 6i, written by the even lane
        const uint32_t hiw = row_xor_u32<1>(w, j);
        if (write) {
            uint8_t* blk = dst + 14 * (j >> 2);
            uint16_t* d16 = reinterpret_cast<uint16_t*>(blk);
            if (l == 0) d16[0] = f32_to_f16_bits(d);
            if ((l & 1) == 0) {
                const uint64_t w48 = (uint64_t)w | ((uint64_t)hiw << 24);
                uint16_t* p = reinterpret_cast<uint16_t*>(blk + 2 + 3 * l);
                p[0] = (uint16_t)(w48 & 0xffff);
                p[1] = (uint16_t)((w48 >> 16) & 0xffff);
                p[2] = (uint16_t)((w48 >> 32) & 0xffff);
            }
        }
    }
}

// float_to_fp8_e4m3 / _e4b15 (src/cuda/turboquant_kernels.cu:47-83, :98-134),
// operation for operation: exponent bias 7 or 15, the mantissa taken as
// (m + 2^18) >> 19 with a carry into the exponent when it exceeds 7,
// exponent 255 -> 0x7C / 0x78, overflow -> 0x7F, values below the smallest
// normal -> exponent field 1 with mantissa min(7, ((1.m >> shift) + 4) >> 4)
__device__ __forceinline__ uint32_t fp8_encode(float v, int e4b15) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, v);
    const uint32_t sign = (bits >> 31) & 1u;
    const int exp_f32 = (int)((bits >> 23) & 0xffu);
    const uint32_t mant_f32 = bits & 0x7fffffu;
    if (exp_f32 == 0 && mant_f32 == 0) return sign << 7;
    if (exp_f32 == 255) return (sign << 7) | (e4b15 ? 0x78u : 0x7Cu);
    int e = exp_f32 - 127 + (e4b15 ? 15 : 7);
    if (e < 1) {
        const int shift = 1 - e;
        if (shift > 24) return sign << 7;
        const uint32_t mant = (0x800000u | mant_f32) >> shift;
        uint32_t m8 = (mant + 4) >> 4;
        if (m8 > 7) m8 = 7;
        return (sign << 7) | (1u << 3) | m8;
    }
    if (e > 15) return (sign << 7) | 0x7Fu;
    uint32_t m8 = (mant_f32 + 0x40000u) >> 19;
    if (m8 > 7) {
        m8 = 0;
        ++e;
        if (e > 15) return (sign << 7) | 0x7Fu;
    }
    return (sign << 7) | ((uint32_t)(e & 0xf) << 3) | (m8 & 7u);
}

// turboquant_k8v4 slot of one (token, head) vector (half_to_fp8_store_kernel,
// turboquant_kernels.cu:188-245): K byte d = fp8(k[d]) at sp + d (lane j:
// bytes 8j .. 8j+7; slots are 196 bytes, so 4-byte aligned), then the V part
template <bool BF16>
__device__ __forceinline__ void k8v4_store_vec(const float* k, const float* vv, int j, uint8_t* sp, bool write,
                                               int e4b15) {
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        w0 |= fp8_encode(k[e], e4b15) << (8 * e);
        w1 |= fp8_encode(k[4 + e], e4b15) << (8 * e);
    }
    if (write) {
        uint32_t* d = reinterpret_cast<uint32_t*>(sp + 8 * j);
        d[0] = w0;
        d[1] = w1;
    }
    tq_store_v<4, BF16>(vv, j, sp + 128, write, 64);
}

}  // namespace vmc
