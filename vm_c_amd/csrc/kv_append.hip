// kv_append.hip -- quantize-on-append of K/V rows into the paged cache.
//
// Replaces vm_c::reshape_and_cache (src/cuda/cache_kernels.cu:14-54, :88-157).
// Page addressing is the reference's (NHD: blk*stride + off*Hkv*E + h*E, HND:
// blk*stride + h*bs*E + off*E, cache_kernels.cu:33-40) with E the entry bytes
// of the format.  q8_0 / q4_0 entries are head_dim/32 GGUF blocks encoded
// exactly as ggml's quantize_row_q8_0_ref / quantize_row_q4_0_ref
// (ggml/src/ggml-quants.c:234-257, :71-104) -- the encoder ggml's set_rows
// uses for a q8_0 / q4_0 KV cache.
//
// One thread per (token, head, 32-value block) for K and V: a block is two
// 16-byte loads of contiguous fp16, so a wave reads 2 KB of consecutive rows.
#include "kv_quant.hpp"

namespace vmc {
namespace {

constexpr int QK = kQK;

template <int FMT, bool SRC_BF16, bool HND>
__global__ void __launch_bounds__(256)
reshape_and_cache_kernel(const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
                         uint8_t* __restrict__ key_cache, uint8_t* __restrict__ value_cache,
                         const int64_t* __restrict__ slot_mapping, int num_tokens, int Hkv,
                         int D, int64_t bs, int64_t stride, int64_t E) {
    // work item = (tensor k/v, token, head, block of 32)
    const int nb = D / QK;
    const int64_t per_tensor = (int64_t)num_tokens * Hkv * nb;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= 2 * per_tensor) return;
    const int is_v = idx >= per_tensor;
    const int64_t r = is_v ? idx - per_tensor : idx;
    const int ib = (int)(r % nb);
    const int h = (int)((r / nb) % Hkv);
    const int64_t t = r / ((int64_t)nb * Hkv);
    const int64_t slot = slot_mapping[t];
    if (slot < 0) return;  // cache_kernels.cu:26
    const int64_t blk = slot / bs, off = slot % bs;
    const int64_t ent = HND ? blk * stride + (int64_t)h * bs * E + off * E
                            : blk * stride + off * Hkv * E + (int64_t)h * E;
    const uint16_t* src = (is_v ? value : key) + (t * Hkv + h) * D + ib * QK;
    append_block32<FMT, SRC_BF16>(src, (is_v ? value_cache : key_cache) + ent, ib);
}

// OCP 8-bit float from fp32 (OFP8 v1.0; E4M3: 3 mantissa bits, bias 7, max
// 448 = 0x7e; E5M2: 2, 15, 57344 = 0x7b): round to nearest even, |x| >= max
// (infinities included) saturated to the largest finite code, NaN to 0x7f.
// Integer arithmetic on the fp32 bits.
template <bool E5M2>
__device__ __forceinline__ uint32_t f32_to_ofp8(float x) {
    constexpr int M = E5M2 ? 2 : 3, B = E5M2 ? 15 : 7;
    constexpr uint32_t maxc = E5M2 ? 0x7bu : 0x7eu;
    constexpr uint32_t maxbits = E5M2 ? 0x47600000u : 0x43e00000u;  // 57344.0f, 448.0f
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const uint32_t s = (u >> 24) & 0x80u, a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7fu;
    if (a >= maxbits) return s | maxc;
    const int E = (int)(a >> 23) - 127;
    if (E >= 1 - B) {  // normal: M mantissa bits, a carry moves into the exponent
        constexpr int sh = 23 - M;
        const uint32_t man = a & 0x7fffffu;
        const uint32_t q = man >> sh, rem = man & ((1u << sh) - 1u);
        const uint32_t up = (rem > (1u << (sh - 1))) || (rem == (1u << (sh - 1)) && (q & 1u));
        return s | (((uint32_t)(E + B) << M) + q + up);
    }
    if (a < 0x00800000u) return s;  // zero, fp32 subnormals
    const int sh = 24 - B - M - E;  // subnormal: (value / 2^(1 - B - M)) = significand >> sh
    if (sh >= 32) return s;
    const uint32_t sig = (a & 0x7fffffu) | 0x800000u;
    const uint32_t q = sig >> sh, rem = sig & ((1u << sh) - 1u), half = 1u << (sh - 1);
    return s | (q + ((rem > half) || (rem == half && (q & 1u))));
}

// fp8 pages: one thread per (tensor, token, head, 16 values): two 16-byte
// loads, E4M3 of x / scale (cache_kernels.cu:43-46: the reference casts to
// __nv_fp8_e4m3 for "fp8_e4m3" and "fp8_e5m2" alike), one 16-byte store
template <bool SRC_BF16, bool HND>
__global__ void __launch_bounds__(256)
reshape_and_cache_fp8_kernel(const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
                             uint8_t* __restrict__ key_cache, uint8_t* __restrict__ value_cache,
                             const int64_t* __restrict__ slot_mapping, int num_tokens, int Hkv, int D,
                             int64_t bs, int64_t stride, float k_scale, float v_scale) {
    const int nc = D / 16;
    const int64_t per_tensor = (int64_t)num_tokens * Hkv * nc;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= 2 * per_tensor) return;
    const int is_v = idx >= per_tensor;
    const int64_t r = is_v ? idx - per_tensor : idx;
    const int ic = (int)(r % nc);
    const int h = (int)((r / nc) % Hkv);
    const int64_t t = r / ((int64_t)nc * Hkv);
    const int64_t slot = slot_mapping[t];
    if (slot < 0) return;  // cache_kernels.cu:26
    const int64_t blk = slot / bs, off = slot % bs;
    // cache_kernels.cu:36-40
    const int64_t ent = HND ? blk * stride + (int64_t)h * bs * D + off * D
                            : blk * stride + off * Hkv * D + (int64_t)h * D;
    const u32x4* src = reinterpret_cast<const u32x4*>((is_v ? value : key) + (t * Hkv + h) * D + ic * 16);
    const float sc = is_v ? v_scale : k_scale;
    const u32x4 w0 = src[0], w1 = src[1];
    u32x4 o;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const u32x4& w = d < 2 ? w0 : w1;
        uint32_t b = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t half = (w[(d & 1) * 2 + (e >> 1)] >> (16 * (e & 1))) & 0xffffu;
            b |= f32_to_ofp8<false>(half_to_f32<SRC_BF16>((uint16_t)half) / sc) << (8 * e);
        }
        o[d] = b;
    }
    *reinterpret_cast<u32x4*>((is_v ? value_cache : key_cache) + ent + ic * 16) = o;
}

// convert_fp8: dst[i] = fp8(src[i] * scale), 16 values per thread (a
// shorter run at the end, or one value per thread when a pointer is not
// 16-byte aligned)
template <bool SRC_BF16, bool E5M2, bool VEC>
__global__ void __launch_bounds__(256)
convert_fp8_kernel(uint8_t* __restrict__ dst, const uint16_t* __restrict__ src, float scale, int64_t n) {
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * (VEC ? 16 : 1);
    if (i0 >= n) return;
    if (VEC && i0 + 16 <= n) {
        const u32x4 w0 = reinterpret_cast<const u32x4*>(src + i0)[0], w1 = reinterpret_cast<const u32x4*>(src + i0)[1];
        u32x4 o;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const u32x4& w = d < 2 ? w0 : w1;
            uint32_t b = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t half = (w[(d & 1) * 2 + (e >> 1)] >> (16 * (e & 1))) & 0xffffu;
                b |= f32_to_ofp8<E5M2>(half_to_f32<SRC_BF16>((uint16_t)half) * scale) << (8 * e);  // cache_kernels.cu:183-184
            }
            o[d] = b;
        }
        *reinterpret_cast<u32x4*>(dst + i0) = o;
        return;
    }
    const int64_t i1 = VEC ? n : i0 + 1;
    for (int64_t i = i0; i < i1; ++i) dst[i] = (uint8_t)f32_to_ofp8<E5M2>(half_to_f32<SRC_BF16>(src[i]) * scale);
}

template <int FMT, bool SRC_BF16>
int launch_append(const void* key, const void* value, void* kc, void* vc, const int64_t* slots,
                  int T, int Hkv, int D, int64_t bs, int64_t stride, int64_t E, bool hnd,
                  hipStream_t stream) {
    const int64_t work = 2LL * T * Hkv * (D / QK);
    const int threads = 256;
    const int64_t grid = (work + threads - 1) / threads;
    if (grid == 0) return VMC_OK;
    if (hnd)
        hipLaunchKernelGGL((reshape_and_cache_kernel<FMT, SRC_BF16, true>), dim3((unsigned)grid),
                           dim3(threads), 0, stream, (const uint16_t*)key, (const uint16_t*)value,
                           (uint8_t*)kc, (uint8_t*)vc, slots, T, Hkv, D, bs, stride, E);
    else
        hipLaunchKernelGGL((reshape_and_cache_kernel<FMT, SRC_BF16, false>), dim3((unsigned)grid),
                           dim3(threads), 0, stream, (const uint16_t*)key, (const uint16_t*)value,
                           (uint8_t*)kc, (uint8_t*)vc, slots, T, Hkv, D, bs, stride, E);
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}

}  // namespace
}  // namespace vmc

using namespace vmc;

extern "C" int64_t vmc_kv_entry_bytes(int kv_format, int head_dim) {
    if (head_dim <= 0 || head_dim % 32 != 0) return -1;
    switch (kv_format) {
        case VMC_KV_F16:
        case VMC_KV_BF16: return (int64_t)head_dim * 2;
        case VMC_KV_Q8_0: return (int64_t)(head_dim / 32) * 34;
        case VMC_KV_Q4_0: return (int64_t)(head_dim / 32) * 18;
        default: return -1;
    }
}

extern "C" int vmc_reshape_and_cache(const void* key, const void* value, void* key_cache,
                                     void* value_cache, const int64_t* slot_mapping,
                                     int num_tokens, int num_kv_heads, int head_dim,
                                     int64_t block_size, int64_t cache_stride, int kv_format,
                                     int src_dtype, int layout, vmc_stream_t stream) {
    const int64_t E = vmc_kv_entry_bytes(kv_format, head_dim);
    if (E < 0 || num_tokens < 0 || num_kv_heads <= 0 || block_size <= 0) return VMC_EINVAL;
    if (src_dtype != VMC_DTYPE_F16 && src_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (layout != VMC_LAYOUT_NHD && layout != VMC_LAYOUT_HND) return VMC_EINVAL;
    if (num_tokens == 0) return VMC_OK;
    if (!key || !value || !key_cache || !value_cache || !slot_mapping) return VMC_EINVAL;
    const int64_t stride = cache_stride > 0 ? cache_stride : block_size * num_kv_heads * E;
    if (stride < block_size * num_kv_heads * E) return VMC_EINVAL;
    if ((kv_format == VMC_KV_F16 || kv_format == VMC_KV_BF16) && (stride % 16) != 0) return VMC_EINVAL;
    const bool hnd = layout == VMC_LAYOUT_HND;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool sb = src_dtype == VMC_DTYPE_BF16;
#define VMC_APPEND_CASE(F)                                                                        \
    case F:                                                                                       \
        return sb ? launch_append<F, true>(key, value, key_cache, value_cache, slot_mapping,      \
                                           num_tokens, num_kv_heads, head_dim, block_size,        \
                                           stride, E, hnd, s)                                     \
                  : launch_append<F, false>(key, value, key_cache, value_cache, slot_mapping,     \
                                            num_tokens, num_kv_heads, head_dim, block_size,       \
                                            stride, E, hnd, s);
    switch (kv_format) {
        VMC_APPEND_CASE(VMC_KV_F16)
        VMC_APPEND_CASE(VMC_KV_BF16)
        VMC_APPEND_CASE(VMC_KV_Q8_0)
        VMC_APPEND_CASE(VMC_KV_Q4_0)
        default: return VMC_EINVAL;
    }
#undef VMC_APPEND_CASE
}

extern "C" int vmc_reshape_and_cache_fp8(const void* key, const void* value, void* key_cache, void* value_cache,
                                         const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                                         int head_dim, int64_t block_size, int64_t cache_stride,
                                         const float* k_scale, const float* v_scale, int src_dtype, int layout,
                                         vmc_stream_t stream) {
    if (num_tokens < 0 || num_kv_heads <= 0 || block_size <= 0 || head_dim <= 0 || head_dim % 16 != 0)
        return VMC_EINVAL;
    if (src_dtype != VMC_DTYPE_F16 && src_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (layout != VMC_LAYOUT_NHD && layout != VMC_LAYOUT_HND) return VMC_EINVAL;
    if (num_tokens == 0) return VMC_OK;
    if (!key || !value || !key_cache || !value_cache || !slot_mapping) return VMC_EINVAL;
    const int64_t min_stride = block_size * num_kv_heads * head_dim;
    const int64_t stride = cache_stride > 0 ? cache_stride : min_stride;
    if (stride < min_stride || stride % 16 != 0) return VMC_EINVAL;
    if ((((uintptr_t)key | (uintptr_t)value | (uintptr_t)key_cache | (uintptr_t)value_cache) & 15) != 0)
        return VMC_EINVAL;
    // the scales are host floats, read here (cache_kernels.cu:103-104); none = 1
    const float ks = k_scale ? *k_scale : 1.0f, vs = v_scale ? *v_scale : 1.0f;
    const int64_t work = 2LL * num_tokens * num_kv_heads * (head_dim / 16);
    const int64_t grid = (work + 255) / 256;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool sb = src_dtype == VMC_DTYPE_BF16, hnd = layout == VMC_LAYOUT_HND;
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), 0, s, (const uint16_t*)key, (const uint16_t*)value,
                           (uint8_t*)key_cache, (uint8_t*)value_cache, slot_mapping, num_tokens, num_kv_heads,
                           head_dim, block_size, stride, ks, vs);
    };
    if (sb) hnd ? go(reshape_and_cache_fp8_kernel<true, true>) : go(reshape_and_cache_fp8_kernel<true, false>);
    else hnd ? go(reshape_and_cache_fp8_kernel<false, true>) : go(reshape_and_cache_fp8_kernel<false, false>);
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}

extern "C" int vmc_convert_fp8(void* dst_cache, const void* src_cache, double scale, int64_t num_elements,
                               int e5m2, int src_dtype, vmc_stream_t stream) {
    if (num_elements < 0) return VMC_EINVAL;
    if (num_elements == 0) return VMC_OK;  // cache_kernels.cu:193
    if (!dst_cache || !src_cache) return VMC_EINVAL;
    if (src_dtype != VMC_DTYPE_F16 && src_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    const float sc = (float)scale;  // cache_kernels.cu:195
    const bool vec = (((uintptr_t)dst_cache | (uintptr_t)src_cache) & 15) == 0;
    const int64_t threads = vec ? (num_elements + 15) / 16 : num_elements;
    const int64_t grid = (threads + 255) / 256;
    if (grid > 0x7fffffff) return VMC_EINVAL;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), 0, s, (uint8_t*)dst_cache,
                           (const uint16_t*)src_cache, sc, num_elements);
    };
    const bool sb = src_dtype == VMC_DTYPE_BF16, e5 = e5m2 != 0;
#define VMC_CVT(SB, E5, V) if (sb == SB && e5 == E5 && vec == V) go(convert_fp8_kernel<SB, E5, V>);
    VMC_CVT(false, false, false) VMC_CVT(false, false, true) VMC_CVT(false, true, false) VMC_CVT(false, true, true)
    VMC_CVT(true, false, false) VMC_CVT(true, false, true) VMC_CVT(true, true, false) VMC_CVT(true, true, true)
#undef VMC_CVT
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}
