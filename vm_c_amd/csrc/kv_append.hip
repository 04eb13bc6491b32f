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
