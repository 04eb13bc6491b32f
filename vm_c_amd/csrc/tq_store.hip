// tq_store.hip -- TurboQuant quantize-on-append, one fused kernel.
//
// Replaces vm_c::turboquant_store (src/cuda/turboquant_kernels.cu:792-860),
// which ran four launches plus a cuBLAS GEMM with fp32 scratch round trips:
//   half_to_float_norm_kernel :145-161   norm = sqrtf(sum k*k)   (fmaf chain)
//   normalize_kernel          :163-175   x = k * (1/(norm + 1e-8f))
//   cublasSgemm               :841-848   y = H x
//   tq_store_mse_kernel       :247-351   codes, norm, V min/max codes, scale, zero
// Here 16 lanes own one (token, kv-head) vector end to end, 8 dims each in
// VGPRs: the norm keeps the reference's sequential fmaf order, y = H x is a
// Walsh-Hadamard transform (butterflies of half-width 1..d/2, then one multiply
// by the reference matrix scale 1/sqrtf(d)) -- the declared rotation order the
// CPU oracle shares -- and the codebook index is the count of midpoints <= y,
// which equals the reference's top-down scan (:283-304) for sorted midpoints.
// Slot addressing: compute_slot_byte_offset (:39-45).
#include "generic_attn.hpp"
#include "vmc_store.hpp"

namespace vmc {
namespace {

template <int D, int KB, int VB, bool BF16>
__global__ void __launch_bounds__(256)
tq_store_kernel(const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
                uint8_t* __restrict__ cache, const int64_t* __restrict__ slot_mapping, int T,
                int Hkv, int64_t bs, int SA, int mse_bytes, int key_packed, int val_data,
                TQTables tab) {
    static_assert(D == kGroup * kDims, "one 16-lane group per 128-dim vector");
    __shared__ __attribute__((aligned(16))) float sq[256 / kGroup][D];  // per-group K for the norm chain
    const int lane = threadIdx.x & 63, j = lane & (kGroup - 1);
    const int gi = threadIdx.x / kGroup;  // group in the workgroup
    const int64_t pid = (int64_t)blockIdx.x * (blockDim.x / kGroup) + gi;
    const bool live = pid < (int64_t)T * Hkv;
    const int64_t pv = live ? pid : 0;  // every lane stays in the shuffles
    const int64_t t = pv / Hkv;
    const int h = (int)(pv % Hkv);
    const int64_t slot = live ? slot_mapping[t] : -1;  // :266-267: slot < 0 skips
    const int64_t blk = slot / bs, off = slot % bs;
    uint8_t* sp = cache + blk * bs * Hkv * SA + off * Hkv * SA + (int64_t)h * SA;
    float y[kDims], vv[kDims];
    // both loads up front (one HBM latency)
    load8<BF16>(key + pv * D + kDims * j, y);
    load8<BF16>(value + pv * D + kDims * j, vv);
    tq_store_vec<D, KB, VB, BF16>(y, vv, j, sp, slot >= 0, sq[gi], tab, mse_bytes, key_packed, val_data);
}

template <int BITS, bool BF16>
__global__ void __launch_bounds__(256)
g32_store_kernel(const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
                 uint8_t* __restrict__ cache, const int64_t* __restrict__ slot_mapping, int T,
                 int Hkv, int64_t bs, G32Signs sg, float rot_c) {
    constexpr int D = kGroup * kDims, P = BITS == 4 ? 80 : 56, S = 2 * P;
    const int lane = threadIdx.x & 63, j = lane & (kGroup - 1);
    const int gi = threadIdx.x / kGroup;
    const int64_t pid = (int64_t)blockIdx.x * (blockDim.x / kGroup) + gi;
    const bool live = pid < (int64_t)T * Hkv;
    const int64_t pv = live ? pid : 0;  // every lane stays in the shuffles
    const int64_t t = pv / Hkv;
    const int h = (int)(pv % Hkv);
    const int64_t slot = live ? slot_mapping[t] : -1;  // slot < 0 skips
    const int64_t blk = slot / bs, off = slot % bs;
    uint8_t* sp = cache + blk * bs * Hkv * S + off * Hkv * S + (int64_t)h * S;
    const uint32_t sbits = (sg.w[j >> 2] >> (8 * (j & 3))) & 0xffu;
    float yk[kDims], yv[kDims];
    load8<BF16>(key + pv * D + kDims * j, yk);
    load8<BF16>(value + pv * D + kDims * j, yv);
    g32_rotate(yk, j, sbits, rot_c);
    g32_quantize<BITS>(yk, j, sp, slot >= 0);
    g32_rotate(yv, j, sbits, rot_c);
    g32_quantize<BITS>(yv, j, sp + P, slot >= 0);
}

// turboquant_k8v4 (half_to_fp8_store_kernel, turboquant_kernels.cu:188-245),
// same 16-lane ownership: fp8 key bytes by the reference's converter, the V
// part as in every TurboQuant slot
template <bool BF16>
__global__ void __launch_bounds__(256)
k8v4_store_kernel(const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
                  uint8_t* __restrict__ cache, const int64_t* __restrict__ slot_mapping, int T,
                  int Hkv, int64_t bs, int e4b15) {
    constexpr int D = kGroup * kDims, S = 196;
    const int lane = threadIdx.x & 63, j = lane & (kGroup - 1);
    const int gi = threadIdx.x / kGroup;
    const int64_t pid = (int64_t)blockIdx.x * (blockDim.x / kGroup) + gi;
    const bool live = pid < (int64_t)T * Hkv;
    const int64_t pv = live ? pid : 0;  // every lane stays in the exchanges
    const int64_t t = pv / Hkv;
    const int h = (int)(pv % Hkv);
    const int64_t slot = live ? slot_mapping[t] : -1;  // :207: slot < 0 skips
    const int64_t blk = slot / bs, off = slot % bs;
    uint8_t* sp = cache + blk * bs * Hkv * S + off * Hkv * S + (int64_t)h * S;
    float yk[kDims], yv[kDims];
    load8<BF16>(key + pv * D + kDims * j, yk);
    load8<BF16>(value + pv * D + kDims * j, yv);
    k8v4_store_vec<BF16>(yk, yv, j, sp, slot >= 0, e4b15);
}

int launch_g32_store(const void* key, const void* value, void* cache, const int64_t* slots, int T,
                     int Hkv, int64_t bs, const vmc_tq_config* c, bool bf16, hipStream_t stream) {
    const int64_t n = (int64_t)T * Hkv;
    const int threads = 256, per_block = threads / kGroup;
    const int64_t grid = (n + per_block - 1) / per_block;
    if (grid > 0x7fffffff) return VMC_EINVAL;
    const G32Signs sg = g32_signs(c->sign_seed);
    const float rot_c = 1.0f / sqrtf(128.0f);
    const auto* k = (const uint16_t*)key;
    const auto* v = (const uint16_t*)value;
    auto* kc = (uint8_t*)cache;
    if (c->key_quant_bits == 4) {
        if (bf16) hipLaunchKernelGGL((g32_store_kernel<4, true>), dim3((unsigned)grid), dim3(threads), 0, stream, k, v, kc, slots, T, Hkv, bs, sg, rot_c);
        else hipLaunchKernelGGL((g32_store_kernel<4, false>), dim3((unsigned)grid), dim3(threads), 0, stream, k, v, kc, slots, T, Hkv, bs, sg, rot_c);
    } else {
        if (bf16) hipLaunchKernelGGL((g32_store_kernel<3, true>), dim3((unsigned)grid), dim3(threads), 0, stream, k, v, kc, slots, T, Hkv, bs, sg, rot_c);
        else hipLaunchKernelGGL((g32_store_kernel<3, false>), dim3((unsigned)grid), dim3(threads), 0, stream, k, v, kc, slots, T, Hkv, bs, sg, rot_c);
    }
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}

template <int D, int KB, int VB>
int launch_store(const void* key, const void* value, void* cache, const int64_t* slots, int T,
                 int Hkv, int64_t bs, const vmc_tq_config* c, bool bf16, hipStream_t stream) {
    const TQTables& tab = tq_tables(D, KB);
    const int64_t n = (int64_t)T * Hkv;
    const int threads = 256, per_block = threads / kGroup;
    const int64_t grid = (n + per_block - 1) / per_block;
    if (grid > 0x7fffffff) return VMC_EINVAL;
    if (bf16)
        hipLaunchKernelGGL((tq_store_kernel<D, KB, VB, true>), dim3((unsigned)grid), dim3(threads),
                           0, stream, (const uint16_t*)key, (const uint16_t*)value,
                           (uint8_t*)cache, slots, T, Hkv, bs, c->slot_size_aligned,
                           c->mse_bytes, c->key_packed_size, c->val_data_bytes, tab);
    else
        hipLaunchKernelGGL((tq_store_kernel<D, KB, VB, false>), dim3((unsigned)grid), dim3(threads),
                           0, stream, (const uint16_t*)key, (const uint16_t*)value,
                           (uint8_t*)cache, slots, T, Hkv, bs, c->slot_size_aligned,
                           c->mse_bytes, c->key_packed_size, c->val_data_bytes, tab);
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}

}  // namespace
}  // namespace vmc

using namespace vmc;

extern "C" int vmc_turboquant_store(const void* key, const void* value, void* kv_cache,
                                    const int64_t* slot_mapping, int num_tokens,
                                    int num_kv_heads, int head_dim, int64_t block_size,
                                    const vmc_tq_config* cfg, int half_dtype,
                                    vmc_stream_t stream) {
    if (!tq_config_valid(cfg) || cfg->head_dim != head_dim) return VMC_EINVAL;
    if (head_dim != 128 && !generic_head_dim(head_dim)) return VMC_EINVAL;
    if (num_tokens < 0 || num_kv_heads <= 0 || block_size <= 0) return VMC_EINVAL;
    if (half_dtype != VMC_DTYPE_F16 && half_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (num_tokens == 0) return VMC_OK;
    if (!key || !value || !kv_cache || !slot_mapping) return VMC_EINVAL;
    if (head_dim != 128)
        return gen_tq_store(key, value, kv_cache, slot_mapping, num_tokens, num_kv_heads, head_dim, block_size,
                            cfg, half_dtype == VMC_DTYPE_BF16, reinterpret_cast<hipStream_t>(stream));
    if (cfg->key_fp8) {
        const int64_t grid = ((int64_t)num_tokens * num_kv_heads + 15) / 16;
        if (grid > 0x7fffffff) return VMC_EINVAL;
        hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        if (half_dtype == VMC_DTYPE_BF16)
            hipLaunchKernelGGL((k8v4_store_kernel<true>), dim3((unsigned)grid), dim3(256), 0, s,
                               (const uint16_t*)key, (const uint16_t*)value, (uint8_t*)kv_cache, slot_mapping,
                               num_tokens, num_kv_heads, block_size, cfg->fp8_e4b15);
        else
            hipLaunchKernelGGL((k8v4_store_kernel<false>), dim3((unsigned)grid), dim3(256), 0, s,
                               (const uint16_t*)key, (const uint16_t*)value, (uint8_t*)kv_cache, slot_mapping,
                               num_tokens, num_kv_heads, block_size, cfg->fp8_e4b15);
        VMC_LAUNCH_CHECK();
        return VMC_OK;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool bf = half_dtype == VMC_DTYPE_BF16;
    if (cfg->group_size != 0)
        return launch_g32_store(key, value, kv_cache, slot_mapping, num_tokens, num_kv_heads, block_size,
                                cfg, bf, s);
    const int kb = cfg->key_quant_bits, vb = cfg->value_quant_bits;
    if (kb == 4 && vb == 4)
        return launch_store<128, 4, 4>(key, value, kv_cache, slot_mapping, num_tokens, num_kv_heads,
                                       block_size, cfg, bf, s);
    if (kb == 3 && vb == 3)
        return launch_store<128, 3, 3>(key, value, kv_cache, slot_mapping, num_tokens, num_kv_heads,
                                       block_size, cfg, bf, s);
    if (kb == 3 && vb == 4)
        return launch_store<128, 3, 4>(key, value, kv_cache, slot_mapping, num_tokens, num_kv_heads,
                                       block_size, cfg, bf, s);
    return VMC_EINVAL;
}
