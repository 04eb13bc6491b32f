// tq_store.hip -- TurboQuant quantize-on-append, one fused kernel.
//
// Replaces vm_c::turboquant_store (src/cuda/turboquant_kernels.cu:792-860),
// which ran four launches plus a cuBLAS GEMM with fp32 scratch round trips:
//   half_to_float_norm_kernel :145-161   norm = sqrtf(sum k*k)   (fmaf chain)
//   normalize_kernel          :163-175   x = k * (1/(norm + 1e-8f))
//   cublasSgemm               :841-848   y = H x
//   tq_store_mse_kernel       :247-351   codes, norm, V min/max codes, scale, zero
// Here one thread owns one (token, kv-head) vector end to end with the vector
// in VGPRs: the norm keeps the reference's sequential fmaf order, y = H x is a
// Walsh-Hadamard transform (butterflies of half-width 1..d/2, then one multiply
// by the reference matrix scale 1/sqrtf(d)) -- the declared rotation order the
// CPU oracle shares -- and the codebook index is the count of midpoints <= y,
// which equals the reference's top-down scan (:283-304) for sorted midpoints.
// Slot addressing: compute_slot_byte_offset (:39-45).
#include "vmc_common.hpp"
#include "vmc_tq.hpp"

namespace vmc {
namespace {

template <int D, bool BF16>
__device__ __forceinline__ void load_vec(const uint16_t* src, float* x) {
    const u32x4* p = reinterpret_cast<const u32x4*>(src);
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
        const u32x4 w = p[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[8 * c + 2 * e] = half_to_f32<BF16>((uint16_t)(w[e] & 0xffffu));
            x[8 * c + 2 * e + 1] = half_to_f32<BF16>((uint16_t)(w[e] >> 16));
        }
    }
}

template <int D>
__device__ __forceinline__ void fwht(float* y) {
#pragma unroll
    for (int h = 1; h < D; h <<= 1) {
#pragma unroll
        for (int i = 0; i < D; i += 2 * h) {
#pragma unroll
            for (int j = i; j < i + h; ++j) {
                const float a = y[j], b = y[j + h];
                y[j] = a + b;
                y[j + h] = a - b;
            }
        }
    }
}

// codes q[D] -> packed bytes written as 16-bit words (dst is 2-byte aligned)
template <int D, int BITS>
__device__ __forceinline__ void store_codes(const int* q, uint8_t* dst) {
    uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
    if constexpr (BITS == 4) {
        // even d in the low nibble (:291)
#pragma unroll
        for (int d = 0; d < D; d += 4)
            d16[d / 4] = (uint16_t)((q[d] & 0xf) | ((q[d + 1] & 0xf) << 4) | ((q[d + 2] & 0xf) << 8) |
                                    ((q[d + 3] & 0xf) << 12));
    } else {
        // 8 codes -> 3 bytes little endian, code i at bits 3i (:294-309); two
        // groups give three 16-bit words
#pragma unroll
        for (int g = 0; g < D / 8; g += 2) {
            uint32_t p0 = 0, p1 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                p0 |= (uint32_t)(q[g * 8 + i] & 7) << (3 * i);
                p1 |= (uint32_t)(q[(g + 1) * 8 + i] & 7) << (3 * i);
            }
            const uint64_t w = (uint64_t)p0 | ((uint64_t)p1 << 24);
            d16[g / 2 * 3 + 0] = (uint16_t)(w & 0xffff);
            d16[g / 2 * 3 + 1] = (uint16_t)((w >> 16) & 0xffff);
            d16[g / 2 * 3 + 2] = (uint16_t)((w >> 32) & 0xffff);
        }
    }
}

template <int D, int KB, int VB, bool BF16>
__global__ void __launch_bounds__(64)
tq_store_kernel(const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
                uint8_t* __restrict__ cache, const int64_t* __restrict__ slot_mapping, int T,
                int Hkv, int64_t bs, int SA, int mse_bytes, int key_packed, int val_data,
                TQTables tab) {
    const int64_t pid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (pid >= (int64_t)T * Hkv) return;
    const int64_t t = pid / Hkv;
    const int h = (int)(pid % Hkv);
    const int64_t slot = slot_mapping[t];
    if (slot < 0) return;  // :266-267
    const int64_t blk = slot / bs, off = slot % bs;
    uint8_t* sp = cache + blk * bs * Hkv * SA + off * Hkv * SA + (int64_t)h * SA;

    float y[D];
    int q[D];
    // ---- K: norm, normalise, rotate, codebook
    load_vec<D, BF16>(key + pid * D, y);
    float nsq = 0.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) nsq = __builtin_fmaf(y[d], y[d], nsq);
    const float norm = sqrtf(nsq);
    const float inv = 1.0f / (norm + 1e-8f);
#pragma unroll
    for (int d = 0; d < D; ++d) y[d] = __fmul_rn(y[d], inv);
    fwht<D>(y);
    constexpr int NC = 1 << KB;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const float v = __fmul_rn(y[d], tab.rot_c);
        int idx = 0;
#pragma unroll
        for (int c = 0; c < NC - 1; ++c) idx += (v >= tab.midpoints[c]) ? 1 : 0;
        q[d] = idx;
    }
    store_codes<D, KB>(q, sp);
    *reinterpret_cast<uint16_t*>(sp + mse_bytes) = f32_to_half<BF16>(norm);

    // ---- V: asymmetric min/max over the whole vector (:314-347)
    load_vec<D, BF16>(value + pid * D, y);
    float vmin = 3.402823466e+38f, vmax = -3.402823466e+38f;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        vmin = fminf(vmin, y[d]);
        vmax = fmaxf(vmax, y[d]);
    }
    constexpr int VMAXQ = VB == 4 ? 15 : 7;
    float vscale = (vmax - vmin) / (float)VMAXQ;
    vscale = fmaxf(vscale, 1e-8f);
#pragma unroll
    for (int d = 0; d < D; ++d) {
        int qq = (int)roundf((y[d] - vmin) / vscale);
        q[d] = qq < 0 ? 0 : (qq > VMAXQ ? VMAXQ : qq);
    }
    uint8_t* vp = sp + key_packed;
    store_codes<D, VB>(q, vp);
    *reinterpret_cast<uint16_t*>(vp + val_data) = f32_to_half<BF16>(vscale);
    *reinterpret_cast<uint16_t*>(vp + val_data + 2) = f32_to_half<BF16>(vmin);
}

template <int D, int KB, int VB>
int launch_store(const void* key, const void* value, void* cache, const int64_t* slots, int T,
                 int Hkv, int64_t bs, const vmc_tq_config* c, bool bf16, hipStream_t stream) {
    const TQTables& tab = tq_tables(D, KB);
    const int64_t n = (int64_t)T * Hkv;
    const int threads = 64;
    const int64_t grid = (n + threads - 1) / threads;
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
    if (head_dim != 128) return VMC_EINVAL;
    if (num_tokens < 0 || num_kv_heads <= 0 || block_size <= 0) return VMC_EINVAL;
    if (half_dtype != VMC_DTYPE_F16 && half_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (num_tokens == 0) return VMC_OK;
    if (!key || !value || !kv_cache || !slot_mapping) return VMC_EINVAL;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool bf = half_dtype == VMC_DTYPE_BF16;
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
