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
#include "vmc_common.hpp"
#include "vmc_tq.hpp"

namespace vmc {
namespace {

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
        const uint32_t hi = (uint32_t)__shfl_xor((int)w, 1, kGroup);
        if ((j & 1) == 0) {
            const uint64_t w48 = (uint64_t)w | ((uint64_t)hi << 24);
            d16[3 * (j >> 1) + 0] = (uint16_t)(w48 & 0xffff);
            d16[3 * (j >> 1) + 1] = (uint16_t)((w48 >> 16) & 0xffff);
            d16[3 * (j >> 1) + 2] = (uint16_t)((w48 >> 32) & 0xffff);
        }
    }
}

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
    int q[kDims];
    // both loads up front (one HBM latency)
    load8<BF16>(key + pv * D + kDims * j, y);
    load8<BF16>(value + pv * D + kDims * j, vv);
    // ---- K: norm by the reference's sequential fmaf chain over d = 0..D-1
    // (every lane of the group runs the same chain from LDS)
#pragma unroll
    for (int e = 0; e < kDims; ++e) sq[gi][kDims * j + e] = y[e];
    __syncthreads();
    float nsq = 0.0f;
#pragma unroll
    for (int d = 0; d < D; d += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(&sq[gi][d]);
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
#pragma unroll
    for (int m = 1; m < kGroup; m <<= 1) {
#pragma unroll
        for (int e = 0; e < kDims; ++e) {
            const float o = __shfl_xor(y[e], m, kGroup);
            y[e] = (j & m) ? o - y[e] : y[e] + o;
        }
    }
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
    if (slot >= 0) {
        store_codes8<KB>(q, sp, j);
        if (j == 0) *reinterpret_cast<uint16_t*>(sp + mse_bytes) = f32_to_half<BF16>(norm);
    }

    // ---- V: asymmetric min/max over the whole vector (:314-347)
#pragma unroll
    for (int e = 0; e < kDims; ++e) y[e] = vv[e];
    float vmin = y[0], vmax = y[0];
#pragma unroll
    for (int e = 1; e < kDims; ++e) {
        vmin = fminf(vmin, y[e]);
        vmax = fmaxf(vmax, y[e]);
    }
#pragma unroll
    for (int m = 1; m < kGroup; m <<= 1) {
        vmin = fminf(vmin, __shfl_xor(vmin, m, kGroup));
        vmax = fmaxf(vmax, __shfl_xor(vmax, m, kGroup));
    }
    constexpr int VMAXQ = VB == 4 ? 15 : 7;
    float vscale = (vmax - vmin) / (float)VMAXQ;
    vscale = fmaxf(vscale, 1e-8f);
#pragma unroll
    for (int e = 0; e < kDims; ++e) {
        int qq = (int)roundf((y[e] - vmin) / vscale);
        q[e] = qq < 0 ? 0 : (qq > VMAXQ ? VMAXQ : qq);
    }
    if (slot >= 0) {
        uint8_t* vp = sp + key_packed;
        store_codes8<VB>(q, vp, j);
        if (j == 0) {
            *reinterpret_cast<uint16_t*>(vp + val_data) = f32_to_half<BF16>(vscale);
            *reinterpret_cast<uint16_t*>(vp + val_data + 2) = f32_to_half<BF16>(vmin);
        }
    }
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
#pragma unroll
    for (int m = 1; m < kGroup; m <<= 1) {
#pragma unroll
        for (int e = 0; e < kDims; ++e) {
            const float o = __shfl_xor(y[e], m, kGroup);
            y[e] = (j & m) ? o - y[e] : y[e] + o;
        }
    }
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
#pragma unroll
        for (int m = 1; m < 4; m <<= 1) {
            mn = fminf(mn, __shfl_xor(mn, m, kGroup));
            mx = fmaxf(mx, __shfl_xor(mx, m, kGroup));
        }
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
        const uint32_t plo = (uint32_t)__shfl_xor((int)lo, 2, kGroup);
        const uint32_t phi = (uint32_t)__shfl_xor((int)hi, 2, kGroup);
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
#pragma unroll
        for (int m = 1; m < 4; m <<= 1) {
            const float a2 = __shfl_xor(amax, m, kGroup);
            const float v2 = __shfl_xor(v, m, kGroup);
            const int i2 = __shfl_xor(idx, m, kGroup);
            if (a2 > amax || (a2 == amax && i2 < idx)) {
                amax = a2;
                v = v2;
                idx = i2;
            }
        }
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
        const uint32_t hiw = (uint32_t)__shfl_xor((int)w, 1, kGroup);
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
    if (head_dim != 128) return VMC_EINVAL;
    if (num_tokens < 0 || num_kv_heads <= 0 || block_size <= 0) return VMC_EINVAL;
    if (half_dtype != VMC_DTYPE_F16 && half_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (num_tokens == 0) return VMC_OK;
    if (!key || !value || !kv_cache || !slot_mapping) return VMC_EINVAL;
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
