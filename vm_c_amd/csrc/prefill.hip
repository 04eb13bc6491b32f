// prefill.hip -- causal flash-attention prefill on MFMA, with optional fused
// quantize-on-append of the K/V rows into the paged cache.
//
// Replaces vm_c::flash_attention_prefill_local (include/vm_c/cuda/
// kernels_flash_attn.h:81-93, src/cuda/flash_attn_v2_kernels.cu:262-393: one
// serial thread block per (token, head)).  Semantics: each sequence's tokens
// are contiguous with positions 0..n-1, so token t attends keys
// [t - pos(t), t]; GQA kv head = q head / (Hq / Hkv).
//
// Tiling (gfx950, wave64, v_mfma_f32_32x32x16_{bf16,f16}):
//   workgroup = 4 waves = 128 query rows of one query head; K/V tiles of 64
//   rows, double-buffered in LDS (row pitch 272 B: 16-byte aligned reads hit
//   distinct banks).
//   S^T[64 kv x 32 q] = K . Q^T  per wave: 2 x 8 MFMAs, Q^T held in registers.
//     The output layout puts one query row per lane column, so the row max /
//     sum of the online softmax are in-lane plus one cross-half shuffle.
//   O[32 q x 128] += P . V       per wave: 4 dim-blocks x 4 kv-chunks MFMAs.
//     P is fed straight from the S^T registers: the contraction index k of an
//     MFMA may be any permutation of the 16 kv rows as long as A and B agree,
//     so logical k = 8h + e maps to kv 16c + 8(e/4) + 4h + e%4, which is what
//     lane half h already holds.  V output columns are permuted (block m,
//     column n -> dim 4n + m) so each lane reads 8 contiguous bytes per kv row.
//   Per-row rescale factors reach the O rows through a 128-byte LDS scratch.
// Fused append: the workgroup of the first query head of each KV group writes
// its 128 K/V rows into the paged cache with the same block encoders as
// vmc_reshape_and_cache (bit-identical pages).
#include "kv_quant.hpp"

namespace vmc {
namespace {

constexpr int kD = 128;
constexpr int BM = 128;    // query rows per workgroup
constexpr int BN = 64;     // kv rows per tile
constexpr int PITCH = 272; // LDS bytes per K/V row
constexpr int TILE_BYTES = BN * PITCH;
constexpr int LDS_BYTES = 4 * TILE_BYTES + 2 * 4 * 32 * 4;
constexpr float kNegInf = -__builtin_inff();

struct PrefillParams {
    uint16_t* out;
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const int32_t* pos;
    int T, Hq, Hkv, G;
    float scale_log2;
    int ntiles;
    // fused append
    uint8_t* kc;
    uint8_t* vc;
    const int64_t* slots;
    int64_t bs, E, stride;
    int hnd;
};

template <bool BF16>
struct MT;
template <>
struct MT<true> {
    using v8 = bf16x8;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint16_t cvt(float x) { return f32_to_bf16_bits(x); }
    static __device__ __forceinline__ float back(uint16_t b) { return bf16_bits_to_f32(b); }
};
template <>
struct MT<false> {
    using v8 = f16x8;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint16_t cvt(float x) { return f32_to_f16_bits(x); }
    static __device__ __forceinline__ float back(uint16_t b) { return f16_bits_to_f32(b); }
};

template <typename V8>
__device__ __forceinline__ V8 as_v8(u32x4 w) {
    return __builtin_bit_cast(V8, w);
}

template <bool BF16, int APPEND_FMT>
__global__ void __launch_bounds__(256, 2)
prefill_kernel(PrefillParams p) {
    using M = MT<BF16>;
    using V8 = typename M::v8;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* kbuf = smem;                      // [2][BN][PITCH]
    uint8_t* vbuf = smem + 2 * TILE_BYTES;     // [2][BN][PITCH]
    float* scratch = reinterpret_cast<float*>(smem + 4 * TILE_BYTES);  // [4 waves][32]

    const int tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63;
    const int c32 = lane & 31, h = lane >> 5;
    const int hq = blockIdx.x % p.Hq;
    const int tile = p.ntiles - 1 - (int)(blockIdx.x / p.Hq);
    const int g = hq / p.G;
    const int T = p.T;
    const int q0 = tile * BM;

    // kv range of the whole workgroup
    const int kv_lo = max(0, q0 - p.pos[q0]);
    const int kv_end = min(q0 + BM, T);
    const int ntile = (kv_end - kv_lo + BN - 1) / BN;

    // this lane's query row and its key window [lo, row]
    const int row = q0 + 32 * w + c32;
    const bool row_ok = row < T;
    const int lo = row_ok ? row - p.pos[row] : 0;
    // wave-uniform bounds
    const int wrow0 = q0 + 32 * w;
    const bool wave_ok = wrow0 < T;
    const int wrow1 = min(wrow0 + 31, T - 1);
    const int wlo0 = wave_ok ? wrow0 - p.pos[wrow0] : 0;
    const int wlo1 = wave_ok ? wrow1 - p.pos[wrow1] : 0;

    // ---- Q^T operand: lane (col = row, half h) holds dims 16s + 8h .. +7
    V8 qb[8];
    {
        const uint16_t* qp = p.q + ((int64_t)row * p.Hq + hq) * kD + 8 * h;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            u32x4 wv = {0u, 0u, 0u, 0u};
            if (row_ok) wv = *reinterpret_cast<const u32x4*>(qp + 16 * s);
            qb[s] = as_v8<V8>(wv);
        }
    }

    f32x16 o[4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[m][i] = 0.0f;
    float m_run = kNegInf, l_part = 0.0f;

    // ---- staging: 1024 16-byte chunks per tensor per tile, 4 per thread
    u32x4 stk[4], stv[4];
    auto stage_load = [&](int t) {
        const int k0 = kv_lo + t * BN;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + 256 * i;
            const int r = c >> 4, ch = c & 15;
            const int kk = k0 + r;
            stk[i] = u32x4{0u, 0u, 0u, 0u};
            stv[i] = u32x4{0u, 0u, 0u, 0u};
            if (kk < kv_end) {
                const int64_t off = ((int64_t)kk * p.Hkv + g) * kD + ch * 8;
                stk[i] = *reinterpret_cast<const u32x4*>(p.k + off);
                stv[i] = *reinterpret_cast<const u32x4*>(p.v + off);
                if constexpr (BF16) {
                    // PV runs in fp16 (P keeps 11 mantissa bits): V bf16 -> fp16,
                    // exact for |v| in [2^-14, 65504]
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t x = stv[i][e];
                        stv[i][e] = (uint32_t)f32_to_f16_bits(bf16_bits_to_f32((uint16_t)(x & 0xffff))) |
                                    ((uint32_t)f32_to_f16_bits(bf16_bits_to_f32((uint16_t)(x >> 16))) << 16);
                    }
                }
            }
        }
    };
    auto stage_store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + 256 * i;
            const int r = c >> 4, ch = c & 15;
            *reinterpret_cast<u32x4*>(kbuf + buf * TILE_BYTES + r * PITCH + ch * 16) = stk[i];
            *reinterpret_cast<u32x4*>(vbuf + buf * TILE_BYTES + r * PITCH + ch * 16) = stv[i];
        }
    };

    stage_load(0);
    stage_store(0);
    __syncthreads();

    for (int t = 0; t < ntile; ++t) {
        const int buf = t & 1;
        if (t + 1 < ntile) stage_load(t + 1);
        const int k0 = kv_lo + t * BN;
        // skip: tile entirely after this wave's last row, or before its first window
        const bool active = wave_ok && k0 <= wrow1 && k0 + BN - 1 >= wlo0;
        if (active) {
            const uint8_t* kt = kbuf + buf * TILE_BYTES;
            const uint8_t* vt = vbuf + buf * TILE_BYTES;
            const bool need_mask = (k0 + BN - 1 > wrow0) || (k0 < wlo1);
            // ---- S^T = K Q^T, two 32-row kv blocks
            f32x16 sacc[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int i = 0; i < 16; ++i) sacc[kb][i] = 0.0f;
                const uint8_t* kr = kt + (kb * 32 + c32) * PITCH + 16 * h;
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    const u32x4 a = *reinterpret_cast<const u32x4*>(kr + 32 * s);
                    sacc[kb] = M::mma(as_v8<V8>(a), qb[s], sacc[kb]);
                }
            }
            // ---- online softmax (log2 domain), one query row per lane column
            float mx = kNegInf;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    float sv = sacc[kb][j] * p.scale_log2;
                    if (need_mask) {
                        const int kv = k0 + kb * 32 + 8 * (j >> 2) + 4 * h + (j & 3);
                        sv = (kv <= row && kv >= lo && row_ok) ? sv : kNegInf;
                    }
                    sacc[kb][j] = sv;
                    mx = fmaxf(mx, sv);
                }
            mx = fmaxf(mx, shfl_xor(mx, 32));
            const float m_new = fmaxf(m_run, mx);
            const float m_use = m_new == kNegInf ? 0.0f : m_new;
            const float alpha = exp2f(m_run - m_use);
            m_run = m_new;
            // P as MFMA A operands, chunk c = kv rows 16c .. 16c+15
            uint32_t pw[4][4];
            float psum = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const int kb = c >> 1;
                    const int j0 = 4 * (2 * (c & 1) + (e >> 2)) + (e & 3);
                    const uint16_t b0 = f32_to_f16_bits(exp2f(sacc[kb][j0] - m_use));
                    const uint16_t b1 = f32_to_f16_bits(exp2f(sacc[kb][j0 + 1] - m_use));
                    psum += f16_bits_to_f32(b0) + f16_bits_to_f32(b1);
                    pw[c][e >> 1] = (uint32_t)b0 | ((uint32_t)b1 << 16);
                }
            l_part = __builtin_fmaf(l_part, alpha, psum);
            // ---- rescale O rows by their query rows' alpha (rows 8b + 4h + i)
            float* sc = scratch + w * 32;
            if (h == 0) sc[c32] = alpha;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            float al[16];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const f32x4 a4 = *reinterpret_cast<const f32x4*>(sc + 8 * b + 4 * h);
#pragma unroll
                for (int i = 0; i < 4; ++i) al[4 * b + i] = a4[i];
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[m][i] *= al[i];
            // ---- O += P V
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const f16x8 pa = as_v8<f16x8>(u32x4{pw[c][0], pw[c][1], pw[c][2], pw[c][3]});
                u32x2 vv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int kv = 16 * c + 8 * (e >> 2) + 4 * h + (e & 3);
                    vv[e] = *reinterpret_cast<const u32x2*>(vt + kv * PITCH + 8 * c32);
                }
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    u32x4 bw;
#pragma unroll
                    for (int e2 = 0; e2 < 4; ++e2) {
                        const uint32_t lo16 = (vv[2 * e2][m >> 1] >> (16 * (m & 1))) & 0xffffu;
                        const uint32_t hi16 = (vv[2 * e2 + 1][m >> 1] >> (16 * (m & 1))) & 0xffffu;
                        bw[e2] = lo16 | (hi16 << 16);
                    }
                    o[m] = MT<false>::mma(pa, as_v8<f16x8>(bw), o[m]);
                }
            }
        }
        if (t + 1 < ntile) stage_store(buf ^ 1);
        __syncthreads();
    }

    // ---- normalise and store: lane holds rows 8b + 4h + i, dims 4*c32 .. +3
    {
        const float l_tot = l_part + shfl_xor(l_part, 32);
        float* sc = scratch + 4 * 32 + w * 32;
        if (h == 0) sc[c32] = l_tot;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const f32x4 l4 = *reinterpret_cast<const f32x4*>(sc + 8 * b + 4 * h);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = wrow0 + 8 * b + 4 * h + i;
                if (r >= T) continue;
                const float inv = l4[i] > 0.0f ? 1.0f / l4[i] : 0.0f;
                const uint32_t d0 = M::cvt(o[0][4 * b + i] * inv), d1 = M::cvt(o[1][4 * b + i] * inv);
                const uint32_t d2 = M::cvt(o[2][4 * b + i] * inv), d3 = M::cvt(o[3][4 * b + i] * inv);
                uint16_t* op = p.out + ((int64_t)r * p.Hq + hq) * kD + 4 * c32;
                *reinterpret_cast<u32x2*>(op) = u32x2{d0 | (d1 << 16), d2 | (d3 << 16)};
            }
        }
    }

    // ---- fused quantize-on-append of this tile's K/V rows (once per KV head)
    if constexpr (APPEND_FMT >= 0) {
        if (hq % p.G == 0) {
            const int nrow = min(BM, T - q0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int item = tid + 256 * j;  // [tensor][row][block]
                const int tensor = item >> 9;
                const int r = (item >> 2) & 127;
                const int blk = item & 3;
                if (r >= nrow) continue;
                const int64_t slot = p.slots[q0 + r];
                if (slot < 0) continue;
                const uint16_t* src = (tensor ? p.v : p.k) + ((int64_t)(q0 + r) * p.Hkv + g) * kD + 32 * blk;
                uint8_t* dst = (tensor ? p.vc : p.kc) +
                               kv_entry_offset(slot, g, p.bs, p.Hkv, p.E, p.stride, p.hnd != 0);
                append_block32<APPEND_FMT, BF16>(src, dst, blk);
            }
        }
    }
}

template <bool BF16, int FMT>
int launch_prefill(PrefillParams& prm, hipStream_t stream) {
    auto kern = prefill_kernel<BF16, FMT>;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES) != hipSuccess)
        return VMC_EIO;
    const int64_t grid = (int64_t)prm.ntiles * prm.Hq;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), LDS_BYTES, stream, prm);
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}

template <bool BF16>
int dispatch_fmt(PrefillParams& prm, int fmt, hipStream_t s) {
    switch (fmt) {
        case -1: return launch_prefill<BF16, -1>(prm, s);
        case VMC_KV_F16: return launch_prefill<BF16, VMC_KV_F16>(prm, s);
        case VMC_KV_BF16: return launch_prefill<BF16, VMC_KV_BF16>(prm, s);
        case VMC_KV_Q8_0: return launch_prefill<BF16, VMC_KV_Q8_0>(prm, s);
        case VMC_KV_Q4_0: return launch_prefill<BF16, VMC_KV_Q4_0>(prm, s);
        default: return VMC_EINVAL;
    }
}

}  // namespace
}  // namespace vmc

using namespace vmc;

extern "C" int vmc_flash_attention_prefill(void* output, const void* query, const void* key,
                                           const void* value, int num_tokens, int num_heads,
                                           int num_kv_heads, int head_dim, float scale,
                                           const int32_t* token_positions, int dtype,
                                           void* key_cache, void* value_cache,
                                           const int64_t* slot_mapping, int64_t block_size,
                                           int kv_format, int layout, vmc_stream_t stream) {
    if (head_dim != kD || num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 ||
        num_heads % num_kv_heads != 0)
        return VMC_EINVAL;
    if (dtype != VMC_DTYPE_F16 && dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (num_tokens == 0) return VMC_OK;
    if (!output || !query || !key || !value || !token_positions) return VMC_EINVAL;
    PrefillParams prm = {};
    prm.out = reinterpret_cast<uint16_t*>(output);
    prm.q = reinterpret_cast<const uint16_t*>(query);
    prm.k = reinterpret_cast<const uint16_t*>(key);
    prm.v = reinterpret_cast<const uint16_t*>(value);
    prm.pos = token_positions;
    prm.T = num_tokens;
    prm.Hq = num_heads;
    prm.Hkv = num_kv_heads;
    prm.G = num_heads / num_kv_heads;
    prm.scale_log2 = scale * kLog2e;
    prm.ntiles = (num_tokens + BM - 1) / BM;
    int fmt = -1;
    if (key_cache) {
        const int64_t E = vmc_kv_entry_bytes(kv_format, head_dim);
        if (E < 0 || !value_cache || !slot_mapping || block_size <= 0) return VMC_EINVAL;
        if (layout != VMC_LAYOUT_NHD && layout != VMC_LAYOUT_HND) return VMC_EINVAL;
        prm.kc = reinterpret_cast<uint8_t*>(key_cache);
        prm.vc = reinterpret_cast<uint8_t*>(value_cache);
        prm.slots = slot_mapping;
        prm.bs = block_size;
        prm.E = E;
        prm.stride = block_size * num_kv_heads * E;
        prm.hnd = layout == VMC_LAYOUT_HND;
        fmt = kv_format;
    }
    if ((int64_t)prm.ntiles * prm.Hq > 0x7fffffffLL) return VMC_EINVAL;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    return dtype == VMC_DTYPE_BF16 ? dispatch_fmt<true>(prm, fmt, s) : dispatch_fmt<false>(prm, fmt, s);
}
