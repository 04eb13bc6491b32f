// fused_norm_rope.hip -- Q/K RMSNorm + RoPE + quantize-on-append in one launch.
//
// Replaces vm_c::fused_qk_norm_rope_store / fused_qk_norm_rope
// (include/vm_c/cuda/kernels_fused_attn.h; src/cuda/fused_attn_kernels.cu:
// 39-313: one 128-thread block per token, serial loops over the heads, the
// K/V rows copied into fp16 pages).  Here 16 lanes own one (token, head) row,
// 8 dims each in VGPRs, and the append writes any of the paged formats --
// fp16/bf16/q8_0/q4_0 pages (NHD/HND), TurboQuant slots, or the per-32-group
// variant -- from the rotated K row still in registers, so K/V make one trip
// through HBM.  Semantics (the reference's intent; its cross-warp reduction
// and its GPT-J read are defects):
//   RMSNorm (:72-124): S = sum of x^2 over the row, inv = 1/sqrtf(S/D + eps),
//     y = (x * inv) * w[h*D + d], rounded to the element type; S in the
//     declared order: lane j's fmaf chain over its 8 dims, then a butterfly
//     over the 16 lanes (distances 1, 2, 4, 8);
//   RoPE (:128-178): cos/sin = cache[pos][0, D/2) / [D/2, D); neox pairs
//     (d, d + D/2), GPT-J pairs (2d, 2d+1); a' = a c - b s, b' = b c + a s,
//     rounded; the rows are written back in place (Q and K);
//   append: the rotated K row (as rounded) and the V row, as
//     vmc_reshape_and_cache / vmc_turboquant_store would write them.
#include "kv_quant.hpp"
#include "vmc_store.hpp"

namespace vmc {
namespace {

enum { ST_NONE = 0, ST_F16 = 1, ST_BF16 = 2, ST_Q8_0 = 3, ST_Q4_0 = 4, ST_TQ = 5, ST_G32 = 6, ST_K8 = 7 };

struct FusedParams {
    uint16_t* q;
    uint16_t* k;
    const uint16_t* v;
    const uint16_t* qw;
    const uint16_t* kw;
    const uint16_t* cs;
    const int64_t* pos;
    uint8_t* kc;
    uint8_t* vc;
    const int64_t* slots;
    int T, Hq, Hkv;
    float eps;
    int neox;
    int64_t bs;
    // paged formats
    int64_t E, stride;
    int hnd;
    // TurboQuant slot
    int SA, mse_bytes, key_packed, val_data;
    TQTables tab;
    G32Signs sg;
    int e4b15;  // turboquant_k8v4 key codes
};

// The fp32 result is materialised before the conversion (opaque): otherwise
// fp16(u * w) becomes one v_fma_mix, a single rounding of the exact product
// where the declared order rounds to fp32 first.
template <bool BF16>
__device__ __forceinline__ float round_half(float x) {
    return half_to_f32<BF16>(f32_to_half<BF16>(opaque(x)));
}

template <bool BF16>
__device__ __forceinline__ u32x4 pack8(const float* x) {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        w[e] = (uint32_t)f32_to_half<BF16>(opaque(x[2 * e])) |
               ((uint32_t)f32_to_half<BF16>(opaque(x[2 * e + 1])) << 16);
    return w;
}

// q8_0 / q4_0 block of 32 values held by lanes 4b .. 4b+3 (lane l: values
// 8l .. 8l+7); the encoders of kv_quant.hpp, element for element
template <int ST>
__device__ __forceinline__ void gguf_block4(const float* x, int j, uint8_t* entry, bool write) {
    const int l = j & 3, ib = j >> 2;
    if constexpr (ST == ST_Q8_0) {
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(x[e]));
        amax = fmaxf(amax, row_xor<1>(amax, j));
        amax = fmaxf(amax, row_xor<2>(amax, j));
        const float d = opaque(amax / 127.0f);
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        if (write) {
            uint16_t* d16 = reinterpret_cast<uint16_t*>(entry + 34 * ib);
            if (l == 0) d16[0] = f32_to_f16_bits(d);
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const int q0 = (int)roundf(x[e] * id);
                const int q1 = (int)roundf(x[e + 1] * id);
                d16[1 + 4 * l + e / 2] = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
            }
        }
    } else {
        // signed value of the first largest |x| (index order)
        float amax = 0.0f, mx = 0.0f;
        int idx = 1 << 20;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float a = fabsf(x[e]);
            if (amax < a) {
                amax = a;
                mx = x[e];
                idx = 8 * l + e;
            }
        }
        static_for<2>([&](auto m) {
            constexpr int M = 1 << decltype(m)::value;
            const float a2 = row_xor<M>(amax, j);
            const float x2 = row_xor<M>(mx, j);
            const int i2 = row_xor<M>(idx, j);
            if (a2 > amax || (a2 == amax && i2 < idx)) {
                amax = a2;
                mx = x2;
                idx = i2;
            }
        });
        const float d = opaque(mx / -8.0f);
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t q[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x0 = __fmul_rn(x[e], id);
            const int t0 = (int)(int8_t)(int)__fadd_rn(x0, 8.5f);
            q[e] = (uint32_t)(t0 < 15 ? t0 : 15);
        }
        // byte i = value i | value i + 16 << 4: lanes 0, 1 take lanes 2, 3's codes
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lo |= q[e] << (8 * e);
            hi |= q[e + 4] << (8 * e);
        }
        const uint32_t plo = row_xor_u32<2>(lo, j);
        const uint32_t phi = row_xor_u32<2>(hi, j);
        if (write) {
            uint16_t* d16 = reinterpret_cast<uint16_t*>(entry + 18 * ib);
            if (l == 0) d16[0] = f32_to_f16_bits(d);
            if (l < 2) {
                const uint32_t w0 = lo | (plo << 4), w1 = hi | (phi << 4);
                d16[1 + 4 * l] = (uint16_t)(w0 & 0xffffu);
                d16[2 + 4 * l] = (uint16_t)(w0 >> 16);
                d16[3 + 4 * l] = (uint16_t)(w1 & 0xffffu);
                d16[4 + 4 * l] = (uint16_t)(w1 >> 16);
            }
        }
    }
}

template <bool BF16>
__device__ __forceinline__ void unpack8(const u32x4 w, float* x) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        x[2 * e] = half_to_f32<BF16>((uint16_t)(w[e] & 0xffffu));
        x[2 * e + 1] = half_to_f32<BF16>((uint16_t)(w[e] >> 16));
    }
}

// Each 16-lane group owns R consecutive rows (heads h0 .. h0+R-1 of one
// token); groups 0 .. T*Hkv/R-1 are the K rows (norm, RoPE, append of K and
// V), the rest the Q rows; 16 groups per 256-thread workgroup.  Every load of
// the group's rows is issued before the first row is processed.
template <bool BF16, int ST, int KB, int VB, int R, int RQ>
__global__ void __launch_bounds__(256)
fused_norm_rope_kernel(FusedParams p) {
    __shared__ __attribute__((aligned(16))) float sq[16][128];  // TurboQuant norm chain, per group
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int gi = threadIdx.x >> 4;
    const int64_t nk = (int64_t)p.T * (p.Hkv / R);
    const int64_t ng = nk + (int64_t)p.T * (p.Hq / RQ);
    const int64_t g0 = (int64_t)blockIdx.x * 16 + gi;
    const bool live = g0 < ng;
    const int64_t g = live ? g0 : 0;  // dead groups repeat row 0 without writing
    const bool is_k = g < nk;
    const int H = is_k ? p.Hkv : p.Hq;
    const int nr = is_k ? R : RQ;  // rows of this group
    const int64_t r0 = is_k ? g * R : (g - nk) * RQ;  // row t*H + h0
    const int64_t t = r0 / H;
    const int h0 = (int)(r0 % H);
    uint16_t* rows = (is_k ? p.k : p.q) + r0 * 128;
    const uint16_t* w = is_k ? p.kw : p.qw;

    // ---- loads
    u32x4 xr[RQ], wr_[RQ], vr[R];
#pragma unroll
    for (int r = 0; r < RQ; ++r)
        if (r < nr) xr[r] = *reinterpret_cast<const u32x4*>(rows + r * 128 + 8 * j);
    if constexpr (ST != ST_NONE) {
        if (is_k) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                vr[r & (R - 1)] = *reinterpret_cast<const u32x4*>(p.v + (r0 + r) * 128 + 8 * j);
        }
    }
    const uint16_t* cs = p.cs + p.pos[t] * 128;
    float c[8], sn[8];
    if (p.neox) {
        // lane j < 8 holds a (dims 8j ..), lane j + 8 the b of the same pairs
        const int d0 = 8 * (j & 7);
        load8<BF16>(cs + d0, c);
        load8<BF16>(cs + 64 + d0, sn);
    } else {
        // pairs (8j + 2i, 8j + 2i + 1), pair index 4j + i
        const uint2 cw = *reinterpret_cast<const uint2*>(cs + 4 * j);
        const uint2 sw = *reinterpret_cast<const uint2*>(cs + 64 + 4 * j);
        const uint32_t cc[2] = {cw.x, cw.y}, ss[2] = {sw.x, sw.y};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[i] = half_to_f32<BF16>((uint16_t)(cc[i >> 1] >> (16 * (i & 1))));
            sn[i] = half_to_f32<BF16>((uint16_t)(ss[i >> 1] >> (16 * (i & 1))));
        }
    }
    if (w) {  // the same in the whole group
#pragma unroll
        for (int r = 0; r < RQ; ++r)
            if (r < nr) wr_[r] = *reinterpret_cast<const u32x4*>(w + (int64_t)(h0 + r) * 128 + 8 * j);
    }
    int64_t slot = -1;
    if constexpr (ST != ST_NONE) {
        if (is_k && live) slot = p.slots[t];
    }

#pragma unroll
    for (int r = 0; r < RQ; ++r) {
        if (r >= nr) break;  // K groups: R rows (r < R below)
        const int h = h0 + r;
        float x[8];
        unpack8<BF16>(xr[r], x);
        if (w) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) s = __builtin_fmaf(x[e], x[e], s);
            s = row_sum16(s);
            const float inv = 1.0f / sqrtf(s / 128.0f + p.eps);
            float wv[8];
            unpack8<BF16>(wr_[r], wv);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float u = x[e] * inv;
                u = u * wv[e];
                x[e] = round_half<BF16>(u);
            }
        }
        // RoPE
        float y[8];
        if (p.neox) {
            float o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = row_xor<8>(x[e], j);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float t0 = x[e] * c[e], t1 = o[e] * sn[e];
                y[e] = j < 8 ? t0 - t1 : t0 + t1;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float a = x[2 * i], b = x[2 * i + 1];
                float t0 = a * c[i], t1 = b * sn[i];
                y[2 * i] = t0 - t1;
                t0 = b * c[i];
                t1 = a * sn[i];
                y[2 * i + 1] = t0 + t1;
            }
        }
        const u32x4 yw = pack8<BF16>(y);
        if (live) *reinterpret_cast<u32x4*>(rows + r * 128 + 8 * j) = yw;

        // ---- append (K rows)
        if constexpr (ST != ST_NONE) {
            if (is_k) {
#pragma unroll
                for (int e = 0; e < 8; ++e) y[e] = round_half<BF16>(y[e]);
                const bool wr = slot >= 0;
                float vv[8];
                if constexpr (ST == ST_TQ || ST == ST_G32 || ST == ST_K8) {
                    unpack8<BF16>(vr[r & (R - 1)], vv);
                    const int64_t blk = slot / p.bs, off = slot % p.bs;
                    uint8_t* sp = p.kc + blk * p.bs * p.Hkv * p.SA + off * p.Hkv * p.SA + (int64_t)h * p.SA;
                    if constexpr (ST == ST_K8) {
                        k8v4_store_vec<BF16>(y, vv, j, sp, wr, p.e4b15);
                    } else if constexpr (ST == ST_TQ) {
                        tq_store_vec<128, KB, VB, BF16>(y, vv, j, sp, wr, sq[gi], p.tab, p.mse_bytes,
                                                        p.key_packed, p.val_data);
                    } else {
                        constexpr int P = KB == 4 ? 80 : 56;
                        const uint32_t sbits = (p.sg.w[j >> 2] >> (8 * (j & 3))) & 0xffu;
                        g32_rotate(y, j, sbits, p.tab.rot_c);
                        g32_quantize<KB>(y, j, sp, wr);
                        g32_rotate(vv, j, sbits, p.tab.rot_c);
                        g32_quantize<KB>(vv, j, sp + P, wr);
                    }
                } else {
                    const int64_t eo = kv_entry_offset(wr ? slot : 0, h, p.bs, p.Hkv, p.E, p.stride, p.hnd != 0);
                    if constexpr (ST == ST_F16 || ST == ST_BF16) {
                        constexpr bool DB = ST == ST_BF16;
                        u32x4 vw = vr[r & (R - 1)], kw = yw;
                        if constexpr (DB != BF16) {
                            unpack8<BF16>(vr[r & (R - 1)], vv);
                            vw = pack8<DB>(vv);
                            kw = pack8<DB>(y);
                        }
                        if (wr) {
                            *reinterpret_cast<u32x4*>(p.kc + eo + 16 * j) = kw;
                            *reinterpret_cast<u32x4*>(p.vc + eo + 16 * j) = vw;
                        }
                    } else {
                        unpack8<BF16>(vr[r & (R - 1)], vv);
                        gguf_block4<ST>(y, j, p.kc + eo, wr);
                        gguf_block4<ST>(vv, j, p.vc + eo, wr);
                    }
                }
            }
        }
    }
}

template <bool BF16, int ST, int KB, int VB, int R, int RQ>
int launch_r(const FusedParams& prm, hipStream_t s) {
    const int64_t ng = (int64_t)prm.T * (prm.Hq / RQ + prm.Hkv / R);
    const int64_t grid = (ng + 15) / 16;
    if (grid > 0x7fffffff) return VMC_EINVAL;
    if (grid == 0) return VMC_OK;
    hipLaunchKernelGGL((fused_norm_rope_kernel<BF16, ST, KB, VB, R, RQ>), dim3((unsigned)grid), dim3(256), 0, s,
                       prm);
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}

// rows per group: Q groups 4 when Hq allows it (four 16-byte loads in flight
// per lane); K groups, which also append (more registers), 2 -- fewer
// registers for the whole kernel, so more waves for the Q rows -- or 4 when
// there is no append; else 2, else 1
template <bool BF16, int ST, int KB = 0, int VB = 0>
int launch_fused(const FusedParams& prm, hipStream_t s) {
    if (prm.Hq % 4 == 0 && prm.Hkv % 2 == 0) return launch_r<BF16, ST, KB, VB, ST == ST_NONE ? 4 : 2, 4>(prm, s);
    if (prm.Hq % 2 == 0 && prm.Hkv % 2 == 0) return launch_r<BF16, ST, KB, VB, 2, 2>(prm, s);
    return launch_r<BF16, ST, KB, VB, 1, 1>(prm, s);
}

template <bool BF16>
int dispatch(const FusedParams& prm, int st, const vmc_tq_config* c, hipStream_t s) {
    switch (st) {
        case ST_NONE: return launch_fused<BF16, ST_NONE>(prm, s);
        case ST_F16: return launch_fused<BF16, ST_F16>(prm, s);
        case ST_BF16: return launch_fused<BF16, ST_BF16>(prm, s);
        case ST_Q8_0: return launch_fused<BF16, ST_Q8_0>(prm, s);
        case ST_Q4_0: return launch_fused<BF16, ST_Q4_0>(prm, s);
        case ST_K8: return launch_fused<BF16, ST_K8>(prm, s);
        case ST_G32:
            return c->key_quant_bits == 4 ? launch_fused<BF16, ST_G32, 4, 4>(prm, s)
                                          : launch_fused<BF16, ST_G32, 3, 3>(prm, s);
        case ST_TQ: {
            const int kb = c->key_quant_bits, vb = c->value_quant_bits;
            if (kb == 4 && vb == 4) return launch_fused<BF16, ST_TQ, 4, 4>(prm, s);
            if (kb == 3 && vb == 3) return launch_fused<BF16, ST_TQ, 3, 3>(prm, s);
            if (kb == 3 && vb == 4) return launch_fused<BF16, ST_TQ, 3, 4>(prm, s);
            return VMC_EINVAL;
        }
        default: return VMC_EINVAL;
    }
}

}  // namespace
}  // namespace vmc

using namespace vmc;

extern "C" int vmc_fused_qk_norm_rope_store(void* q_buf, void* k_buf, const void* v_buf,
                                            const void* q_norm_weight, const void* k_norm_weight,
                                            const void* cos_sin_cache, const int64_t* position_ids,
                                            void* key_cache, void* value_cache,
                                            const int64_t* slot_mapping, int num_tokens,
                                            int num_heads, int num_kv_heads, int head_dim,
                                            float rms_norm_eps, int is_neox, int64_t block_size,
                                            int64_t cache_stride, int kv_format, int layout,
                                            const vmc_tq_config* tq_config, int dtype,
                                            vmc_stream_t stream) {
    if (head_dim != 128 || num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0) return VMC_EINVAL;
    if (dtype != VMC_DTYPE_F16 && dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (num_tokens == 0) return VMC_OK;
    if (!q_buf || !k_buf || !cos_sin_cache || !position_ids) return VMC_EINVAL;
    FusedParams prm = {};
    prm.q = reinterpret_cast<uint16_t*>(q_buf);
    prm.k = reinterpret_cast<uint16_t*>(k_buf);
    prm.v = reinterpret_cast<const uint16_t*>(v_buf);
    prm.qw = reinterpret_cast<const uint16_t*>(q_norm_weight);
    prm.kw = reinterpret_cast<const uint16_t*>(k_norm_weight);
    prm.cs = reinterpret_cast<const uint16_t*>(cos_sin_cache);
    prm.pos = position_ids;
    prm.T = num_tokens;
    prm.Hq = num_heads;
    prm.Hkv = num_kv_heads;
    prm.eps = rms_norm_eps;
    prm.neox = is_neox != 0;
    int st = ST_NONE;
    if (key_cache) {
        if (!v_buf || !slot_mapping || block_size <= 0) return VMC_EINVAL;
        prm.kc = reinterpret_cast<uint8_t*>(key_cache);
        prm.slots = slot_mapping;
        prm.bs = block_size;
        if (tq_config) {
            if (!tq_config_valid(tq_config) || tq_config->head_dim != head_dim) return VMC_EINVAL;
            prm.SA = tq_config->slot_size_aligned;
            prm.mse_bytes = tq_config->mse_bytes;
            prm.key_packed = tq_config->key_packed_size;
            prm.val_data = tq_config->val_data_bytes;
            if (tq_config->key_fp8) {
                prm.e4b15 = tq_config->fp8_e4b15 ? 1 : 0;
                st = ST_K8;
            } else {
                prm.tab = tq_tables(head_dim, tq_config->key_quant_bits);
                prm.sg = g32_signs(tq_config->sign_seed);
                st = tq_config->group_size != 0 ? ST_G32 : ST_TQ;
            }
        } else {
            const int64_t E = vmc_kv_entry_bytes(kv_format, head_dim);
            if (E < 0 || !value_cache) return VMC_EINVAL;
            if (layout != VMC_LAYOUT_NHD && layout != VMC_LAYOUT_HND) return VMC_EINVAL;
            prm.vc = reinterpret_cast<uint8_t*>(value_cache);
            prm.E = E;
            prm.stride = cache_stride > 0 ? cache_stride : block_size * num_kv_heads * E;
            // a page must hold block_size * num_kv_heads entries, and f16/bf16
            // pages are written with 16-byte stores
            if (prm.stride < block_size * num_kv_heads * E) return VMC_EINVAL;
            if ((kv_format == VMC_KV_F16 || kv_format == VMC_KV_BF16) && (prm.stride % 16) != 0)
                return VMC_EINVAL;
            prm.hnd = layout == VMC_LAYOUT_HND;
            st = kv_format == VMC_KV_F16 ? ST_F16 : kv_format == VMC_KV_BF16 ? ST_BF16
               : kv_format == VMC_KV_Q8_0 ? ST_Q8_0 : ST_Q4_0;
        }
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    return dtype == VMC_DTYPE_BF16 ? dispatch<true>(prm, st, tq_config, s) : dispatch<false>(prm, st, tq_config, s);
}
