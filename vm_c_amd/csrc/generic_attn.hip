// generic_attn.hip -- head_dim 64 and 256.
//
// The head_dim 128 kernels are tuned per format (16 lanes x 8 dims per
// vector, MFMA tiles of 128-dim rows).  The other head sizes the reference
// accepts (TQConfig::kMaxSupportedHeadDim = 256, kernels_turboquant.h:11;
// prefill head dims 64 / 128 / 256, attention_kernels.cu:270-371) run here,
// written once for every source:
//   gen_tq_store_kernel: one wave per (token, kv head) vector, the TurboQuant
//     slot in the reference's order of operations (turboquant_kernels.cu:
//     145-351; the rotation in the butterfly order the oracle declares),
//     bit-identical to the oracle's store.
//   gen_attn_kernel: one wave per (query row, query head).  Keys go 64 at a
//     time, one per lane: the lane dequantizes its key's K entry and takes the
//     dot product with q (in LDS; rotated for TurboQuant codebook keys), the
//     wave runs the online softmax over the 64 scores, then every lane
//     accumulates its D / 64 output dims over the 64 keys' V entries.
// Sources: f16 / bf16 / q8_0 / q4_0 pages (NHD or HND), TurboQuant slots
// (codebook keys with norm correction, or fp8 keys; 3- or 4-bit values), and
// this step's contiguous K/V rows (local prefill).
#include "generic_attn.hpp"
#include "vmc_common.hpp"
#include "vmc_store.hpp"
#include "vmc_tq.hpp"

namespace vmc {
namespace {

constexpr int kWpb = 4;  // waves (vectors / query heads) per workgroup

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
    return v;
}
__device__ __forceinline__ float wave_min_f(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fminf(v, shfl_xor(v, m));
    return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
    return v;
}

// y = butterflies of half-width 1, 2, .., D/2 over LDS y[0..D) (the
// declared rotation order), by the 64 lanes of one wave; the caller scales
template <int D>
__device__ __forceinline__ void wht_lds(float* y, int lane) {
#pragma unroll
    for (int hw = 1; hw < D; hw <<= 1) {
#pragma unroll
        for (int b0 = 0; b0 < D / 2; b0 += 64) {
            const int b = b0 + lane;
            if (b < D / 2) {
                const int j = (b / hw) * 2 * hw + (b % hw);
                const float a = y[j], c = y[j + hw];
                y[j] = a + c;
                y[j + hw] = a - c;
            }
        }
        wave_sync();
    }
}

// fp8 key byte -> float (fp8_e4m3_to_float / fp8_e4b15_to_float,
// turboquant_kernels.cu:85-96, :136-143): (1 + m/8) 2^(e - bias), zero codes
// signed zero
__device__ __forceinline__ float fp8_decode(uint32_t b, int e4b15) {
    const uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
    float v = 0.0f;
    if (e != 0 || m != 0) v = ldexpf(1.0f + (float)m * 0.125f, (int)e - (e4b15 ? 15 : 7));
    return (b & 0x80u) ? -v : v;
}

// codes 8g .. 8g+7 of a packed TurboQuant code array (2-byte aligned):
// 4-bit -> 4 bytes at 4g (even d low nibble), 3-bit -> 3 bytes at 3g, code
// i at bits 3i; returned as a word with code i at bits BITS * i
template <int BITS>
__device__ __forceinline__ uint32_t codes8(const uint8_t* p, int g) {
    if constexpr (BITS == 4) {
        return ld_u16(p + 4 * g) | (ld_u16(p + 4 * g + 2) << 16);
    } else {
        const int o = 3 * g, a = o & ~1;
        const uint32_t w = ld_u16(p + a) | (ld_u16(p + a + 2) << 16);
        return (w >> (8 * (o & 1))) & 0xffffffu;
    }
}
template <int BITS>
__device__ __forceinline__ uint32_t code_at(const uint8_t* p, int d) {
    if constexpr (BITS == 4) {
        return (p[d >> 1] >> (4 * (d & 1))) & 0xfu;
    } else {
        return (codes8<3>(p, d >> 3) >> (3 * (d & 7))) & 7u;
    }
}

template <bool BF>
__device__ __forceinline__ float ld_half(const uint8_t* p) {
    return half_to_f32<BF>((uint16_t)ld_u16(p));
}

// ------------------------------------------------------------------ store

template <int D, int KB, int VB, bool BF, bool FP8>
__global__ void __launch_bounds__(64 * kWpb)
gen_tq_store_kernel(const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
                    uint8_t* __restrict__ cache, const int64_t* __restrict__ slots, int T, int Hkv,
                    int64_t bs, int S, int mse_bytes, int key_packed, int val_data, int e4b15,
                    TQTables tab) {
    constexpr int NPL = D / 64;
    __shared__ float ys[kWpb][D];
    __shared__ uint8_t cs[kWpb][D];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t pid = (int64_t)blockIdx.x * kWpb + w;
    if (pid >= (int64_t)T * Hkv) return;
    const int64_t t = pid / Hkv;
    const int h = (int)(pid % Hkv);
    const int64_t slot = slots[t];
    if (slot < 0) return;  // turboquant_kernels.cu:266-267
    const int64_t blk = slot / bs, off = slot % bs;
    uint8_t* sp = cache + blk * bs * Hkv * S + off * Hkv * S + (int64_t)h * S;
    float* y = ys[w];
    uint8_t* c = cs[w];
    float kf[NPL], vf[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        kf[i] = half_to_f32<BF>(key[pid * D + lane + 64 * i]);
        vf[i] = half_to_f32<BF>(value[pid * D + lane + 64 * i]);
    }
    // codes of 8 dims -> the packed array at p (4-bit: 4 bytes at 4g; 3-bit: 3 bytes at 3g)
    auto pack = [&](uint8_t* p, int bits) {
        if (lane < D / 8) {
            const int g = lane;
            uint32_t wv = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) wv |= (uint32_t)c[8 * g + i] << (bits * i);
            if (bits == 4) {
                reinterpret_cast<uint16_t*>(p)[2 * g] = (uint16_t)(wv & 0xffffu);
                reinterpret_cast<uint16_t*>(p)[2 * g + 1] = (uint16_t)(wv >> 16);
            } else {
                p[3 * g] = (uint8_t)(wv & 0xffu);
                p[3 * g + 1] = (uint8_t)((wv >> 8) & 0xffu);
                p[3 * g + 2] = (uint8_t)((wv >> 16) & 0xffu);
            }
        }
        wave_sync();
    };
    if constexpr (FP8) {
        // half_to_fp8_store_kernel (:188-245): K byte d = fp8(k[d])
#pragma unroll
        for (int i = 0; i < NPL; ++i) sp[lane + 64 * i] = (uint8_t)fp8_encode(kf[i], e4b15);
    } else {
        // norm: the sequential fmaf chain over d = 0 .. D-1 (:145-161), every
        // lane the same chain; x = k * (1 / (norm + 1e-8f)) (:163-175)
#pragma unroll
        for (int i = 0; i < NPL; ++i) y[lane + 64 * i] = kf[i];
        wave_sync();
        float nsq = 0.0f;
        for (int d = 0; d < D; ++d) nsq = __builtin_fmaf(y[d], y[d], nsq);
        const float norm = sqrtf(nsq);
        const float inv = 1.0f / (norm + 1e-8f);
        wave_sync();
#pragma unroll
        for (int i = 0; i < NPL; ++i) y[lane + 64 * i] = __fmul_rn(kf[i], inv);
        wave_sync();
        wht_lds<D>(y, lane);
        // code = #midpoints <= y / sqrt(D) (the reference's top-down scan, :283-304)
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const float v = __fmul_rn(y[lane + 64 * i], tab.rot_c);
            int idx = 0;
#pragma unroll
            for (int m = 0; m < (1 << KB) - 1; ++m) idx += (v >= tab.midpoints[m]) ? 1 : 0;
            c[lane + 64 * i] = (uint8_t)idx;
        }
        wave_sync();
        pack(sp, KB);
        if (lane == 0) *reinterpret_cast<uint16_t*>(sp + mse_bytes) = f32_to_half<BF>(norm);
    }
    // V: asymmetric min / max codes, scale and zero (:314-350)
    float lo = vf[0], hi = vf[0];
#pragma unroll
    for (int i = 1; i < NPL; ++i) {
        lo = fminf(lo, vf[i]);
        hi = fmaxf(hi, vf[i]);
    }
    const float vmin = wave_min_f(lo), vmax = wave_max_f(hi);
    constexpr int VMAXQ = VB == 4 ? 15 : 7;
    const float vscale = fmaxf((vmax - vmin) / (float)VMAXQ, 1e-8f);
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int qq = (int)roundf((vf[i] - vmin) / vscale);
        c[lane + 64 * i] = (uint8_t)(qq < 0 ? 0 : (qq > VMAXQ ? VMAXQ : qq));
    }
    wave_sync();
    uint8_t* vp = sp + key_packed;
    pack(vp, VB);
    if (lane == 0) {
        *reinterpret_cast<uint16_t*>(vp + val_data) = f32_to_half<BF>(vscale);
        *reinterpret_cast<uint16_t*>(vp + val_data + 2) = f32_to_half<BF>(vmin);
    }
}

// ------------------------------------------------------------------ attention

template <int D, int SRC, int KB, int VB, bool BF>
__global__ void __launch_bounds__(64 * kWpb)
gen_attn_kernel(GenArgs a, TQTables tab) {
    constexpr int NPL = D / 64;
    __shared__ float qsm[kWpb][D];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x;
    const int hq = blockIdx.y * kWpb + w;
    if (hq >= a.Hq) return;
    const int g = hq / (a.Hq / a.Hkv);
    uint16_t* op = reinterpret_cast<uint16_t*>(a.out) + ((int64_t)row * a.Hq + hq) * D;

    // the row's keys: n of them, positions 0 .. n-1 of sequence seq, or local
    // tokens base .. base + n - 1
    int n = 0, seq = 0, base = 0;
    if constexpr (SRC == GEN_LOCAL) {
        n = a.pos[row] + 1;
        base = row - a.pos[row];
    } else if (!a.tok_seq) {
        seq = row;
        n = a.seq_lens[row];
    } else {
        seq = a.tok_seq[row];
        n = a.pos[row] + 1;
        if (a.num_seqs >= 0 && (seq < 0 || seq >= a.num_seqs)) n = 0;
    }
    // paged rows: no further than the block-table row reaches
    if constexpr (SRC != GEN_LOCAL) n = (int)min((int64_t)n, a.max_blocks * a.bs);
    if (n <= 0) {
#pragma unroll
        for (int i = 0; i < NPL; ++i) op[lane + 64 * i] = f32_to_half<BF>(0.0f);
        return;
    }

    // q in LDS as fp32; TurboQuant codebook keys: q_rot = H q / sqrt(D)
    float* qs = qsm[w];
    const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q) + ((int64_t)row * a.Hq + hq) * D;
#pragma unroll
    for (int i = 0; i < NPL; ++i) qs[lane + 64 * i] = half_to_f32<BF>(qp[lane + 64 * i]);
    wave_sync();
    constexpr bool kRot = SRC == GEN_TQ && KB != 8;
    if constexpr (kRot) {
        wht_lds<D>(qs, lane);
#pragma unroll
        for (int i = 0; i < NPL; ++i) qs[lane + 64 * i] = qs[lane + 64 * i] * tab.rot_c;
        wave_sync();
    }

    const int64_t seq_bt = (int64_t)seq * a.max_blocks;
    // byte address of position k's entry in pool p (null when its page is a hole)
    auto entry_of = [&](const uint8_t* p, int k) -> const uint8_t* {
        const int32_t pg = a.bt[seq_bt + k / a.bs];
        if (pg < 0) return nullptr;
        const int64_t r = k % a.bs;
        const int64_t idx = a.hnd ? ((int64_t)pg * a.Hkv + g) * a.bs + r : ((int64_t)pg * a.bs + r) * a.Hkv + g;
        return p + idx * a.entry;
    };

    float m = -__builtin_inff(), l = 0.0f, acc[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) acc[i] = 0.0f;
    for (int k0 = 0; k0 < n; k0 += 64) {
        const int kk = k0 + lane;
        const uint8_t* ke = nullptr;
        const uint8_t* ve = nullptr;
        bool valid = kk < n;
        if (valid) {
            if constexpr (SRC == GEN_LOCAL) {
                const int64_t o = (((int64_t)base + kk) * a.Hkv + g) * D * 2;
                ke = reinterpret_cast<const uint8_t*>(a.k) + o;
                ve = reinterpret_cast<const uint8_t*>(a.v) + o;
            } else {
                ke = entry_of(a.kp, kk);
                ve = SRC == GEN_TQ ? ke : (ke ? entry_of(a.vp, kk) : nullptr);
                valid = ke != nullptr;
            }
        }
        // ---- score of this lane's key
        float s = -__builtin_inff();
        if (valid) {
            float dot = 0.0f;
            if constexpr (SRC == GEN_F16 || SRC == GEN_BF16 || SRC == GEN_LOCAL) {
                constexpr bool KBF = SRC == GEN_BF16 || (SRC == GEN_LOCAL && BF);
                for (int d = 0; d < D; d += 2) {
                    const uint32_t wv = *reinterpret_cast<const uint32_t*>(ke + 2 * d);
                    dot = __builtin_fmaf(qs[d], half_to_f32<KBF>((uint16_t)(wv & 0xffffu)), dot);
                    dot = __builtin_fmaf(qs[d + 1], half_to_f32<KBF>((uint16_t)(wv >> 16)), dot);
                }
            } else if constexpr (SRC == GEN_Q8 || SRC == GEN_Q4) {
                constexpr int BE = SRC == GEN_Q8 ? 34 : 18;
                for (int b = 0; b < D / 32; ++b) {
                    const uint8_t* blk = ke + BE * b;
                    const float db = ld_half<false>(blk);
                    float part = 0.0f;
                    for (int j = 0; j < 32; ++j) {
                        int x;
                        if constexpr (SRC == GEN_Q8) x = (int)(int8_t)blk[2 + j];
                        else x = (int)((blk[2 + (j & 15)] >> (j < 16 ? 0 : 4)) & 0xf) - 8;
                        part = __builtin_fmaf(qs[32 * b + j], (float)x, part);
                    }
                    dot = __builtin_fmaf(db, part, dot);
                }
            } else if constexpr (KB == 8) {
                // fp8 keys: q not rotated, no norm
                for (int d = 0; d < D; ++d) dot = __builtin_fmaf(qs[d], fp8_decode(ke[d], a.fp8_e4b15), dot);
            } else {
                // codebook keys: C[code] / ||C[codes]|| * norm (tq_decode_stage1 :416-450)
                float cn = 0.0f;
                for (int gq = 0; gq < D / 8; ++gq) {
                    const uint32_t cw = codes8<KB>(ke, gq);
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const float cv = tab.centroids[(cw >> (KB * i)) & ((1u << KB) - 1)];
                        dot = __builtin_fmaf(qs[8 * gq + i], cv, dot);
                        cn = __builtin_fmaf(cv, cv, cn);
                    }
                }
                const float ci = a.norm_correction ? 1.0f / sqrtf(cn + 1e-16f) : 1.0f;
                dot = dot * ci * ld_half<BF>(ke + a.mse_bytes);
            }
            s = dot * a.scale;
        }
        // ---- online softmax over the 64 keys
        const float mc = wave_max_f(s);
        const float m_new = fmaxf(m, mc);
        if (m_new == -__builtin_inff()) continue;  // no key so far (uniform)
        const float alpha = expf(m - m_new);  // 0 from -inf
        const float p = valid ? expf(s - m_new) : 0.0f;
        l = l * alpha + wave_sum_f(p);
#pragma unroll
        for (int i = 0; i < NPL; ++i) acc[i] *= alpha;
        m = m_new;
        // ---- O += p V: lane owns dims lane + 64 i
        const uintptr_t vaddr = (uintptr_t)ve;
        for (int j = 0; j < 64 && k0 + j < n; ++j) {
            const float pj = shfl(p, j);
            if (pj == 0.0f) continue;  // masked, a hole, or underflow (uniform)
            const uint32_t lo32 = (uint32_t)__shfl((int)(uint32_t)vaddr, j, kWave);
            const uint32_t hi32 = (uint32_t)__shfl((int)(uint32_t)(vaddr >> 32), j, kWave);
            const uint8_t* vj = reinterpret_cast<const uint8_t*>(((uint64_t)hi32 << 32) | lo32);
            float vs = 0.0f, vz = 0.0f;
            if constexpr (SRC == GEN_TQ) {
                vs = ld_half<BF>(vj + a.key_packed + a.val_data);
                vz = ld_half<BF>(vj + a.key_packed + a.val_data + 2);
            }
#pragma unroll
            for (int i = 0; i < NPL; ++i) {
                const int d = lane + 64 * i;
                float v;
                if constexpr (SRC == GEN_F16 || SRC == GEN_BF16 || SRC == GEN_LOCAL) {
                    constexpr bool VBF = SRC == GEN_BF16 || (SRC == GEN_LOCAL && BF);
                    v = ld_half<VBF>(vj + 2 * d);
                } else if constexpr (SRC == GEN_Q8) {
                    const uint8_t* blk = vj + 34 * (d >> 5);
                    v = ld_half<false>(blk) * (float)(int8_t)blk[2 + (d & 31)];
                } else if constexpr (SRC == GEN_Q4) {
                    const uint8_t* blk = vj + 18 * (d >> 5);
                    const int j5 = d & 31;
                    v = ld_half<false>(blk) * (float)((int)((blk[2 + (j5 & 15)] >> (j5 < 16 ? 0 : 4)) & 0xf) - 8);
                } else {
                    v = __builtin_fmaf((float)code_at<VB>(vj + a.key_packed, d), vs, vz);
                }
                acc[i] = __builtin_fmaf(pj, v, acc[i]);
            }
        }
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) op[lane + 64 * i] = f32_to_half<BF>(acc[i] * inv);
}

template <int D, int SRC, int KB, int VB, bool BF>
int launch_gen(const GenArgs& a, const TQTables& tab, hipStream_t s) {
    const dim3 grid((unsigned)a.rows, (unsigned)((a.Hq + kWpb - 1) / kWpb));
    hipLaunchKernelGGL((gen_attn_kernel<D, SRC, KB, VB, BF>), grid, dim3(64 * kWpb), 0, s, a, tab);
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}

template <int D, bool BF>
int dispatch_src(const GenArgs& a, hipStream_t s) {
    TQTables none = {};
    switch (a.src) {
        case GEN_F16: return launch_gen<D, GEN_F16, 0, 0, BF>(a, none, s);
        case GEN_BF16: return launch_gen<D, GEN_BF16, 0, 0, BF>(a, none, s);
        case GEN_Q8: return launch_gen<D, GEN_Q8, 0, 0, BF>(a, none, s);
        case GEN_Q4: return launch_gen<D, GEN_Q4, 0, 0, BF>(a, none, s);
        case GEN_LOCAL: return launch_gen<D, GEN_LOCAL, 0, 0, BF>(a, none, s);
        case GEN_TQ: {
            if (a.key_fp8) {
                if (a.vb != 4) return VMC_EINVAL;
                return launch_gen<D, GEN_TQ, 8, 4, BF>(a, none, s);
            }
            const TQTables& tab = tq_tables(D, a.kb);
            if (a.kb == 4 && a.vb == 4) return launch_gen<D, GEN_TQ, 4, 4, BF>(a, tab, s);
            if (a.kb == 3 && a.vb == 3) return launch_gen<D, GEN_TQ, 3, 3, BF>(a, tab, s);
            if (a.kb == 3 && a.vb == 4) return launch_gen<D, GEN_TQ, 3, 4, BF>(a, tab, s);
            return VMC_EINVAL;
        }
        default: return VMC_EINVAL;
    }
}

template <int D, int KB, int VB, bool BF, bool FP8>
int launch_store_gen(const void* key, const void* value, void* cache, const int64_t* slots, int T, int Hkv,
                     int64_t bs, const vmc_tq_config* c, hipStream_t s) {
    const int64_t n = (int64_t)T * Hkv;
    const int64_t grid = (n + kWpb - 1) / kWpb;
    if (grid > 0x7fffffff) return VMC_EINVAL;
    const TQTables tab = FP8 ? TQTables{} : tq_tables(D, KB);
    hipLaunchKernelGGL((gen_tq_store_kernel<D, KB, VB, BF, FP8>), dim3((unsigned)grid), dim3(64 * kWpb), 0, s,
                       (const uint16_t*)key, (const uint16_t*)value, (uint8_t*)cache, slots, T, Hkv, bs,
                       c->slot_size_aligned, c->mse_bytes, c->key_packed_size, c->val_data_bytes,
                       c->fp8_e4b15, tab);
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}

template <int D, bool BF>
int store_dispatch(const void* key, const void* value, void* cache, const int64_t* slots, int T, int Hkv,
                   int64_t bs, const vmc_tq_config* c, hipStream_t s) {
    if (c->key_fp8) {
        if (c->value_quant_bits != 4) return VMC_EINVAL;
        return launch_store_gen<D, 8, 4, BF, true>(key, value, cache, slots, T, Hkv, bs, c, s);
    }
    const int kb = c->key_quant_bits, vb = c->value_quant_bits;
    if (kb == 4 && vb == 4) return launch_store_gen<D, 4, 4, BF, false>(key, value, cache, slots, T, Hkv, bs, c, s);
    if (kb == 3 && vb == 3) return launch_store_gen<D, 3, 3, BF, false>(key, value, cache, slots, T, Hkv, bs, c, s);
    if (kb == 3 && vb == 4) return launch_store_gen<D, 3, 4, BF, false>(key, value, cache, slots, T, Hkv, bs, c, s);
    return VMC_EINVAL;
}

}  // namespace

int gen_attention(const GenArgs& a, hipStream_t s) {
    if ((a.D != 64 && a.D != 128 && a.D != 256) || a.rows < 0 || a.Hq <= 0 || a.Hkv <= 0 || a.Hq % a.Hkv != 0)
        return VMC_EINVAL;
    if (a.rows == 0) return VMC_OK;
    if (a.rows > 0x7fffffff) return VMC_EINVAL;
    if (a.D == 64) return a.q_bf16 ? dispatch_src<64, true>(a, s) : dispatch_src<64, false>(a, s);
    if (a.D == 128) return a.q_bf16 ? dispatch_src<128, true>(a, s) : dispatch_src<128, false>(a, s);
    return a.q_bf16 ? dispatch_src<256, true>(a, s) : dispatch_src<256, false>(a, s);
}

int gen_tq_store(const void* key, const void* value, void* cache, const int64_t* slots, int T, int Hkv, int D,
                 int64_t bs, const vmc_tq_config* c, bool bf16, hipStream_t s) {
    if (!generic_head_dim(D) || c->group_size != 0) return VMC_EINVAL;
    if (D == 64)
        return bf16 ? store_dispatch<64, true>(key, value, cache, slots, T, Hkv, bs, c, s)
                    : store_dispatch<64, false>(key, value, cache, slots, T, Hkv, bs, c, s);
    return bf16 ? store_dispatch<256, true>(key, value, cache, slots, T, Hkv, bs, c, s)
                : store_dispatch<256, false>(key, value, cache, slots, T, Hkv, bs, c, s);
}

}  // namespace vmc
