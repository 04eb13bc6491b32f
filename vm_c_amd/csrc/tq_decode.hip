// tq_decode.hip -- split-KV paged decode over TurboQuant slots, gfx950:
// the reference layout (turboquant_4bit_nc / k3v4_nc, and 3bit_nc with other
// than 8 KV heads -- tq_stream.hip takes 3-bit slots with 8) with at most 8
// query heads per KV head, and (G32) the per-32-group variant of the same
// slots (turboquant_4bit_g32 / 3bit_g32; its format is defined in
// vmc_attn.h, the reference has no code for it).
//
// Replaces the decode of vm_c::turboquant_decode_attention
// (src/cuda/turboquant_kernels.cu:939-1007: q rotation, stage 1 :353-506,
// stage 2 :508-547); the arithmetic is that of paged_decode.hip's TurboQuant
// path (K = C[code] * norm / ||C[codes]||, V = code * scale + zero, fp32
// online softmax, the same page-range plan and merge), restructured for
// latency hiding:
//
//  * every wave streams its own KV head: its DMA ring holds the head's
//    16 token runs of each page (slot bytes at a 16-byte window), fetched by
//    load-to-LDS transfers the wave issues and waits for itself -- no
//    workgroup barrier inside the page loop;
//  * token rows sit in LDS at an odd number of 16-byte chunks, so the 16 rows
//    a lane group reads fall on 16 distinct bank groups;
//  * the transfers are ordinary (cached) loads: the 16-byte windows of
//    neighbouring heads share their boundary chunks, which L2 then serves
//    once (measured: a non-temporal hint fetches 1.37x the bytes and runs
//    ~10% slower);
//  * three page pairs are in flight per wave (four pages of transfers behind
//    the pair whose bytes are being read), and the raw bytes of pair k+1
//    (key code words, norms, value code runs, scales and zeros) are read
//    from LDS while pair k is computed from registers: the LDS latency of
//    one pair hides behind the arithmetic of the other.
//
// Per wave and page pair (32 tokens x G <= 8 query heads), as in
// paged_decode.hip: S^T = K . Q^T on v_mfma_f32_16x16x32_f16 with the
// first page's heads in S columns 0-7 and the second's in 8-15 (a
// block-diagonal Q^T), ||C[codes]||^2 from the Gram diagonal K K^T, online
// softmax in the log2 domain with a lazy reference max, O += P . V with the V
// codes as exact fp16 subnormals and sum(P * zero) kept apart.
#include "decode_plan.hpp"

namespace vmc {
namespace {

// Compile-time geometry of one slot layout: the reference's
// (turboquant_kernels.cu:29-45), or the per-32-group variant (G32: K part
// then V part, four blocks of be bytes each -- fp16 d and 12 code bytes at
// 3 bits, fp16 d, m and 16 code bytes at 4 bits).
template <int KB, int VB, bool G32 = false>
struct TqGeo {
    static constexpr int mse = 16 * KB, kp = mse + 2, vd = 16 * VB;
    static constexpr int be = KB == 3 ? 14 : 20;  // G32 block bytes
    static constexpr int part = 4 * be;           // G32 K part bytes
    static constexpr int slot = G32 ? 2 * part : (kp + vd + 4 + 1) / 2 * 2;
    // a head's run starts at most 14 bytes into its 16-byte window
    static constexpr int nch = (14 + slot + 15) / 16;
    static constexpr int nchp = nch | 1;  // odd: 16 rows -> 16 distinct bank groups
    static constexpr int row = 16 * nchp;  // LDS bytes per token row
    static constexpr int page = kBs * row;  // one page of one KV head
    static constexpr int waves = 8;
    // page buffers per wave: four pairs where they fit the LDS beside the
    // tables, else three (the 3-bit key table takes 32 KB)
    static constexpr int npair = waves * 8 * page + 12 * 1024 + (KB == 3 ? 32768 : 0) <= 160 * 1024 ? 4 : 3;
    static constexpr int nb = 2 * npair;
    static constexpr int spt = (kBs * nchp + 63) / 64;  // transfers per page
    static_assert(spt == 3, "the vmcnt bookkeeping counts three transfers per page");
    static_assert(nb * page < 60000, "a wave's ring offsets must fit the LDS instruction offset");
};

template <int KB, int VB, bool G32>
struct alignas(16) TqLds {
    using TG = TqGeo<KB, VB, G32>;
    // 3-bit keys: four fp16 centroids per 12 bits of codes (8-byte entries;
    // measured faster than the conflict-free 64-entry pair table, whose two
    // lookups per 12 bits cost more index arithmetic than the conflicts cost);
    // G32: four exact fp16 (code - 4), keys and values
    u32x2 lut4[KB == 3 ? 4096 : 1];
    uint32_t lut[256];  // key code pair -> two fp16 centroids
    uint8_t ring[TG::waves][TG::nb][TG::page];
    float wscr[TG::waves][80];  // per-wave exchange
    int32_t bt[256];            // block of each page of the chunk
    int32_t info[256];          // b << 6 | valid tokens << 1 | piece ends
    int32_t seg_b[256], seg_ps[256], seg_L[256];
    WGPlan plan;
    int n_seg;
};

// per-32-group variant: two exact fp16 values times d (one packed multiply,
// one rounding each)
__device__ __forceinline__ uint32_t g32_mul(uint32_t c2, f16x2 d2) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, c2) * d2);
}
// 4-bit: two codes of the 16 code bytes (byte i = value i | value i + 16 << 4):
// bytes 2 odd, 2 odd + 1 of w, low nibbles or high (hi), to packed fp16
// code * d + m (fp16 1024 + code under 0x64, a packed subtract, one packed
// FMA)
__device__ __forceinline__ uint32_t g32_nib2(uint32_t w, int odd, bool hi, f16x2 d2, f16x2 m2) {
    const uint32_t sp = __builtin_amdgcn_perm(0u, w, odd ? 0x0c030c02u : 0x0c010c00u);
    const uint32_t z = ((sp >> (hi ? 4 : 0)) & 0x000f000fu) | 0x64006400u;
    const f16x2 c = __builtin_bit_cast(f16x2, z) - f16x2{(_Float16)1024.0f, (_Float16)1024.0f};
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, d2, m2));
}

// one 16-byte-per-lane load-to-LDS transfer, an ordinary cached load: lane
// L's 16 bytes from base + off land at LDS address m0 + 16 L.  Issued from asm, so the
// compiler does not track it (it would make every later LDS read wait for
// all transfers); the kernel counts its own transfers.
__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t off, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(m0) : "memory");
}

// Raw bytes of a page pair in registers.  TqCodes is consumed by the first
// phase of a pair (key table lookups issued, value bytes permuted), so the
// next pair's codes are read into the same registers before the second phase
// runs (G32: the value code words only after it, since its second phase
// still reads this pair's from the copies the first phase made); TqHalves is used by the second phase, and the next pair's halves are
// read into it after that phase (the next step's first phase covers their
// latency).
// wait until at most the transfers of N page pairs (6 each) are outstanding
template <int N>
__device__ __forceinline__ void vmcnt_pairs() {
    static_assert(N >= 1 && N <= 3, "ring depth");
    if constexpr (N == 1) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    else if constexpr (N == 2) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(18)" ::: "memory");
}

template <int KB, int VB>
struct TqCodes {
    uint32_t kd[2][KB == 3 ? 4 : 5];  // key code words of the lane's 32 dims, from the 4-byte floor
    uint32_t cw[2][4][2];             // value code runs of tokens 4*grp + i: two words from the 4-byte floor
};
struct TqHalves {
    uint32_t nrm;        // 16-bit norms of token r16, first page | second << 16
    uint32_t hsz[4][2];  // scale, zero of the lane's page's token 4*grp + i: two words from the 4-byte floor
};

template <int KB, int VB, bool BF, bool G32>
__global__ void __launch_bounds__(512) tq_decode_kernel(DecodeParams p) {
    using TG = TqGeo<KB, VB, G32>;
    using AT = f16x8;
    using CODES = TqCodes<KB, VB>;
    __shared__ TqLds<KB, VB, G32> lds;
    WGPlan& plan = lds.plan;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int r16 = lane & 15, grp = lane >> 4;
    const int w = (int)blockIdx.x;

    // ---- this workgroup's page range (paged_decode.hip's plan)
    if (wave == 0) {
        WGPlan wp;
        if (p.per_seq) {
            int ps = 0, L = 0;
            for (int b0 = 0; b0 < p.B; b0 += 64) {
                const int b = b0 + lane;
                int v = b < w ? seq_pages(p, b, &L) : 0;
#pragma unroll
                for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
                ps += v;
            }
            const int pg = seq_pages(p, w, &L);
            wp = {ps, ps + pg, w, w, 0, 0};
        } else {
            const int T = total_pages(p, lane);
            const int n = effective_wgs(p, T, p.grid);
            wp.p_lo = w < n ? (int)((int64_t)w * T / n) : 0;
            wp.p_hi = w < n ? (int)((int64_t)(w + 1) * T / n) : 0;
            wp.first_b = wp.last_b = -1;
            wp.first_cut = wp.last_cut = 0;
        }
        if (lane == 0) plan = wp;
    }
    __syncthreads();
    const int p_lo = __builtin_amdgcn_readfirstlane(plan.p_lo);
    const int p_hi = __builtin_amdgcn_readfirstlane(plan.p_hi);

    const int g = wave;  // KV head of this wave
    float* wscr = lds.wscr[wave];
    const int G = p.G;
    const int hq0 = g * G;
    const int qh = r16 & 7;  // query head of S column r16
    const bool q_ok = qh < G;

    if (p_lo >= p_hi) {
        if (p.per_seq && w < p.B && r16 < G) {
            uint16_t* o = reinterpret_cast<uint16_t*>(p.out) + ((int64_t)w * p.Hq + hq0 + r16) * kD + 32 * grp;
#pragma unroll
            for (int c = 0; c < 4; ++c) reinterpret_cast<u32x4*>(o)[c] = u32x4{0u, 0u, 0u, 0u};
        }
        return;
    }

    // ---- key centroid pair table; G32 3-bit: the exact (code - 4) table
    if constexpr (G32) {
        if constexpr (KB == 3) {
            for (int e = tid; e < 4096; e += blockDim.x) {
                uint32_t w2[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float lo = (float)((int)((e >> (6 * h)) & 7) - 4);
                    const float hi = (float)((int)((e >> (6 * h + 3)) & 7) - 4);
                    w2[h] = (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
                }
                lds.lut4[e] = u32x2{w2[0], w2[1]};
            }
        }
    } else {
        build_pair_lut<KB>(lds.lut, p.tab);
        if constexpr (KB == 3) {
            __syncthreads();
            for (int e = tid; e < 4096; e += blockDim.x) lds.lut4[e] = u32x2{lds.lut[e & 63], lds.lut[e >> 6]};
        }
    }

    // ---- Q operand: lane (r16, grp) holds dims 32 grp + 8 j + e of head qh
    // (columns c and c + 8 both hold head c), rotated (H q / sqrt(d))
    AT qb[4];
    auto load_q = [&](int b) __attribute__((always_inline)) {
        const int64_t qrow = ((int64_t)b * p.Hq + hq0 + qh) * kD;
        float y[32];
        if (q_ok) {
            const u32x4* src = reinterpret_cast<const u32x4*>(p.q + qrow + 32 * grp);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const u32x4 wv = src[c];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    y[8 * c + 2 * e] = half_to_f32<BF>((uint16_t)(wv[e] & 0xffff));
                    y[8 * c + 2 * e + 1] = half_to_f32<BF>((uint16_t)(wv[e] >> 16));
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 32; ++e) y[e] = 0.0f;
        }
        if constexpr (G32) {  // the variant's rotation: H (s q) / sqrt(d)
            const uint32_t sb = p.sgn[grp];  // dims 32 grp .. + 31
#pragma unroll
            for (int e = 0; e < 32; ++e) y[e] = ((sb >> e) & 1u) ? -y[e] : y[e];
        }
        // Walsh-Hadamard: half-widths 1..16 inside the lane, 32 and 64 across
        // the lane groups (dim bit 32 = grp bit 0, dim bit 64 = grp bit 1)
#pragma unroll
        for (int hw = 1; hw < 32; hw <<= 1)
#pragma unroll
            for (int i = 0; i < 32; i += 2 * hw)
#pragma unroll
                for (int j = i; j < i + hw; ++j) {
                    const float a = y[j], c = y[j + hw];
                    y[j] = a + c;
                    y[j + hw] = a - c;
                }
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const float o = shfl_xor(y[e], 16);
            y[e] = (grp & 1) ? o - y[e] : y[e] + o;
        }
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const float o = shfl_xor(y[e], 32);
            y[e] = (grp & 2) ? o - y[e] : y[e] + o;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) qb[j][e] = (_Float16)__fmul_rn(y[8 * j + e], p.tab.rot_c);
    };

    // ---- running state of the current piece
    f32x4 oacc[8];
    float m_run, l_part, z_part, m_thr;
    auto reset_state = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < 8; ++c) oacc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        m_run = kNegInf;
        m_thr = kNegInf;
        l_part = 0.0f;
        z_part = 0.0f;
    };
    reset_state();
    int cur_b = -1;

    // ---- finish a piece of sequence b: the rows, or the partial slot
    // (TurboQuant: O chunk c in units of its code field's fp16 subnormal)
    auto vscale = [](int c) { return G32 ? 1.0f : kVScale<FMT_TQ, VB>(c); };
    auto finalize = [&](int b) __attribute__((always_inline)) {
        const bool cut_before = b == __builtin_amdgcn_readfirstlane(plan.first_b) &&
                                __builtin_amdgcn_readfirstlane(plan.first_cut);
        const bool cut_after = b == __builtin_amdgcn_readfirstlane(plan.last_b) &&
                               __builtin_amdgcn_readfirstlane(plan.last_cut);
        const bool whole = !cut_before && !cut_after;
        const int slot = cut_before ? 2 * w : 2 * w + 1;
        float l_tot = sum_over_groups(l_part);
        float z_tot = sum_over_groups(z_part);
        // columns r16 and r16 ^ 8 hold the same head; O rows m and m + 8
        // (lane groups grp and grp + 2) too
        l_tot += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, l_tot), 0x128, 0xf, 0xf, false));
        z_tot += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, z_tot), 0x128, 0xf, 0xf, false));
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) oacc[c][i] += __shfl_xor(oacc[c][i], 32, 64);
        if constexpr (G32) {
            // O back from the rotated domain, s (H O_r) / sqrt(d) (linear: the
            // partial rows of cut pieces too); oacc[c][i] = dim 8 r16 + c:
            // half-widths 1..4 in the lane, 8..64 across r16
#pragma unroll
            for (int hw = 1; hw < 8; hw <<= 1)
#pragma unroll
                for (int c0 = 0; c0 < 8; c0 += 2 * hw)
#pragma unroll
                    for (int c = c0; c < c0 + hw; ++c)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float x = oacc[c][i], y = oacc[c + hw][i];
                            oacc[c][i] = x + y;
                            oacc[c + hw][i] = x - y;
                        }
#pragma unroll
            for (int m = 1; m < 16; m <<= 1)
#pragma unroll
                for (int c = 0; c < 8; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float o = __shfl_xor(oacc[c][i], m, 64);
                        oacc[c][i] = (r16 & m) ? o - oacc[c][i] : oacc[c][i] + o;
                    }
            const uint32_t sb = (p.sgn[r16 >> 2] >> (8 * (r16 & 3))) & 0xffu;  // dims 8 r16 .. + 7
#pragma unroll
            for (int c = 0; c < 8; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float v = oacc[c][i] * p.tab.rot_c;
                    oacc[c][i] = ((sb >> c) & 1u) ? -v : v;
                }
        }
        const f32x4 lh4 = gather4_from_row0(l_tot, wscr, r16, grp);
        const f32x4 zh4 = gather4_from_row0(z_tot, wscr + 16, r16, grp);
        const f32x4 mh4 = gather4_from_row0(m_run, wscr + 32, r16, grp);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int hh = 4 * grp + i;
            const float lh = lh4[i], zh = zh4[i], mh = mh4[i];
            if (hh >= G) continue;
            const int hq = hq0 + hh;
            if (whole) {
                const float inv = lh > 0.0f ? 1.0f / lh : 0.0f;
                uint32_t wd[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v0 = __builtin_fmaf(oacc[2 * e][i], vscale(2 * e), zh) * inv;
                    const float v1 = __builtin_fmaf(oacc[2 * e + 1][i], vscale(2 * e + 1), zh) * inv;
                    wd[e] = (uint32_t)f32_to_half<BF>(v0) | ((uint32_t)f32_to_half<BF>(v1) << 16);
                }
                uint16_t* o = reinterpret_cast<uint16_t*>(p.out) + ((int64_t)b * p.Hq + hq) * kD + 8 * r16;
                *reinterpret_cast<u32x4*>(o) = u32x4{wd[0], wd[1], wd[2], wd[3]};
            } else {
                float* o = p.part + ((int64_t)slot * p.Hq + hq) * kPartRow;
                float* od = o + 8 * r16;
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                    f32x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = __builtin_fmaf(oacc[4 * h2 + e][i], vscale(4 * h2 + e), zh);
                    *reinterpret_cast<f32x4*>(od + 4 * h2) = v;
                }
                if (r16 == 0) *reinterpret_cast<float2*>(o + kD) = make_float2(mh, lh);
            }
        }
        reset_state();
    };

    // ---- per-wave page geometry.  A page in HBM is 16 token rows of Hkv
    // slots (row_bytes each, turboquant_kernels.cu:39-45); this head's run of
    // token row r starts at a = r * row_bytes + g * slot, fetched as the
    // 16-byte window from a & ~15, and lands in LDS row r of the page buffer
    // at mis(r) = a & 15.
    const int row_bytes = p.row_bytes;
    auto mis_of = [&](int r) { return (r * row_bytes + g * TG::slot) & 15; };
    uint8_t* const ring = &lds.ring[wave][0][0];
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)ring;
    // DMA: transfer c of a page, lane -> chunk j of row r (q = 64 c + lane =
    // r * nchp + j); chunks past the run re-read the window's first chunk
    // (never read back), lanes past the page's 16 * nchp chunks issue nothing
    uint32_t doff[TG::spt];
#pragma unroll
    for (int c = 0; c < TG::spt; ++c) {
        const int q = 64 * c + lane;
        const int r = min(q / TG::nchp, kBs - 1), j = q - r * TG::nchp;
        const int a = r * row_bytes + g * TG::slot;
        const int nchr = ((a & 15) + TG::slot + 15) >> 4;
        doff[c] = (uint32_t)((a & ~15) + (j < nchr ? 16 * j : 0));
    }
    constexpr int kLastLanes = kBs * TG::nchp - 64 * (TG::spt - 1);
    const int64_t page_bytes = p.page_bytes;
    auto dma_page = [&](int32_t blk, int buf) __attribute__((always_inline)) {
        const uint8_t* src = p.kc + (int64_t)blk * page_bytes;
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(ring_lds + buf * TG::page);
#pragma unroll
        for (int c = 0; c < TG::spt - 1; ++c) dma16(src, doff[c], m0 + 1024 * c);
        if (lane < kLastLanes) dma16(src, doff[TG::spt - 1], m0 + 1024 * (TG::spt - 1));
    };

    // loop-invariant LDS offsets inside a page buffer: the key run of token
    // r16 (its 4-byte floor; the run starts ks bytes in, the same for every
    // row of this head), the value code runs of tokens 4 grp + i (even i from
    // ve, odd from vo; the 16-bit-aligned start of dims 8 r16 .. + 7), and the
    // scales/zeros of the lane's own page (columns 0-7: first page)
    const int kq = r16 * TG::row + mis_of(r16);
    const int ks = kq & 3;  // 0 or 2, wave-uniform
    const int kfl = (kq + (KB == 3 ? 12 : 16) * grp) & ~3;
    const int vqe = 4 * grp * TG::row + mis_of(4 * grp), vqo = (4 * grp + 1) * TG::row + mis_of(4 * grp + 1);
    // the value runs and the scale/zero pairs start at the same offset modulo 4
    // in every row of this head (row strides and mis differ by multiples of 4)
    const int vce = vqe + TG::kp + VB * r16, vco = vqo + TG::kp + VB * r16;
    const uint32_t vsh = (uint32_t)(vce & 3);
    const int sze = vqe + TG::kp + TG::vd + (r16 >= 8 ? TG::page : 0);
    const int szo = vqo + TG::kp + TG::vd + (r16 >= 8 ? TG::page : 0);
    const uint32_t zsh = (uint32_t)(sze & 3);
    // byte-permute selectors that gather code bytes 0 .. 3 of two tokens' runs
    constexpr uint32_t vsel0 = 0x05040100u, vsel1 = 0x06050201u, vsel2 = 0x07060302u;
    // Gram diagonal: lane (r16, grp) picks element r16 % 4; the exchange slot
    // of its row factor is r16 on the diagonal (grp == r16 / 4), else 16 + r16
    const uint32_t odd_mask = (r16 & 1) ? ~0u : 0u, hi_mask = (r16 & 2) ? ~0u : 0u;
    const int diag_slot = ((r16 >> 2) == grp ? 0 : 16) + r16;

    // G32 (slots in whole 16-byte chunks, so mis = 0): the key block of token
    // r16 (block grp; its 4-byte floor, the block starting gks = 0 or 2 bytes
    // in), and the value block r16 / 4 of token 4 grp (+ i rows for token
    // 4 grp + i): d (| m) at gvb, the codes of dims 8 r16 .. + 7 from the
    // 4-byte floor of gvc, gvsh bytes in
    const int gk = kq + TG::be * grp;
    const int gkfl = gk & ~3;
    const uint32_t gks = (uint32_t)(gk & 3);
    const int gvb = 4 * grp * TG::row + TG::part + TG::be * (r16 >> 2);
    const int gvc = gvb + (KB == 3 ? 2 + 3 * (r16 & 3) : 4 + 8 * (r16 & 1));
    const uint32_t gvsh = (uint32_t)(gvc & 3);

    // raw bytes of the pair in page buffers 2 PS, 2 PS + 1
    auto read_codes = [&](auto ps_c, CODES& R) __attribute__((always_inline)) {
        constexpr int PS = decltype(ps_c)::value;
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            const uint8_t* pg = ring + (2 * PS + pp) * TG::page;
            if constexpr (G32) {  // the value codes: read_vcodes
#pragma unroll
                for (int i = 0; i < (KB == 3 ? 4 : 5); ++i) R.kd[pp][i] = lds32(pg + gkfl + 4 * i);
                continue;
            }
#pragma unroll
            for (int i = 0; i < (KB == 3 ? 4 : 5); ++i) R.kd[pp][i] = lds32(pg + kfl + 4 * i);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint8_t* cr = pg + ((((i & 1) ? vco : vce) & ~3) + (i >> 1) * 2 * TG::row);
                R.cw[pp][i][0] = lds32(cr);
                R.cw[pp][i][1] = lds32(cr + 4);
            }
        }
    };
    // G32: the value code words of the pair, read after the previous pair's
    // phase 2 has consumed its own (so one pair's words are live at a time)
    auto read_vcodes = [&](auto ps_c, CODES& R) __attribute__((always_inline)) {
        constexpr int PS = decltype(ps_c)::value;
        if constexpr (G32) {
#pragma unroll
            for (int pp = 0; pp < 2; ++pp)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint8_t* cr = ring + (2 * PS + pp) * TG::page + (gvc & ~3) + i * TG::row;
                    R.cw[pp][i][0] = lds32(cr);
                    R.cw[pp][i][1] = lds32(cr + 4);
                }
        }
    };
    // TurboQuant: the norms of token r16 on both pages, the scales / zeros of
    // tokens 4 grp + i of the lane's own page; G32: hsz[i][pp] = d (| m) of
    // token 4 grp + i on page pp (value block r16 / 4)
    auto read_halves = [&](auto ps_c, TqHalves& H) __attribute__((always_inline)) {
        constexpr int PS = decltype(ps_c)::value;
        const uint8_t* pg = ring + 2 * PS * TG::page;
        if constexpr (G32) {
            H.nrm = 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int pp = 0; pp < 2; ++pp) {
                    const uint8_t* vb = pg + pp * TG::page + gvb + i * TG::row;
                    H.hsz[i][pp] = KB == 3 ? lds16(vb) : lds32(vb);
                }
            return;
        }
        H.nrm = lds16(pg + kq + TG::mse) | (lds16(pg + TG::page + kq + TG::mse) << 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint8_t* sz = pg + ((((i & 1) ? szo : sze) & ~3) + (i >> 1) * 2 * TG::row);
            H.hsz[i][0] = lds32(sz);
            H.hsz[i][1] = lds32(sz + 4);
        }
    };

    // ---- phase 1 of a pair: key operands looked up (the table reads issued),
    // value code bytes of token pairs gathered by byte permutes (wv[pp][hh][r]:
    // run bytes r .. r + 1 of tokens 4 grp + 2 hh and + 1 in the two halves)
    constexpr int NW = VB == 4 ? 4 : 3;
    auto phase1 = [&](const CODES& R, AT (&a)[2][4], uint32_t (&wv)[2][2][NW]) __attribute__((always_inline)) {
        if constexpr (G32) {
            // keys: code * d + m (4-bit) or (code - 4) * d (3-bit, the exact
            // table then one packed multiply), fp16, MFMA j values 8j .. 8j+7
            // of block grp; values: the code words of tokens 4 grp + i
            // (3-bit: wv[pp][i >> 1][i & 1] = 24 code bits; 4-bit:
            // wv[pp][i >> 1][2 (i & 1) + k] = code dword k)
#pragma unroll
            for (int pp = 0; pp < 2; ++pp) {
                u32x4 aw[4];
                if constexpr (KB == 3) {
                    const bool off2 = gks != 0u;
                    const uint32_t d16 = off2 ? R.kd[pp][0] >> 16 : R.kd[pp][0] & 0xffffu;
                    const uint32_t c0 = off2 ? R.kd[pp][1] : __builtin_amdgcn_alignbyte(R.kd[pp][1], R.kd[pp][0], 2);
                    const uint32_t c1 = off2 ? R.kd[pp][2] : __builtin_amdgcn_alignbyte(R.kd[pp][2], R.kd[pp][1], 2);
                    const uint32_t c2 = off2 ? R.kd[pp][3] : __builtin_amdgcn_alignbyte(R.kd[pp][3], R.kd[pp][2], 2);
                    const uint32_t g24[4] = {c0 & 0xffffffu, (c0 >> 24) | ((c1 & 0xffffu) << 8),
                                             (c1 >> 16) | ((c2 & 0xffu) << 16), c2 >> 8};
                    const f16x2 d2 = __builtin_bit_cast(f16x2, d16 * 0x10001u);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const u32x2 lo = lds.lut4[g24[j] & 0xfffu], hi = lds.lut4[g24[j] >> 12];
                        aw[j] = u32x4{g32_mul(lo[0], d2), g32_mul(lo[1], d2), g32_mul(hi[0], d2), g32_mul(hi[1], d2)};
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        wv[pp][i >> 1][i & 1] = __builtin_amdgcn_alignbyte(R.cw[pp][i][1], R.cw[pp][i][0], gvsh) & 0xffffffu;
                } else {
                    const uint32_t dm = R.kd[pp][0];
                    const f16x2 d2 = __builtin_bit_cast(f16x2, (dm & 0xffffu) * 0x10001u);
                    const f16x2 m2 = __builtin_bit_cast(f16x2, (dm >> 16) * 0x10001u);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            aw[j][e] = g32_nib2(R.kd[pp][1 + 2 * (j & 1) + (e >> 1)], e & 1, j >= 2, d2, m2);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        wv[pp][i >> 1][2 * (i & 1)] = R.cw[pp][i][0];
                        wv[pp][i >> 1][2 * (i & 1) + 1] = R.cw[pp][i][1];
                    }
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) a[pp][j] = __builtin_bit_cast(AT, aw[j]);
            }
            return;
        }
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            u32x4 aw[4];
            if constexpr (KB == 3) {
                // 12 code bytes = eight 12-bit fields; each indexes the table of
                // four packed fp16 centroids
                const uint32_t c0 = __builtin_amdgcn_alignbyte(R.kd[pp][1], R.kd[pp][0], ks);
                const uint32_t c1 = __builtin_amdgcn_alignbyte(R.kd[pp][2], R.kd[pp][1], ks);
                const uint32_t c2 = __builtin_amdgcn_alignbyte(R.kd[pp][3], R.kd[pp][2], ks);
                const uint32_t f[8] = {c0 & 0xfffu, (c0 >> 12) & 0xfffu,
                                       __builtin_amdgcn_alignbit(c1, c0, 24) & 0xfffu, (c1 >> 4) & 0xfffu,
                                       (c1 >> 16) & 0xfffu, __builtin_amdgcn_alignbit(c2, c1, 28) & 0xfffu,
                                       (c2 >> 8) & 0xfffu, c2 >> 20};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const u32x2 lo = lds.lut4[f[2 * j]], hi = lds.lut4[f[2 * j + 1]];
                    aw[j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
                }
            } else {
                // 16 code bytes; each byte (two 4-bit codes) indexes the pair table
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t wd = __builtin_amdgcn_alignbyte(R.kd[pp][j + 1], R.kd[pp][j], ks);
#pragma unroll
                    for (int e = 0; e < 4; ++e) aw[j][e] = lds.lut[(wd >> (8 * e)) & 0xffu];
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) a[pp][j] = __builtin_bit_cast(AT, aw[j]);
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const uint32_t A = __builtin_amdgcn_alignbyte(R.cw[pp][2 * hh][1], R.cw[pp][2 * hh][0], vsh);
                const uint32_t Bw = __builtin_amdgcn_alignbyte(R.cw[pp][2 * hh + 1][1], R.cw[pp][2 * hh + 1][0], vsh);
                wv[pp][hh][0] = __builtin_amdgcn_perm(Bw, A, vsel0);
                wv[pp][hh][1] = __builtin_amdgcn_perm(Bw, A, vsel1);
                wv[pp][hh][2] = __builtin_amdgcn_perm(Bw, A, vsel2);
                if constexpr (VB == 4) wv[pp][hh][3] = __builtin_amdgcn_perm(Bw, A, 0x0c070c03u);
            }
        }
    };

    // ---- phase 2: S, softmax and O += P . V for the pair; nv0 / nv1 valid
    // tokens of the first / second page (0: the page contributes nothing)
    auto phase2 = [&](const AT (&a)[2][4], uint32_t (&wv)[2][2][NW], const TqHalves& H, int nv0, int nv1)
                      __attribute__((always_inline)) {
        if constexpr (G32) {
            // values first: d (| m) of tokens 4 grp + i on both pages, zero past
            // a page's end (so those rows are 0 whatever their bytes), and the
            // 3-bit tables read early
            uint32_t dv[2][4];
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                dv[0][i2] = H.hsz[i2][0];
                dv[1][i2] = H.hsz[i2][1];
            }
            u32x2 vlo[2][4], vhi[2][4];
            if constexpr (KB == 3) {
#pragma unroll
                for (int pp = 0; pp < 2; ++pp)
#pragma unroll
                    for (int i2 = 0; i2 < 4; ++i2) {
                        const uint32_t w = wv[pp][i2 >> 1][i2 & 1];
                        vlo[pp][i2] = lds.lut4[w & 0xfffu];
                        vhi[pp][i2] = lds.lut4[w >> 12];
                    }
            }
            // S^T per page against the same Q^T (column r16 >= 8: the second
            // page), times scale log2(e)
            f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) s0 = mfma16x16x32(a[0][j], qb[j], s0);
#pragma unroll
            for (int j = 0; j < 4; ++j) s1 = mfma16x16x32(a[1][j], qb[j], s1);
            const bool second = r16 >= 8;
            float sv[4];
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) sv[i2] = (second ? s1[i2] : s0[i2]) * p.scale_log2;
            if (nv0 < kBs || nv1 < kBs) {  // tokens past a page's end may hold anything
                const int nvl = second ? nv1 : nv0;
#pragma unroll
                for (int i2 = 0; i2 < 4; ++i2) {
                    sv[i2] = 4 * grp + i2 < nvl ? sv[i2] : kNegInf;
                    dv[0][i2] = 4 * grp + i2 < nv0 ? dv[0][i2] : 0u;
                    dv[1][i2] = 4 * grp + i2 < nv1 ? dv[1][i2] : 0u;
                }
            }
            // lazy reference max; a head's max spans columns c, c ^ 8
            const float mloc = vmax(vmax(sv[0], sv[1]), vmax(sv[2], sv[3]));
            if (__ballot(mloc > m_thr)) {
                float mx = vmax_over_groups(mloc);
                mx = vmax(mx, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, mx), 0x128, 0xf, 0xf, false)));
                const bool upd = mx > m_thr;
                const float m_new = upd ? mx : m_run;
                const float alpha = upd ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
                l_part *= alpha;
                const f32x4 al = gather4_from_row0(alpha, wscr + 64, r16, grp);
#pragma unroll
                for (int i2 = 0; i2 < 4; ++i2)
#pragma unroll
                    for (int c = 0; c < 8; ++c) oacc[c][i2] *= al[i2];
                m_run = m_new;
                m_thr = m_run + 8.0f;
            }
            const float m_use = m_run == kNegInf ? 0.0f : m_run;
            float psum = 0.0f;
            f16x4 pw;
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                const float pv = __builtin_amdgcn_exp2f(sv[i2] - m_use);
                psum += pv;
                pw[i2] = (_Float16)pv;
            }
            l_part += psum;
            // P: rows 0-7 take k = 8 grp + i (first page, token 4 grp + i),
            // rows 8-15 k = 8 grp + 4 + i (second page)
            const u32x2 pw2 = __builtin_bit_cast(u32x2, pw);
            const uint32_t lo_m = r16 < 8 ? ~0u : 0u;
            const AT pa = __builtin_bit_cast(AT, u32x4{pw2[0] & lo_m, pw2[1] & lo_m, pw2[0] & ~lo_m, pw2[1] & ~lo_m});
            // V values of tokens 4 grp + i, dims 8 r16 + 2e, + 1, one e at a
            // time: B operands {token 0,1}, {token 2,3} of those dims, first
            // page then second, for chunks 2e and 2e + 1; O += P . V
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t ve[2][4];
#pragma unroll
                for (int pp = 0; pp < 2; ++pp)
#pragma unroll
                    for (int i2 = 0; i2 < 4; ++i2) {
                        const f16x2 d2 = __builtin_bit_cast(f16x2, (dv[pp][i2] & 0xffffu) * 0x10001u);
                        if constexpr (KB == 3) {
                            ve[pp][i2] = g32_mul(e < 2 ? vlo[pp][i2][e] : vhi[pp][i2][e - 2], d2);
                        } else {
                            const f16x2 m2 = __builtin_bit_cast(f16x2, (dv[pp][i2] >> 16) * 0x10001u);
                            const uint32_t w = wv[pp][i2 >> 1][2 * (i2 & 1) + (e >> 1)];
                            ve[pp][i2] = g32_nib2(w, e & 1, (r16 & 3) >= 2, d2, m2);
                        }
                    }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t sel = h ? 0x07060302u : 0x05040100u;
                    const AT vb = __builtin_bit_cast(
                        AT, u32x4{__builtin_amdgcn_perm(ve[0][1], ve[0][0], sel), __builtin_amdgcn_perm(ve[0][3], ve[0][2], sel),
                                  __builtin_amdgcn_perm(ve[1][1], ve[1][0], sel), __builtin_amdgcn_perm(ve[1][3], ve[1][2], sel)});
                    oacc[2 * e + h] = mfma16x16x32(pa, vb, oacc[2 * e + h]);
                }
            }
            return;
        }
        // ||C[codes]||^2 per token: the Gram diagonal (token r16's value in
        // the lanes with grp == r16 / 4, element r16 % 4); the row factor
        // scale * norm / ||C|| (scale * norm without the norm correction)
        float rowf[2];
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            f32x4 gram = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) gram = mfma16x16x32(a[pp][j], a[pp][j], gram);
            const float csq = sel_bits(sel_bits(gram[0], gram[1], odd_mask), sel_bits(gram[2], gram[3], odd_mask),
                                       hi_mask);
            const uint16_t nb16 = (uint16_t)(pp ? H.nrm >> 16 : H.nrm & 0xffffu);
            rowf[pp] = p.scale_log2 * half_to_f32<BF>(nb16) * (p.norm_corr ? __builtin_amdgcn_rsqf(csq + 1e-16f) : 1.0f);
        }
        // S^T per page against the same Q^T; S column c < 8 keeps the first
        // page's scores (head c), c >= 8 the second's (head c - 8)
        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) s0 = mfma16x16x32(a[0][j], qb[j], s0);
#pragma unroll
        for (int j = 0; j < 4; ++j) s1 = mfma16x16x32(a[1][j], qb[j], s1);
        wscr[diag_slot] = rowf[0];
        wscr[32 + diag_slot] = rowf[1];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const f32x4 rf = *reinterpret_cast<const f32x4*>(wscr + (r16 >= 8 ? 32 : 0) + 4 * grp);
        __builtin_amdgcn_wave_barrier();
        const bool second = r16 >= 8;
        float sv[4];
        uint32_t hsz[4];
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
            sv[i2] = (second ? s1[i2] : s0[i2]) * rf[i2];
            hsz[i2] = __builtin_amdgcn_alignbyte(H.hsz[i2][1], H.hsz[i2][0], zsh);
        }
        const int nvl = second ? nv1 : nv0;
        if (nv0 < kBs || nv1 < kBs) {  // tokens past a page's end may hold anything
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                const bool ok = 4 * grp + i2 < nvl;
                sv[i2] = ok ? sv[i2] : kNegInf;
                hsz[i2] = ok ? hsz[i2] : 0u;
            }
        }
        // lazy reference max: m_run moves only when a head's max passes it by
        // more than 8 (log2 units), so P <= 2^8; when a value scale of the pair
        // exceeds 65504 / 2^8 the max is taken exactly (P <= 1), so that
        // fp16(P * scale) cannot overflow.  A head's max spans columns c, c ^ 8
        float scf[4];
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) scf[i2] = half_to_f32<BF>((uint16_t)(hsz[i2] & 0xffffu));
        const float smax = vmax(vmax(scf[0], scf[1]), vmax(scf[2], scf[3]));
        const bool exact = __ballot(smax > 255.875f) != 0;  // wave-uniform, rare
        const float thr = exact ? m_run : m_thr;
        const float mloc = vmax(vmax(sv[0], sv[1]), vmax(sv[2], sv[3]));
        if (__ballot(mloc > thr)) {
            float mx = vmax_over_groups(mloc);
            mx = vmax(mx, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, mx), 0x128, 0xf, 0xf, false)));
            const bool upd = mx > thr;
            const float m_new = upd ? vmax(mx, m_run) : m_run;
            const float alpha = m_new > m_run ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
            l_part *= alpha;
            z_part *= alpha;
            const f32x4 al = gather4_from_row0(alpha, wscr + 64, r16, grp);
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2)
#pragma unroll
                for (int c = 0; c < 8; ++c) oacc[c][i2] *= al[i2];
            m_run = m_new;
            m_thr = m_run + 8.0f;
        }
        const float m_use = m_run == kNegInf ? 0.0f : m_run;
        float psum = 0.0f, zsum = 0.0f;
        f16x4 pw;
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
            const float pv = __builtin_amdgcn_exp2f(sv[i2] - m_use);
            psum += pv;
            zsum = __builtin_fmaf(pv, half_to_f32<BF>((uint16_t)(hsz[i2] >> 16)), zsum);
            pw[i2] = (_Float16)__builtin_fmaf(pv, scf[i2], 0.0f);
        }
        l_part += psum;
        z_part += zsum;
        // O += P . V: rows 0-7 take k = 8 grp + i (first page, token 4 grp + i),
        // rows 8-15 k = 8 grp + 4 + i (second page); the V operand of output
        // chunk c is its code field masked where it lies (an fp16 subnormal
        // code * 2^(shift - 24), kVShift)
        const u32x2 pw2 = __builtin_bit_cast(u32x2, pw);
        const uint32_t lo_m = r16 < 8 ? ~0u : 0u;
        const AT pa = __builtin_bit_cast(AT, u32x4{pw2[0] & lo_m, pw2[1] & lo_m, pw2[0] & ~lo_m, pw2[1] & ~lo_m});
        // (an empty asm "redefines" the permuted words here, so the masked
        // operands are built next to their MFMAs, not hoisted out of the piece
        // loop where they would hold 32 registers)
#pragma unroll
        for (int pp = 0; pp < 2; ++pp)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int r = 0; r < NW; ++r) asm volatile("" : "+v"(wv[pp][hh][r]));
        const uint32_t (&wl)[2][2][NW] = wv;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            uint32_t m, wi;
            if constexpr (VB == 4) {
                wi = c >> 1;
                m = (c & 1) ? 0x00f000f0u : 0x000f000fu;
            } else {
                constexpr uint32_t kM[8] = {0x00070007u, 0x00380038u, 0x01c001c0u, 0x000e000eu,
                                            0x00700070u, 0x03800380u, 0x001c001cu, 0x00e000e0u};
                wi = c < 3 ? 0 : c < 6 ? 1 : 2;
                m = kM[c];
            }
            const AT vb = __builtin_bit_cast(AT, u32x4{wl[0][0][wi] & m, wl[0][1][wi] & m, wl[1][0][wi] & m,
                                                         wl[1][1][wi] & m});
            oacc[c] = mfma16x16x32(pa, vb, oacc[c]);
        }
    };

    // ---- the pair of pages (i, i + 1) of the chunk from codes R and halves
    // H; between the phases, the codes of the next pair are read into R (from
    // page buffers NEXT; G32: its key words only), after them its halves
    // into H (G32: and its value code words into R).  A pair that a piece
    // boundary splits runs phase 2 twice, each time with one page masked.
    auto process_pair = [&](CODES& R, TqHalves& H, auto next_c, int i, int npc) __attribute__((always_inline)) {
        AT a[2][4];
        uint32_t wv[2][2][NW];
        phase1(R, a, wv);
        // the next pair's transfers have landed once at most those of the
        // NP - 2 pairs after it are outstanding (a wave's transfers retire in
        // issue order; loads and stores the compiler issues in between only
        // make the wait stricter)
        vmcnt_pairs<TG::npair - 2>();
        read_codes(next_c, R);
        const int info0 = __builtin_amdgcn_readfirstlane(lds.info[i]);
        const bool has1 = i + 1 < npc;
        const int info1 = has1 ? __builtin_amdgcn_readfirstlane(lds.info[i + 1]) : info0;
        const bool split = (info0 & 1) && has1;
        int b = info0 >> 6;
        int nva = (info0 >> 1) & 31, nvb = has1 && !split ? (info1 >> 1) & 31 : 0;
        int ends = split ? info0 : info1;
        for (int part = 0;; ++part) {
            if (b != cur_b) {  // a new sequence starts here
                load_q(b);
                cur_b = b;
            }
            phase2(a, wv, H, nva, nvb);
            if (ends & 1) finalize(b);
            if (!split || part == 1) break;
            b = info1 >> 6;
            nva = 0;
            nvb = (info1 >> 1) & 31;
            ends = info1;
        }
        read_vcodes(next_c, R);
        read_halves(next_c, H);
    };

    // ---- chunks of up to 256 pages: stage the block-table slice and the
    // per-page sequence info in LDS, then stream the pages
    for (int c_lo = p_lo; c_lo < p_hi; c_lo += 256) {
        const int c_hi = min(p_hi, c_lo + 256);
        const int npc = c_hi - c_lo;
        if (wave == 0) {
            const int ns = collect_segments(p, c_lo, c_hi, lane, lds.seg_b, lds.seg_ps, lds.seg_L, &plan,
                                            c_lo == p_lo && !p.per_seq);
            if (lane == 0) lds.n_seg = ns;
        }
        __syncthreads();
        const int ns = lds.n_seg;
        for (int i = tid; i < npc; i += blockDim.x) {
            const int gp = c_lo + i;
            int lo = 0, hi = ns - 1;  // last segment with seg_ps <= gp
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (lds.seg_ps[mid] <= gp) lo = mid;
                else hi = mid - 1;
            }
            const int b = lds.seg_b[lo], L = lds.seg_L[lo], pp = gp - lds.seg_ps[lo];
            const int pages_b = (L + kBs - 1) / kBs;
            const int32_t blk = p.bt[(int64_t)(p.row_seq ? p.row_seq[b] : b) * p.max_blocks + pp];
            const int nv = blk < 0 ? 0 : min(kBs, L - pp * kBs);
            const int ends = pp == pages_b - 1 || gp == p_hi - 1;
            lds.bt[i] = blk;
            lds.info[i] = (b << 6) | (nv << 1) | ends;
        }
        __syncthreads();

        // Pair k of the chunk sits in page buffers 2 (k % NP), 2 (k % NP) + 1
        // (NP = npair).  Step k: phase 1 of pair k from registers; wait until
        // pair k+1 has landed (pairs k+1 .. k+NP-1 were in flight) and read
        // its bytes; phase 2 of pair k; issue pair k+NP into pair k's buffers.
        // A transfer has NP - 1.5 steps to land.  Past the chunk's last page
        // block 0 is re-read into buffers no step reads, so every step issues
        // the same transfers.
        const int npairs = (npc + 1) >> 1;
        auto blk_of = [&](int i) -> int32_t {
            return __builtin_amdgcn_readfirstlane(i < npc ? max(lds.bt[i], 0) : 0);
        };
        constexpr int NP = TG::npair, NPH = NP;
#pragma unroll
        for (int k = 0; k < NP; ++k) {
            dma_page(blk_of(2 * k), 2 * k);
            dma_page(blk_of(2 * k + 1), 2 * k + 1);
        }
        vmcnt_pairs<NP - 1>();
        CODES rc;
        TqHalves hz;
        read_codes(std::integral_constant<int, 0>{}, rc);
        read_vcodes(std::integral_constant<int, 0>{}, rc);
        read_halves(std::integral_constant<int, 0>{}, hz);
        for (int k0 = 0; k0 < npairs; k0 += NPH) {
            static_for<NPH>([&](auto ph) __attribute__((always_inline)) {
                constexpr int P = decltype(ph)::value;
                const int k = k0 + P;
                if (k < npairs) {  // uniform over the wave
                    process_pair(rc, hz, std::integral_constant<int, (P + 1) % NP>{}, 2 * k, npc);
                    // pair k's buffers are free (their bytes were read at step
                    // k - 1, and every LDS read has returned): pair k + NP goes there
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    dma_page(blk_of(2 * (k + NP)), 2 * (P % NP));
                    dma_page(blk_of(2 * (k + NP) + 1), 2 * (P % NP) + 1);
                }
            });
        }
        // no transfer may still target LDS when the tables are restaged or
        // the workgroup ends
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
}

}  // namespace

// TurboQuant decode (reference layout, G <= 8) with the pipelined kernel;
// returns VMC_EINVAL when the layout is not one it was built for.
template <int KB, int VB, bool BF, bool G32 = false>
int launch_tq_decode(DecodeParams& prm, hipStream_t stream) {
    using TG = TqGeo<KB, VB, G32>;
    if (G32 ? prm.entry_bytes != TG::slot
            : (prm.entry_bytes != TG::slot || prm.mse_bytes != TG::mse || prm.key_packed != TG::kp ||
               prm.val_data != TG::vd))
        return VMC_EINVAL;
    if (prm.G > 8 || prm.Hkv > TG::waves) return VMC_EINVAL;
    prm.row_bytes = prm.Hkv * TG::slot;
    prm.grid = prm.per_seq ? prm.B : tq_ranges(prm.B, prm.Hkv, prm.max_blocks, prm.max_splits, num_cus());
    hipLaunchKernelGGL((tq_decode_kernel<KB, VB, BF, G32>), dim3(prm.grid), dim3(64 * prm.Hkv), 0, stream, prm);
    VMC_LAUNCH_CHECK();
    if (!prm.per_seq) {
        hipLaunchKernelGGL(decode_merge_kernel, dim3(prm.B, prm.Hkv), dim3(64 * prm.G), 0, stream, prm);
        VMC_LAUNCH_CHECK();
    }
    return VMC_OK;
}

// the per-32-group variant (fp16 activations, 3- or 4-bit) on the same kernel
int launch_g32_decode(DecodeParams& prm, int bits, hipStream_t s) {
    return bits == 3 ? launch_tq_decode<3, 3, false, true>(prm, s) : launch_tq_decode<4, 4, false, true>(prm, s);
}

int launch_tq_decode_any(DecodeParams& prm, int kb, int vb, bool bf, hipStream_t s) {
    if (kb == 3 && vb == 3) return bf ? launch_tq_decode<3, 3, true>(prm, s) : launch_tq_decode<3, 3, false>(prm, s);
    if (kb == 4 && vb == 4) return bf ? launch_tq_decode<4, 4, true>(prm, s) : launch_tq_decode<4, 4, false>(prm, s);
    if (kb == 3 && vb == 4) return bf ? launch_tq_decode<3, 4, true>(prm, s) : launch_tq_decode<3, 4, false>(prm, s);
    return VMC_EINVAL;
}

}  // namespace vmc
