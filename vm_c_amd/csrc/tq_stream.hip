// tq_stream.hip -- split-KV paged decode over 3-bit TurboQuant slots in the
// reference layout (turboquant_3bit_nc, 102-byte slots): 8 KV heads, at most
// 8 query heads per KV head.
//
// Replaces the decode of vm_c::turboquant_decode_attention
// (src/cuda/turboquant_kernels.cu:939-1007: q rotation, stage 1 :353-506,
// stage 2 :508-547).  The arithmetic per page is paged_decode.hip's
// TurboQuant path (K = C[code] * norm / ||C[codes]||, V = code * scale +
// zero, fp32 online softmax, the same page-range plan and merge); what
// differs is how the bytes arrive:
//
//  * one workgroup per page range: 8 waves, one KV head each, so a page's
//    13,056 bytes (102 whole 128-byte lines) are fetched exactly once, as a
//    contiguous block, by non-temporal load-to-LDS transfers spread over the
//    waves (a split of the heads over two workgroups fetches the lines that
//    straddle the split twice: 1.29x the bytes at 128-byte granularity);
//  * two workgroups per CU (four waves per SIMD, at most 128 registers);
//    the rotated q operands sit in LDS, not in registers;
//  * two page-pair buffers, one workgroup barrier per pair: the transfers of
//    pair k + 1 are issued when pair k's compute starts;
//  * a token row is 816 bytes = 51 chunks, an odd count, so the page's LDS
//    copy (a byte copy) puts 16 rows on distinct bank groups for 16-byte reads;
//  * key codes are looked up two at a time in an LDS table of packed fp16
//    centroid pairs (64 entries), replicated 32 times so that the 32 lanes of
//    a half wave read 32 distinct banks: no conflicts.  (A lane permute of a
//    64-entry register table measured slower: ds_bpermute conflicts as a
//    64-entry LDS table does.)
//
// Per wave and page pair (32 tokens x G <= 8 query heads): S^T = K . Q^T on
// v_mfma_f32_16x16x32_f16 with the first page's heads in S columns 0-7 and
// the second's in 8-15 (a block-diagonal Q^T), ||C[codes]||^2 from the Gram
// diagonal K K^T, online softmax in the log2 domain with a lazy reference
// max, O += P . V with the V codes as exact fp16 subnormals and sum(P * zero)
// kept apart; both pages' P rows are moved into O rows 0-7 (a row rotation),
// so O needs no cross-lane sum.  P enters the product as fp16(P * scale):
// with the lazy max P is at most 2^8, so a page pair whose largest value
// scale exceeds 65504 / 2^8 takes the exact running max instead (P <= 1),
// which keeps every product in the fp16 range for any fp16 scale.
#include "decode_plan.hpp"

namespace vmc {
namespace {

constexpr int kStPages = 96;  // pages per staged slice of the block table

template <int KB, int VB>
struct StGeo {
    static constexpr int mse = 16 * KB, kp = mse + 2, vd = 16 * VB;
    static constexpr int slot = (kp + vd + 4 + 1) / 2 * 2;
    static constexpr int hpg = 8;  // waves per workgroup: one per KV head, every head of a page
    // a token row of 8 slots is a whole, odd number of 16-byte chunks (51,
    // 67, 59), so a page buffer in LDS is a byte copy of the page in HBM whose
    // 16 rows fall on distinct bank groups for 16-byte reads
    static constexpr int nc = hpg * slot / 16;
    static_assert(hpg * slot % 16 == 0 && (nc & 1), "token rows of an odd number of whole chunks");
    static constexpr int rowl = 16 * nc;     // bytes per token row, HBM and LDS
    static constexpr int page = kBs * rowl;  // one page
    // the second page of a pair starts 16 bytes past the first's end, so the
    // lanes that read the same offset of both pages use different banks
    static constexpr int pstr = page + 16;
    static constexpr int pair = 2 * pstr;
    // key table: 64 (3-bit) or 256 (4-bit) code-pair entries, replicated so
    // that lanes l and l' of a half wave read the same bank only when
    // l = l' mod copies (32 copies of the 3-bit table: never; 4 of the 4-bit
    // table, which has to leave room for its larger pages)
    static constexpr int lut_log2c = KB == 3 ? 5 : 2;
    static constexpr int lut_words = (KB == 3 ? 64 : 256) << lut_log2c;
    // two workgroups per CU (four waves per SIMD), two page-pair buffers each
    static constexpr int npb = 2;
    static constexpr int lds_bytes = 4 * lut_words + npb * pair + hpg * 80 * 4 + hpg * 2048 + 5 * kStPages * 4 + 64;
    static constexpr bool fits = 2 * lds_bytes <= 160 * 1024;  // two workgroups per CU
    // transfers: each wave fetches cw chunks of a page, in tr load-to-LDS
    // instructions (the last with last_lanes active lanes)
    static constexpr int page_chunks = kBs * nc;
    static_assert(page_chunks % hpg == 0, "a page's chunks split evenly over the waves");
    static constexpr int cw = page_chunks / hpg;
    static constexpr int tr = (cw + 63) / 64;
    static constexpr int last_lanes = cw - 64 * (tr - 1);
};

template <int KB, int VB>
struct alignas(16) StLds {
    using SG = StGeo<KB, VB>;
    uint32_t lut[SG::lut_words];  // key code pair (x copies) -> two fp16 centroids
    uint8_t ring[SG::npb][SG::pair];
    float wscr[SG::hpg][80];  // per-wave exchange
    // rotated q of each wave's heads as S^T operands: [wave][j][grp][head]
    // 16 bytes (dims 32 grp + 8 j .. + 7 of head), so the 8 heads a lane
    // group reads for one j fill the 32 banks once
    u32x4 qop[SG::hpg][4][4][8];
    int32_t bt[kStPages];     // block of each page of the slice
    int32_t info[kStPages];   // b << 6 | valid tokens << 1 | piece ends
    int32_t seg_b[kStPages], seg_ps[kStPages], seg_L[kStPages];
    WGPlan plan;
    int n_seg;
};

// one 16-byte-per-lane load-to-LDS transfer with the non-temporal hint: lane
// L's 16 bytes from base + off land at LDS address m0 + 16 L.  Issued from
// asm, so the compiler does not track it; the kernel counts its own
// transfers (vmcnt).
__device__ __forceinline__ void dma16_nt(const uint8_t* base, uint32_t off, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "{m0}"(m0) : "memory");
}

// After a global store of v: redefine v's registers in place, so the
// compiler waits for the store to read them here -- on the rare path that
// stores -- rather than at the first reuse of those registers in the page
// loop, where its wait (vmcnt) would also drain the load-to-LDS transfers in
// flight.
template <typename V>
__device__ __forceinline__ void store_done(V& v) {
    asm volatile("" : "+v"(v));
}

// LDS address of a pointer into the workgroup's LDS
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(const T* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

template <int KB, int VB, bool BF>
__global__ void __launch_bounds__(512, 4) tq_stream_kernel(DecodeParams p) {
    using SG = StGeo<KB, VB>;
    using AT = f16x8;
    __shared__ StLds<KB, VB> lds;
    WGPlan& plan = lds.plan;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int r16 = lane & 15, grp = lane >> 4;
    constexpr int hpg = SG::hpg;  // waves of the workgroup = KV heads of the group
    const int nranges = p.grid;
    const int w = (int)blockIdx.x;

    // key table: entry e (codes c0 | c1 << KB) = fp16(C[c0]) | fp16(C[c1]) << 16
    // at LDS words (e << lut_log2c) + copy.  Built by waves 1.. while wave 0
    // plans, four words (copies of one entry) per 16-byte write.
    static_assert(SG::lut_log2c >= 2, "a 16-byte group holds copies of one entry");
    if (wave != 0) {
        for (int i = tid - 64; i < SG::lut_words / 4; i += 64 * (hpg - 1)) {
            const int e = (4 * i) >> SG::lut_log2c;
            const int c0 = e & ((1 << KB) - 1), c1 = e >> KB;
            float a = 0.0f, b = 0.0f;
#pragma unroll
            for (int c = 0; c < (1 << KB); ++c) {
                a = c == c0 ? p.tab.centroids[c] : a;
                b = c == c1 ? p.tab.centroids[c] : b;
            }
            const uint32_t v = (uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
            reinterpret_cast<u32x4*>(lds.lut)[i] = u32x4{v, v, v, v};
        }
    }

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
            int T = 0, nz = 0;
            batch_pages(p, lane, &T, &nz);
            const int n = effective_wgs(p, T, nranges);
            // boundaries on the axis where a sequence switch counts as V pages
            const int V = switch_pages(p, n, T);
            const int Tv = T + V * max(nz - 1, 0);
            const int v_lo = w < n ? range_lo(p, w, n, Tv) : 0;
            const int v_hi = w < n ? range_lo(p, w + 1, n, Tv) : 0;
            if (V > 0) {
                real_pages(p, lane, V, v_lo, v_hi, &wp.p_lo, &wp.p_hi);
            } else {
                wp.p_lo = v_lo;
                wp.p_hi = v_hi;
            }
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

    // ---- Q operand: lane (r16, grp) reads dims 32 grp + 8 j + e of head qh
    // (columns c and c + 8 both hold head c), rotated (H q / sqrt(d)), from
    // the wave's LDS copy, one j at a time (no registers held across pairs)
    u32x4 (&qop)[4][4][8] = lds.qop[wave];
    auto q_at = [&](int j) -> AT { return __builtin_bit_cast(AT, qop[j][grp][qh]); };
    auto load_q = [&](int b) __attribute__((always_inline)) {
        // lane (r16, grp) rotates dims 32 grp + 16 hf .. + 15 of head qh
        // (hf = r16 / 8: the two lanes of a head's column pair split the
        // lane group's 32 dims) and writes their two 8-dim operand words
        const int hf = r16 >> 3;
        const int64_t qrow = ((int64_t)b * p.Hq + hq0 + qh) * kD;
        float y[16];
        if (q_ok) {
            const u32x4* src = reinterpret_cast<const u32x4*>(p.q + qrow + 32 * grp + 16 * hf);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const u32x4 wv = src[c];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    y[8 * c + 2 * e] = half_to_f32<BF>((uint16_t)(wv[e] & 0xffff));
                    y[8 * c + 2 * e + 1] = half_to_f32<BF>((uint16_t)(wv[e] >> 16));
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) y[e] = 0.0f;
        }
        // Walsh-Hadamard: half-widths 1..8 inside the lane, 16 across the
        // column pair (dim bit 16 = r16 bit 3: a row rotation by 8 lanes), 32
        // and 64 across the lane groups (grp bits 0 and 1).  The upper element
        // of a butterfly becomes partner - own: fma(-1, own, partner), exact.
#pragma unroll
        for (int hw = 1; hw < 16; hw <<= 1)
#pragma unroll
            for (int i = 0; i < 16; i += 2 * hw)
#pragma unroll
                for (int j = i; j < i + hw; ++j) {
                    const float a = y[j], c = y[j + hw];
                    y[j] = a + c;
                    y[j + hw] = a - c;
                }
        const float s8 = hf ? -1.0f : 1.0f, s16 = (grp & 1) ? -1.0f : 1.0f, s32 = (grp & 2) ? -1.0f : 1.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float o = __builtin_bit_cast(
                float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, y[e]), 0x128, 0xf, 0xf, false));
            y[e] = __builtin_fmaf(s8, y[e], o);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) y[e] = __builtin_fmaf(s16, y[e], shfl_xor(y[e], 16));
#pragma unroll
        for (int e = 0; e < 16; ++e) y[e] = __builtin_fmaf(s32, y[e], shfl_xor(y[e], 32));
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            AT v;
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (_Float16)__fmul_rn(y[8 * jj + e], p.tab.rot_c);
            qop[2 * hf + jj][grp][qh] = __builtin_bit_cast(u32x4, v);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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

    // ---- finish a piece of sequence b: the rows, or the partial slot (O
    // chunk c in units of its code field's fp16 subnormal)
    auto finalize = [&](int b) __attribute__((always_inline)) {
        const bool cut_before = b == __builtin_amdgcn_readfirstlane(plan.first_b) &&
                                __builtin_amdgcn_readfirstlane(plan.first_cut);
        const bool cut_after = b == __builtin_amdgcn_readfirstlane(plan.last_b) &&
                               __builtin_amdgcn_readfirstlane(plan.last_cut);
        const bool whole = !cut_before && !cut_after;
        const int slot = cut_before ? 2 * w : 2 * w + 1;
        float l_tot = sum_over_groups(l_part);
        float z_tot = sum_over_groups(z_part);
        // columns r16 and r16 ^ 8 hold the same head (O rows 0-7 already hold
        // both pages' sums: lane groups 0 and 1)
        l_tot += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, l_tot), 0x128, 0xf, 0xf, false));
        z_tot += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, z_tot), 0x128, 0xf, 0xf, false));
        const f32x4 lh4 = gather4_from_row0(l_tot, wscr, r16, grp);
        const f32x4 zh4 = gather4_from_row0(z_tot, wscr + 16, r16, grp);
        const f32x4 mh4 = gather4_from_row0(m_run, wscr + 32, r16, grp);
        // uniform row bases (scalar) plus 32-bit lane offsets: head hq0 + 4 grp
        // + i, dims 8 r16 .. + 7 (only lane groups 0 and 1 hold heads < 8)
        uint8_t* const obase = reinterpret_cast<uint8_t*>(p.out) + ((int64_t)b * p.Hq + hq0) * (2 * kD);
        uint8_t* const pbase = reinterpret_cast<uint8_t*>(p.part) + ((int64_t)slot * p.Hq + hq0) * (4 * kPartRow);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int hh = 4 * grp + i;
            const float lh = lh4[i], zh = zh4[i], mh = mh4[i];
            if (hh >= G) continue;
            if (whole) {
                const float inv = lh > 0.0f ? 1.0f / lh : 0.0f;
                uint32_t wd[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v0 = __builtin_fmaf(oacc[2 * e][i], kVScale<FMT_TQ, VB>(2 * e), zh) * inv;
                    const float v1 = __builtin_fmaf(oacc[2 * e + 1][i], kVScale<FMT_TQ, VB>(2 * e + 1), zh) * inv;
                    wd[e] = (uint32_t)f32_to_half<BF>(v0) | ((uint32_t)f32_to_half<BF>(v1) << 16);
                }
                const uint32_t off = (uint32_t)(hh * (2 * kD) + 16 * r16);
                u32x4 v = u32x4{wd[0], wd[1], wd[2], wd[3]};
                *reinterpret_cast<u32x4*>(obase + off) = v;
                store_done(v);
            } else {
                const uint32_t off = (uint32_t)(hh * (4 * kPartRow) + 32 * r16);
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                    u32x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v[e] = __builtin_bit_cast(uint32_t, __builtin_fmaf(oacc[4 * h2 + e][i], kVScale<FMT_TQ, VB>(4 * h2 + e), zh));
                    *reinterpret_cast<u32x4*>(pbase + off + 16 * h2) = v;
                    store_done(v);
                }
                if (r16 == 0) {
                    u32x2 v = {__builtin_bit_cast(uint32_t, mh), __builtin_bit_cast(uint32_t, lh)};
                    *reinterpret_cast<u32x2*>(pbase + (uint32_t)(hh * (4 * kPartRow) + 4 * kD)) = v;
                    store_done(v);
                }
            }
        }
        reset_state();
    };

    // ---- page transfers.  A page in HBM is 16 token rows of 8 slots (rowl
    // bytes each; turboquant_kernels.cu:39-45); its LDS buffer is a byte copy.
    // Wave w fetches chunks c = cw * w + 64 i + lane, i < tr: HBM and LDS
    // offset 16 c of the page.
    const int c_beg = SG::cw * wave;
    const int64_t page_bytes = p.page_bytes;
    const uint32_t ring_lds = lds_addr(&lds.ring[0][0]);
    auto dma_page = [&](int32_t blk, int buf, int pp) __attribute__((always_inline)) {
        const uint8_t* src = p.kc + (int64_t)blk * page_bytes + 16 * c_beg;
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(ring_lds + buf * SG::pair + pp * SG::pstr + 16 * c_beg);
        // 16 * lane, recomputed here (an asm the compiler cannot hoist) so no
        // register holds it across the loop: a spilled copy would be reloaded
        // from scratch, and that load's wait would drain the transfers
        uint32_t doff;
        asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0\n\tv_lshlrev_b32 %0, 4, %0"
                     : "=v"(doff));
#pragma unroll
        for (int i = 0; i < SG::tr - 1; ++i) dma16_nt(src + 1024 * i, doff, m0 + 1024 * i);
        if (lane < SG::last_lanes) dma16_nt(src + 1024 * (SG::tr - 1), doff, m0 + 1024 * (SG::tr - 1));
    };

    // loop-invariant LDS offsets inside a page buffer: the key run of token
    // r16 (its 4-byte floor; the run starts ks bytes in, the same for every
    // row and lane of this wave), the value code runs of tokens 4 grp + i
    // (dims 8 r16 .. + 7, from the 4-byte floor, vsh bytes in), the norms
    // (token r16) and the scale / zero pairs of tokens 4 grp + i on the
    // lane's own page (columns 0-7: first page)
    const int run0 = wave * SG::slot;
    const int kq = r16 * SG::rowl + run0 + (KB == 3 ? 12 : 16) * grp;
    const int kfl = kq & ~3;
    const uint32_t ks = (uint32_t)__builtin_amdgcn_readfirstlane(kq & 3);
    const int nq = r16 * SG::rowl + run0 + SG::mse;
    const int vq = 4 * grp * SG::rowl + run0 + SG::kp + VB * r16;
    const int vfl = vq & ~3;
    const uint32_t vsh = (uint32_t)(vq & 3);
    const int zq = 4 * grp * SG::rowl + run0 + SG::kp + SG::vd + (r16 >= 8 ? SG::pstr : 0);
    const int zfl = zq & ~3;
    const uint32_t zsh = (uint32_t)__builtin_amdgcn_readfirstlane(zq & 3);
    // byte-permute selectors that gather code bytes 0 .. 3 of two tokens' runs
    constexpr uint32_t vsel0 = 0x05040100u, vsel1 = 0x06050201u, vsel2 = 0x07060302u;
    // Gram diagonal: lane (r16, grp) picks element r16 % 4 (bit selects); the
    // exchange slot of its row factor is r16 on the diagonal (grp == r16 / 4),
    // else 16 + r16
    const uint32_t odd_mask = (r16 & 1) ? ~0u : 0u, hi_mask = (r16 & 2) ? ~0u : 0u;
    const int diag_slot = ((r16 >> 2) == grp ? 0 : 16) + r16;
    const uint8_t* const lutb = reinterpret_cast<const uint8_t*>(lds.lut);
    // the table copy of this lane, as a byte offset
    const uint32_t lut_lane = (uint32_t)(lane & ((1 << SG::lut_log2c) - 1)) << 2;
    auto lut_at = [&](uint32_t e) -> uint32_t {
        return lds32(lutb + ((e << (2 + SG::lut_log2c)) | lut_lane));
    };

    constexpr int NW = VB == 4 ? 4 : 3;
    // ---- one page pair from ring buffer pb: S, softmax, O += P . V; nv0 /
    // nv1 valid tokens of the first / second page (0: the page adds nothing)
    auto compute_pair = [&](const uint8_t* pg, int nv0, int nv1) __attribute__((always_inline)) {
        // the key code words of token r16 (both pages) and its norms
        uint32_t kd[2][KB == 3 ? 4 : 5];
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
            for (int i = 0; i < (KB == 3 ? 4 : 5); ++i) kd[pp][i] = lds32(pg + pp * SG::pstr + kfl + 4 * i);
        }
        const uint32_t nrm = lds16(pg + nq) | (lds16(pg + SG::pstr + nq) << 16);
        // one page at a time: the key operands (two codes per table entry),
        // then ||C[codes]||^2 per token from the Gram diagonal (token r16's
        // value in the lanes with grp == r16 / 4, element r16 % 4), the row
        // factor scale * norm / ||C|| (scale * norm without the norm
        // correction), and S^T against Q^T (S column c < 8 keeps the first
        // page's scores, head c; c >= 8 the second's, head c - 8).
        float rowf[2];
        f32x4 sp[2];
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            u32x4 aw[4];
            if constexpr (KB == 3) {
                // 12 code bytes = sixteen 6-bit fields (two codes each)
                uint32_t c[3];
#pragma unroll
                for (int i = 0; i < 3; ++i) c[i] = __builtin_amdgcn_alignbyte(kd[pp][i + 1], kd[pp][i], ks);
#pragma unroll
                for (int f = 0; f < 16; ++f) {
                    const int bit = 6 * f, wi = bit >> 5, o = bit & 31;
                    const uint32_t e = o <= 26 ? (c[wi] >> o) & 63u : __builtin_amdgcn_alignbit(c[wi + 1], c[wi], o) & 63u;
                    aw[f >> 2][f & 3] = lut_at(e);
                }
            } else {
                // 16 code bytes; each byte (two 4-bit codes) indexes the table
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t wd = __builtin_amdgcn_alignbyte(kd[pp][j + 1], kd[pp][j], ks);
#pragma unroll
                    for (int e = 0; e < 4; ++e) aw[j][e] = lut_at((wd >> (8 * e)) & 0xffu);
                }
            }
            AT a[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) a[j] = __builtin_bit_cast(AT, aw[j]);
            f32x4 gram = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) gram = mfma16x16x32(a[j], a[j], gram);
            f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) sacc = mfma16x16x32(a[j], q_at(j), sacc);
            sp[pp] = sacc;
            const float csq = sel_bits(sel_bits(gram[0], gram[1], odd_mask), sel_bits(gram[2], gram[3], odd_mask), hi_mask);
            const uint16_t nb16 = (uint16_t)(pp ? nrm >> 16 : nrm & 0xffffu);
            rowf[pp] = p.scale_log2 * half_to_f32<BF>(nb16) * (p.norm_corr ? __builtin_amdgcn_rsqf(csq + 1e-16f) : 1.0f);
        }
        wscr[diag_slot] = rowf[0];
        wscr[32 + diag_slot] = rowf[1];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const f32x4 rf = *reinterpret_cast<const f32x4*>(wscr + (r16 >= 8 ? 32 : 0) + 4 * grp);
        __builtin_amdgcn_wave_barrier();
        // scale / zero words of tokens 4 grp + i on the lane's page
        uint32_t hz[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            hz[i][0] = lds32(pg + zfl + i * SG::rowl);
            hz[i][1] = lds32(pg + zfl + i * SG::rowl + 4);
        }
        const bool second = r16 >= 8;
        float sv[4];
        uint32_t hsz[4];
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
            sv[i2] = (second ? sp[1][i2] : sp[0][i2]) * rf[i2];
            hsz[i2] = __builtin_amdgcn_alignbyte(hz[i2][1], hz[i2][0], zsh);
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
        float scf[4];
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) scf[i2] = half_to_f32<BF>((uint16_t)(hsz[i2] & 0xffffu));
        // lazy reference max: m_run moves only when a head's max passes it by
        // more than 8 (log2 units), so P <= 2^8; when a value scale of the
        // pair exceeds 65504 / 2^8 the max is taken exactly (P <= 1), so that
        // fp16(P * scale) cannot overflow.  A head's max spans columns c, c ^ 8
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
        // O += P . V: row h < 8 takes k = 8 grp + i from column h (first page,
        // token 4 grp + i) and k = 8 grp + 4 + i from column h + 8 (second
        // page; a row rotation by 8 lanes brings it over), so O rows 0-7 sum
        // both pages.  Rows 8-15 take the same columns the other way round:
        // their O rows are never read, and the rows of a product do not mix,
        // so they need no zeroing.  The V operand of output chunk c is its
        // code field masked where it lies (an fp16 subnormal
        // code * 2^(shift - 24), kVShift)
        const u32x2 pw2 = __builtin_bit_cast(u32x2, pw);
        // row_ror:8 (every lane has a source, so no old value is kept)
        const uint32_t pb0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)pw2[0], 0x128, 0xf, 0xf, false);
        const uint32_t pb1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)pw2[1], 0x128, 0xf, 0xf, false);
        const AT pa = __builtin_bit_cast(AT, u32x4{pw2[0], pw2[1], pb0, pb1});
        // value code words of tokens 4 grp + i (both pages), dims 8 r16 .. + 7
        uint32_t cw2[2][4][2];
#pragma unroll
        for (int pp = 0; pp < 2; ++pp)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                cw2[pp][i][0] = lds32(pg + pp * SG::pstr + vfl + i * SG::rowl);
                cw2[pp][i][1] = lds32(pg + pp * SG::pstr + vfl + i * SG::rowl + 4);
            }
        uint32_t wv[2][2][NW];
#pragma unroll
        for (int pp = 0; pp < 2; ++pp)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const uint32_t A = __builtin_amdgcn_alignbyte(cw2[pp][2 * hh][1], cw2[pp][2 * hh][0], vsh);
                const uint32_t Bw = __builtin_amdgcn_alignbyte(cw2[pp][2 * hh + 1][1], cw2[pp][2 * hh + 1][0], vsh);
                wv[pp][hh][0] = __builtin_amdgcn_perm(Bw, A, vsel0);
                wv[pp][hh][1] = __builtin_amdgcn_perm(Bw, A, vsel1);
                wv[pp][hh][2] = __builtin_amdgcn_perm(Bw, A, vsel2);
                if constexpr (VB == 4) wv[pp][hh][3] = __builtin_amdgcn_perm(Bw, A, 0x0c070c03u);
            }
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
            const AT vb = __builtin_bit_cast(AT, u32x4{wv[0][0][wi] & m, wv[0][1][wi] & m, wv[1][0][wi] & m,
                                                         wv[1][1][wi] & m});
            oacc[c] = mfma16x16x32(pa, vb, oacc[c]);
        }
    };

    // ---- the pair of pages (i, i + 1) of the slice in ring buffer pb.  A
    // pair that a piece boundary splits runs twice, each time with one page
    // masked.
    auto process_pair = [&](const uint8_t* pg, int i, int npc) __attribute__((always_inline)) {
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
            compute_pair(pg, nva, nvb);
            if (ends & 1) finalize(b);
            if (!split || part == 1) break;
            b = info1 >> 6;
            nva = 0;
            nvb = (info1 >> 1) & 31;
            ends = info1;
        }
    };

    // ---- slices of up to kStPages pages: stage the block-table slice and the
    // per-page sequence info in LDS, then stream the pages
    for (int c_lo = p_lo; c_lo < p_hi; c_lo += kStPages) {
        const int c_hi = min(p_hi, c_lo + kStPages);
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
            int lo_s = 0, hi_s = ns - 1;  // last segment with seg_ps <= gp
            while (lo_s < hi_s) {
                const int mid = (lo_s + hi_s + 1) >> 1;
                if (lds.seg_ps[mid] <= gp) lo_s = mid;
                else hi_s = mid - 1;
            }
            const int b = lds.seg_b[lo_s], L = lds.seg_L[lo_s], pp = gp - lds.seg_ps[lo_s];
            const int pages_b = (L + kBs - 1) / kBs;
            const int32_t blk = p.bt[(int64_t)(p.row_seq ? p.row_seq[b] : b) * p.max_blocks + pp];
            const int nv = blk < 0 ? 0 : min(kBs, L - pp * kBs);
            const int ends = pp == pages_b - 1 || gp == p_hi - 1;
            lds.bt[i] = blk;
            lds.info[i] = (b << 6) | (nv << 1) | ends;
        }
        __syncthreads();

        // Pair k of the slice sits in ring buffer k % 2.  Step k waits for this
        // wave's transfers of pair k (the only ones in flight), then a
        // workgroup barrier (every wave's transfers of pair k have landed, and
        // every wave has finished pair k - 1, whose buffer is free), issues
        // pair k + 1 into that buffer and computes pair k: a pair's transfers
        // have one step to land.
        const int npairs = (npc + 1) >> 1;
        auto blk_of = [&](int i) -> int32_t {
            return __builtin_amdgcn_readfirstlane(i < npc ? max(lds.bt[i], 0) : 0);
        };
        auto issue_pair = [&](int k, int buf) __attribute__((always_inline)) {
            dma_page(blk_of(2 * k), buf, 0);
            if (2 * k + 1 < npc) dma_page(blk_of(2 * k + 1), buf, 1);
        };
        // q of the slice's first sequence before any transfer is in flight:
        // its loads' wait (vmcnt) would otherwise also wait for them
        if (npairs > 0) {
            const int b0 = __builtin_amdgcn_readfirstlane(lds.info[0]) >> 6;
            if (b0 != cur_b) {
                load_q(b0);
                cur_b = b0;
            }
            issue_pair(0, 0);
        }
        for (int k0 = 0; k0 < npairs; k0 += 2) {
            static_for<2>([&](auto pc) __attribute__((always_inline)) {
                constexpr int P = decltype(pc)::value;
                const int k = k0 + P;
                if (k < npairs) {  // uniform over the workgroup
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    __syncthreads();
                    if (k + 1 < npairs) issue_pair(k + 1, P ^ 1);
                    process_pair(&lds.ring[P][0], 2 * k, npc);
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

// TurboQuant 3-bit decode (reference layout, 8 KV heads, G <= 8) with the
// streaming kernel; VMC_EINVAL when the shape is not one it takes (4-bit and
// k3v4 pages do not fit two workgroups' rings in a CU's LDS).
template <int KB, int VB, bool BF>
int launch_tq_stream(DecodeParams& prm, hipStream_t stream) {
    using SG = StGeo<KB, VB>;
    static_assert(SG::fits, "two workgroups per CU");
    if (prm.entry_bytes != SG::slot || prm.mse_bytes != SG::mse || prm.key_packed != SG::kp ||
        prm.val_data != SG::vd)
        return VMC_EINVAL;
    if (prm.G > 8 || prm.Hkv != SG::hpg) return VMC_EINVAL;
    prm.row_bytes = SG::rowl;
    if (prm.page_bytes != SG::page) return VMC_EINVAL;
    prm.hpw = SG::hpg;
    prm.hgroups = 1;
    prm.grid = prm.per_seq ? prm.B : tq_stream_ranges(prm.B, prm.Hkv, prm.max_blocks, prm.max_splits, num_cus());
    // With two workgroups on every CU, workgroups w and w + CUs share one,
    // and the first, dispatched ahead, wins the instruction issue: on the
    // ragged 32k batch it ended at 111-121 us median against 147-158 us for
    // its partner, which then ran alone.  It takes 5 of 8 parts of the pair's
    // pages: both then end together, and the kernel took 155.0 against
    // 160.2 us (162.4-164.7 against 169.4-170.9 us per call, the same GPU).
    const int cus = num_cus();
    prm.split_h = !prm.per_seq && prm.grid == 2 * cus ? cus : 0;
    prm.split_wa = 5;
    prm.split_wb = 3;
    // A range that holds a sequence switch (the last piece's rows, the next
    // sequence's q loaded and rotated, the pair across the boundary computed
    // twice) took ~7 us longer on the ragged 32k batch, and the 20 slowest of
    // 256 CUs all held one.  Counting each switch as 8 pages evens that out:
    // 166.0 against 167.9 us per call (the same GPU, three alternations).
    prm.split_v = 8;
    hipLaunchKernelGGL((tq_stream_kernel<KB, VB, BF>), dim3(prm.grid), dim3(64 * SG::hpg), 0, stream, prm);
    VMC_LAUNCH_CHECK();
    if (!prm.per_seq) {
        hipLaunchKernelGGL(decode_merge_kernel, dim3(prm.B, prm.Hkv), dim3(64 * prm.G), 0, stream, prm);
        VMC_LAUNCH_CHECK();
    }
    return VMC_OK;
}

int launch_tq_stream_any(DecodeParams& prm, int kb, int vb, bool bf, hipStream_t s) {
    if (kb == 3 && vb == 3) return bf ? launch_tq_stream<3, 3, true>(prm, s) : launch_tq_stream<3, 3, false>(prm, s);
    return VMC_EINVAL;
}

}  // namespace vmc
