// tq_decode_d256.hip -- split-KV paged decode over TurboQuant slots of
// head_dim 256 (the reference layout, turboquant_4bit_nc / 3bit_nc: 262 /
// 198-byte slots), 1, 2 or 4 KV heads, at most 8 query heads per KV head.
// The reference's deployment of this size (Qwen3.5-A3B: head_dim 256, 16
// query / 2 KV heads, src/distributed/tp_runtime.cpp:257-261) runs here.
//
// Replaces the decode of vm_c::turboquant_decode_attention
// (src/cuda/turboquant_kernels.cu:939-1007) for head_dim 256: q rotated by
// the 256-point Walsh-Hadamard transform, K = C[code] * norm / ||C[codes]||,
// V = code * scale + zero, fp32 online softmax, a split over page ranges
// merged in a second pass (stage 2, :508-547).
//
// Organisation:
//  * a workgroup of 8 waves = Hkv heads x S page streams (S = 8 / Hkv), one
//    per CU; each stream is a page range of its own (its own plan, pieces
//    and partial slots), and each wave (head, stream) runs one page of its
//    stream per step;
//  * per step the workgroup fetches the S pages (every KV head of each, a
//    contiguous block) by load-to-LDS transfers into one of three buffers,
//    two steps in flight;
//  * per wave and page (16 tokens x G <= 8 query heads): S^T = K . Q^T on
//    v_mfma_f32_16x16x32_f16 over 8 steps of 32 dims (lane (r16, grp) holds
//    dims 64 grp .. + 63 of token r16; Q^T columns c and c + 8 both hold head
//    c), ||C[codes]||^2 from the Gram diagonal K K^T, lazy-max online
//    softmax, O += P . V on v_mfma_f32_16x16x16_f16 over the page's 16
//    tokens, 16 output tiles of 16 dims (lane r16 owns dims 16 r16 .. + 15),
//    V codes as exact fp16 subnormals and sum(P * zero) kept apart;
//  * key codes go through an LDS table of packed fp16 centroid pairs (code
//    pair -> two fp16) in 32 copies, lane l reading copy l % 32 (no two
//    lanes of a half wave share a bank); P enters the PV product as fp16(P * scale), with the exact running
//    max for a page whose largest value scale exceeds 65504 / 2^8.
#include "decode_plan.hpp"

namespace vmc {
namespace {

constexpr int kD2 = 256;
constexpr int kPages2 = 64;
constexpr int kPartRow2 = kD2 + 4;  // split partial row: o[256], m, l, padding to 16 bytes  // pages per staged slice of a stream's block table

template <int KB, int HK>
struct D2Geo {
    static constexpr int mse = 32 * KB, kp = mse + 2, vd = 32 * KB;
    static constexpr int slot = (kp + vd + 4 + 1) / 2 * 2;  // 262 (4-bit), 198 (3-bit)
    static constexpr int row = HK * slot;                   // one token row, every KV head
    static constexpr int page = kBs * row;                  // a multiple of 16 bytes
    static constexpr int ns = 8 / HK;                       // page streams per workgroup (HK waves each)
    static constexpr int nb = 3;                            // page buffers per stream
    // a page is HK * slot 16-byte chunks: wave h of a stream fetches chunks
    // h * slot .. + slot - 1, in ni transfers (the last of `last` lanes)
    static constexpr int ni = (slot + 63) / 64;
    static constexpr int last = slot - 64 * (ni - 1);
    // key table: entry e (codes c0 | c1 << KB) at words (e << log2c) + copy,
    // 32 copies: lane l reads copy l % 32, its own bank
    static constexpr int log2c = 5;
    static constexpr int lut_words = (KB == 3 ? 64 : 256) << log2c;
    static constexpr int kw = KB == 3 ? 7 : 9;  // key words of a lane (its 64 dims, from the 4-byte floor)
};

template <int KB, int HK>
struct alignas(16) D2Lds {
    using DG = D2Geo<KB, HK>;
    uint32_t lut[DG::lut_words];
    uint8_t ring[DG::ns][DG::nb][DG::page];  // [stream][buffer]: a buffer within 64 KB of its stream's
    float wscr[8][80];                       // per-wave exchange
    uint32_t ctab[16];                       // fp16 centroids (table build)
    int32_t bt[DG::ns][kPages2];
    int32_t info[DG::ns][kPages2];  // b << 6 | valid tokens << 1 | piece ends
    int32_t seg_b[DG::ns][kPages2], seg_ps[DG::ns][kPages2], seg_L[DG::ns][kPages2];
    WGPlan plan[DG::ns];
    int n_seg[DG::ns];
};

__device__ __forceinline__ void dma16_d2(const uint8_t* base, uint32_t off, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "{m0}"(m0) : "memory");
}

template <typename T>
__device__ __forceinline__ uint32_t lds_addr2(const T* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// After a global store of v: redefine v's registers, so the compiler waits
// for the store to read them on the storing path, not at their first reuse in
// the page loop (a wait there would also drain the transfers in flight).
template <typename V>
__device__ __forceinline__ void store_done2(V& v) {
    asm volatile("" : "+v"(v));
}

// the V operand of output tile c from the packed words of two tokens: 3-bit
// byte-window words (wv[0..2]: run bytes (0,1), (1,2), (2,3)), 4-bit (wv[0..3]:
// bytes 0, 1, 2, 3); the code field masked where it lies
template <int KB>
__device__ __forceinline__ uint32_t v_field(const uint32_t (&wv)[4], int c) {
    if constexpr (KB == 4) {
        return wv[c >> 1] & ((c & 1) ? 0x00f000f0u : 0x000f000fu);
    } else {
        constexpr uint32_t kM[8] = {0x00070007u, 0x00380038u, 0x01c001c0u, 0x000e000eu,
                                    0x00700070u, 0x03800380u, 0x001c001cu, 0x00e000e0u};
        return wv[c < 3 ? 0 : c < 6 ? 1 : 2] & kM[c];
    }
}

template <int KB, int HK, bool BF>
__global__ void __launch_bounds__(512, 1) tq_decode_d256_kernel(DecodeParams p) {
    using DG = D2Geo<KB, HK>;
    using AT = f16x8;
    __shared__ D2Lds<KB, HK> lds;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int r16 = lane & 15, grp = lane >> 4;
    const int head = wave % HK, stream = wave / HK;
    const int nranges = p.grid;  // page ranges = workgroups x streams
    const int w = (int)blockIdx.x * DG::ns + stream;  // this wave's range

    // ---- the page range of each stream (the first wave of the stream)
    if (head == 0) {
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
            const int pg = w < p.B ? seq_pages(p, w, &L) : 0;
            wp = {ps, ps + pg, w, w, 0, 0};
        } else {
            const int T = total_pages(p, lane);
            const int n = effective_wgs(p, T, nranges);
            wp.p_lo = w < n ? (int)((int64_t)w * T / n) : 0;
            wp.p_hi = w < n ? (int)((int64_t)(w + 1) * T / n) : 0;
            wp.first_b = wp.last_b = -1;
            wp.first_cut = wp.last_cut = 0;
        }
        if (lane == 0) lds.plan[stream] = wp;
    }
    // key table: the fp16 centroids, then each entry's 32 copies (four per
    // 16-byte store)
    if (tid < (1 << KB)) lds.ctab[tid] = f32_to_f16_bits(p.tab.centroids[tid]);
    __syncthreads();
    for (int i = tid; i < DG::lut_words / 4; i += 512) {
        const int e = i >> (DG::log2c - 2);
        const uint32_t v = lds.ctab[e & ((1 << KB) - 1)] | (lds.ctab[e >> KB] << 16);
        reinterpret_cast<u32x4*>(lds.lut)[i] = u32x4{v, v, v, v};
    }
    __syncthreads();
    WGPlan& plan = lds.plan[stream];
    const int p_lo = __builtin_amdgcn_readfirstlane(plan.p_lo);
    const int p_hi = __builtin_amdgcn_readfirstlane(plan.p_hi);
    const int G = p.G;
    const int hq0 = head * G;
    const int qh = r16 & 7;  // query head of S column r16
    float* wscr = lds.wscr[wave];

    // every stream's number of pages, in slices of kPages2: the workgroup
    // steps together, a stream past its end idles
    int steps = 0;
#pragma unroll
    for (int s = 0; s < DG::ns; ++s)
        steps = max(steps, __builtin_amdgcn_readfirstlane(lds.plan[s].p_hi - lds.plan[s].p_lo));
    // a sequence without pages (per-sequence mode): zero rows (the flat
    // mode's merge pass writes those)
    if (p.per_seq && w < p.B && p_hi == p_lo && lane < 32) {
        for (int hh = 0; hh < G; ++hh)
            reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(p.out) + ((int64_t)w * p.Hq + hq0 + hh) * kD2)[lane] =
                u32x4{0u, 0u, 0u, 0u};
    }
    if (steps == 0) return;

    // ---- Q operand: lane (r16, grp) holds dims 64 grp + 8 j + e of head
    // r16 % 8 for MFMA j, rotated (H q / sqrt(256)).  The rotation runs with
    // lane (h, t) = (lane / 8, lane % 8) holding dims 32 t .. + 31 of head h
    // (three cross-lane stages by DPP); lane permutes then gather the
    // operand: dims 64 grp .. + 31 from lane 8 h + 2 grp, the next 32 from
    // lane 8 h + 2 grp + 1.
    AT qb[8];
    const int qlh = lane >> 3, qlt = lane & 7;
    auto fetch_q = [&](int b, u32x4 (&raw)[4]) __attribute__((always_inline)) {
        if (qlh < G) {
            const u32x4* src = reinterpret_cast<const u32x4*>(p.q + ((int64_t)b * p.Hq + hq0 + qlh) * kD2 + 32 * qlt);
#pragma unroll
            for (int c = 0; c < 4; ++c) raw[c] = src[c];
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) raw[c] = u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto rotate_q = [&](const u32x4 (&raw)[4]) __attribute__((always_inline)) {
        float y[32];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                y[8 * c + 2 * e] = half_to_f32<BF>((uint16_t)(raw[c][e] & 0xffff));
                y[8 * c + 2 * e + 1] = half_to_f32<BF>((uint16_t)(raw[c][e] >> 16));
            }
        // Walsh-Hadamard: half-widths 1..16 inside the lane, 32, 64, 128 across
        // lanes (dim bits 5, 6, 7 = lane bits 0, 1, 2)
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
            const float o = row_xor<1>(y[e], lane);
            y[e] = (lane & 1) ? o - y[e] : y[e] + o;
        }
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const float o = row_xor<2>(y[e], lane);
            y[e] = (lane & 2) ? o - y[e] : y[e] + o;
        }
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const float o = row_xor<4>(y[e], lane);
            y[e] = (lane & 4) ? o - y[e] : y[e] + o;
        }
        uint32_t wq[16];  // fp16 pairs: dims 32 t + 2 k, + 1
#pragma unroll
        for (int k = 0; k < 16; ++k)
            wq[k] = (uint32_t)f32_to_f16_bits(__fmul_rn(y[2 * k], p.tab.rot_c)) |
                    ((uint32_t)f32_to_f16_bits(__fmul_rn(y[2 * k + 1], p.tab.rot_c)) << 16);
        const int src0 = (8 * qh + 2 * grp) << 2;  // byte address of the source lane
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            u32x4 v;
#pragma unroll
            for (int d = 0; d < 4; ++d)
                v[d] = (uint32_t)__builtin_amdgcn_ds_bpermute(src0 + ((j >> 2) << 2), (int)wq[4 * (j & 3) + d]);
            qb[j] = __builtin_bit_cast(AT, v);
        }
    };
    auto load_q = [&](int b) __attribute__((always_inline)) {
        u32x4 raw[4];
        fetch_q(b, raw);
        rotate_q(raw);
    };

    // ---- running state of the current piece
    f32x4 oacc[16];
    float m_run, l_part, z_part, m_thr;
    auto reset_state = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < 16; ++c) oacc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        m_run = kNegInf;
        m_thr = kNegInf;
        l_part = 0.0f;
        z_part = 0.0f;
    };
    reset_state();
    int cur_b = -1;

    // ---- finish a piece of sequence b: the rows (lane groups 0 and 1 hold
    // O rows 0-7 = heads 0-7; O tile c holds dim 16 r16 + c, in units of its
    // code field's fp16 subnormal), or the partial slot
    auto finalize = [&](int b) __attribute__((always_inline)) {
        const bool cut_before = b == __builtin_amdgcn_readfirstlane(plan.first_b) &&
                                __builtin_amdgcn_readfirstlane(plan.first_cut);
        const bool cut_after = b == __builtin_amdgcn_readfirstlane(plan.last_b) &&
                               __builtin_amdgcn_readfirstlane(plan.last_cut);
        const bool whole = !cut_before && !cut_after;
        const int slot = cut_before ? 2 * w : 2 * w + 1;
        const float l_tot = sum_over_groups(l_part);
        const float z_tot = sum_over_groups(z_part);
        const f32x4 lh4 = gather4_from_row0(l_tot, wscr, r16, grp);
        const f32x4 zh4 = gather4_from_row0(z_tot, wscr + 16, r16, grp);
        const f32x4 mh4 = gather4_from_row0(m_run, wscr + 32, r16, grp);
        uint8_t* const obase = reinterpret_cast<uint8_t*>(p.out) + ((int64_t)b * p.Hq + hq0) * (2 * kD2);
        uint8_t* const pbase = reinterpret_cast<uint8_t*>(p.part) + ((int64_t)slot * p.Hq + hq0) * (4 * kPartRow2);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int hh = 4 * grp + i;
            const float lh = lh4[i], zh = zh4[i], mh = mh4[i];
            if (hh >= G) continue;
            if (whole) {
                const float inv = lh > 0.0f ? 1.0f / lh : 0.0f;
                uint32_t wd[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float v0 = __builtin_fmaf(oacc[2 * e][i], kVScale<FMT_TQ, KB>(2 * e & 7), zh) * inv;
                    const float v1 = __builtin_fmaf(oacc[2 * e + 1][i], kVScale<FMT_TQ, KB>((2 * e + 1) & 7), zh) * inv;
                    wd[e] = (uint32_t)f32_to_half<BF>(v0) | ((uint32_t)f32_to_half<BF>(v1) << 16);
                }
                const uint32_t off = (uint32_t)(hh * (2 * kD2) + 32 * r16);
                u32x4 v0 = u32x4{wd[0], wd[1], wd[2], wd[3]}, v1 = u32x4{wd[4], wd[5], wd[6], wd[7]};
                *reinterpret_cast<u32x4*>(obase + off) = v0;
                *reinterpret_cast<u32x4*>(obase + off + 16) = v1;
                store_done2(v0);
                store_done2(v1);
            } else {
                const uint32_t off = (uint32_t)(hh * (4 * kPartRow2) + 64 * r16);
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    u32x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v[e] = __builtin_bit_cast(uint32_t, __builtin_fmaf(oacc[4 * q4 + e][i], kVScale<FMT_TQ, KB>((4 * q4 + e) & 7), zh));
                    *reinterpret_cast<u32x4*>(pbase + off + 16 * q4) = v;
                    store_done2(v);
                }
                if (r16 == 0) {
                    u32x2 v = {__builtin_bit_cast(uint32_t, mh), __builtin_bit_cast(uint32_t, lh)};
                    *reinterpret_cast<u32x2*>(pbase + (uint32_t)(hh * (4 * kPartRow2) + 4 * kD2)) = v;
                    store_done2(v);
                }
            }
        }
        reset_state();
    };

    // ---- loop-invariant LDS offsets from buffer 0 of this wave's stream (a
    // byte copy of the page; token row r at r * row, this head's run at
    // head * slot of it): the key words of token r16 (dims 64 grp .. + 63,
    // from the 4-byte floor), its norm, the value runs of tokens 4 grp + i
    // (dims 16 r16 .. + 15) and their scale / zero pairs
    const int run0 = stream * DG::nb * DG::page + head * DG::slot;
    const int kq = r16 * DG::row + run0 + (KB == 3 ? 24 : 32) * grp;
    const int kfl = kq & ~3;
    const uint32_t ksh = (uint32_t)(kq & 3);
    const int nq = r16 * DG::row + run0 + DG::mse;
    // value runs: 4 tokens, each its own 4-byte floor and shift (rows may
    // differ in alignment)
    // (half h of a run: its codes 8 h .. 8 h + 7, from byte 3 h (3-bit) or
    // 4 h (4-bit))
    int vfl[2][4], zfl[4];
    uint32_t vsh[2][4], zsh[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int vq = (4 * grp + i) * DG::row + run0 + DG::kp + 2 * KB * r16 + (KB == 3 ? 3 : 4) * h;
            vfl[h][i] = vq & ~3;
            vsh[h][i] = (uint32_t)(vq & 3);
        }
        const int zq = (4 * grp + i) * DG::row + run0 + DG::kp + DG::vd;
        zfl[i] = zq & ~3;
        zsh[i] = (uint32_t)(zq & 3);
    }
    const uint32_t odd_mask = (r16 & 1) ? ~0u : 0u, hi_mask = (r16 & 2) ? ~0u : 0u;
    const int diag_slot = ((r16 >> 2) == grp ? 0 : 16) + r16;
    const uint8_t* const lutb = reinterpret_cast<const uint8_t*>(lds.lut);
    const uint32_t lut_lane = (uint32_t)(lane & ((1 << DG::log2c) - 1)) << 2;
    auto lut_at = [&](uint32_t e) -> uint32_t { return lds32(lutb + ((e << (2 + DG::log2c)) | lut_lane)); };
    constexpr uint32_t vsel0 = 0x05040100u, vsel1 = 0x06050201u, vsel2 = 0x07060302u;

    // ---- one page (16 tokens, nv valid) from LDS page buffer pg
    auto compute_page = [&](const uint8_t* pg, int nv) __attribute__((always_inline)) {
        uint32_t kd[DG::kw];
#pragma unroll
        for (int i = 0; i < DG::kw; ++i) kd[i] = lds32(pg + kfl + 4 * i);
        const float nrm = half_to_f32<BF>((uint16_t)lds16(pg + nq));
        // key operands: MFMA j takes dims 64 grp + 8 j .. + 7 (4 table entries)
        AT a[8];
        if constexpr (KB == 3) {
            uint32_t c[6];
#pragma unroll
            for (int i = 0; i < 6; ++i) c[i] = __builtin_amdgcn_alignbyte(kd[i + 1], kd[i], ksh);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                u32x4 aw;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int f = 4 * j + e, bit = 6 * f, wi = bit >> 5, o = bit & 31;
                    const uint32_t x = o <= 26 ? (c[wi] >> o) & 63u : __builtin_amdgcn_alignbit(c[wi + 1], c[wi], o) & 63u;
                    aw[e] = lut_at(x);
                }
                a[j] = __builtin_bit_cast(AT, aw);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t wd = __builtin_amdgcn_alignbyte(kd[j + 1], kd[j], ksh);
                u32x4 aw;
#pragma unroll
                for (int e = 0; e < 4; ++e) aw[e] = lut_at((wd >> (8 * e)) & 0xffu);
                a[j] = __builtin_bit_cast(AT, aw);
            }
        }
        // ||C[codes]||^2 (Gram diagonal) and S^T = K . Q^T
        f32x4 gram = {0.f, 0.f, 0.f, 0.f}, sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 8; ++j) gram = mfma16x16x32(a[j], a[j], gram);
#pragma unroll
        for (int j = 0; j < 8; ++j) sacc = mfma16x16x32(a[j], qb[j], sacc);
        const float csq = sel_bits(sel_bits(gram[0], gram[1], odd_mask), sel_bits(gram[2], gram[3], odd_mask), hi_mask);
        const float rowf = p.scale_log2 * nrm * (p.norm_corr ? __builtin_amdgcn_rsqf(csq + 1e-16f) : 1.0f);
        wscr[diag_slot] = rowf;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const f32x4 rf = *reinterpret_cast<const f32x4*>(wscr + 4 * grp);
        __builtin_amdgcn_wave_barrier();
        // scale / zero of tokens 4 grp + i
        float sv[4], scf[4], zf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t hz = __builtin_amdgcn_alignbyte(lds32(pg + zfl[i] + 4), lds32(pg + zfl[i]), zsh[i]);
            const bool ok = 4 * grp + i < nv;  // tokens past a page's end may hold anything
            sv[i] = ok ? sacc[i] * rf[i] : kNegInf;
            scf[i] = ok ? half_to_f32<BF>((uint16_t)(hz & 0xffffu)) : 0.0f;
            zf[i] = ok ? half_to_f32<BF>((uint16_t)(hz >> 16)) : 0.0f;
        }
        // lazy reference max (P <= 2^8), exact when a value scale of the page
        // exceeds 65504 / 2^8 (P <= 1: fp16(P * scale) in range)
        const float smax = vmax(vmax(scf[0], scf[1]), vmax(scf[2], scf[3]));
        const bool exact = __ballot(smax > 255.875f) != 0;
        const float thr = exact ? m_run : m_thr;
        const float mloc = vmax(vmax(sv[0], sv[1]), vmax(sv[2], sv[3]));
        if (__ballot(mloc > thr)) {
            const float mx = vmax_over_groups(mloc);
            const bool upd = mx > thr;
            const float m_new = upd ? vmax(mx, m_run) : m_run;
            const float alpha = m_new > m_run ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
            l_part *= alpha;
            z_part *= alpha;
            const f32x4 al = gather4_from_row0(alpha, wscr + 64, r16, grp);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int c = 0; c < 16; ++c) oacc[c][i] *= al[i];
            m_run = m_new;
            m_thr = m_run + 8.0f;
        }
        const float m_use = m_run == kNegInf ? 0.0f : m_run;
        float psum = 0.0f, zsum = 0.0f;
        f16x4 pa;  // A operand of the PV MFMA: row r16 (head), k = 4 grp + i (token)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float pv = __builtin_amdgcn_exp2f(sv[i] - m_use);
            psum += pv;
            zsum = __builtin_fmaf(pv, zf[i], zsum);
            pa[i] = (_Float16)__builtin_fmaf(pv, scf[i], 0.0f);
        }
        l_part += psum;
        z_part += zsum;
        uint32_t vw[2][4];  // half h, token 4 grp + i: the run's words from its floor, aligned
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                vw[h][i] = __builtin_amdgcn_alignbyte(lds32(pg + vfl[h][i] + 4), lds32(pg + vfl[h][i]), vsh[h][i]);
        // value operands: tile c = dim 16 r16 + c; tokens 4 grp + 0, 1 in dword
        // 0 and + 2, 3 in dword 1; the run's first 8 codes from its bytes
        // 0 .. 3, the last 8 from the bytes after (3-bit: bytes 3 .. 6, 4-bit:
        // 4 .. 7)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            uint32_t wv[2][4];
#pragma unroll
            for (int tp = 0; tp < 2; ++tp) {
                const uint32_t A = vw[half][2 * tp], B = vw[half][2 * tp + 1];
                wv[tp][0] = __builtin_amdgcn_perm(B, A, vsel0);
                wv[tp][1] = __builtin_amdgcn_perm(B, A, vsel1);
                wv[tp][2] = __builtin_amdgcn_perm(B, A, vsel2);
                wv[tp][3] = KB == 4 ? __builtin_amdgcn_perm(B, A, 0x0c070c03u) : 0u;
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const f16x4 vb = __builtin_bit_cast(f16x4, u32x2{v_field<KB>(wv[0], c), v_field<KB>(wv[1], c)});
                oacc[8 * half + c] = mfma16x16x16(pa, vb, oacc[8 * half + c]);
            }
        }
    };

    // ---- pages of a stream: staged per slice (block and sequence info).
    // Wave h of a stream fetches chunks h * slot .. + slot - 1 of the stream's
    // page of a step: always ni transfers (a stream without a page in the
    // step fetches block 0 unused), so that vmcnt counts steps.
    const uint32_t ring_lds = lds_addr2(&lds.ring[stream][0][0]) + 16 * head * DG::slot;
    auto dma_step = [&](int k, int buf) __attribute__((always_inline)) {
        const int info = __builtin_amdgcn_readfirstlane(lds.info[stream][k]);
        const int32_t blk = (info & (1 << 30)) ? __builtin_amdgcn_readfirstlane(max(lds.bt[stream][k], 0)) : 0;
        const uint8_t* src = p.kc + (int64_t)blk * p.page_bytes + 16 * head * DG::slot;
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(ring_lds + buf * DG::page);
        uint32_t doff;
        asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0\n\tv_lshlrev_b32 %0, 4, %0"
                     : "=v"(doff));
#pragma unroll
        for (int i = 0; i < DG::ni - 1; ++i) dma16_d2(src + 1024 * i, doff, m0 + 1024 * i);
        if (lane < DG::last) dma16_d2(src + 1024 * (DG::ni - 1), doff, m0 + 1024 * (DG::ni - 1));
    };

    for (int c0 = 0; c0 < steps; c0 += kPages2) {
        const int cn = min(kPages2, steps - c0);  // steps of this slice
        // stage each stream's slice: pages p_lo + c0 .. of its range
        if (head == 0) {
            const int slo = min(p_hi, p_lo + c0), shi = min(p_hi, p_lo + c0 + cn);
            int ns = 0;
            if (slo < shi)
                ns = collect_segments(p, slo, shi, lane, lds.seg_b[stream], lds.seg_ps[stream], lds.seg_L[stream],
                                      &plan, c0 == 0 && !p.per_seq);
            if (lane == 0) lds.n_seg[stream] = ns;
        }
        __syncthreads();
        for (int e = tid; e < DG::ns * cn; e += 512) {
            const int s = e / cn, i = e - s * cn;
            const int lo_s = lds.plan[s].p_lo, hi_s = lds.plan[s].p_hi;
            const int gp = lo_s + c0 + i;
            int32_t blk = -1, info = 0;
            if (gp < hi_s) {
                const int nsg = lds.n_seg[s];
                int a = 0, z = nsg - 1;  // last segment with seg_ps <= gp
                while (a < z) {
                    const int mid = (a + z + 1) >> 1;
                    if (lds.seg_ps[s][mid] <= gp) a = mid;
                    else z = mid - 1;
                }
                const int b = lds.seg_b[s][a], L = lds.seg_L[s][a], pp = gp - lds.seg_ps[s][a];
                const int pages_b = (L + kBs - 1) / kBs;
                blk = p.bt[(int64_t)(p.row_seq ? p.row_seq[b] : b) * p.max_blocks + pp];
                const int nv = blk < 0 ? 0 : min(kBs, L - pp * kBs);
                const int ends = pp == pages_b - 1 || gp == hi_s - 1;
                info = (b << 6) | (nv << 1) | ends | (1 << 30);  // bit 30: the step holds a page
            }
            lds.bt[s][i] = blk;
            lds.info[s][i] = info;
        }
        __syncthreads();

        // Step k sits in buffer k % 3; two steps in flight.  At step k: wait
        // for this wave's transfers of step k (those of step k + 1 may stay
        // in flight), a workgroup barrier (every wave's have landed, and
        // every wave has finished step k - 1, whose buffer is free), issue
        // step k + 2 there, compute step k.
        // q of the range's first sequence: its loads in flight with the first
        // transfers
        const int info0 = __builtin_amdgcn_readfirstlane(lds.info[stream][0]);
        const bool pre = c0 == 0 && (info0 & (1 << 30));
        u32x4 raw[4];
        if (pre) fetch_q((info0 >> 6) & 0xffffff, raw);
        dma_step(0, 0);
        if (cn > 1) dma_step(1, 1);
        if (pre) {
            rotate_q(raw);
            cur_b = (info0 >> 6) & 0xffffff;
        }
        for (int k0 = 0; k0 < cn; k0 += 3) {
            static_for<3>([&](auto pc) __attribute__((always_inline)) {
                constexpr int P = decltype(pc)::value;
                const int k = k0 + P;
                if (k < cn) {
                    if (k + 1 < cn) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DG::ni) : "memory");
                    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    __syncthreads();
                    if (k + 2 < cn) dma_step(k + 2, (P + 2) % 3);
                    const int info = __builtin_amdgcn_readfirstlane(lds.info[stream][k]);
                    if (info & (1 << 30)) {  // uniform over the wave
                        const int b = (info >> 6) & 0xffffff;
                        if (b != cur_b) {
                            load_q(b);
                            cur_b = b;
                        }
                        compute_page(&lds.ring[0][P][0], (info >> 1) & 31);
                        if (info & 1) finalize(b);
                    }
                }
            });
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
}

// Combines the pieces of sequences cut by range boundaries (head_dim 256):
// decode_merge_kernel's rule over rows of kPartRow2 floats (o unnormalised, m,
// l).  Grid (B, Hq), 4 waves per (sequence, query head): wave w takes pieces
// w, w + 4, ... (sixteen rows in flight), lane l dims 4 l .. + 3; the four
// partial sums are combined through LDS.
__global__ void __launch_bounds__(256) decode_merge_d256_kernel(DecodeParams p) {
    __shared__ __attribute__((aligned(16))) float red[4][kD2 + 4];  // rows 16-byte aligned
    const int b = blockIdx.x, hq = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int carry = 0, ps_b = 0, pg_b = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
        int L = 0;
        const int pg = b0 + lane < p.B ? seq_pages(p, b0 + lane, &L) : 0;
        const int incl = wave_incl_scan(pg, lane);
        if (b >= b0 && b < b0 + 64) {  // uniform over the wave
            ps_b = __shfl(carry + incl - pg, b - b0, 64);
            pg_b = __shfl(pg, b - b0, 64);
        }
        carry += __shfl(incl, 63, 64);
    }
    const int T = carry;
    uint16_t* orow = reinterpret_cast<uint16_t*>(p.out) + ((int64_t)b * p.Hq + hq) * kD2;
    if (pg_b == 0) {
        if (wave == 0) reinterpret_cast<u32x2*>(orow)[lane] = u32x2{0u, 0u};
        return;
    }
    const int n = effective_wgs(p, T, p.grid);
    const int w0 = wg_of_page(ps_b, n, T), w1 = wg_of_page(ps_b + pg_b - 1, n, T);
    if (w0 == w1) return;  // written by its range
    const int nseg = w1 - w0 + 1;
    const int64_t rs = (int64_t)p.Hq * kPartRow2;
    auto row = [&](int s) {  // piece s = range w0 + s
        const int slot = s == 0 ? 2 * w0 + 1 : 2 * (w0 + s);
        return p.part + slot * rs + (int64_t)hq * kPartRow2;
    };
    float M = kNegInf, L = 0.0f;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = wave; s0 < nseg; s0 += 64) {
        // (rows are 8-byte aligned: float2 loads)
        float2 o[16][2], ml[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const float* r = row(min(s0 + 4 * u, nseg - 1));
            ml[u] = *reinterpret_cast<const float2*>(r + kD2);
            o[u][0] = *reinterpret_cast<const float2*>(r + 4 * lane);
            o[u][1] = *reinterpret_cast<const float2*>(r + 4 * lane + 2);
        }
        float mx = M;
#pragma unroll
        for (int u = 0; u < 16; ++u) mx = s0 + 4 * u < nseg ? fmaxf(mx, ml[u].x) : mx;
        if (mx > M && M != kNegInf) {  // wave-uniform
            const float f = __builtin_amdgcn_exp2f(M - mx);
            L *= f;
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] *= f;
        }
        M = mx;
        const float Mu = M == kNegInf ? 0.0f : M;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const float wu = s0 + 4 * u < nseg ? __builtin_amdgcn_exp2f(ml[u].x - Mu) : 0.0f;
            L = __builtin_fmaf(ml[u].y, wu, L);
            acc[0] = __builtin_fmaf(o[u][0].x, wu, acc[0]);
            acc[1] = __builtin_fmaf(o[u][0].y, wu, acc[1]);
            acc[2] = __builtin_fmaf(o[u][1].x, wu, acc[2]);
            acc[3] = __builtin_fmaf(o[u][1].y, wu, acc[3]);
        }
    }
    *reinterpret_cast<f32x4*>(&red[wave][4 * lane]) = f32x4{acc[0], acc[1], acc[2], acc[3]};
    if (lane == 0) {
        red[wave][kD2] = M;
        red[wave][kD2 + 1] = L;
    }
    __syncthreads();
    if (wave != 0) return;
    float Mg = kNegInf;
#pragma unroll
    for (int w = 0; w < 4; ++w) Mg = fmaxf(Mg, red[w][kD2]);
    const float Mgu = Mg == kNegInf ? 0.0f : Mg;
    float Lg = 0.0f;
    f32x4 og = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float f = red[w][kD2] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(red[w][kD2] - Mgu);
        Lg = __builtin_fmaf(red[w][kD2 + 1], f, Lg);
        const f32x4 v = *reinterpret_cast<const f32x4*>(&red[w][4 * lane]);
#pragma unroll
        for (int e = 0; e < 4; ++e) og[e] = __builtin_fmaf(v[e], f, og[e]);
    }
    const float inv = Lg > 0.0f ? 1.0f / Lg : 0.0f;
    uint32_t w2[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint16_t x0 = p.q_bf16 ? f32_to_bf16_bits(og[2 * e] * inv) : f32_to_f16_bits(og[2 * e] * inv);
        const uint16_t x1 = p.q_bf16 ? f32_to_bf16_bits(og[2 * e + 1] * inv) : f32_to_f16_bits(og[2 * e + 1] * inv);
        w2[e] = (uint32_t)x0 | ((uint32_t)x1 << 16);
    }
    reinterpret_cast<u32x2*>(orow)[lane] = u32x2{w2[0], w2[1]};
}

template <int KB, int HK, bool BF>
int launch_d256(DecodeParams& prm, hipStream_t stream) {
    using DG = D2Geo<KB, HK>;
    if (prm.entry_bytes != DG::slot || prm.mse_bytes != DG::mse || prm.key_packed != DG::kp ||
        prm.val_data != DG::vd || prm.page_bytes != DG::page)
        return VMC_EINVAL;
    // ranges: one per sequence (per-sequence mode), else d256_ranges'
    prm.grid = prm.per_seq ? prm.B : d256_ranges(prm.B, prm.Hkv, prm.max_blocks, prm.max_splits, num_cus());
    const int nwg = (prm.grid + DG::ns - 1) / DG::ns;
    hipLaunchKernelGGL((tq_decode_d256_kernel<KB, HK, BF>), dim3(nwg), dim3(512), 0, stream, prm);
    VMC_LAUNCH_CHECK();
    if (!prm.per_seq) {
        hipLaunchKernelGGL(decode_merge_d256_kernel, dim3(prm.B, prm.Hq), dim3(256), 0, stream, prm);
        VMC_LAUNCH_CHECK();
    }
    return VMC_OK;
}

template <int KB, bool BF>
int launch_d256_heads(DecodeParams& prm, hipStream_t s) {
    switch (prm.Hkv) {
        case 1: return launch_d256<KB, 1, BF>(prm, s);
        case 2: return launch_d256<KB, 2, BF>(prm, s);
        case 4: return launch_d256<KB, 4, BF>(prm, s);
        default: return VMC_EINVAL;
    }
}

}  // namespace

int launch_tq_decode_d256(DecodeParams& prm, int bits, bool bf, hipStream_t s) {
    if (prm.G > 8) return VMC_EINVAL;
    if (bits == 4) return bf ? launch_d256_heads<4, true>(prm, s) : launch_d256_heads<4, false>(prm, s);
    if (bits == 3) return bf ? launch_d256_heads<3, true>(prm, s) : launch_d256_heads<3, false>(prm, s);
    return VMC_EINVAL;
}

}  // namespace vmc
