// paged_decode.hip -- split-KV paged decode attention for gfx950.
//
// Replaces vm_c::paged_attention_v1/_v2 (src/cuda/attention_kernels.cu:438-473)
// and vm_c::turboquant_decode_attention (src/cuda/turboquant_kernels.cu:
// 939-1007).  Semantics: softmax(q k^T * scale) v per query head over the
// sequence's tokens, read through the block table, GQA kv head = q head /
// (Hq / Hkv) (ggml flash_attn_ext broadcast, ggml-cpu/ops.cpp:8260-8265).
//
// Work decomposition ("flat").  The batch's pages are numbered sequence after
// sequence (pages_b = ceil(L_b / bs)); workgroup w of n takes the equal share
// [w T / n, (w+1) T / n) of the T pages, whatever sequences it crosses, so
// every workgroup does the same work and the grid is one resident wave of
// workgroups.  Each workgroup recomputes the layout from seq_lens (no host
// round trip).  A sequence that lies inside one workgroup's range is written
// directly; a sequence cut by a range boundary leaves an fp32 partial (o, m, l)
// per piece -- at most two per workgroup, slot 2w for the piece that continues
// from the previous range and 2w+1 for the piece that continues into the next
// -- and a small second kernel merges them.  max_num_kv_splits == 1 instead
// gives each sequence its own workgroup (no partials, no workspace).
//
// The workgroup has one wave per KV head; a page of the reference layout holds
// all heads of 16 tokens contiguously, so the workgroup reads whole pages with
// 16-byte loads (quantized formats stage the page in LDS; f16/bf16 pages are
// read straight into MFMA operand registers).
//
// Per wave and page (16 tokens x G query heads of one KV head):
//   S^T[16 tok x 16 heads] = K[16 x 128] . Q^T  : 4 x mfma 16x16x32 (f16/bf16)
//   online softmax in the log2 domain, fp32 running max / sum per head
//   O[16 heads x 128] += P[16 x 16 tok] . V      : 8 x mfma 16x16x16
// S^T comes out of the MFMA in exactly the A-operand layout the PV MFMA needs
// (lane l: head l%16, tokens 4*(l/16)+i), so P never leaves registers.  The PV
// output columns are permuted (chunk c, column n -> dim 8n + c) so each lane's
// V operand is one contiguous 8-dim run of a token.
//
// TurboQuant: K = C[code] * norm / ||C[codes]||, so S = scale*norm/||C|| *
// (C[codes] . q_rot): the MFMA runs on fp16 centroids and the per-token factor
// is applied to the S row.  V = code*scale + zero, so P.V = (P*scale).codes +
// sum(P*zero): the MFMA runs on the exact small-integer codes.
// q_rot = H q is a Walsh-Hadamard transform done in registers (the order the
// oracle and the store kernel share).
#include "decode_plan.hpp"
#include "generic_attn.hpp"
#include "kv_quant.hpp"
#include "prefill_api.hpp"

#include <mutex>
#include <utility>

namespace vmc {
namespace {

// Compile-time geometry of a page format (head_dim 128, block 16, at most 8
// KV heads): TurboQuant slot fields (kernels_turboquant.h:29-45), GGUF entry
// sizes, and the staging of LDS-staged formats -- SPP 16-byte chunks per
// thread per page (one wave per KV head) and PF pages in flight.  GGUF pages
// go through registers into one LDS buffer per ring slot (K page, then V page
// at kHalf); TurboQuant pages go straight from HBM into LDS (load-to-LDS DMA)
// with PF + 2 buffers, each one head group's share of a page: two pages are
// read while PF more land.
template <int FMT, int KB, int VB>
struct Geo {
    static constexpr int mse = 16 * KB, key_packed = mse + 2, val_data = 16 * VB;
    // K and V in one slot per (token, head), one pool
    static constexpr bool combined = FMT == FMT_TQ || FMT == FMT_G4 || FMT == FMT_G3 || FMT == FMT_K8;
    static constexpr int entry = FMT == FMT_TQ ? (key_packed + val_data + 4 + 1) / 2 * 2
                                 : FMT == FMT_K8 ? 196
                                 : FMT == FMT_G4 ? 160 : FMT == FMT_G3 ? 112
                                 : FMT == FMT_Q8_0 ? 136 : FMT == FMT_Q4_0 ? 72 : 256;
    static constexpr int per_thread = combined ? entry : 2 * entry;  // staged bytes per token-head
    static constexpr bool staged = FMT >= FMT_Q8_0;
    static constexpr int spp = staged ? (per_thread + 63) / 64 : 1;
    static constexpr bool dma = FMT == FMT_TQ;
    static constexpr int kHalf = kBs * 8 * entry;  // one cache's page, 8 heads
    // staged NHD pages sit in LDS with a 16-byte pad after each token row, so
    // the 16 rows a lane group reads fall on distinct LDS banks (a row of
    // 8 x 160 B is a multiple of the 256-byte bank cycle: all 16 would hit one)
    static constexpr int kPad = 16;
    static constexpr int kHalfP = kHalf + kBs * kPad;
    // TurboQuant: a head group (<= 4 heads) of 16 tokens, each token's run
    // fetched as a window of whole 16-byte chunks (at most nc_max of them)
    static constexpr int nc_of(int h) { return (h * entry + 30) / 16; }
    static constexpr int spt_of(int h) { return (kBs * nc_of(h) + 64 * h - 1) / (64 * h); }
    static constexpr int nc_max = nc_of(4);
    // chunks per lane per page for any group size (1..4 heads, one wave each)
    static constexpr int spt = std::max(std::max(spt_of(1), spt_of(2)), std::max(spt_of(3), spt_of(4)));
    static constexpr int kBuf = dma ? kBs * nc_max * 16 : combined ? kHalfP : 2 * kHalfP;  // one LDS buffer
    // pages whose block-table entries are staged in LDS at once, and waves per
    // workgroup (TurboQuant: one head group of at most 4 KV heads)
    static constexpr int chunk = 256;
    static constexpr int waves = dma ? 4 : 8;
    // TurboQuant: two pages in flight behind the pair being read (four
    // measured no faster: the kernel is bound by its K/V decode, not by the
    // bytes in flight)
    static constexpr int pf = !staged ? 1 : dma ? 2 : (spp <= 2 ? 4 : (spp <= 3 ? 3 : 2));
    static constexpr int nbuf = dma ? pf + 2 : pf;
};

// per-32-group variant: the codes of values 8j .. 8j+7 of the 32-value
// block at blk (LDS, even address), value v of the 8 at bits 4v (4-bit:
// byte i of the 16 holds values i and i + 16) or 3v (3-bit: 8 codes per 3
// bytes, little endian)
template <int FMT>
__device__ __forceinline__ uint32_t g32_codes8(const uint8_t* blk, int j) {
    if constexpr (FMT == FMT_G4) {
        const uint8_t* cb = blk + 4 + 8 * (j & 1);
        const uint32_t w0 = lds16(cb) | (lds16(cb + 2) << 16);
        const uint32_t w1 = lds16(cb + 4) | (lds16(cb + 6) << 16);
        const int sh = j < 2 ? 0 : 4;
        uint32_t cw = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            cw |= ((w0 >> (8 * e + sh)) & 0xfu) << (4 * e);
            cw |= ((w1 >> (8 * e + sh)) & 0xfu) << (4 * e + 16);
        }
        return cw;
    } else {
        const int o = 2 + 3 * j;  // the block start is even: o's parity is j's
        const uint8_t* cb = blk + (o & ~1);
        const uint32_t w = lds16(cb) | (lds16(cb + 2) << 16);
        return (w >> (8 * (o & 1))) & 0xffffffu;
    }
}
// two exact fp16 values times d, one rounding each (v_pk_mul_f16)
__device__ __forceinline__ uint32_t g32_times(uint32_t c2, f16x2 d2) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, c2) * d2);
}
template <int FMT>
__device__ __forceinline__ float g32_code(uint32_t cw, int v) {
    return FMT == FMT_G4 ? (float)((cw >> (4 * v)) & 0xfu) : (float)((cw >> (3 * v)) & 7u);
}

template <int FMT>
__device__ __forceinline__ int entry_off(int tok, int g, int Hkv, int E, int hnd) {
    return hnd ? (g * kBs + tok) * E : (tok * Hkv + g) * E;
}

// ------------------------------------------------------------------ kernel

// Every LDS byte of the decode kernel in one object, the page ring first, so
// a ring slot's reads carry compile-time offsets (below 64 KiB they fold into
// the LDS instruction) and need no address arithmetic.
template <int FMT, int KB, int VB, bool PAIRS>
struct alignas(16) DecodeLds {
    using GE = Geo<FMT, KB, VB>;
    // staged page pairs (PAIRS): two pairs of buffers, the one being read
    // and the one being filled
    uint8_t ring[GE::staged ? (PAIRS ? 4 : GE::nbuf) * GE::kBuf : 16];
    // 3-bit codes, 12 bits -> four packed fp16 values: TurboQuant key
    // centroids, or the per-32-group variant's exact code - 4
    u32x2 lut4[(FMT == FMT_TQ && KB == 3) || FMT == FMT_G3 ? 4096 : 1];
    uint32_t lut[FMT == FMT_TQ ? 256 : 1];              // key code pair -> two fp16 centroids
    float wscr[GE::waves][80];                          // per-wave exchange
    int32_t bt[GE::chunk];                              // block of each page of the chunk
    int32_t info[GE::chunk];                            // b << 6 | valid tokens << 1 | piece ends
    int32_t seg_b[GE::chunk], seg_ps[GE::chunk], seg_L[GE::chunk];
    WGPlan plan;
    int n_seg;
};

// HALF (the per-32-group formats with at most 8 query heads per KV head;
// TurboQuant slots with G <= 8 run tq_decode.hip's kernel instead): the 16
// columns of the S tile hold the heads for the step's first page (columns
// 0-7) and for its second page (columns 8-15): K of both pages runs against a
// block-diagonal Q^T, so every lane's scores are real and one softmax covers
// two pages.  The PV product keeps the page of each row apart (rows 0-7 first
// page, 8-15 second) and the halves are added when the piece ends.  Two pages
// are staged and processed per workgroup barrier.
template <int FMT, int KB, int VB, bool MBF16, bool HALF>
__global__ void __launch_bounds__(512)
paged_decode_kernel(DecodeParams p) {
    // TurboQuant: MBF16 says that q, out and the stored norms, scales and
    // zeros are bf16 (the reference's USE_BF16 instantiation,
    // turboquant_kernels.cu:353, :445-461); its MFMA operands stay fp16
    // (centroids and exact codes)
    constexpr bool kTqBf16 = FMT == FMT_TQ && MBF16;
    using AT = typename std::conditional<MBF16 && FMT != FMT_TQ, bf16x8, f16x8>::type;
    using PT = typename std::conditional<MBF16 && FMT != FMT_TQ, s16x4, f16x4>::type;
    static_assert(!HALF || FMT == FMT_G4 || FMT == FMT_G3, "page pairs: the per-32-group formats");
    constexpr bool kPairs = HALF;  // staged: two pages per step
    __shared__ DecodeLds<FMT, KB, VB, kPairs> lds;
    uint8_t* const smem = lds.ring;
    WGPlan& plan = lds.plan;
    int32_t* const bt_lds = lds.bt;
    int32_t* const info_lds = lds.info;
    int32_t* const seg_b = lds.seg_b;
    int32_t* const seg_ps = lds.seg_ps;
    int32_t* const seg_L = lds.seg_L;
    uint32_t* const lut = lds.lut;
    u32x2* const lut4 = lds.lut4;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int r16 = lane & 15, grp = lane >> 4;
    // workgroup = (KV-head group hg, page range or sequence w); the groups of
    // one range are p.grid ids apart, so with p.grid a multiple of 8 they
    // share an XCD (and its L2)
    const int hg = (int)blockIdx.x / p.grid;
    const int w = (int)blockIdx.x - hg * p.grid;
    constexpr bool kStaged = FMT >= FMT_Q8_0;

    // ---- this workgroup's page range
    if (wave == 0) {
        WGPlan wp;
        if (p.per_seq) {
            int ps = 0, pg = 0, L = 0;
            for (int b0 = 0; b0 < p.B; b0 += 64) {  // pages before sequence w
                const int b = b0 + lane;
                int v = b < w ? seq_pages(p, b, &L) : 0;
#pragma unroll
                for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
                ps += v;
            }
            pg = seq_pages(p, w, &L);
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

    const int g = hg * p.hpw + wave;  // kv head of this wave
    float* wscr = lds.wscr[wave];
    const int G = p.G;
    const int hq0 = g * G;
    const bool head_ok = r16 < G;
    const int qh = HALF ? (r16 & 7) : r16;  // query head of S column r16
    const bool q_ok = qh < G;

    if (p_lo >= p_hi) {
        // no pages: per-sequence mode writes the sequence's zero rows
        if (p.per_seq && w < p.B && head_ok) {
            uint16_t* o = reinterpret_cast<uint16_t*>(p.out) + ((int64_t)w * p.Hq + hq0 + r16) * kD + 32 * grp;
#pragma unroll
            for (int c = 0; c < 4; ++c) reinterpret_cast<u32x4*>(o)[c] = u32x4{0u, 0u, 0u, 0u};
        }
        return;
    }

    // key centroid tables (their addresses are compile-time offsets of each
    // read); 3-bit keys: a 12-bit table of four packed fp16 centroids
    if constexpr (FMT == FMT_TQ) {
        build_pair_lut<KB>(lut, p.tab);
        if constexpr (KB == 3) {
            __syncthreads();
            for (int e = tid; e < 4096; e += blockDim.x) lut4[e] = u32x2{lut[e & 63], lut[e >> 6]};
        }
    }
    if constexpr (FMT == FMT_G3) {
        for (int e = tid; e < 4096; e += blockDim.x) {
            uint32_t w[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float lo = (float)((int)((e >> (6 * h)) & 7) - 4), hi = (float)((int)((e >> (6 * h + 3)) & 7) - 4);
                w[h] = (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
            }
            lut4[e] = u32x2{w[0], w[1]};
        }
    }

    // ---- Q operand: lane (r16 = head, grp) holds dims 32*grp + 8*j + e, j = MFMA index
    // HALF: qb[0..3] hold the heads in columns 0-7 (zero in 8-15), qb[4..7]
    // the heads in columns 8-15 (zero in 0-7)
    AT qb[HALF ? 8 : 4];
    auto load_q = [&](int b) __attribute__((always_inline)) {
        const int64_t qrow = ((int64_t)b * p.Hq + hq0 + qh) * kD;
        if constexpr (FMT == FMT_TQ || FMT == FMT_G4 || FMT == FMT_G3) {
            // q in the rotated domain of the keys: H (s q) / sqrt(d), s = +1 for
            // the reference layout
            float y[32];
            if (q_ok) {
                const u32x4* src = reinterpret_cast<const u32x4*>(p.q + qrow + 32 * grp);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const u32x4 wv = src[c];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint16_t lo = (uint16_t)(wv[e] & 0xffff), hi = (uint16_t)(wv[e] >> 16);
                        y[8 * c + 2 * e] = p.q_bf16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
                        y[8 * c + 2 * e + 1] = p.q_bf16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 32; ++e) y[e] = 0.0f;
            }
            if constexpr (FMT != FMT_TQ) {
                const uint32_t sb = p.sgn[grp];  // dims 32*grp .. +31
#pragma unroll
                for (int e = 0; e < 32; ++e) y[e] = ((sb >> e) & 1u) ? -y[e] : y[e];
            }
            // Walsh-Hadamard: half-widths 1..16 inside the lane, 32 and 64 across
            // the lane groups (dim bit 32 = grp bit 0, dim bit 64 = grp bit 1).
#pragma unroll
            for (int h = 1; h < 32; h <<= 1)
#pragma unroll
                for (int i = 0; i < 32; i += 2 * h)
#pragma unroll
                    for (int j = i; j < i + h; ++j) {
                        const float a = y[j], c = y[j + h];
                        y[j] = a + c;
                        y[j + h] = a - c;
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
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                u32x4 wv = {0u, 0u, 0u, 0u};
                if (q_ok) wv = *reinterpret_cast<const u32x4*>(p.q + qrow + 32 * grp + 8 * j);
                const bool qbf = p.q_bf16 != 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint16_t lo = (uint16_t)(wv[e] & 0xffff), hi = (uint16_t)(wv[e] >> 16);
                    if constexpr (MBF16) {
                        const uint16_t l2 = qbf ? lo : f32_to_bf16_bits(f16_bits_to_f32(lo));
                        const uint16_t h2 = qbf ? hi : f32_to_bf16_bits(f16_bits_to_f32(hi));
                        qb[j][2 * e] = __builtin_bit_cast(__bf16, l2);
                        qb[j][2 * e + 1] = __builtin_bit_cast(__bf16, h2);
                    } else {
                        qb[j][2 * e] = qbf ? (_Float16)bf16_bits_to_f32(lo) : __builtin_bit_cast(_Float16, lo);
                        qb[j][2 * e + 1] = qbf ? (_Float16)bf16_bits_to_f32(hi) : __builtin_bit_cast(_Float16, hi);
                    }
                }
            }
        }
        if constexpr (HALF) {
            const uint32_t lo_m = r16 < 8 ? ~0u : 0u;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4 v = __builtin_bit_cast(u32x4, qb[j]);
                qb[4 + j] = __builtin_bit_cast(AT, u32x4{v[0] & ~lo_m, v[1] & ~lo_m, v[2] & ~lo_m, v[3] & ~lo_m});
                qb[j] = __builtin_bit_cast(AT, u32x4{v[0] & lo_m, v[1] & lo_m, v[2] & lo_m, v[3] & lo_m});
            }
        }
    };

    // ---- running state of the current piece
    f32x4 oacc[8];
    float m_run, l_part, z_part;  // m_run per head r16 (log2 domain), l/z partial over this lane's tokens
    auto reset_state = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < 8; ++c) oacc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        m_run = kNegInf;
        l_part = 0.0f;
        z_part = 0.0f;
    };
    reset_state();
    int cur_b = -1;

    const int Hkv = p.Hkv, hnd = p.hnd;
    const int64_t page_bytes = p.page_bytes;
    const int nthreads = blockDim.x;

    // ---- finish a piece of sequence b: write the rows, or the partial slot
    auto finalize = [&](int b) __attribute__((always_inline)) {
        const bool cut_before = b == __builtin_amdgcn_readfirstlane(plan.first_b) &&
                                __builtin_amdgcn_readfirstlane(plan.first_cut);
        const bool cut_after = b == __builtin_amdgcn_readfirstlane(plan.last_b) &&
                               __builtin_amdgcn_readfirstlane(plan.last_cut);
        const bool whole = !cut_before && !cut_after;
        const int slot = cut_before ? 2 * w : 2 * w + 1;
        if constexpr (FMT == FMT_G4 || FMT == FMT_G3) {
            // O back from the rotated domain: s (H O_r) / sqrt(d) (linear, so
            // partial rows may be rotated before the merge).  oacc[c][i] =
            // dim 8*r16 + c: half-widths 1..4 in the lane, 8..64 across r16.
#pragma unroll
            for (int hw = 1; hw < 8; hw <<= 1)
#pragma unroll
                for (int c0 = 0; c0 < 8; c0 += 2 * hw)
#pragma unroll
                    for (int c = c0; c < c0 + hw; ++c)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float a = oacc[c][i], bb = oacc[c + hw][i];
                            oacc[c][i] = a + bb;
                            oacc[c + hw][i] = a - bb;
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
            const uint32_t sb = (p.sgn[r16 >> 2] >> (8 * (r16 & 3))) & 0xffu;  // dims 8*r16 .. +7
#pragma unroll
            for (int c = 0; c < 8; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float v = oacc[c][i] * p.tab.rot_c;
                    oacc[c][i] = ((sb >> c) & 1u) ? -v : v;
                }
        }
        float l_tot = sum_over_groups(l_part);
        float z_tot = (FMT == FMT_TQ) ? sum_over_groups(z_part) : 0.0f;
        if constexpr (HALF) {
            // columns r16 and r16 ^ 8 hold the same head; O rows m and m + 8
            // (lane groups grp and grp + 2) too
            l_tot += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, l_tot), 0x128, 0xf, 0xf, false));
            z_tot += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, z_tot), 0x128, 0xf, 0xf, false));
            // (a lane-permute read per element: a loop of permlane32 swaps is
            // miscompiled by this toolchain, which reuses one swap's result)
#pragma unroll
            for (int c = 0; c < 8; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i) oacc[c][i] += __shfl_xor(oacc[c][i], 32, 64);
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
                    const float v0 = __builtin_fmaf(oacc[2 * e][i], kVScale<FMT, VB>(2 * e), zh) * inv;
                    const float v1 = __builtin_fmaf(oacc[2 * e + 1][i], kVScale<FMT, VB>(2 * e + 1), zh) * inv;
                    const uint16_t b0 = p.q_bf16 ? f32_to_bf16_bits(v0) : f32_to_f16_bits(v0);
                    const uint16_t b1 = p.q_bf16 ? f32_to_bf16_bits(v1) : f32_to_f16_bits(v1);
                    wd[e] = (uint32_t)b0 | ((uint32_t)b1 << 16);
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
                    for (int e = 0; e < 4; ++e) v[e] = __builtin_fmaf(oacc[4 * h2 + e][i], kVScale<FMT, VB>(4 * h2 + e), zh);
                    *reinterpret_cast<f32x4*>(od + 4 * h2) = v;
                }
                if (r16 == 0) *reinterpret_cast<float2*>(o + kD) = make_float2(mh, lh);
            }
        }
        reset_state();
    };

    int npc = 0;  // pages of the current chunk

    // staged formats: PF pages in flight in registers -> LDS double buffer
    using GE = Geo<FMT, KB, VB>;
    constexpr int SPP = GE::spp, PF = GE::pf;
    const int n16_k = (int)(page_bytes / 16);
    const int n16 = GE::combined ? n16_k : 2 * n16_k;
    u32x4 stage[kPairs ? 2 : PF][SPP];  // page pairs: the next pair's two pages
    auto stage_load = [&](auto slot_c, int i) __attribute__((always_inline)) {
        constexpr int S = decltype(slot_c)::value;
        // Branch-free so the compiler can count outstanding loads exactly (a
        // hole reads page 0, whose tokens are then masked; chunks past the
        // page re-read its last chunk and are not stored).
        const int32_t blk = max(bt_lds[i], 0);
        const u32x4* ks = reinterpret_cast<const u32x4*>(p.kc + (int64_t)blk * page_bytes);
        const u32x4* vs = reinterpret_cast<const u32x4*>(p.vc + (int64_t)blk * page_bytes);
#pragma unroll
        for (int c = 0; c < SPP; ++c) {
            const int idx = min(tid + c * nthreads, n16 - 1);
            const u32x4* src = (GE::combined || idx < n16_k) ? ks + idx : vs + (idx - n16_k);
            stage[S][c] = *src;
        }
    };
    // slot S of the register ring goes to LDS buffer S (V half at kHalfP);
    // chunk ci of a padded page lands in row ci / row_chunks
    const bool lds_pad = p.lds_pad != 0;
    const int lds_row = p.lds_row, row_chunks = p.row_chunks;
    const uint32_t rc_inv = (uint32_t)p.rc_inv;
    auto stage_store_to = [&](auto slot_c, auto buf_c) __attribute__((always_inline)) {
        constexpr int S = decltype(slot_c)::value;
        uint8_t* buf = smem + decltype(buf_c)::value * GE::kBuf;
#pragma unroll
        for (int c = 0; c < SPP; ++c) {
            const int idx = tid + c * nthreads;
            const bool kpart = GE::combined || idx < n16_k;
            const int ci = kpart ? idx : idx - n16_k;
            int off = 16 * ci;
            if (lds_pad) {
                const int row = (int)(((uint32_t)ci * rc_inv) >> 20);
                off = row * lds_row + 16 * (ci - row * row_chunks);
            }
            if (!kpart) off += GE::kHalfP;
            if (idx < n16) *reinterpret_cast<u32x4*>(buf + off) = stage[S][c];
        }
    };
    auto stage_store = [&](auto slot_c) __attribute__((always_inline)) { stage_store_to(slot_c, slot_c); };

    // TurboQuant: page i of the chunk straight into LDS buffer buf: 16-byte
    // chunk c*nthreads + tid of the page goes to the same offset of the
    // buffer; lanes past the page issue nothing.  Past the chunk's last page
    // (i >= npc) block 0 is re-read (every workgroup shares it, so it stays
    // in the cache) into a buffer no step reads.
    // TurboQuant (NHD pages: token rows of Hkv slots): the buffer holds this
    // group's run of every token row, [t*row + hg*run, +run), as a window of
    // NC 16-byte chunks starting at the run's 16-byte-aligned start; window
    // chunk j of token t sits at LDS offset 16 * (t*NC + j).  The run starts
    // mis(t) = (t*row + hg*run) % 16 bytes into its window.  Chunks past the
    // page end (the last window's tail) re-read the page's last chunk; they
    // are never read back.
    constexpr int SPT = GE::spt;
    const int tq_nc = p.tq_nc, run_bytes = p.hpw * GE::entry;
    auto run_mis = [&](int t) { return (t * p.row_bytes + hg * run_bytes) & 15; };
    uint32_t dma_off[SPT];  // loop-invariant source offset of this lane's chunks in the page
    bool dma_on[SPT];
#pragma unroll
    for (int c = 0; c < SPT; ++c) {
        const int q = c * nthreads + tid, t = q / max(tq_nc, 1), j = q - t * tq_nc;
        const int a = ((t * p.row_bytes + hg * run_bytes) & ~15) + 16 * j;
        dma_on[c] = FMT == FMT_TQ && t < kBs;
        dma_off[c] = (uint32_t)min(a, (int)page_bytes - 16);
    }
    auto dma_page = [&](int i, int buf) __attribute__((always_inline)) {
        const int32_t blk = i < npc ? max(bt_lds[i], 0) : 0;
        const uint8_t* src = p.kc + (int64_t)__builtin_amdgcn_readfirstlane(blk) * page_bytes;
#pragma unroll
        for (int c = 0; c < SPT; ++c) {
            uint8_t* dst = smem + buf * GE::kBuf + 16 * (c * nthreads + 64 * wave);
            if (dma_on[c])
                __builtin_amdgcn_global_load_lds(
                    (const void __attribute__((address_space(1)))*)(src + dma_off[c]),
                    (void __attribute__((address_space(3)))*)dst, 16, 0, 0);  // cached: windows overlap
        }
    };

    // loop-invariant LDS offsets of this lane's entries inside a page
    // (staged in LDS, or in HBM for f16/bf16):
    // K of token r16, V of tokens 4*grp + i
    // (TurboQuant: this group's window layout, local head = wave)
    auto lds_entry = [&](int t) {
        return FMT == FMT_TQ ? t * tq_nc * 16 + run_mis(t) + wave * GE::entry
                             : lds_pad ? t * lds_row + g * GE::entry : entry_off<FMT>(t, g, Hkv, GE::entry, hnd);
    };
    const int k_off = lds_entry(r16);
    int v_off[4];
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) v_off[i2] = lds_entry(4 * grp + i2);

    // direct formats: per-lane operand registers for one page
    u32x4 kreg[4], vreg[4];
    auto direct_load = [&](int i) __attribute__((always_inline)) {
        const int32_t blk = bt_lds[i];
        const int nv = (info_lds[i] >> 1) & 31;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            kreg[c] = u32x4{0u, 0u, 0u, 0u};
            vreg[c] = u32x4{0u, 0u, 0u, 0u};
        }
        if (blk < 0) return;
        const uint8_t* kp = p.kc + (int64_t)blk * page_bytes;
        const uint8_t* vp = p.vc + (int64_t)blk * page_bytes;
        if (r16 < nv) {
            const u32x4* src = reinterpret_cast<const u32x4*>(kp + k_off + 64 * grp);
#pragma unroll
            for (int c = 0; c < 4; ++c) kreg[c] = src[c];
        }
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
            const int tok = 4 * grp + i2;
            if (tok < nv)
                vreg[i2] = *reinterpret_cast<const u32x4*>(vp + v_off[i2] + 16 * r16);
        }
    };


    // ---- TurboQuant: two pages (32 tokens) per online-softmax step.  Slot pp
    // of a step is ring buffer BUF0 + pp (compile time); a slot without valid
    // tokens (nv 0) contributes nothing.
    // Per-lane loop-invariant LDS offsets inside a page: the even start of
    // the four bytes holding token (4*grp + i)'s V code run (dims 8*r16 ..
    // +7), which begins d = 0 or 1 bytes in (3-bit runs at odd offsets), and
    // the byte-permute selectors that gather code bytes d .. d+2 of two tokens.
    int vc_al[4];
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) vc_al[i2] = (v_off[i2] + GE::key_packed + VB * r16) & ~1;
    const uint32_t vd = (uint32_t)((v_off[0] + GE::key_packed + VB * r16) & 1) * 0x01010101u;
    const uint32_t vsel0 = 0x05040100u + vd, vsel1 = 0x06050201u + vd, vsel2 = 0x07060302u + vd;
    // Gram diagonal: lane (r16, grp) picks element r16 % 4 (two bit masks);
    // the exchange slot of its row factor is r16 on the diagonal (grp ==
    // r16 / 4) and 16 + r16 elsewhere (written, never read), so the write
    // needs no branch.
    const uint32_t odd_mask = (r16 & 1) ? ~0u : 0u, hi_mask = (r16 & 2) ? ~0u : 0u;
    const int diag_slot = ((r16 >> 2) == grp ? 0 : 16) + r16;
    float m_thr = kNegInf;  // m_run + 8: the lazy max moves only past it
    auto process_tq = [&](auto buf0_c, int nv0, int nv1, auto masked_c) __attribute__((always_inline)) {
        constexpr bool kMasked = decltype(masked_c)::value;  // a slot has fewer than 16 valid tokens
        constexpr int BUF0 = decltype(buf0_c)::value;
        if constexpr (FMT == FMT_TQ) {
        const uint8_t* pg[2] = {smem + BUF0 * GE::kBuf, smem + (BUF0 + 1) * GE::kBuf};
        const int nvp[2] = {nv0, nv1};
        AT a[2][4];
        float rowf[2];
        uint16_t vsc[2][4], vzr[2][4];  // fp16 scale and zero of token 4*grp + i
        uint32_t bop[2][8][2];  // PV B operands: dim 8*r16 + c, tokens {0,1} / {2,3}
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            // K: lane group grp owns dims 32*grp .. +31 of token r16; the codes
            // index LUTs of packed fp16 centroids.
            const uint8_t* ke = pg[pp] + k_off;
            u32x4 aw[4];
            if constexpr (KB == 4) {
                const uint8_t* cb = ke + 16 * grp;  // 16 bytes, 2-byte aligned
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t wv = lds16(cb + 4 * j) | (lds16(cb + 4 * j + 2) << 16);
#pragma unroll
                    for (int e = 0; e < 4; ++e) aw[j][e] = lut[(wv >> (8 * e)) & 0xffu];
                }
            } else {
                // 12 bytes = four 8-code groups; each 12-bit half indexes the
                // table of four packed fp16 centroids
                const uint8_t* cb = ke + 12 * grp;
                uint32_t h[6];
#pragma unroll
                for (int q = 0; q < 6; ++q) h[q] = lds16(cb + 2 * q);
                const uint32_t g24[4] = {h[0] | ((h[1] & 0xffu) << 16), (h[1] >> 8) | (h[2] << 8),
                                         h[3] | ((h[4] & 0xffu) << 16), (h[4] >> 8) | (h[5] << 8)};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const u32x2 lo = lut4[g24[j] & 0xfffu], hi = lut4[g24[j] >> 12];
                    aw[j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) a[pp][j] = __builtin_bit_cast(AT, aw[j]);
            // ||C[codes]||^2 of every token: the diagonal of the Gram matrix
            // K K^T (fp16 products exact, sums fp32); token r16's value sits in
            // the lanes with grp == r16 / 4, element r16 % 4.
            f32x4 gram = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) gram = mfma16x16x32(a[pp][j], a[pp][j], gram);
            const float csq = sel_bits(sel_bits(gram[0], gram[1], odd_mask), sel_bits(gram[2], gram[3], odd_mask),
                                       hi_mask);
            const float nrm = half_to_f32<kTqBf16>((uint16_t)lds16(ke + GE::mse));
            rowf[pp] = p.scale_log2 * nrm * (p.norm_corr ? __builtin_amdgcn_rsqf(csq + 1e-16f) : 1.0f);
            // V: the four bytes around token 4*grp + i's code run, its scale
            // and zero
            uint32_t cw[4];
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                const uint8_t* cr = pg[pp] + vc_al[i2];
                cw[i2] = lds16(cr) | (lds16(cr + 2) << 16);
                const uint8_t* ve = pg[pp] + v_off[i2] + GE::key_packed + GE::val_data;
                vsc[pp][i2] = (uint16_t)lds16(ve);
                vzr[pp][i2] = (uint16_t)lds16(ve + 2);
            }
            if constexpr (kMasked) {  // tokens past the end may hold anything
#pragma unroll
                for (int i2 = 0; i2 < 4; ++i2) {
                    const bool ok = 4 * grp + i2 < nvp[pp];
                    vsc[pp][i2] = ok ? vsc[pp][i2] : (uint16_t)0;
                    vzr[pp][i2] = ok ? vzr[pp][i2] : (uint16_t)0;
                }
            }
            // B operands {token a, token b} per dim: byte permutes put both
            // tokens' code bytes in the two halves of a dword, then each
            // chunk's field is masked where it lies (kVShift).
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const uint32_t A = cw[2 * hh], Bw = cw[2 * hh + 1];
                const uint32_t w0 = __builtin_amdgcn_perm(Bw, A, vsel0);  // run bytes 0-1
                const uint32_t w1 = __builtin_amdgcn_perm(Bw, A, vsel1);  // run bytes 1-2
                const uint32_t w2 = __builtin_amdgcn_perm(Bw, A, vsel2);  // run bytes 2-3 (4-bit)
                if constexpr (VB == 4) {
                    const uint32_t w3 = __builtin_amdgcn_perm(Bw, A, 0x0c070c03u);  // run byte 3
                    bop[pp][0][hh] = w0 & 0x000f000fu;
                    bop[pp][1][hh] = w0 & 0x00f000f0u;
                    bop[pp][2][hh] = w1 & 0x000f000fu;
                    bop[pp][3][hh] = w1 & 0x00f000f0u;
                    bop[pp][4][hh] = w2 & 0x000f000fu;
                    bop[pp][5][hh] = w2 & 0x00f000f0u;
                    bop[pp][6][hh] = w3 & 0x000f000fu;
                    bop[pp][7][hh] = w3 & 0x00f000f0u;
                } else {
                    bop[pp][0][hh] = w0 & 0x00070007u;  // code bits 0-2 of the run
                    bop[pp][1][hh] = w0 & 0x00380038u;  // 3-5
                    bop[pp][2][hh] = w0 & 0x01c001c0u;  // 6-8
                    bop[pp][3][hh] = w1 & 0x000e000eu;  // 9-11
                    bop[pp][4][hh] = w1 & 0x00700070u;  // 12-14
                    bop[pp][5][hh] = w1 & 0x03800380u;  // 15-17
                    bop[pp][6][hh] = w2 & 0x001c001cu;  // 18-20 (w2's high bytes unused)
                    bop[pp][7][hh] = w2 & 0x00e000e0u;  // 21-23
                }
            }
        }
        // ---- S^T = K . Q^T per page, times the per-token factor
        f32x4 sacc[2];
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            sacc[pp] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) sacc[pp] = mfma16x16x32(a[pp][j], qb[j], sacc[pp]);
        }
        wscr[diag_slot] = rowf[0];
        wscr[32 + diag_slot] = rowf[1];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const f32x4 rf0 = *reinterpret_cast<const f32x4*>(wscr + 4 * grp);
        const f32x4 rf1 = *reinterpret_cast<const f32x4*>(wscr + 32 + 4 * grp);
        __builtin_amdgcn_wave_barrier();
        float sv[2][4];
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
            sv[0][i2] = sacc[0][i2] * rf0[i2];
            sv[1][i2] = sacc[1][i2] * rf1[i2];
        }
        if constexpr (kMasked) {
#pragma unroll
            for (int pp = 0; pp < 2; ++pp)
#pragma unroll
                for (int i2 = 0; i2 < 4; ++i2) sv[pp][i2] = 4 * grp + i2 < nvp[pp] ? sv[pp][i2] : kNegInf;
        }
        // Lazy reference max: m_run moves only when a head's max exceeds it by
        // more than 8 (log2 units), so p <= 256 and most steps skip the O
        // rescale.  Every term of l, z and O uses the same reference: exact.
        // The cross-group max is taken only when some lane's own max passes
        // the threshold.
        // P enters the PV product as fp16(p * scale), so p <= 256 needs every
        // value scale <= 65504 / 256: a step whose largest scale is above that
        // takes the exact running max instead (p <= 1; in range for any fp16
        // scale)
        float scf[2][4];
#pragma unroll
        for (int pp = 0; pp < 2; ++pp)
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) scf[pp][i2] = half_to_f32<kTqBf16>(vsc[pp][i2]);
        const float smax = vmax(vmax(vmax(scf[0][0], scf[0][1]), vmax(scf[0][2], scf[0][3])),
                                vmax(vmax(scf[1][0], scf[1][1]), vmax(scf[1][2], scf[1][3])));
        const bool exact = __ballot(smax > 255.875f) != 0;  // wave-uniform, rare
        const float thr = exact ? m_run : m_thr;
        const float mloc = vmax(vmax(vmax(sv[0][0], sv[0][1]), vmax(sv[0][2], sv[0][3])),
                                vmax(vmax(sv[1][0], sv[1][1]), vmax(sv[1][2], sv[1][3])));
        if (__ballot(mloc > thr)) {  // wave-uniform
            const float mx = vmax_over_groups(mloc);
            const bool upd = mx > thr;  // the same in every lane of head r16
            const float m_new = upd ? vmax(mx, m_run) : m_run;
            const float alpha = m_new > m_run ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;  // 0 when m_run = -inf
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
        AT pa;  // A operand of the PV MFMA: k = 8*grp + 4*pp + i <-> page pp, token 4*grp + i
#pragma unroll
        for (int pp = 0; pp < 2; ++pp)
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                const float pv = __builtin_amdgcn_exp2f(sv[pp][i2] - m_use);
                const float zr = half_to_f32<kTqBf16>(vzr[pp][i2]);
                psum += pv;
                zsum = __builtin_fmaf(pv, zr, zsum);
                pa[4 * pp + i2] = (_Float16)__builtin_fmaf(pv, scf[pp][i2], 0.0f);
            }
        l_part += psum;
        z_part += zsum;
        // ---- O += P . V over the 32 tokens of both pages
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const AT vb = __builtin_bit_cast(AT, u32x4{bop[0][c][0], bop[0][c][1], bop[1][c][0], bop[1][c][1]});
            oacc[c] = mfma16x16x32(pa, vb, oacc[c]);
        }
        }
    };

    // ---- staged formats: the K operand of token r16 (a) and the V values of
    // tokens 4*grp + i, dims 8*r16 .. +7 (vw) of one page in LDS; nv valid
    // tokens (V rows past them are zero)
    auto dequant = [&](const uint8_t* kpage, const uint8_t* vpage, int nv, AT (&a)[4], uint32_t (&vw)[4][4])
                       __attribute__((always_inline)) {
        // ---- K operand for token r16
        const uint8_t* ke = kpage + k_off;
        if constexpr (FMT == FMT_K8) {
            // fp8 keys: lane group grp owns bytes 32*grp .. +31 (MFMA j
            // takes 8j .. 8j+7); every code is exact in fp16
            const uint8_t* kb = ke + 32 * grp;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t w0 = lds32(kb + 8 * j), w1 = lds32(kb + 8 * j + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a[j][e] = __builtin_bit_cast(_Float16, fp8_f16_bits(w0 >> (8 * e), p.fp8_e4b15));
                    a[j][4 + e] = __builtin_bit_cast(_Float16, fp8_f16_bits(w1 >> (8 * e), p.fp8_e4b15));
                }
            }
            // V of tokens 4*grp + i, dims 8*r16 .. +7: bytes 4*r16 .. +3
            // (even dim in the low nibble), code * scale + zero
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                const uint8_t* vb = vpage + v_off[i2];
                const float sc = f16_bits_to_f32((uint16_t)lds16(vb + 64));
                const float zr = f16_bits_to_f32((uint16_t)lds16(vb + 66));
                const uint32_t cw = lds32(vb + 4 * r16);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float x0 = __builtin_fmaf((float)((cw >> (8 * e)) & 0xfu), sc, zr);
                    const float x1 = __builtin_fmaf((float)((cw >> (8 * e + 4)) & 0xfu), sc, zr);
                    vw[i2][e] = (uint32_t)f32_to_f16_bits(x0) | ((uint32_t)f32_to_f16_bits(x1) << 16);
                }
            }
        } else if constexpr (FMT == FMT_G4 || FMT == FMT_G3) {
            // block grp of the K part (dims 32*grp .. +31): code * d + m (4-bit)
            // or (code - 4) * d (3-bit); MFMA j takes values 8j .. 8j+7
            constexpr int BE = FMT == FMT_G4 ? 20 : 14;
            const uint8_t* kb = ke + BE * grp;
            if constexpr (FMT == FMT_G4) {
                // 20-byte blocks, 4-byte aligned: d | m, then bytes 0-15
                // (value v < 16: low nibble of byte v, else high nibble of
                // byte v - 16); MFMA j: values 8j .. 8j+7
                const uint32_t dm = lds32(kb);
                const uint32_t q[4] = {lds32(kb + 4), lds32(kb + 8), lds32(kb + 12), lds32(kb + 16)};
                const f16x2 d2 = __builtin_bit_cast(f16x2, (dm & 0xffffu) * 0x10001u);
                const f16x2 m2 = __builtin_bit_cast(f16x2, (dm >> 16) * 0x10001u);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    u32x4 kw;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t w = q[2 * (j & 1) + (e >> 1)];
                        const uint32_t sp = __builtin_amdgcn_perm(0u, w, (e & 1) ? 0x0c030c02u : 0x0c010c00u);
                        const uint32_t z = ((sp >> (j >= 2 ? 4 : 0)) & 0x000f000fu) | 0x64006400u;
                        const f16x2 c = __builtin_bit_cast(f16x2, z) - f16x2{(_Float16)1024.0f, (_Float16)1024.0f};
                        kw[e] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, d2, m2));
                    }
                    a[j] = __builtin_bit_cast(AT, kw);
                }
            } else {
                // 14-byte blocks, 2-byte aligned: four dwords from the
                // 4-byte floor (inside the 112-byte entry), realigned so
                // c0..c2 hold the 12 code bytes
                const bool off2 = ((uint32_t)(uintptr_t)kb & 2u) != 0u;
                const uint32_t* aw4 = reinterpret_cast<const uint32_t*>(kb - (off2 ? 2 : 0));
                const uint32_t a0 = aw4[0], a1 = aw4[1], a2 = aw4[2], a3 = aw4[3];
                const uint32_t d16 = off2 ? a0 >> 16 : a0 & 0xffffu;
                const uint32_t c0 = off2 ? a1 : __builtin_amdgcn_alignbyte(a1, a0, 2);
                const uint32_t c1 = off2 ? a2 : __builtin_amdgcn_alignbyte(a2, a1, 2);
                const uint32_t c2 = off2 ? a3 : __builtin_amdgcn_alignbyte(a3, a2, 2);
                const uint32_t g24[4] = {c0 & 0xffffffu, (c0 >> 24) | ((c1 & 0xffffu) << 8),
                                         (c1 >> 16) | ((c2 & 0xffu) << 16), c2 >> 8};
                const f16x2 d2 = __builtin_bit_cast(f16x2, d16 * 0x10001u);
                // four codes per table entry, exact (code - 4) in fp16, then
                // one packed multiply by d: fp16((code - 4) * d)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const u32x2 lo = lut4[g24[j] & 0xfffu], hi = lut4[g24[j] >> 12];
                    const u32x4 kw = {g32_times(lo[0], d2), g32_times(lo[1], d2), g32_times(hi[0], d2),
                                      g32_times(hi[1], d2)};
                    a[j] = __builtin_bit_cast(AT, kw);
                }
            }
            // V of tokens 4*grp + i, dims 8*r16 .. +7: block r16 / 4, values 8 (r16 % 4) ..
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                const uint8_t* vb = vpage + v_off[i2] + BE * (r16 >> 2);
                if constexpr (FMT == FMT_G4) {
                    // 20-byte block, 4-byte aligned: d | m, then the 8 code
                    // bytes of values 8l .. 8l+7 (l = r16 % 4) as two words
                    const int l = r16 & 3;
                    const uint32_t dm = lds32(vb);
                    const uint32_t q0 = lds32(vb + 4 + 8 * (l & 1)), q1 = lds32(vb + 8 + 8 * (l & 1));
                    const f16x2 dv2 = __builtin_bit_cast(f16x2, (dm & 0xffffu) * 0x10001u);
                    const f16x2 mv2 = __builtin_bit_cast(f16x2, (dm >> 16) * 0x10001u);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t w = (e >> 1) ? q1 : q0;
                        const uint32_t sp = __builtin_amdgcn_perm(0u, w, (e & 1) ? 0x0c030c02u : 0x0c010c00u);
                        const uint32_t z = ((sp >> (l >= 2 ? 4 : 0)) & 0x000f000fu) | 0x64006400u;
                        const f16x2 c = __builtin_bit_cast(f16x2, z) - f16x2{(_Float16)1024.0f, (_Float16)1024.0f};
                        vw[i2][e] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, dv2, mv2));
                    }
                } else {
                    const uint32_t dv16 = lds16(vb);
                    const f16x2 dv2 = __builtin_bit_cast(f16x2, dv16 | (dv16 << 16));
                    const uint32_t cw = g32_codes8<FMT>(vb, r16 & 3);
                    const u32x2 lo = lut4[cw & 0xfffu], hi = lut4[cw >> 12];
                    vw[i2][0] = g32_times(lo[0], dv2);
                    vw[i2][1] = g32_times(lo[1], dv2);
                    vw[i2][2] = g32_times(hi[0], dv2);
                    vw[i2][3] = g32_times(hi[1], dv2);
                }
            }
        } else {
            // GGUF blocks: lane group grp owns block grp (dims 32*grp .. +31)
            constexpr int BE = FMT == FMT_Q8_0 ? 34 : 18;
            const uint8_t* kb = ke + BE * grp;
            // the block (2-byte aligned) read as 4-byte words from its
            // 4-byte floor and realigned: c[] = the code bytes (the read
            // ends at most 2 bytes past the block, inside the buffer)
            constexpr int NC = FMT == FMT_Q8_0 ? 8 : 4;  // code dwords
            const bool off2 = ((uint32_t)(uintptr_t)kb & 2u) != 0u;
            const uint32_t* kw4 = reinterpret_cast<const uint32_t*>(kb - (off2 ? 2 : 0));
            uint32_t av[NC + 1], c[NC];
#pragma unroll
            for (int i = 0; i <= NC; ++i) av[i] = kw4[i];
#pragma unroll
            for (int i = 0; i < NC; ++i) c[i] = off2 ? av[i + 1] : __builtin_amdgcn_alignbyte(av[i + 1], av[i], 2);
            const uint32_t d16 = off2 ? av[0] >> 16 : av[0] & 0xffffu;
            const f16x2 d2 = __builtin_bit_cast(f16x2, d16 * 0x10001u);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                u32x4 kw;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (FMT == FMT_Q8_0) {
                        // values 8j + 2e, +1: bytes of dword 2j + e/2
                        const uint32_t w = c[2 * j + (e >> 1)];
                        kw[e] = q8_pair_f16((e & 1) ? w >> 16 : w, d2);
                    } else {
                        // byte i = value i | value i + 16 << 4
                        const uint32_t w = c[2 * (j & 1) + (e >> 1)];
                        kw[e] = q4_pair_f16((e & 1) ? w >> 16 : w, j >= 2 ? 4 : 0, d2);
                    }
                }
                a[j] = __builtin_bit_cast(AT, kw);
            }
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                const uint8_t* vb = vpage + v_off[i2] + BE * (r16 >> 2);
                const uint32_t dv16 = lds16(vb);
                const f16x2 dv2 = __builtin_bit_cast(f16x2, dv16 | (dv16 << 16));
                const int q0 = 8 * (r16 & 3);  // index inside the block
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    uint32_t x;
                    if constexpr (FMT == FMT_Q8_0) {
                        x = q8_pair_f16(lds16(vb + 2 + q0 + 2 * e), dv2);
                    } else {
                        const int jj = q0 + 2 * e;
                        x = q4_pair_f16(lds16(vb + 2 + (jj & 15)), jj < 16 ? 0 : 4, dv2);
                    }
                    vw[i2][e] = x;
                }
            }
        }
        if (nv < kBs) {  // rows past the page's valid tokens may hold anything
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                const bool ok = 4 * grp + i2 < nv;
#pragma unroll
                for (int e = 0; e < 4; ++e) vw[i2][e] = ok ? vw[i2][e] : 0u;
            }
        }
    };

    auto process = [&](int i, auto buf_c) __attribute__((always_inline)) {
        constexpr int BUF = decltype(buf_c)::value;
        const uint8_t* kpage = smem + BUF * GE::kBuf;
        // V entries: the other cache's page, or the slot's V part
        const uint8_t* vpage = kpage + (FMT == FMT_K8 ? 128 : GE::combined ? GE::entry / 2 : GE::kHalfP);
        const int info = __builtin_amdgcn_readfirstlane(info_lds[i]);
        const int b = info >> 6;
        const int nv = (info >> 1) & 31;  // valid tokens in this page
        if (b != cur_b) {  // a new sequence starts on this page
            load_q(b);
            cur_b = b;
        }
        AT a[4];
        // V operand pieces (tokens 4*grp + i, dims 8*r16 .. +7) as fp16/bf16 bits
        uint32_t vw[4][4];  // [token i][dword e] = dims (2e, 2e+1)
        uint32_t bop[8][2];  // PV B operands: dim 8*r16 + c, tokens {0,1} / {2,3}

        if constexpr (kStaged) {
            dequant(kpage, vpage, nv, a, vw);
        } else {
            // f16 / bf16: operands straight from the registers loaded last iteration
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4 wv = kreg[j];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (MBF16) {
                        a[j][2 * e] = __builtin_bit_cast(__bf16, (uint16_t)(wv[e] & 0xffff));
                        a[j][2 * e + 1] = __builtin_bit_cast(__bf16, (uint16_t)(wv[e] >> 16));
                    } else {
                        a[j][2 * e] = __builtin_bit_cast(_Float16, (uint16_t)(wv[e] & 0xffff));
                        a[j][2 * e + 1] = __builtin_bit_cast(_Float16, (uint16_t)(wv[e] >> 16));
                    }
                }
            }
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2)
#pragma unroll
                for (int e = 0; e < 4; ++e) vw[i2][e] = vreg[i2][e];
            if (i + 1 < npc) direct_load(i + 1);
        }

        // ---- S^T = K . Q^T
        f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) sacc = mfma16x16x32(a[j], qb[j], sacc);

        float sv[4];
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) sv[i2] = sacc[i2] * p.scale_log2;
        if (nv < kBs) {
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) sv[i2] = 4 * grp + i2 < nv ? sv[i2] : kNegInf;
        }
        float mx = vmax(vmax(sv[0], sv[1]), vmax(sv[2], sv[3]));
        mx = max_over_groups(mx);
        // Lazy reference max: m_run moves only when a head's max exceeds it by
        // more than 8 (log2 units), so p <= 256 and most pages skip the O
        // rescale.  Every term of l, z and O uses the same reference: exact.
        const bool upd = mx > m_run + 8.0f;
        if (__ballot(upd)) {  // wave-uniform
            const float m_new = upd ? mx : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 when m_run = -inf
            l_part *= alpha;
            const f32x4 al = gather4_from_row0(alpha, wscr + 16, r16, grp);
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2)
#pragma unroll
                for (int c = 0; c < 8; ++c) oacc[c][i2] *= al[i2];
            m_run = m_new;
        }
        const float m_use = m_run == kNegInf ? 0.0f : m_run;
        float pv[4], psum = 0.0f;
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
            pv[i2] = __builtin_amdgcn_exp2f(sv[i2] - m_use);
            psum += pv[i2];
        }
        l_part += psum;

        // ---- O += P . V
        PT pa;
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
            if constexpr (MBF16) pa[i2] = (short)f32_to_bf16_bits(pv[i2]);
            else pa[i2] = (_Float16)pv[i2];
        }
        // {token 0,1} and {token 2,3} halves of dims (2e, 2e+1)
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
            bop[c][0] = __builtin_amdgcn_perm(vw[1][c >> 1], vw[0][c >> 1], sel);
            bop[c][1] = __builtin_amdgcn_perm(vw[3][c >> 1], vw[2][c >> 1], sel);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const PT vb = __builtin_bit_cast(PT, u32x2{bop[c][0], bop[c][1]});
            oacc[c] = mfma16x16x16(pa, vb, oacc[c]);
        }
        if (info & 1) finalize(b);  // last page of this sequence's piece
    };

    // ---- staged formats, HALF: the page pair in buffers BUF0, BUF0 + 1 with
    // nv0 / nv1 valid tokens (0: the page contributes nothing).  One S tile
    // (the first page's heads in columns 0-7, the second's in 8-15), one
    // softmax, O += P . V over the 32 tokens on v_mfma_f32_16x16x32.
    auto process2 = [&](auto buf0_c, int nv0, int nv1) __attribute__((always_inline)) {
        constexpr int BUF0 = decltype(buf0_c)::value;
        AT a[2][4];
        uint32_t vw[2][4][4];
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            const uint8_t* kpage = smem + (BUF0 + pp) * GE::kBuf;
            const uint8_t* vpage = kpage + (FMT == FMT_K8 ? 128 : GE::combined ? GE::entry / 2 : GE::kHalfP);
            dequant(kpage, vpage, pp ? nv1 : nv0, a[pp], vw[pp]);
        }
        f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) sacc = mfma16x16x32(a[0][j], qb[j], sacc);
#pragma unroll
        for (int j = 0; j < 4; ++j) sacc = mfma16x16x32(a[1][j], qb[4 + j], sacc);
        float sv[4];
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) sv[i2] = sacc[i2] * p.scale_log2;
        if (nv0 < kBs || nv1 < kBs) {  // tokens past a page's end may hold anything
            const int nvl = r16 >= 8 ? nv1 : nv0;
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) sv[i2] = 4 * grp + i2 < nvl ? sv[i2] : kNegInf;
        }
        // lazy reference max; a head's max spans columns c and c ^ 8
        const float mloc = vmax(vmax(sv[0], sv[1]), vmax(sv[2], sv[3]));
        if (__ballot(mloc > m_thr)) {  // wave-uniform
            float mx = vmax_over_groups(mloc);
            mx = vmax(mx, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, mx), 0x128, 0xf, 0xf, false)));
            const bool upd = mx > m_thr;  // the same in every lane of the head
            const float m_new = upd ? mx : m_run;
            const float alpha = upd ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;  // 0 when m_run = -inf
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
        uint16_t pw[4];
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
            const float pv = __builtin_amdgcn_exp2f(sv[i2] - m_use);
            psum += pv;
            pw[i2] = MBF16 ? f32_to_bf16_bits(pv) : f32_to_f16_bits(pv);
        }
        l_part += psum;
        // P: rows 0-7 take k = 8*grp + i (first page, token 4*grp + i), rows
        // 8-15 k = 8*grp + 4 + i (second page)
        const uint32_t p01 = (uint32_t)pw[0] | ((uint32_t)pw[1] << 16);
        const uint32_t p23 = (uint32_t)pw[2] | ((uint32_t)pw[3] << 16);
        const uint32_t lo_m = r16 < 8 ? ~0u : 0u;
        const AT pa = __builtin_bit_cast(AT, u32x4{p01 & lo_m, p23 & lo_m, p01 & ~lo_m, p23 & ~lo_m});
        // V: {token 0,1} and {token 2,3} halves of dims (2e, 2e+1), first page
        // then second
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
            const AT vb = __builtin_bit_cast(AT, u32x4{__builtin_amdgcn_perm(vw[0][1][c >> 1], vw[0][0][c >> 1], sel),
                                                       __builtin_amdgcn_perm(vw[0][3][c >> 1], vw[0][2][c >> 1], sel),
                                                       __builtin_amdgcn_perm(vw[1][1][c >> 1], vw[1][0][c >> 1], sel),
                                                       __builtin_amdgcn_perm(vw[1][3][c >> 1], vw[1][2][c >> 1], sel)});
            oacc[c] = mfma16x16x32(pa, vb, oacc[c]);
        }
    };

    // ---- chunks of up to GE::chunk pages: stage the block-table slice and
    // the per-page sequence info in LDS, then stream the pages
    for (int c_lo = p_lo; c_lo < p_hi; c_lo += GE::chunk) {
        const int c_hi = min(p_hi, c_lo + GE::chunk);
        npc = c_hi - c_lo;
        if (wave == 0) {
            const int ns = collect_segments(p, c_lo, c_hi, lane, seg_b, seg_ps, seg_L, &plan,
                                            c_lo == p_lo && !p.per_seq);
            if (lane == 0) lds.n_seg = ns;
        }
        __syncthreads();
        const int ns = lds.n_seg;
        for (int i = tid; i < npc; i += nthreads) {
            const int gp = c_lo + i;
            int lo = 0, hi = ns - 1;  // last segment with seg_ps <= gp
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (seg_ps[mid] <= gp) lo = mid;
                else hi = mid - 1;
            }
            const int b = seg_b[lo], L = seg_L[lo], pp = gp - seg_ps[lo];
            const int pages_b = (L + kBs - 1) / kBs;
            const int32_t blk = p.bt[(int64_t)(p.row_seq ? p.row_seq[b] : b) * p.max_blocks + pp];
            const int nv = blk < 0 ? 0 : min(kBs, L - pp * kBs);
            const int ends = pp == pages_b - 1 || gp == p_hi - 1;
            bt_lds[i] = blk;
            info_lds[i] = (b << 6) | (nv << 1) | ends;
        }
        __syncthreads();

        if constexpr (GE::dma) {
            // Ring of NB = PF + 2 LDS buffers fed by load-to-LDS.  Steps take the
            // aligned page pairs (2k, 2k+1) of the chunk; step k reads buffers
            // 2k % NB and 2k % NB + 1 (compile-time: the loop is unrolled over
            // the NB / 2 ring phases).  Pages 2k .. 2k+PF-1 are in flight when
            // step k starts: each wave waits until only its transfers of the
            // PF - 2 pages after the pair are outstanding (a wave issues nw
            // transfers per page; vmcnt retires loads in issue order and later
            // stores only make the wait stricter), the barrier makes every
            // wave's share visible and shows that every wave is done with the
            // previous step's buffers, which then receive pages 2k+PF and
            // 2k+PF+1.  The barrier is the raw instruction and the asm's memory
            // clobber keeps LDS reads below it.  A pair that a piece boundary
            // splits runs twice, each time with one slot masked.
            constexpr int NB = GE::nbuf, NPH = NB / 2;
            static_assert(NB == PF + 2 && NB % 2 == 0 && PF <= 4 && SPT <= 3, "pair steps over an even ring");
            // transfers this wave issues per page (its first lane decides)
            int nw = 0;
#pragma unroll
            for (int c = 0; c < SPT; ++c) nw += c * nthreads + 64 * wave < kBs * tq_nc;
            nw = __builtin_amdgcn_readfirstlane(nw);
#pragma unroll
            for (int s2 = 0; s2 < PF; ++s2) dma_page(s2, s2);
            for (int i0 = 0; i0 < npc; i0 += NB) {
                static_for<NPH>([&](auto ph) __attribute__((always_inline)) {
                    constexpr int S0 = 2 * decltype(ph)::value;
                    const int i = i0 + S0;
                    if (i < npc) {  // uniform over the workgroup
                        // at most SPP * (PF - 2) <= 6 of this wave's transfers may stay
                        switch (nw * (PF - 2)) {
                        case 0: asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory"); break;
                        case 1: asm volatile("s_waitcnt vmcnt(1)\n\ts_barrier" ::: "memory"); break;
                        case 2: asm volatile("s_waitcnt vmcnt(2)\n\ts_barrier" ::: "memory"); break;
                        case 3: asm volatile("s_waitcnt vmcnt(3)\n\ts_barrier" ::: "memory"); break;
                        case 4: asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory"); break;
                        default: asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory"); break;
                        }
                        dma_page(i + PF, (S0 + PF) % NB);
                        dma_page(i + PF + 1, (S0 + PF + 1) % NB);
                        const int info0 = __builtin_amdgcn_readfirstlane(info_lds[i]);
                        const bool has1 = i + 1 < npc;
                        const int info1 = has1 ? __builtin_amdgcn_readfirstlane(info_lds[i + 1]) : info0;
                        const bool split = (info0 & 1) && has1;  // page i ends its piece, i + 1 starts one
                        int b = info0 >> 6;
                        int nva = (info0 >> 1) & 31, nvb = has1 && !split ? (info1 >> 1) & 31 : 0;
                        int ends = split ? info0 : info1;
                        for (int part = 0;; ++part) {
                            if (b != cur_b) {  // a new sequence starts here
                                load_q(b);
                                cur_b = b;
                            }
                            if (nva == kBs && nvb == kBs)
                                process_tq(std::integral_constant<int, S0>{}, nva, nvb, std::false_type{});
                            else
                                process_tq(std::integral_constant<int, S0>{}, nva, nvb, std::true_type{});
                            if (ends & 1) {  // last page of this sequence's piece
                                finalize(b);
                                m_thr = kNegInf;
                            }
                            if (!split || part == 1) break;
                            b = info1 >> 6;
                            nva = 0;
                            nvb = (info1 >> 1) & 31;
                            ends = info1;
                        }
                    }
                });
            }
            // no transfer may still target LDS when the buffers are reused or the
            // workgroup ends
            asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        } else if constexpr (kPairs) {
            // Page pairs: register slots 0 and 1 hold the next pair while pair
            // j is computed from LDS buffers 2 (j % 2), 2 (j % 2) + 1; the step
            // then stores the registers into the other two buffers (read by
            // step j - 1, which every wave has left: the barrier) and loads pair
            // j + 2.  Loads and LDS stores are unconditional (tail pages clamp
            // to the last page).  A pair that a piece boundary splits runs
            // twice, each time with one page masked.
            using I0 = std::integral_constant<int, 0>;
            using I1 = std::integral_constant<int, 1>;
            stage_load(I0{}, 0);
            stage_load(I1{}, min(1, npc - 1));
            stage_store_to(I0{}, I0{});
            stage_store_to(I1{}, I1{});
            stage_load(I0{}, min(2, npc - 1));
            stage_load(I1{}, min(3, npc - 1));
            __syncthreads();
            for (int i0 = 0; i0 < npc; i0 += 4) {
                static_for<2>([&](auto qc) __attribute__((always_inline)) {
                    constexpr int Q = decltype(qc)::value;
                    const int i = i0 + 2 * Q;
                    if (i < npc) {  // uniform over the workgroup
                        const int info0 = __builtin_amdgcn_readfirstlane(info_lds[i]);
                        const bool has1 = i + 1 < npc;
                        const int info1 = has1 ? __builtin_amdgcn_readfirstlane(info_lds[i + 1]) : info0;
                        const bool split = (info0 & 1) && has1;  // page i ends its piece, i + 1 starts one
                        int b = info0 >> 6;
                        int nva = (info0 >> 1) & 31, nvb = has1 && !split ? (info1 >> 1) & 31 : 0;
                        int ends = split ? info0 : info1;
                        for (int part = 0;; ++part) {
                            if (b != cur_b) {  // a new sequence starts here
                                load_q(b);
                                cur_b = b;
                            }
                            process2(std::integral_constant<int, 2 * Q>{}, nva, nvb);
                            if (ends & 1) {  // last page of this sequence's piece
                                finalize(b);
                                m_thr = kNegInf;
                            }
                            if (!split || part == 1) break;
                            b = info1 >> 6;
                            nva = 0;
                            nvb = (info1 >> 1) & 31;
                            ends = info1;
                        }
                    }
                    stage_store_to(I0{}, std::integral_constant<int, 2 * (1 - Q)>{});
                    stage_store_to(I1{}, std::integral_constant<int, 2 * (1 - Q) + 1>{});
                    stage_load(I0{}, min(i + 4, npc - 1));
                    stage_load(I1{}, min(i + 5, npc - 1));
                    __syncthreads();
                });
            }
        } else if constexpr (kStaged) {
            // Ring of PF register slots: slot S holds page base+S+PF while page
            // base+S is computed from LDS.  Loads and LDS stores are unconditional
            // (tail pages clamp to the last page), so the only branch holds no
            // memory loads and the compiler keeps exact load counters: each LDS
            // store waits only for its own slot, PF-1 pages stay in flight.
            static_for<PF>([&](auto sc) __attribute__((always_inline)) {
                stage_load(sc, min((int)decltype(sc)::value, npc - 1));
            });
            stage_store(std::integral_constant<int, 0>{});
            __syncthreads();
            for (int base = 0; base < npc; base += PF) {
                static_for<PF>([&](auto sc) __attribute__((always_inline)) {
                    constexpr int S = decltype(sc)::value;
                    const int i = base + S;
                    if (i < npc) process(i, sc);  // uniform over the workgroup
                    stage_load(sc, min(i + PF, npc - 1));
                    stage_store(std::integral_constant<int, (S + 1) % PF>{});
                    __syncthreads();
                });
            }
        } else {
            direct_load(0);
            for (int i = 0; i < npc; ++i) process(i, std::integral_constant<int, 0>{});
            __syncthreads();  // the next chunk rewrites the page tables
        }
    }
}

template <int FMT, int KB, int VB, bool MBF16, bool HALF = false>
int launch_decode(DecodeParams& prm, hipStream_t stream) {
    using GE = Geo<FMT, KB, VB>;
    // the compile-time geometry must be the one the caller described
    if (prm.entry_bytes != GE::entry || (FMT == FMT_TQ && (prm.mse_bytes != GE::mse ||
                                                           prm.key_packed != GE::key_packed ||
                                                           prm.val_data != GE::val_data)))
        return VMC_EINVAL;
    auto kern = paged_decode_kernel<FMT, KB, VB, MBF16, HALF>;
    if constexpr (FMT == FMT_TQ) {
        prm.hpw = tq_heads_per_group(prm.Hkv);
        prm.hgroups = prm.Hkv / prm.hpw;
        prm.row_bytes = prm.Hkv * GE::entry;
        prm.tq_nc = GE::nc_of(prm.hpw);
        prm.grid = prm.per_seq ? prm.B : tq_ranges(prm.B, prm.Hkv, prm.max_blocks, prm.max_splits, num_cus());
    } else {
        prm.hpw = prm.Hkv;
        prm.hgroups = 1;
        const int rowb = prm.Hkv * GE::entry;
        prm.lds_pad = GE::staged && !prm.hnd && rowb % 16 == 0;
        prm.row_chunks = rowb / 16;
        prm.lds_row = rowb + GE::kPad;
        prm.rc_inv = prm.row_chunks > 0 ? ((1 << 20) + prm.row_chunks - 1) / prm.row_chunks : 0;
        prm.grid = prm.per_seq ? prm.B : flat_grid(prm.B, prm.Hkv, prm.max_blocks, prm.max_splits, num_cus());
    }
    hipLaunchKernelGGL(kern, dim3(prm.grid * prm.hgroups), dim3(64 * prm.hpw), 0, stream, prm);
    VMC_LAUNCH_CHECK();
    if (!prm.per_seq) {
        hipLaunchKernelGGL(decode_merge_kernel, dim3(prm.B, prm.Hkv), dim3(64 * prm.G), 0, stream, prm);
        VMC_LAUNCH_CHECK();
    }
    return VMC_OK;
}

int setup_common(DecodeParams& prm, void* out, const void* query, const int32_t* bt,
                 const int32_t* seq_lens, int B, int Hq, int Hkv, int D, int bs, int max_blocks,
                 float scale, int max_splits, void* ws, size_t ws_bytes) {
    if (D != kD || bs != kBs) return VMC_EINVAL;
    if (B < 0 || Hq <= 0 || Hkv <= 0 || Hkv > 8 || Hq % Hkv != 0 || Hq / Hkv > 16) return VMC_EINVAL;
    if (max_blocks <= 0) return VMC_EINVAL;
    if (B > (1 << 24)) return VMC_EINVAL;
    if (B > 0 && (!out || !query || !bt || !seq_lens)) return VMC_EINVAL;
    const size_t need = workspace_bytes_for(B, Hq, Hkv, max_blocks, max_splits, num_cus());
    if (need > 0 && (!ws || ws_bytes < need)) return ws ? VMC_ENOMEM : VMC_EINVAL;
    prm.out = out;
    prm.q = reinterpret_cast<const uint16_t*>(query);
    prm.bt = bt;
    prm.seq_lens = seq_lens;
    prm.B = B;
    prm.Hq = Hq;
    prm.Hkv = Hkv;
    prm.G = Hq / Hkv;
    prm.max_blocks = max_blocks;
    prm.scale_log2 = scale * kLog2e;
    prm.part = reinterpret_cast<float*>(ws);
    prm.per_seq = max_splits == 1;
    prm.pps_min = kPpsMin;
    prm.max_splits = max_splits;
    return VMC_OK;
}

}  // namespace
}  // namespace vmc

using namespace vmc;

extern "C" size_t vmc_paged_decode_workspace_size(int batch_size, int num_heads, int num_kv_heads,
                                                  int head_dim, int max_num_blocks_per_req,
                                                  int block_size, int max_num_kv_splits) {
    (void)head_dim;
    (void)block_size;
    if (batch_size < 0 || num_heads <= 0 || num_kv_heads <= 0 || max_num_blocks_per_req <= 0) return 0;
    return workspace_bytes_for(batch_size, num_heads, num_kv_heads, max_num_blocks_per_req,
                               max_num_kv_splits, num_cus());
}

extern "C" size_t vmc_turboquant_decode_workspace_size(int batch_size, int num_heads, int num_kv_heads,
                                                       int head_dim, int64_t max_num_blocks_per_req,
                                                       int64_t block_size, int max_num_kv_splits) {
    const int mb = (int)std::min<int64_t>(max_num_blocks_per_req, 0x7fffffff);
    const size_t n = vmc_paged_decode_workspace_size(batch_size, num_heads, num_kv_heads, head_dim, mb,
                                                     (int)block_size, max_num_kv_splits);
    // head_dim 256 (tq_decode_d256.hip): rows of 256 + 2 floats
    if (head_dim == 256 && batch_size >= 0 && num_heads > 0 && num_kv_heads > 0 && mb > 0)
        return std::max(n, workspace_bytes_d256(batch_size, num_heads, num_kv_heads, mb, max_num_kv_splits,
                                                num_cus()));
    return n;
}

namespace {
int paged_decode_rows(void* out, const void* query, const void* key_cache, const void* value_cache,
                      const int32_t* block_tables, const int32_t* seq_lens, const int32_t* row_seq,
                      const int32_t* row_pos, int batch_size, int num_heads, int num_kv_heads,
                      int head_dim, int block_size, int max_num_blocks_per_req, float scale,
                      int q_dtype, int kv_format, int layout, int max_num_kv_splits, void* workspace,
                      size_t workspace_bytes, vmc_stream_t stream) {
    if (generic_head_dim(head_dim) || beyond_tuned_decode(head_dim, num_heads, num_kv_heads)) {
        // head_dim 64 / 256, and head counts past the tuned kernels' (see
        // beyond_tuned_decode): one wave per (row, query head), no workspace
        if (batch_size < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
            block_size <= 0 || max_num_blocks_per_req <= 0)
            return VMC_EINVAL;
        if (q_dtype != VMC_DTYPE_F16 && q_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
        if (layout != VMC_LAYOUT_NHD && layout != VMC_LAYOUT_HND) return VMC_EINVAL;
        const int64_t E = vmc_kv_entry_bytes(kv_format, head_dim);
        if (E < 0) return VMC_EINVAL;
        if (batch_size == 0) return VMC_OK;
        if (!out || !query || !block_tables || !key_cache || !value_cache || !seq_lens) return VMC_EINVAL;
        GenArgs a = {};
        a.out = out;
        a.q = query;
        a.q_bf16 = q_dtype == VMC_DTYPE_BF16;
        a.src = kv_format == VMC_KV_F16 ? GEN_F16 : kv_format == VMC_KV_BF16 ? GEN_BF16
              : kv_format == VMC_KV_Q8_0 ? GEN_Q8 : GEN_Q4;
        a.kp = reinterpret_cast<const uint8_t*>(key_cache);
        a.vp = reinterpret_cast<const uint8_t*>(value_cache);
        a.entry = E;
        a.hnd = layout == VMC_LAYOUT_HND;
        a.bs = block_size;
        a.bt = block_tables;
        a.max_blocks = max_num_blocks_per_req;
        a.seq_lens = seq_lens;
        a.tok_seq = row_seq;
        a.pos = row_pos;
        a.num_seqs = -1;
        a.rows = batch_size;
        a.Hq = num_heads;
        a.Hkv = num_kv_heads;
        a.D = head_dim;
        a.scale = scale;
        return gen_attention(a, reinterpret_cast<hipStream_t>(stream));
    }
    DecodeParams prm = {};
    int rc = setup_common(prm, out, query, block_tables, seq_lens, batch_size, num_heads,
                          num_kv_heads, head_dim, block_size, max_num_blocks_per_req, scale,
                          max_num_kv_splits, workspace, workspace_bytes);
    if (rc != VMC_OK) return rc;
    prm.row_seq = row_seq;
    prm.row_pos = row_pos;
    if (q_dtype != VMC_DTYPE_F16 && q_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (layout != VMC_LAYOUT_NHD && layout != VMC_LAYOUT_HND) return VMC_EINVAL;
    const int64_t E = vmc_kv_entry_bytes(kv_format, head_dim);
    if (E < 0) return VMC_EINVAL;
    if (batch_size == 0) return VMC_OK;
    if (!key_cache || !value_cache) return VMC_EINVAL;
    prm.kc = reinterpret_cast<const uint8_t*>(key_cache);
    prm.vc = reinterpret_cast<const uint8_t*>(value_cache);
    prm.q_bf16 = q_dtype == VMC_DTYPE_BF16;
    prm.entry_bytes = (int)E;
    prm.page_bytes = (int64_t)kBs * num_kv_heads * E;
    prm.hnd = layout == VMC_LAYOUT_HND;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (kv_format == VMC_KV_Q8_0 || kv_format == VMC_KV_Q4_0) {
        if ((prm.page_bytes % 16) != 0) return VMC_EINVAL;
    }
    switch (kv_format) {
        case VMC_KV_F16: return launch_decode<FMT_F16, 0, 0, false>(prm, s);
        case VMC_KV_BF16: return launch_decode<FMT_BF16, 0, 0, true>(prm, s);
        // (GGUF pages stay one page per step: page pairs measured slower on
        // q8_0, 44.4 vs 38.4 us on batch 16)
        case VMC_KV_Q8_0: return launch_decode<FMT_Q8_0, 0, 0, false>(prm, s);
        case VMC_KV_Q4_0: return launch_decode<FMT_Q4_0, 0, 0, false>(prm, s);
        default: return VMC_EINVAL;
    }
}
}  // namespace

extern "C" int vmc_paged_attention_decode(void* out, const void* query, const void* key_cache,
                                          const void* value_cache, const int32_t* block_tables,
                                          const int32_t* seq_lens, int batch_size, int num_heads,
                                          int num_kv_heads, int head_dim, int block_size,
                                          int max_num_blocks_per_req, float scale, int q_dtype,
                                          int kv_format, int layout, int max_num_kv_splits,
                                          void* workspace, size_t workspace_bytes,
                                          vmc_stream_t stream) {
    return paged_decode_rows(out, query, key_cache, value_cache, block_tables, seq_lens, nullptr,
                             nullptr, batch_size, num_heads, num_kv_heads, head_dim, block_size,
                             max_num_blocks_per_req, scale, q_dtype, kv_format, layout,
                             max_num_kv_splits, workspace, workspace_bytes, stream);
}

extern "C" int vmc_paged_attention_prefill(void* out, const void* query, const void* key_cache,
                                           const void* value_cache, int num_tokens, int num_heads,
                                           int num_kv_heads, int head_dim, float scale,
                                           int block_size, int max_num_blocks_per_req,
                                           const int32_t* block_tables,
                                           const int32_t* token_to_seq,
                                           const int32_t* token_positions, int q_dtype,
                                           int kv_format, int layout, int max_num_kv_splits,
                                           void* workspace, size_t workspace_bytes,
                                           vmc_stream_t stream) {
    if (num_tokens > 0 && (!token_to_seq || !token_positions)) return VMC_EINVAL;
    // token_positions stands in for seq_lens (not read when rows are indirect)
    return paged_decode_rows(out, query, key_cache, value_cache, block_tables, token_positions,
                             token_to_seq, token_positions, num_tokens, num_heads, num_kv_heads,
                             head_dim, block_size, max_num_blocks_per_req, scale, q_dtype,
                             kv_format, layout, max_num_kv_splits, workspace, workspace_bytes,
                             stream);
}

namespace {
// at most 8 query heads per KV head: the pipelined kernel of tq_decode.hip
// (two pages share the S tile's columns); 16: this file's kernel, one page
// per S tile
template <bool BF>
int launch_tq(DecodeParams& prm, int kb, int vb, bool half, hipStream_t s) {
    if (half) {
        const int rc = launch_tq_stream_any(prm, kb, vb, BF, s);
        if (rc != VMC_EINVAL) return rc;
        return launch_tq_decode_any(prm, kb, vb, BF, s);
    }
    if (kb == 4 && vb == 4) return launch_decode<FMT_TQ, 4, 4, BF>(prm, s);
    if (kb == 3 && vb == 3) return launch_decode<FMT_TQ, 3, 3, BF>(prm, s);
    if (kb == 3 && vb == 4) return launch_decode<FMT_TQ, 3, 4, BF>(prm, s);
    return VMC_EINVAL;
}

// TurboQuant decode rows that the one-wave-per-(row, head) kernel takes:
// head_dim 64 / 256, fp8 keys with bf16 halves, head counts past the tuned
// kernels' (no workspace)
bool tq_generic_route(const vmc_tq_config* cfg, int head_dim, int num_heads, int num_kv_heads, int half_dtype) {
    return generic_head_dim(head_dim) || (cfg->key_fp8 && half_dtype == VMC_DTYPE_BF16) ||
           beyond_tuned_decode(head_dim, num_heads, num_kv_heads);
}

// head_dim 256 over reference-layout slots with equal key and value bits (3
// or 4), 1, 2 or 4 KV heads and at most 8 query heads per KV head -- the
// reference's deployment of this size, 262-byte slots with 16 query / 2 KV
// heads (src/distributed/tp_runtime.cpp:257-261) -- with q, out and the pool
// 16-byte aligned: the MFMA decode of tq_decode_d256.hip
bool tq_d256_route(const vmc_tq_config* cfg, int head_dim, int num_heads, int num_kv_heads, int64_t block_size,
                   const void* q, const void* out, const void* pool) {
    return head_dim == 256 && cfg->group_size == 0 && !cfg->key_fp8 &&
           cfg->key_quant_bits == cfg->value_quant_bits &&
           (cfg->key_quant_bits == 3 || cfg->key_quant_bits == 4) && block_size == kBs &&
           (num_kv_heads == 1 || num_kv_heads == 2 || num_kv_heads == 4) && num_heads > 0 &&
           num_heads % num_kv_heads == 0 && num_heads / num_kv_heads <= 8 &&
           (((uintptr_t)q | (uintptr_t)out | (uintptr_t)pool) & 15) == 0;
}

int tq_d256_rows(void* output, const void* query, const void* kv_cache, const int32_t* block_tables,
                 const int32_t* seq_lens, const int32_t* row_seq, const int32_t* row_pos, int batch_size,
                 int num_heads, int num_kv_heads, float scale, int64_t max_num_blocks_per_req,
                 const vmc_tq_config* cfg, int half_dtype, int max_num_kv_splits, void* workspace,
                 size_t workspace_bytes, vmc_stream_t stream) {
    if (batch_size < 0 || max_num_blocks_per_req <= 0 || batch_size > (1 << 24)) return VMC_EINVAL;
    if (batch_size == 0) return VMC_OK;
    if (!output || !query || !kv_cache || !block_tables || !seq_lens) return VMC_EINVAL;
    const int mb = (int)max_num_blocks_per_req;
    const size_t need = workspace_bytes_d256(batch_size, num_heads, num_kv_heads, mb, max_num_kv_splits, num_cus());
    if (need > 0 && (!workspace || workspace_bytes < need)) return workspace ? VMC_ENOMEM : VMC_EINVAL;
    DecodeParams prm = {};
    prm.out = output;
    prm.q = reinterpret_cast<const uint16_t*>(query);
    prm.bt = block_tables;
    prm.seq_lens = seq_lens;
    prm.row_seq = row_seq;
    prm.row_pos = row_pos;
    prm.B = batch_size;
    prm.Hq = num_heads;
    prm.Hkv = num_kv_heads;
    prm.G = num_heads / num_kv_heads;
    prm.max_blocks = mb;
    prm.scale_log2 = scale * kLog2e;
    prm.part = reinterpret_cast<float*>(workspace);
    prm.per_seq = max_num_kv_splits == 1;
    prm.pps_min = kPpsMin;
    prm.max_splits = max_num_kv_splits;
    prm.kc = reinterpret_cast<const uint8_t*>(kv_cache);
    prm.vc = prm.kc;
    prm.q_bf16 = half_dtype == VMC_DTYPE_BF16 ? 1 : 0;
    prm.entry_bytes = cfg->slot_size_aligned;
    prm.page_bytes = (int64_t)kBs * num_kv_heads * cfg->slot_size_aligned;
    prm.mse_bytes = cfg->mse_bytes;
    prm.key_packed = cfg->key_packed_size;
    prm.val_data = cfg->val_data_bytes;
    prm.norm_corr = cfg->norm_correction != 0;
    prm.tab = tq_tables(256, cfg->key_quant_bits);
    return launch_tq_decode_d256(prm, cfg->key_quant_bits, prm.q_bf16 != 0, reinterpret_cast<hipStream_t>(stream));
}

int tq_decode_rows(void* output, const void* query, const void* kv_cache, const int32_t* block_tables,
                   const int32_t* seq_lens, const int32_t* row_seq, const int32_t* row_pos, int batch_size,
                   int num_heads, int num_kv_heads, int head_dim, float scale, int64_t block_size,
                   int64_t max_num_blocks_per_req, const vmc_tq_config* cfg, int half_dtype,
                   int max_num_kv_splits, void* workspace, size_t workspace_bytes, vmc_stream_t stream) {
    if (!tq_config_valid(cfg) || cfg->head_dim != head_dim) return VMC_EINVAL;
    if (half_dtype != VMC_DTYPE_F16 && half_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (max_num_blocks_per_req > 0x7fffffff) return VMC_EINVAL;
    if (tq_d256_route(cfg, head_dim, num_heads, num_kv_heads, block_size, query, output, kv_cache))
        return tq_d256_rows(output, query, kv_cache, block_tables, seq_lens, row_seq, row_pos, batch_size, num_heads,
                            num_kv_heads, scale, max_num_blocks_per_req, cfg, half_dtype, max_num_kv_splits, workspace,
                            workspace_bytes, stream);
    if (tq_generic_route(cfg, head_dim, num_heads, num_kv_heads, half_dtype)) {
        // head_dim 64 / 256, fp8 keys with bf16 halves, and head counts past
        // the tuned kernels': one wave per (row, query head), no workspace;
        // q, out and the stored halves are half_dtype (the per-32-group
        // variant has no such kernel)
        if (cfg->group_size != 0) return VMC_EINVAL;
        if (batch_size < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
            block_size <= 0 || max_num_blocks_per_req <= 0)
            return VMC_EINVAL;
        if (batch_size == 0) return VMC_OK;
        if (!output || !query || !kv_cache || !block_tables || !seq_lens) return VMC_EINVAL;
        GenArgs a = {};
        a.out = output;
        a.q = query;
        a.q_bf16 = half_dtype == VMC_DTYPE_BF16;
        a.src = GEN_TQ;
        a.kp = a.vp = reinterpret_cast<const uint8_t*>(kv_cache);
        a.entry = cfg->slot_size_aligned;
        a.hnd = 0;
        a.bs = block_size;
        a.bt = block_tables;
        a.max_blocks = max_num_blocks_per_req;
        a.seq_lens = seq_lens;
        a.tok_seq = row_seq;
        a.pos = row_pos;
        a.num_seqs = -1;
        a.rows = batch_size;
        a.Hq = num_heads;
        a.Hkv = num_kv_heads;
        a.D = head_dim;
        a.scale = scale;
        a.kb = cfg->key_quant_bits;
        a.vb = cfg->value_quant_bits;
        a.key_fp8 = cfg->key_fp8;
        a.fp8_e4b15 = cfg->fp8_e4b15;
        a.mse_bytes = cfg->mse_bytes;
        a.key_packed = cfg->key_packed_size;
        a.val_data = cfg->val_data_bytes;
        a.norm_correction = cfg->norm_correction;
        return gen_attention(a, reinterpret_cast<hipStream_t>(stream));
    }
    DecodeParams prm = {};
    if (cfg->group_size != 0) {
        // per-32-group variant: fp16 queries; d and m are fp16 whatever the
        // stored half_dtype of the reference layout would be
        if (half_dtype != VMC_DTYPE_F16) return VMC_EINVAL;
        int rc = setup_common(prm, output, query, block_tables, seq_lens, batch_size, num_heads,
                              num_kv_heads, head_dim, (int)block_size, (int)max_num_blocks_per_req,
                              scale, max_num_kv_splits, workspace, workspace_bytes);
        if (rc != VMC_OK) return rc;
        prm.row_seq = row_seq;
        prm.row_pos = row_pos;
        if (batch_size == 0) return VMC_OK;
        if (!kv_cache) return VMC_EINVAL;
        prm.kc = reinterpret_cast<const uint8_t*>(kv_cache);
        prm.vc = prm.kc;
        prm.q_bf16 = 0;
        prm.entry_bytes = cfg->slot_size_aligned;
        prm.page_bytes = (int64_t)kBs * num_kv_heads * cfg->slot_size_aligned;
        prm.hnd = 0;
        prm.tab = tq_tables(head_dim, cfg->key_quant_bits);
        const G32Signs sg = g32_signs(cfg->sign_seed);
        for (int i = 0; i < 4; ++i) prm.sgn[i] = sg.w[i];
        hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        if (prm.G <= 8) {  // the pipelined kernel of tq_decode.hip, else page pairs
            const int rc = launch_g32_decode(prm, cfg->key_quant_bits, s);
            if (rc != VMC_EINVAL) return rc;
        }
        if (prm.G <= 8)
            return cfg->key_quant_bits == 4 ? launch_decode<FMT_G4, 0, 0, false, true>(prm, s)
                                            : launch_decode<FMT_G3, 0, 0, false, true>(prm, s);
        return cfg->key_quant_bits == 4 ? launch_decode<FMT_G4, 0, 0, false>(prm, s)
                                        : launch_decode<FMT_G3, 0, 0, false>(prm, s);
    }
    if (cfg->key_fp8) {
        // turboquant_k8v4: fp8 keys (q not rotated, no norm), 4-bit values;
        // fp16 q, out, scale and zero (bf16 takes the branch above)
        if (half_dtype != VMC_DTYPE_F16) return VMC_EINVAL;
        int rc = setup_common(prm, output, query, block_tables, seq_lens, batch_size, num_heads,
                              num_kv_heads, head_dim, (int)block_size, (int)max_num_blocks_per_req,
                              scale, max_num_kv_splits, workspace, workspace_bytes);
        if (rc != VMC_OK) return rc;
        prm.row_seq = row_seq;
        prm.row_pos = row_pos;
        if (batch_size == 0) return VMC_OK;
        if (!kv_cache) return VMC_EINVAL;
        prm.kc = reinterpret_cast<const uint8_t*>(kv_cache);
        prm.vc = prm.kc;
        prm.q_bf16 = 0;
        prm.entry_bytes = cfg->slot_size_aligned;
        prm.page_bytes = (int64_t)kBs * num_kv_heads * cfg->slot_size_aligned;
        prm.hnd = 0;
        prm.fp8_e4b15 = cfg->fp8_e4b15 ? 1 : 0;
        // (fp8 keys stay one page per step: the pair kernel spills)
        return launch_decode<FMT_K8, 0, 0, false>(prm, reinterpret_cast<hipStream_t>(stream));
    }
    int rc = setup_common(prm, output, query, block_tables, seq_lens, batch_size, num_heads,
                          num_kv_heads, head_dim, (int)block_size, (int)max_num_blocks_per_req,
                          scale, max_num_kv_splits, workspace, workspace_bytes);
    if (rc != VMC_OK) return rc;
    prm.row_seq = row_seq;
    prm.row_pos = row_pos;
    if (batch_size == 0) return VMC_OK;
    if (!kv_cache) return VMC_EINVAL;
    // q, out and the stored norm/scale/zero are half_dtype
    const bool bf = half_dtype == VMC_DTYPE_BF16;
    prm.kc = reinterpret_cast<const uint8_t*>(kv_cache);
    prm.vc = prm.kc;
    prm.q_bf16 = bf ? 1 : 0;
    prm.entry_bytes = cfg->slot_size_aligned;
    prm.page_bytes = (int64_t)kBs * num_kv_heads * cfg->slot_size_aligned;
    prm.hnd = 0;
    prm.mse_bytes = cfg->mse_bytes;
    prm.key_packed = cfg->key_packed_size;
    prm.val_data = cfg->val_data_bytes;
    prm.norm_corr = cfg->norm_correction != 0;
    prm.tab = tq_tables(head_dim, cfg->key_quant_bits);
    if ((prm.page_bytes % 16) != 0) return VMC_EINVAL;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int kb = cfg->key_quant_bits, vb = cfg->value_quant_bits;
    // at most 8 query heads per KV head: two pages share the S tile's columns
    const bool half = prm.G <= 8;
    return bf ? launch_tq<true>(prm, kb, vb, half, s) : launch_tq<false>(prm, kb, vb, half, s);
}
}  // namespace

extern "C" int vmc_turboquant_decode_attention(void* output, const void* query, const void* kv_cache,
                                               const int32_t* block_tables, const int32_t* seq_lens,
                                               int batch_size, int num_heads, int num_kv_heads,
                                               int head_dim, float scale, int64_t block_size,
                                               int64_t max_num_blocks_per_req,
                                               const vmc_tq_config* cfg, int half_dtype,
                                               int max_num_kv_splits, void* workspace,
                                               size_t workspace_bytes, vmc_stream_t stream) {
    return tq_decode_rows(output, query, kv_cache, block_tables, seq_lens, nullptr, nullptr, batch_size,
                          num_heads, num_kv_heads, head_dim, scale, block_size, max_num_blocks_per_req, cfg,
                          half_dtype, max_num_kv_splits, workspace, workspace_bytes, stream);
}

// ---- allocation-free variant of vmc_turboquant_decode_attention ----------
//
// The split partials (fp32 o, m, l rows of sequences cut by a page-range
// boundary) go to a file-scope device array instead of a caller workspace.
// Each device holds its own copy, resolved once per device by
// hipGetSymbolAddress; the array's host-side name is never passed to a kernel.
// Nothing needs clearing between calls: the merge reads only the rows that the
// same call's split pass wrote.  Calls that overlap on one device share the
// array and race.
namespace {
constexpr size_t kNoAllocScratchBytes = size_t{64} << 20;  // 64 MiB per device
__device__ __align__(256) unsigned char noalloc_scratch[kNoAllocScratchBytes];

void* noalloc_scratch_ptr() {
    static std::mutex mu;
    static void* ptrs[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lk(mu);
    if (!ptrs[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch)) != hipSuccess || !p) return nullptr;
        ptrs[dev] = p;
    }
    return ptrs[dev];
}
}  // namespace

extern "C" size_t vmc_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int vmc_turboquant_decode_attention_noalloc(
    void* output, const void* query, const void* kv_cache, const int32_t* block_tables,
    const int32_t* seq_lens, int batch_size, int num_heads, int num_kv_heads, int head_dim, float scale,
    int64_t block_size, int64_t max_num_blocks_per_req, const vmc_tq_config* cfg, int half_dtype,
    int max_num_kv_splits, vmc_stream_t stream) {
    if (num_heads <= 0 || num_kv_heads <= 0 || batch_size < 0) return VMC_EINVAL;
    if (!tq_config_valid(cfg) || cfg->head_dim != head_dim) return VMC_EINVAL;
    // the shapes of the one-wave-per-row kernel need no split partials
    const bool d256 = tq_d256_route(cfg, head_dim, num_heads, num_kv_heads, block_size, query, output, kv_cache);
    const size_t need = !d256 && tq_generic_route(cfg, head_dim, num_heads, num_kv_heads, half_dtype)
                            ? 0
                            : vmc_turboquant_decode_workspace_size(batch_size, num_heads, num_kv_heads, head_dim,
                                                                   max_num_blocks_per_req, block_size,
                                                                   max_num_kv_splits);
    if (need > kNoAllocScratchBytes) return VMC_ENOMEM;
    void* ws = nullptr;
    if (need > 0 && !(ws = noalloc_scratch_ptr())) return VMC_EIO;
    return tq_decode_rows(output, query, kv_cache, block_tables, seq_lens, nullptr, nullptr, batch_size,
                          num_heads, num_kv_heads, head_dim, scale, block_size, max_num_blocks_per_req, cfg,
                          half_dtype, max_num_kv_splits, ws, ws ? kNoAllocScratchBytes : 0, stream);
}

extern "C" int vmc_turboquant_prefill_attention(void* output, const void* query, const void* kv_cache,
                                                const int32_t* block_tables, const int32_t* token_to_seq,
                                                const int32_t* token_positions, int num_tokens,
                                                int num_heads, int num_kv_heads, int head_dim, float scale,
                                                int64_t block_size, int64_t max_num_blocks_per_req,
                                                const vmc_tq_config* cfg, int half_dtype,
                                                int max_num_kv_splits, void* workspace,
                                                size_t workspace_bytes, vmc_stream_t stream) {
    if (num_tokens > 0 && (!token_to_seq || !token_positions)) return VMC_EINVAL;
    // chunks of 16 tokens or more over reference-layout slots: the tiled
    // prefill (each 64-key tile of a sequence read once per block of query
    // rows); fewer tokens and the per-32-group variant: one decode row per
    // token
    if (head_dim == kD && block_size == kBs && num_tokens >= 16 && tq_config_valid(cfg) && cfg->head_dim == kD &&
        cfg->group_size == 0 && ((uintptr_t)kv_cache & 3) == 0)
        return tq_prefill_tiled(output, query, kv_cache, block_tables, token_to_seq, token_positions, num_tokens,
                                num_heads, num_kv_heads, scale, max_num_blocks_per_req, cfg, half_dtype,
                                reinterpret_cast<hipStream_t>(stream));
    // token_positions stands in for seq_lens (not read when rows are indirect)
    return tq_decode_rows(output, query, kv_cache, block_tables, token_positions, token_to_seq,
                          token_positions, num_tokens, num_heads, num_kv_heads, head_dim, scale, block_size,
                          max_num_blocks_per_req, cfg, half_dtype, max_num_kv_splits, workspace,
                          workspace_bytes, stream);
}
