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
//   workgroup = 8 waves = up to 4 query heads of one KV head x 32-row query
//   blocks, so every K/V tile of 64 keys in LDS serves 256 query rows.  Tiles
//   arrive by load-to-LDS transfers in a 3-slot ring (rows of 256 B, 16-byte
//   chunk ch of row r at position ch ^ swz(r)); before a tile is published
//   each wave transposes the V rows it loaded into an fp16 V^T tile.
//   S^T[64 kv x 32 q] = K . Q^T per wave: 16 MFMAs, Q^T held in registers,
//     the two 32-key chains interleaved with K operand reads two steps
//     ahead.  One query row per lane column: the row max / sum of the online
//     softmax are in-lane plus one cross-half shuffle.
//   O[32 q x 128] += P . V per wave: 16 fp16 MFMAs.  P is fed straight from
//     the S^T registers: the contraction index k of an MFMA may be any
//     permutation of the 16 keys as long as A and B agree, so logical k =
//     8h + e maps to kv 16c + 8(e/4) + 4h + e%4, which is what lane half h
//     already holds; V^T stores each 16-key block in that order, so a B
//     operand is one 16-byte read.
//   Per-row rescale factors reach the O rows through a small LDS scratch.
// bf16 V that fp16 would overflow (|v| >= 65536), or rows of V entirely
// below 2^-8 with values fp16 keeps only on its subnormal grid, are caught
// in the V^T pass; the workgroup then reruns in an exact mode: raw bf16 V
// rows as B operands, P in fp32 split into bf16 hi + lo, two bf16 MFMAs per
// product.
// Fused append: head group 0 of each KV head writes the block's K/V rows into
// the paged cache with the same block encoders as vmc_reshape_and_cache
// (bit-identical pages).
#include "generic_attn.hpp"
#include "kv_quant.hpp"
#include "prefill_api.hpp"
#include "vmc_tq.hpp"

namespace vmc {
namespace {

constexpr int kD = 128;
constexpr int NW = 8;      // waves per workgroup (32 query rows each)
constexpr int BN = 64;     // kv rows per tile
constexpr int NSLOT = 3;   // K/V tile slots in LDS
constexpr int kBsP = 16;   // tokens per page (paged sources)
constexpr float kNegInf = -__builtin_inff();
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// K/V sources of the kernel: this step's contiguous rows, or the paged cache
// (f16 / bf16 pages by load-to-LDS transfers; q8_0 / q4_0 and TurboQuant
// pages (key / value bits 3/3, 4/4, 3/4; fp8 keys with 4-bit values)
// dequantized to fp16 through registers)
constexpr int SRC_LOCAL = 0, SRC_PAGED = 1, SRC_Q8 = 2, SRC_Q4 = 3, SRC_TQ33 = 4, SRC_TQ44 = 5, SRC_TQ34 = 6,
              SRC_K8 = 7;

struct PrefillParams {
    uint16_t* out;
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const int32_t* pos;
    // paged sources: pools, block tables [seq][max_blocks], token -> sequence
    const uint8_t* kp;
    const uint8_t* vp;
    const int32_t* bt;
    const int32_t* tok_seq;
    int64_t max_blocks, page_bytes;
    int num_seqs;        // rows of a sequence outside [0, num_seqs) get no keys
    int q_bf16;          // paged: q / out (TurboQuant: and the stored halves) are bf16
    // TurboQuant slots: Lloyd-Max centroids, 1 / sqrt(d), field offsets
    float cent[16];
    float rot_c;
    int mse_bytes, key_packed, val_data;
    int norm_corr;  // keys scaled by 1 / ||C[codes]|| (else by the stored norm alone)
    int fp8_e4b15;  // fp8 keys: e4b15 (1) or e4m3 (0) codes
    int T, Hq, Hkv, G;
    float scale_log2;
    int ntiles;          // query blocks of qb rows
    int hw, rb, qb;      // heads per workgroup, 32-row blocks per head, rows per block
    int hgroups;         // workgroups per KV head and query block (G / hw)
    // fused append
    uint8_t* kc;
    uint8_t* vc;
    const int64_t* slots;
    int64_t bs, E, stride;
    int hnd;
    // local K/V with a workspace: the V^T tiles of every 64-key tile of the
    // step (vt_prep_kernel) and their exact-mode flags, vt_tiles per KV head
    const uint8_t* vt;
    const uint8_t* vt_flag;
    int vt_tiles;
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

// One 16-byte-per-lane load-to-LDS transfer: lane L's 16 bytes from src land
// at LDS address m0 + 16 L.  Issued from asm so the compiler does not track it: it
// would otherwise make every later LDS read wait for all transfers in
// flight (it cannot tell the slots apart); the kernel waits for them itself.
__device__ __forceinline__ void dma16m(const void* src, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}
// The same transfer from a wave-uniform base (SGPRs) plus a 32-bit per-lane
// offset: no per-lane 64-bit address arithmetic.
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(m0) : "memory");
}

// All LDS of the kernel: the per-wave exchange, the fp16 V^T tiles (128
// rows of 64 keys, 16-byte chunk i of row d at position i ^ ((d >> 1) & 7)),
// then the K / raw V tile ring (rows of 256 B, 16-byte chunk ch of row r
// stored at chunk position ch ^ swz(r)).  In that order every V^T read and
// the K reads of slot 0 sit below 64 KB, where their constant part fits the
// 16-bit offset of the LDS instruction (above it, each address costs a
// vector add: 704-710 vs 712-720 us on the 4 x 4096 prefill).  swz(r) rotates the low
// 4 row bits by two: a bijection on 16 consecutive rows (the 32-row K
// operand reads spread over all banks) whose bits 2-3 differ for 4
// consecutive rows (the transpose reads of 4 rows x 16 dims spread too).
struct PrefillLds {
    float scratch[2][NW][32];            // [alpha, l][wave][row]
    alignas(8) uint8_t wide[NSLOT][NW];  // bf16: wave w's V rows of the tile need the exact mode
    float cent[16];                      // TurboQuant key centroids
    alignas(16) uint8_t vtr[NSLOT][kD * BN * 2];  // [slot][dim][kv position] fp16 V^T
    uint8_t tile[NSLOT][2][BN * 256];             // [slot][K, V][row][position]
};

__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

__device__ __forceinline__ int wave_max_int(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m, kWave));
    return v;
}

// Workgroup = 8 waves = hw query heads of one KV head x rb blocks of 32
// query rows (hw * rb = 8): every K/V tile in LDS serves 256 query rows,
// which halves the tile traffic from L2 against 4-wave, one-head
// workgroups.  Grid: query block (largest first) x KV head x head group.
// BF16 is the type of the S MFMA and of V (paged: the page type; q8_0 /
// q4_0 pages dequantize to fp16).
template <bool BF16, int APPEND_FMT, int SRC, bool VT>
__global__ void __launch_bounds__(512, 1)
prefill_kernel(PrefillParams p) {
    using M = MT<BF16>;
    using V8 = typename M::v8;
    constexpr bool kPaged = SRC != SRC_LOCAL;
    __shared__ PrefillLds lds;

    const int tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63;
    const int c32 = lane & 31, h = lane >> 5;
    const int per_blk = p.Hkv * p.hgroups;
    const int qblk = p.ntiles - 1 - (int)(blockIdx.x / per_blk);
    const int gi = (int)blockIdx.x % per_blk;
    const int g = gi / p.hgroups, hgrp = gi % p.hgroups;
    const int hq = g * p.G + hgrp * p.hw + w / p.rb;  // this wave's query head
    const int T = p.T;
    const int q0 = qblk * p.qb;
    const int q_end = min(q0 + p.qb, T);
    // q / out dtype: the MFMA type for local rows, the caller's for pages
    const bool qbf = kPaged ? p.q_bf16 != 0 : BF16;

    // this lane's query row
    const int wr = 32 * (w % p.rb);  // this wave's rows: q0 + wr .. +31
    const int row = q0 + wr + c32;
    const bool row_ok = row < T;
    const int wrow0 = q0 + wr;

    // pass state: the workgroup's kv range [kv_lo, kv_end) in ntile tiles,
    // this lane's key window [lo, hi] (hi < 0: none) and the wave's bounds of
    // both; rows [cur, rend) are the pass's.  Local rows: one pass, kv index =
    // token index, window [row - pos(row), row].  Pages: one pass per
    // sequence among the workgroup's rows, kv index = position, window
    // [0, pos(row)] through that sequence's block table.
    int kv_lo = 0, kv_end = 0, ntile = 0, lo = 0, hi = -1;
    int wlo_min = 0, wlo_max = 0, whi_min = -1, whi_max = -1;
    int cur = q0, rend = q_end;
    // block-table row of the pass's sequence, read through the constant
    // address space so that wave-uniform lookups are scalar loads (a vector
    // load would need a vmcnt wait, which also waits for the tile transfers)
    using cint = const __attribute__((address_space(4))) int32_t;
    cint* bt_row = (cint*)p.bt;
    int last_page = 0;

    // ---- Q^T operand: lane (col = row, half h) holds dims 16s + 8h .. +7.
    // A negative scale flips Q's sign bits (exact) so that c = |scale| log2 e
    // is positive and the largest raw score is the largest scaled one.  Paged
    // q of the other half type is rounded to the MFMA type.
    const float csc = fabsf(p.scale_log2);
    const uint32_t qflip = p.scale_log2 < 0.0f ? 0x80008000u : 0u;
    V8 qb[8];
    {
        const uint16_t* qp = p.q + ((int64_t)row * p.Hq + hq) * kD + 8 * h;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            u32x4 wv = {0u, 0u, 0u, 0u};
            if (row_ok) wv = *reinterpret_cast<const u32x4*>(qp + 16 * s);
            if constexpr (kPaged) {
                if (qbf != BF16) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float f0 = qbf ? __builtin_bit_cast(float, wv[e] << 16) : f16_bits_to_f32(wv[e] & 0xffff);
                        const float f1 = qbf ? __builtin_bit_cast(float, wv[e] & 0xffff0000u) : f16_bits_to_f32(wv[e] >> 16);
                        wv[e] = BF16 ? ((uint32_t)f32_to_bf16_bits(f0) | ((uint32_t)f32_to_bf16_bits(f1) << 16))
                                     : ((uint32_t)f32_to_f16_bits(f0) | ((uint32_t)f32_to_f16_bits(f1) << 16));
                    }
                }
            }
            qb[s] = as_v8<V8>(u32x4{wv[0] ^ qflip, wv[1] ^ qflip, wv[2] ^ qflip, wv[3] ^ qflip});
        }
    }
    if constexpr (SRC >= SRC_TQ33 && SRC != SRC_K8) {
        // TurboQuant keys are stored rotated: q_rot = H q / sqrt(d), in fp32
        // from the raw q.  Dim 16 s + 8 h + e: butterflies over e (half-widths
        // 1, 2, 4) and s (16, 32, 64) in the lane, over h (8) with the lane
        // 32 apart; then fp16.
        const uint16_t* qp = p.q + ((int64_t)row * p.Hq + hq) * kD + 8 * h;
        float y[8][8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            u32x4 wv = {0u, 0u, 0u, 0u};
            if (row_ok) wv = *reinterpret_cast<const u32x4*>(qp + 16 * s);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                y[s][2 * e] = qbf ? __builtin_bit_cast(float, wv[e] << 16) : f16_bits_to_f32(wv[e] & 0xffff);
                y[s][2 * e + 1] = qbf ? __builtin_bit_cast(float, wv[e] & 0xffff0000u) : f16_bits_to_f32(wv[e] >> 16);
            }
        }
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int hw = 1; hw < 8; hw <<= 1)
#pragma unroll
                for (int i = 0; i < 8; i += 2 * hw)
#pragma unroll
                    for (int j = i; j < i + hw; ++j) {
                        const float a = y[s][j], b = y[s][j + hw];
                        y[s][j] = a + b;
                        y[s][j + hw] = a - b;
                    }
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float o = shfl_xor(y[s][e], 32);
                y[s][e] = h ? o - y[s][e] : y[s][e] + o;
            }
#pragma unroll
        for (int hw = 1; hw < 8; hw <<= 1)
#pragma unroll
            for (int i = 0; i < 8; i += 2 * hw)
#pragma unroll
                for (int j = i; j < i + hw; ++j)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float a = y[j][e], b = y[j + hw][e];
                        y[j][e] = a + b;
                        y[j + hw][e] = a - b;
                    }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            uint32_t wd[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                wd[e] = ((uint32_t)f32_to_f16_bits(y[s][2 * e] * p.rot_c) |
                         ((uint32_t)f32_to_f16_bits(y[s][2 * e + 1] * p.rot_c) << 16)) ^ qflip;
            qb[s] = as_v8<V8>(u32x4{wd[0], wd[1], wd[2], wd[3]});
        }
        if (tid < 16) lds.cent[tid] = p.cent[tid];
        __syncthreads();
    }

    f32x16 o[4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[m][i] = 0.0f;
    // m_run: the row's reference max (log2 units); it moves only when a score
    // exceeds it by more than 8, so P <= 256 and most tiles skip the rescale
    float m_run = kNegInf, m_thr = kNegInf, l_part = 0.0f;

    // ---- tile loads: load-to-LDS, 2 rounds of 32 rows per tensor; lane
    // (wave w, lane L) of round i fills row 32 i + 4 w + L / 16 at chunk
    // position L % 16, i.e. source chunk (L % 16) ^ swz(row)
    const int ld_row = 4 * w + (lane >> 4);
    const uint32_t ld_col = 16u * (uint32_t)((lane & 15) ^ swz(ld_row));
    const int64_t row_stride = (int64_t)p.Hkv * kD * 2;  // bytes between kv rows
    const uint8_t* kg = reinterpret_cast<const uint8_t*>(p.k) + (int64_t)g * kD * 2 + ld_col;
    const uint8_t* vg = reinterpret_cast<const uint8_t*>(p.v) + (int64_t)g * kD * 2 + ld_col;
    // pages: the 4 rows a 16-lane group covers lie in one page, so round i's
    // page is wave-uniform (a scalar block-table read); a hole reads page 0
    // and its keys are masked
    const int wu = __builtin_amdgcn_readfirstlane(w);
    auto page_at = [&](int k) __attribute__((always_inline)) {
        const int32_t pg = bt_row[min(k >> 4, last_page)];
        return max(pg, 0);
    };
    // byte offset of kv row k (< kv_end) inside its page
    auto row_in_page = [&](int k) __attribute__((always_inline)) {
        const int r = k & (kBsP - 1);
        return p.hnd ? (int64_t)(g * kBsP + r) * p.E : (int64_t)(r * p.Hkv + g) * p.E;
    };
    // local K/V: this lane's row of a tile starting at key k0 is k0 + ld_row
    // (+ 32 in the second round); the LDS rows of this wave in slot 0 (the
    // other slots and the V half at fixed offsets)
    // the fast path's transfers: uniform bases (this KV head's dims at the
    // tile's rows) plus this lane's row and chunk as a 32-bit offset
    const uint32_t ld_off = (uint32_t)ld_row * (uint32_t)row_stride + ld_col;
    const uint8_t* const kgu = reinterpret_cast<const uint8_t*>(p.k) + (int64_t)g * kD * 2;
    const uint8_t* const vgu = reinterpret_cast<const uint8_t*>(p.v) + (int64_t)g * kD * 2;
    const uint32_t lds_w = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)&lds.tile[0][0][1024 * w]);
    constexpr uint32_t kSlotB = 2 * BN * 256, kPartB = BN * 256;
    // prebuilt V^T tiles: wave w fetches bytes 2048 w .. + 2047 of the tile
    // into the same bytes of the slot's V^T tile
    const uint32_t vt_w = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)&lds.vtr[0][2048 * w]);
    const uint32_t lane16 = 16u * (uint32_t)lane;
    auto load_tile = [&](int t, auto slot_c, auto vt_c) __attribute__((always_inline)) {
        constexpr int SL = decltype(slot_c)::value;
        constexpr bool FROM_VT = decltype(vt_c)::value;
        const int k0 = kv_lo + t * BN;
        if constexpr (FROM_VT) {
            // kv_lo is a multiple of BN here, so the tile is prebuilt tile k0 / BN
            const uint8_t* src = p.vt + (((int64_t)g * p.vt_tiles + (k0 / BN)) << 14) + 2048 * wu;
            dma16s(src, lane16, vt_w + SL * (uint32_t)(kD * BN * 2));
            dma16s(src + 1024, lane16, vt_w + SL * (uint32_t)(kD * BN * 2) + 1024u);
        }
        if constexpr (SRC == SRC_LOCAL) {
            if (k0 + BN <= kv_end) {  // uniform: every row of the tile in range
                const int64_t toff = (int64_t)k0 * row_stride;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int64_t off = toff + (int64_t)(32 * i) * row_stride;
                    dma16s(kgu + off, ld_off, lds_w + SL * kSlotB + 8192u * i);
                    if constexpr (!FROM_VT) dma16s(vgu + off, ld_off, lds_w + SL * kSlotB + kPartB + 8192u * i);
                }
                return;
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            // rows past the range re-read the last row (masked later)
            const int kk = min(k0 + 32 * i + ld_row, kv_end - 1);
            if constexpr (SRC == SRC_LOCAL) {
                const int64_t off = (int64_t)kk * row_stride;
                dma16m(kg + off, lds_w + SL * kSlotB + 8192u * i);
                if constexpr (!FROM_VT) dma16m(vg + off, lds_w + SL * kSlotB + kPartB + 8192u * i);
            } else {
                const int64_t off = (int64_t)page_at(min(k0 + 32 * i + 4 * wu, kv_end - 1)) * p.page_bytes +
                                    row_in_page(kk) + ld_col;
                dma16m(p.kp + off, lds_w + SL * kSlotB + 8192u * i);
                dma16m(p.vp + off, lds_w + SL * kSlotB + kPartB + 8192u * i);
            }
        }
    };
    // q8_0 / q4_0 pages: lane L of wave w holds 32-dim block L & 3 of row
    // 32 (r >> 2) + 4 w + (r & 3), r = (L >> 2) & 7, of K (L < 32) or V --
    // the rows whose V this wave transposes -- as the block's bytes read
    // from their 4-byte floor (a block is 2-byte aligned; the read stays in
    // the entry)
    constexpr bool kTQ = SRC >= SRC_TQ33;
    constexpr bool kK8 = SRC == SRC_K8;  // fp8 keys: one byte per dim, 4-byte aligned
    constexpr int TKB = SRC == SRC_TQ44 ? 4 : kK8 ? 8 : 3, TVB = SRC == SRC_TQ33 ? 3 : 4;
    constexpr int kBE = SRC == SRC_Q8 ? 34 : 18;        // block bytes
    // words read per lane: GGUF block from its 4-byte floor; TurboQuant:
    // the 32 codes (12 / 16 / 32 bytes) from their floor, TKB + 1 words for K
    // lanes and TVB + 1 for V lanes (the reads end inside the slot), then the
    // norm (K) or the scale and zero (V) as 16-bit reads
    constexpr int kNC = kTQ ? (4 * (TKB > TVB ? TKB : TVB)) / 4 + 1 : 0;
    constexpr int kNW = SRC == SRC_Q8 ? 9 : SRC == SRC_Q4 ? 5 : kTQ ? kNC + 1 : 1;
    const int qr = 32 * ((lane >> 4) & 1) + 4 * w + ((lane >> 2) & 3);
    const int qblk_ = lane & 3;
    uint32_t qraw[kPaged && SRC != SRC_PAGED ? kNW : 1];
    uint32_t tq_sh = 0;  // TurboQuant: the code run's offset past its 4-byte floor (0 or 2)
    auto issue_q = [&](int t) __attribute__((always_inline)) {
        if constexpr (kTQ) {
            const int k0 = kv_lo + t * BN;
            const int kk = min(k0 + qr, kv_end - 1);
            const int pg0 = page_at(min(k0 + 4 * wu, kv_end - 1));
            const int pg1 = page_at(min(k0 + 32 + 4 * wu, kv_end - 1));
            const int pg = (lane & 16) ? pg1 : pg0;
            // slot fields: K codes at 0, the norm at mse_bytes, V codes at
            // key_packed, scale and zero at key_packed + val_data; block b's
            // codes at 4 bits b (the field offsets are multiples of 4 but for
            // key_packed, and a slot is 2-byte aligned)
            const uint8_t* slot = p.kp + (int64_t)pg * p.page_bytes + row_in_page(kk);
            const uint8_t* codes = lane < 32 ? slot + 4 * TKB * qblk_ : slot + p.key_packed + 4 * TVB * qblk_;
            const uint8_t* halves = lane < 32 ? slot + p.mse_bytes : slot + p.key_packed + p.val_data;
            tq_sh = (uint32_t)((uintptr_t)codes & 2u);
            const uint32_t* c4 = reinterpret_cast<const uint32_t*>((uintptr_t)codes & ~(uintptr_t)3);
            const uint16_t* h2 = reinterpret_cast<const uint16_t*>(halves);
#pragma unroll
            for (int i = 0; i < kNC; ++i) qraw[i] = (lane < 32 ? i <= TKB : i <= TVB) ? c4[i] : 0u;
            qraw[kNC] = (uint32_t)h2[0] | (lane < 32 ? 0u : (uint32_t)h2[1] << 16);
        } else if constexpr (SRC == SRC_Q8 || SRC == SRC_Q4) {
            const int k0 = kv_lo + t * BN;
            const int kk = min(k0 + qr, kv_end - 1);
            const int pg0 = page_at(min(k0 + 4 * wu, kv_end - 1));
            const int pg1 = page_at(min(k0 + 32 + 4 * wu, kv_end - 1));
            const int pg = (lane & 16) ? pg1 : pg0;
            // entries are whole dwords (136 / 72 bytes), so block b starts
            // 2 (b & 1) bytes past a dword
            const uint8_t* src = (lane < 32 ? p.kp : p.vp) + (int64_t)pg * p.page_bytes + row_in_page(kk) +
                                 kBE * qblk_ - 2 * (qblk_ & 1);
            const uint32_t* w4 = reinterpret_cast<const uint32_t*>(src);
#pragma unroll
            for (int i = 0; i < kNW; ++i) qraw[i] = w4[i];
        }
    };
    // dequantize the held block into the K or V tile of slot SL (fp16 rows
    // in the swizzled layout of the load-to-LDS path).  The 16 lanes of a
    // 16-byte write pass hold 4 rows x 4 blocks; written in order, lane
    // (row e, block b) puts chunk j at position 4 (b ^ e) + (j ^ const): 4
    // distinct positions, a 4-way bank conflict.  TurboQuant rows write chunk
    // (j + e) & 3 at step j instead: 16 distinct positions, all 64 banks.
    auto store_q = [&](auto slot_c) __attribute__((always_inline)) {
        if constexpr (SRC == SRC_Q8 || SRC == SRC_Q4 || kTQ) {
            constexpr int SL = decltype(slot_c)::value;
            if constexpr (kTQ) {
                u32x4 kw[4];
                const bool kpart = lane < 32;
                constexpr int NC = 4 * (TKB > TVB ? TKB : TVB) / 4;  // code dwords
                uint32_t c[NC];
#pragma unroll
                for (int i = 0; i < NC; ++i) c[i] = __builtin_amdgcn_alignbyte(qraw[i + 1], qraw[i], tq_sh);
                const uint32_t hw2 = qraw[kNC];
                auto half_f = [&](uint32_t b) {
                    return qbf ? __builtin_bit_cast(float, b << 16) : f16_bits_to_f32(b & 0xffffu);
                };
                const int bits = kpart ? TKB : TVB;
                uint32_t code[32];
#pragma unroll
                for (int j = 0; j < 32; ++j) {
                    // 3-bit: code j at bits 3j of c[0..2]; 4-bit: at bits 4j
                    uint32_t code3 = 0, code4 = 0;
                    if constexpr (TKB == 3 || TVB == 3) {
                        const int b0 = 3 * j, wi = b0 >> 5, sh = b0 & 31;
                        code3 = (sh <= 29 ? (c[wi] >> sh) : __builtin_amdgcn_alignbit(c[wi + 1], c[wi], sh)) & 7u;
                    }
                    if constexpr (NC >= 4) code4 = (c[j >> 3] >> (4 * (j & 7))) & 15u;
                    code[j] = bits == 3 ? code3 : code4;
                }
                auto kw_from = [&](const float (&v)[32]) __attribute__((always_inline)) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            kw[j][e] = (uint32_t)f32_to_f16_bits(v[8 * j + 2 * e]) |
                                       ((uint32_t)f32_to_f16_bits(v[8 * j + 2 * e + 1]) << 16);
                };
                float v[32];
                if (kpart) {
                    if constexpr (kK8) {
                        // fp8 keys: each of the lane's 32 bytes is exact in fp16
#pragma unroll
                        for (int j = 0; j < 4; ++j)
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int b = 8 * j + 2 * e;  // bytes b and b + 1 share a word
                                const uint32_t wv = c[b >> 2] >> (8 * (b & 3));
                                kw[j][e] = (uint32_t)fp8_f16_bits(wv, p.fp8_e4b15) |
                                           ((uint32_t)fp8_f16_bits(wv >> 8, p.fp8_e4b15) << 16);
                            }
                    } else {
                        // K = C[code] * norm / ||C[codes]|| over the row's 128 dims
                        // (C[code] * norm without the norm correction)
                        // (the four lanes of a quad hold its four blocks)
                        float ss = 0.0f;
#pragma unroll
                        for (int j = 0; j < 32; ++j) {
                            v[j] = lds.cent[code[j]];
                            ss = __builtin_fmaf(v[j], v[j], ss);
                        }
                        ss += __shfl_xor(ss, 1, kWave);
                        ss += __shfl_xor(ss, 2, kWave);
                        const float f = half_f(hw2) * (p.norm_corr ? __builtin_amdgcn_rsqf(ss + 1e-16f) : 1.0f);
#pragma unroll
                        for (int j = 0; j < 32; ++j) v[j] *= f;
                        kw_from(v);
                    }
                } else {
                    // V = code * scale + zero
                    const float vs = half_f(hw2), vz = half_f(hw2 >> 16);
#pragma unroll
                    for (int j = 0; j < 32; ++j) v[j] = __builtin_fmaf((float)code[j], vs, vz);
                    kw_from(v);
                }
                // chunk (j + rot) & 3 at step j, by two selects on the bits
                // of rot (a select by the chunk index compiles to divergent
                // branches)
                uint8_t* dst = lds.tile[SL][lane >> 5] + qr * 256;
                const int rot = qr & 3;
                const bool b0 = (rot & 1) != 0, b1 = (rot & 2) != 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    u32x4 x;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t t0 = b0 ? kw[(j + 1) & 3][e] : kw[j][e];
                        const uint32_t t1 = b0 ? kw[(j + 3) & 3][e] : kw[(j + 2) & 3][e];
                        x[e] = b1 ? t1 : t0;
                    }
                    *reinterpret_cast<u32x4*>(dst + 16 * ((4 * qblk_ + ((j + rot) & 3)) ^ swz(qr))) = x;
                }
            } else {
                // q8_0 / q4_0: each chunk written as soon as it is converted,
                // in order (measured faster here than the conflict-free order,
                // which needs all four chunks held)
                const bool off2 = (qblk_ & 1) != 0;
                constexpr int NC = SRC == SRC_Q8 ? 8 : 4;  // code dwords
                uint32_t c[NC];
#pragma unroll
                for (int i = 0; i < NC; ++i)
                    c[i] = off2 ? qraw[i + 1] : __builtin_amdgcn_alignbyte(qraw[i + 1], qraw[i], 2);
                const uint32_t d16 = off2 ? qraw[0] >> 16 : qraw[0] & 0xffffu;
                const f16x2 d2 = __builtin_bit_cast(f16x2, d16 * 0x10001u);
                uint8_t* dst = lds.tile[SL][lane >> 5] + qr * 256;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    u32x4 kw;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (SRC == SRC_Q8) {
                            const uint32_t wv = c[2 * j + (e >> 1)];  // values 8j + 2e, +1
                            kw[e] = q8_pair_f16((e & 1) ? wv >> 16 : wv, d2);
                        } else {
                            const uint32_t wv = c[2 * (j & 1) + (e >> 1)];  // byte i: value i | value i+16 << 4
                            kw[e] = q4_pair_f16((e & 1) ? wv >> 16 : wv, j >= 2 ? 4 : 0, d2);
                        }
                    }
                    *reinterpret_cast<u32x4*>(dst + 16 * ((4 * qblk_ + j) ^ swz(qr))) = kw;
                }
            }
        }
    };

    // ---- loop-invariant LDS read offsets
    // K (S^T A operand): lane reads row 32 kb + c32, chunk 2 s + h
    int k_rd[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) k_rd[s] = c32 * 256 + 16 * ((2 * s + h) ^ swz(c32));
    // V^T (PV B operand): lane (n = c32, h) reads dim 32 m + n, kv positions
    // 16 c + 8 h .. +7 = 16-byte chunk 2 c + h of the 128-byte row, stored at
    // chunk (2 c + h) ^ ((dim >> 1) & 7); m enters as an immediate offset
    int vt_rd[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) vt_rd[c] = c32 * 128 + 16 * ((2 * c + h) ^ ((c32 >> 1) & 7));
    // transposing LDS reads: lane (e, q) of a 16-lane group addresses row
    // base + e, dims 4q .. 4q+3 of a 16-dim block; lane j receives dim j of
    // the 4 rows
    const int tq_e = (lane >> 2) & 3, tq_q = lane & 3, tq_j = lane & 15;

    auto process = [&](int t, auto slot_c, auto exact_c) __attribute__((always_inline)) {
        constexpr int SL = decltype(slot_c)::value;
        constexpr bool EXACT = decltype(exact_c)::value;
        const int k0 = kv_lo + t * BN;
        // skip: tile entirely after this wave's last key, or before its first window
        const bool active = k0 <= whi_max && k0 + BN - 1 >= wlo_min;
        if (!active) return;
        const uint8_t* kt = lds.tile[SL][0];
        const uint8_t* vtt = lds.vtr[SL];
        // pages: bit q set when page q of the tile is a hole (its keys masked)
        uint32_t holes = 0;
        if constexpr (kPaged) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int pi = (k0 >> 4) + q;
                holes |= (pi <= last_page && bt_row[pi] < 0) ? 1u << q : 0u;
            }
        }
        const bool need_mask = (k0 + BN - 1 > whi_min) || (k0 < wlo_max) || holes != 0;
        // ---- S^T = K Q^T, two 32-row kv blocks
        f32x16 sacc[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) sacc[kb][i] = 0.0f;
        {
            // the two kv blocks' chains interleaved; K operands read two
            // steps ahead of their MFMAs
            u32x4 ka[8][2];
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
                    ka[s][kb] = *reinterpret_cast<const u32x4*>(kt + kb * 32 * 256 + k_rd[s]);
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) sacc[kb] = M::mma(as_v8<V8>(ka[s][kb]), qb[s], sacc[kb]);
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                if (s < 6) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            }
        }
        // ---- online softmax (log2 domain), one query row per lane column;
        // masked scores become -inf (only tiles that cross a window edge)
        if (need_mask) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int kv = k0 + kb * 32 + 8 * (j >> 2) + 4 * h + (j & 3);
                    const bool ok = kv <= hi && kv >= lo && !((holes >> (2 * kb + (j >> 3))) & 1u);
                    sacc[kb][j] = ok ? sacc[kb][j] : kNegInf;
                }
        }
        float mloc = kNegInf;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int j = 0; j < 16; ++j) mloc = fmaxf(mloc, sacc[kb][j]);
        if (__ballot(mloc * csc > m_thr)) {  // wave-uniform; rare after the first tiles
            const float mrow = fmaxf(mloc, shfl_xor(mloc, 32)) * csc;
            const bool upd = mrow > m_thr;  // the same in both halves of the row
            const float m_new = upd ? mrow : m_run;
            const float alpha = upd ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;  // 0 from -inf
            l_part *= alpha;
            m_run = m_new;
            m_thr = m_run + 8.0f;
            // rescale O rows by their query rows' alpha (rows 8b + 4h + i)
            float* sc = lds.scratch[0][w];
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
        }
        const float m_use = m_run == kNegInf ? 0.0f : m_run;
        if constexpr (EXACT) {
            // ---- exact mode (bf16 V that fp16 cannot hold): P = 2^(s c - m)
            // in fp32 splits into bf16 hi + lo (16 significant bits, fp32
            // range), the row sum adds the same parts, and O += P V runs as two
            // bf16 MFMAs on the raw bf16 V rows, read by transposing reads:
            // lane (n = c32, h) gets kv 16c + 4h + 0..3 and 16c + 8 + 4h + 0..3
            // at dim 32m + n, the k order of the fp16 path.  Row
            // 16c + 8sec + 4h + e has swz = 4e + ((2 sec + h) & 3), so chunk
            // 4m + cb sits at 4 (m ^ e) + (cb ^ h ^ 2 sec).  The lane id is
            // opaque here so that none of this is computed ahead, in
            // registers the fast pass needs.
            uint32_t phi[4][4], plo[4][4];
            float psum = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const int kb = c >> 1;
                    const int j0 = 4 * (2 * (c & 1) + (e >> 2)) + (e & 3);
                    uint32_t hb[2], lb[2];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][j0 + u], csc, -m_use));
                        hb[u] = __builtin_bit_cast(uint32_t, pv) & 0xffff0000u;
                        const float r = pv - __builtin_bit_cast(float, hb[u]);  // exact
                        lb[u] = __builtin_bit_cast(uint32_t, r) & 0xffff0000u;
                        psum += __builtin_bit_cast(float, hb[u]) + __builtin_bit_cast(float, lb[u]);
                    }
                    phi[c][e >> 1] = (hb[0] >> 16) | hb[1];
                    plo[c][e >> 1] = (lb[0] >> 16) | lb[1];
                }
            l_part += psum;
            int ln = lane;
            asm volatile("" : "+v"(ln));
            const int le = (ln >> 2) & 3, lq = ln & 3, lh = ln >> 5;
            const int cbh = (2 * ((ln >> 4) & 1) + (lq >> 1)) ^ lh;
            const uint32_t vbase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)
                                       lds.tile[SL][1] +
                                   (uint32_t)((4 * lh + le) * 256 + 8 * (lq & 1));
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const bf16x8 ah = as_v8<bf16x8>(u32x4{phi[c][0], phi[c][1], phi[c][2], phi[c][3]});
                const bf16x8 al = as_v8<bf16x8>(u32x4{plo[c][0], plo[c][1], plo[c][2], plo[c][3]});
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    s16x4 part[2];
#pragma unroll
                    for (int sec = 0; sec < 2; ++sec) {
                        const uint32_t a = vbase + (uint32_t)(4096 * c + 2048 * sec + 64 * (m ^ le) +
                                                              16 * (cbh ^ (2 * sec)));
                        part[sec] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (__attribute__((address_space(3))) s16x4*)(uintptr_t)a);
                    }
                    const u32x2 p0 = __builtin_bit_cast(u32x2, part[0]);
                    const u32x2 p1 = __builtin_bit_cast(u32x2, part[1]);
                    const bf16x8 vb = as_v8<bf16x8>(u32x4{p0[0], p0[1], p1[0], p1[1]});
                    o[m] = MT<true>::mma(ah, vb, o[m]);
                    o[m] = MT<true>::mma(al, vb, o[m]);
                }
            }
        } else {
            // P = 2^(s c - m) in fp16 (11 bits, also for bf16 inputs) as MFMA A
            // operands, chunk c = kv rows 16c .. 16c+15; the row sum adds the
            // rounded values the MFMA uses
            uint32_t pw[4][4];
            float psum = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const int kb = c >> 1;
                    const int j0 = 4 * (2 * (c & 1) + (e >> 2)) + (e & 3);
                    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][j0], csc, -m_use));
                    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][j0 + 1], csc, -m_use));
                    const f16x2 ph = {(_Float16)p0, (_Float16)p1};
                    psum = __builtin_amdgcn_fdot2(ph, f16x2{(_Float16)1.0f, (_Float16)1.0f}, psum, false);
                    pw[c][e >> 1] = __builtin_bit_cast(uint32_t, ph);
                }
            l_part += psum;
            // ---- O += P V (fp16): k = 8h + e <-> kv 16c + 8(e/4) + 4h + e%4 (the
            // S^T registers' order); V arrives transposed, output column n = dim 32m + n
            u32x4 vb[4][4];
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int m = 0; m < 4; ++m)
                    vb[c][m] = *reinterpret_cast<const u32x4*>(vtt + m * 32 * 128 + vt_rd[c]);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const f16x8 pa = as_v8<f16x8>(u32x4{pw[c][0], pw[c][1], pw[c][2], pw[c][3]});
#pragma unroll
                for (int m = 0; m < 4; ++m) o[m] = MT<false>::mma(pa, as_v8<f16x8>(vb[c][m]), o[m]);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (i < 14) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
        }
    };

    // V^T pass: each wave transposes the 8 V rows its own transfers wrote
    // (rows 32 rs + 4 w + 0..3, rs = 0, 1) into the fp16 V^T tile, by
    // transpose reads (16-lane group: 4 rows x 16 dims) and 8-byte writes.
    // Within each 16-key block, kv 8a + 4h + e sits at position 8h + 4a + e,
    // so the PV B operand of lane half h is one contiguous 16-byte chunk.
    // bf16 inputs are converted to fp16 here, which keeps every bit for
    // 2^-17 <= |v| < 65536 and rounds smaller magnitudes to the subnormal
    // grid (absolute error <= 2^-25).  The wave's rows are marked in
    // lds.wide (exact mode for the workgroup) when they hold |v| >= 65536 or
    // a NaN, or when they hold a value below 2^-17 but none of 2^-8 or more;
    // otherwise the rounding error is at most 2^-17 of their largest |v|.
    auto v_transpose = [&](auto slot_c) __attribute__((always_inline)) {
        constexpr int SL = decltype(slot_c)::value;
        const uint8_t* vr = lds.tile[SL][1];
        uint8_t* vtt = lds.vtr[SL];
        u16x2 amax = {0, 0}, amin1 = {0xffff, 0xffff};  // |bits|, |bits| - 1 (0 wraps)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int combo = 4 * i + (lane >> 4);
            const int rs = combo & 1, dblk = combo >> 1;
            const int r = 32 * rs + 4 * w + tq_e;
            const int chunk = 2 * dblk + (tq_q >> 1);
            const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4*)(vr + r * 256 + 16 * (chunk ^ swz(r)) + 8 * (tq_q & 1)));
            u32x2 y = __builtin_bit_cast(u32x2, x);
            if constexpr (BF16) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const u16x2 a = __builtin_bit_cast(u16x2, y[e] & 0x7fff7fffu);
                    amax = __builtin_elementwise_max(amax, a);
                    amin1 = __builtin_elementwise_min(amin1, a - u16x2{1, 1});
                    const f16x2 hh = {(_Float16)__builtin_bit_cast(float, y[e] << 16),
                                      (_Float16)__builtin_bit_cast(float, y[e] & 0xffff0000u)};
                    y[e] = __builtin_bit_cast(uint32_t, hh);
                }
            }
            const int dim = 16 * dblk + tq_j;
            const int ci = 2 * (2 * rs + (w >> 2)) + (w & 1);
            *reinterpret_cast<u32x2*>(vtt + dim * 128 + 16 * (ci ^ ((dim >> 1) & 7)) + 8 * ((w >> 1) & 1)) = y;
        }
        if constexpr (BF16) {
            // bf16 bit patterns: 0x477f = 65280 (largest below 2^16),
            // 0x3700 = 2^-17, 0x3b80 = 2^-8
            const uint32_t mx = max((uint32_t)amax[0], (uint32_t)amax[1]);
            const uint32_t mn1 = min((uint32_t)amin1[0], (uint32_t)amin1[1]);
            const bool ovf = __ballot(mx > 0x477fu) != 0;
            const bool small = __ballot(mn1 < 0x36ffu) != 0;
            const bool big = __ballot(mx >= 0x3b80u) != 0;
            if (lane == 0) lds.wide[SL][w] = ovf || (small && !big);
        }
    };

    // ---- NSLOT LDS slots: tile t in slot t % NSLOT; the next NSLOT - 1 tiles
    // are in flight while t runs.  Before tile t each wave waits until only
    // the transfers of tiles t+1 .. t+NSLOT-2 are outstanding (4 per tile:
    // vmcnt retires loads in order), converts its own V chunks, and the
    // barrier makes the tile visible and shows slot (t-1) % NSLOT free, which
    // then receives tile t + NSLOT - 1.
    // bf16: when a tile's V is not fp16-exact (a flag every wave reads after
    // the tile's barrier) the pass returns true and the workgroup starts over
    // in the exact mode, which skips the V^T pass and multiplies the raw bf16
    // rows.  The pass runs to its end rather than leaving early: an early
    // exit costs the common case registers.
    // q8_0 / q4_0 pages instead hold the next tile in registers while a
    // tile runs and dequantize it into its slot before that tile's barrier.
    // With prebuilt V^T tiles (FROM_VT) the transfers bring the V^T tile
    // instead of the raw V rows and there is no V^T pass; the exact mode was
    // decided before the pass from the tiles' flags.
    static_assert(NSLOT == 3, "wait counts below assume three slots");
    constexpr bool kDma = SRC == SRC_LOCAL || SRC == SRC_PAGED;
    auto run = [&](auto exact_c, auto vt_c) __attribute__((always_inline)) {
        constexpr bool EXACT = decltype(exact_c)::value;
        constexpr bool FROM_VT = decltype(vt_c)::value;
        bool redo = false;
        if constexpr (kDma) {
            load_tile(0, std::integral_constant<int, 0>{}, vt_c);
            if (1 < ntile) load_tile(1, std::integral_constant<int, 1>{}, vt_c);
        } else {
            issue_q(0);
        }
        for (int t0 = 0; t0 < ntile; t0 += NSLOT) {
            static_for<NSLOT>([&](auto sc) __attribute__((always_inline)) {
                constexpr int S = decltype(sc)::value;
                const int t = t0 + S;
                if (t < ntile) {  // uniform over the workgroup
                    if constexpr (kDma) {
                        if (t + 1 < ntile) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
                        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    } else {
                        store_q(sc);
                    }
                    if constexpr (!EXACT && !FROM_VT) v_transpose(sc);
                    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                    if constexpr (BF16 && !EXACT && !FROM_VT) {
                        const uint64_t wf = *reinterpret_cast<const uint64_t*>(lds.wide[S]);
                        redo |= (__builtin_amdgcn_readfirstlane((uint32_t)wf) |
                                 __builtin_amdgcn_readfirstlane((uint32_t)(wf >> 32))) != 0;
                    }
                    if constexpr (kDma) {
                        if (t + 2 < ntile) load_tile(t + 2, std::integral_constant<int, (S + 2) % NSLOT>{}, vt_c);
                    } else {
                        if (t + 1 < ntile) issue_q(t + 1);
                    }
                    process(t, sc, exact_c);
                }
            });
        }
        if constexpr (kDma) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return redo;
    };
    auto run_pass = [&]() __attribute__((always_inline)) {
        if (run(std::false_type{}, std::false_type{})) {
            if constexpr (BF16) {
                __syncthreads();  // every wave is past its last read of the ring
                // the pass's rows start over: O rows 8b + 4h + i, this lane's row
#pragma unroll
                for (int b = 0; b < 4; ++b)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int r = wrow0 + 8 * b + 4 * h + i;
                        if (r >= cur && r < rend) {
#pragma unroll
                            for (int m = 0; m < 4; ++m) o[m][4 * b + i] = 0.0f;
                        }
                    }
                if (row >= cur && row < rend) {
                    m_run = kNegInf;
                    m_thr = kNegInf;
                    l_part = 0.0f;
                }
                run(std::true_type{}, std::false_type{});
            }
        }
    };

    if constexpr (SRC == SRC_LOCAL) {
        kv_lo = __builtin_amdgcn_readfirstlane(max(0, q0 - p.pos[q0]));  // uniform: scalar tile addresses
        kv_end = q_end;
        ntile = (kv_end - kv_lo + BN - 1) / BN;
        lo = row_ok ? row - p.pos[row] : 0;
        hi = row_ok ? row : -1;
        if (wrow0 < T) {  // rows increase, and so do their window starts
            const int wrow1 = min(wrow0 + 31, T - 1);
            whi_min = wrow0;
            whi_max = wrow1;
            wlo_min = wrow0 - p.pos[wrow0];
            wlo_max = wrow1 - p.pos[wrow1];
        }
        // prebuilt V^T tiles serve a workgroup whose tiles start on a 64-key
        // boundary; a workgroup whose sequence starts elsewhere transposes
        // its own tiles
        bool prebuilt = false;
        if constexpr (VT) {
            if ((kv_lo % BN) == 0) {
                bool flagged = false;
                const uint8_t* fl = p.vt_flag + (int64_t)g * p.vt_tiles + kv_lo / BN;
                for (int t0 = 0; t0 < ntile; t0 += 64)
                    flagged |= __ballot(t0 + lane < ntile && fl[t0 + lane] != 0) != 0;
                // a flagged tile: bf16 runs the exact mode; fp16 (whose flag
                // marks an inf or NaN, possibly in another sequence's rows of
                // the tile) transposes its own rows, which stop at kv_end
                if (!flagged) {
                    run(std::false_type{}, std::true_type{});
                    prebuilt = true;
                } else if constexpr (BF16) {
                    run(std::true_type{}, std::false_type{});
                    prebuilt = true;
                }
            }
        }
        if (!prebuilt) run_pass();
    } else {
        // runs of rows of one sequence: every wave scans the workgroup's rows
        // and finds the same runs
        while (cur < q_end) {
            const int sq = p.tok_seq[cur];
            rend = q_end;
            int pmax = -1;
            for (int r0 = cur; r0 < rend; r0 += 64) {
                const int r = r0 + lane;
                const int sr = r < rend ? p.tok_seq[r] : sq;
                const uint64_t diff = __ballot(sr != sq);
                if (diff) rend = r0 + (int)__builtin_ctzll(diff);
                pmax = max(pmax, wave_max_int(r < rend ? p.pos[r] : -1));
            }
            pmax = __builtin_amdgcn_readfirstlane(pmax);
            if (sq >= 0 && sq < p.num_seqs && pmax >= 0) {
                kv_lo = 0;
                kv_end = pmax + 1;
                ntile = (kv_end + BN - 1) / BN;
                bt_row = (cint*)(p.bt + (int64_t)sq * p.max_blocks);
                last_page = min((kv_end - 1) >> 4, (int)p.max_blocks - 1);
                const bool in = row_ok && row >= cur && row < rend;
                hi = in ? p.pos[row] : -1;
                lo = 0;
                whi_max = __builtin_amdgcn_readfirstlane(wave_max_int(hi));
                whi_min = __builtin_amdgcn_readfirstlane(-wave_max_int(-hi));
                wlo_min = 0;
                wlo_max = 0;
                __syncthreads();  // the previous pass's last tiles are read before the ring refills
                run_pass();
            }
            cur = rend;
        }
    }

    // ---- normalise and store: lane holds rows 8b + 4h + i, dims 32m + c32
    {
        const float l_tot = l_part + shfl_xor(l_part, 32);
        float* sc = lds.scratch[1][w];
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
                uint16_t* op = p.out + ((int64_t)r * p.Hq + hq) * kD + c32;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const float x = o[m][4 * b + i] * inv;
                    op[32 * m] = qbf ? f32_to_bf16_bits(x) : f32_to_f16_bits(x);
                }
            }
        }
    }

    // ---- fused quantize-on-append of this tile's K/V rows (once per KV head)
    if constexpr (APPEND_FMT >= 0) {
        if (hgrp == 0) {
            const int nrow = min(p.qb, T - q0);
            for (int item = tid; item < 2 * p.qb * 4; item += NW * 64) {  // [tensor][row][block]
                const int tensor = item / (p.qb * 4);
                const int r = (item >> 2) % p.qb;
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

// ---- V^T tiles of the local prefill, built once per (64-key tile, KV head)
// rather than by every workgroup that reads the tile.  Tile tau of head g is
// the byte image of prefill_kernel's LDS V^T tile: fp16 V[64 tau + 16c + 8a
// + 4h + e][d] at byte d * 128 + 16 * ((2c + h) ^ ((d >> 1) & 7)) + 8a + 2e
// (keys past the step: zero).  flag[g][tau] = 1 when some row of the tile
// holds, for bf16 V, |v| >= 65536 or a NaN, or a value below 2^-17 and none
// of 2^-8 or more (per row: every case the kernel's own pass flags for its
// rows' groups is flagged); for fp16 V, an inf or NaN.
template <bool BF16>
__global__ void __launch_bounds__(256) vt_prep_kernel(const uint16_t* __restrict__ v, uint8_t* __restrict__ vt,
                                                      uint8_t* __restrict__ flag, int T, int Hkv, int ntT) {
    // rows padded to 65 dwords: the 8 lanes that gather one dim from 8 rows
    // of the tile hit 8 banks in pairs, not one bank
    __shared__ alignas(16) uint16_t tl[BN][kD + 2];
    const int tau = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    bool fl = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;
        const int r = c >> 4, cc = c & 15;  // row of the tile, 16-byte chunk of the row
        const int k = BN * tau + r;
        u32x4 w = {0u, 0u, 0u, 0u};
        if (k < T) w = *reinterpret_cast<const u32x4*>(v + ((int64_t)k * Hkv + g) * kD + 8 * cc);
        uint32_t mx = 0, mn1 = 0xffffu;
        u16x2 amax = {0, 0}, amin1 = {0xffff, 0xffff};  // |bits|, |bits| - 1 (0 wraps)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const u16x2 a = __builtin_bit_cast(u16x2, w[e] & 0x7fff7fffu);
            amax = __builtin_elementwise_max(amax, a);
            amin1 = __builtin_elementwise_min(amin1, a - u16x2{1, 1});
            if constexpr (BF16) {
                const f16x2 hh = {(_Float16)__builtin_bit_cast(float, w[e] << 16),
                                  (_Float16)__builtin_bit_cast(float, w[e] & 0xffff0000u)};
                w[e] = __builtin_bit_cast(uint32_t, hh);
            }
        }
        mx = max((uint32_t)amax[0], (uint32_t)amax[1]);
        mn1 = min((uint32_t)amin1[0], (uint32_t)amin1[1]);
        // a row's 16 chunks sit in lanes 16j .. 16j + 15
#pragma unroll
        for (int m = 1; m < 16; m <<= 1) {
            mx = max(mx, (uint32_t)__shfl_xor((int)mx, m, kWave));
            mn1 = min(mn1, (uint32_t)__shfl_xor((int)mn1, m, kWave));
        }
        // bf16 bit patterns: 0x477f = 65280 (largest below 2^16), 0x3700 =
        // 2^-17, 0x3b80 = 2^-8; fp16: 0x7c00 = inf
        if constexpr (BF16)
            fl |= mx > 0x477fu || (mn1 < 0x36ffu && mx < 0x3b80u);
        else
            fl |= mx >= 0x7c00u;
#pragma unroll
        for (int e = 0; e < 4; ++e) *reinterpret_cast<uint32_t*>(&tl[r][8 * cc + 2 * e]) = w[e];
    }
    const int any = __syncthreads_or(fl ? 1 : 0);
    if (tid == 0) flag[(int64_t)g * ntT + tau] = any ? 1 : 0;
    // the tile's 16 KB as 1024 chunks, chunk q = tid + 256 i (consecutive
    // lanes, consecutive bytes): dim row d = q >> 3 at position q & 7, which
    // holds logical chunk ci = (q & 7) ^ ((d >> 1) & 7)
    uint8_t* out = vt + (((int64_t)g * ntT + tau) << 14);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = tid + 256 * i, d = q >> 3;
        const int ci = (q & 7) ^ ((d >> 1) & 7), c = ci >> 1, h = ci & 1;
        uint32_t x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = tl[16 * c + 8 * (u >> 2) + 4 * h + (u & 3)][d];
        const u32x4 o = {x[0] | (x[1] << 16), x[2] | (x[3] << 16), x[4] | (x[5] << 16), x[6] | (x[7] << 16)};
        *reinterpret_cast<u32x4*>(out + 16 * q) = o;
    }
}

template <bool BF16, int FMT, int SRC = SRC_LOCAL, bool VT = false>
int launch_prefill(PrefillParams& prm, hipStream_t stream) {
    auto kern = prefill_kernel<BF16, FMT, SRC, VT>;
    const int64_t grid = (int64_t)prm.ntiles * prm.Hkv * prm.hgroups;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * NW), 0, stream, prm);
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}

template <bool BF16, bool VT>
int dispatch_fmt(PrefillParams& prm, int fmt, hipStream_t s) {
    switch (fmt) {
        case -1: return launch_prefill<BF16, -1, SRC_LOCAL, VT>(prm, s);
        case VMC_KV_F16: return launch_prefill<BF16, VMC_KV_F16, SRC_LOCAL, VT>(prm, s);
        case VMC_KV_BF16: return launch_prefill<BF16, VMC_KV_BF16, SRC_LOCAL, VT>(prm, s);
        case VMC_KV_Q8_0: return launch_prefill<BF16, VMC_KV_Q8_0, SRC_LOCAL, VT>(prm, s);
        case VMC_KV_Q4_0: return launch_prefill<BF16, VMC_KV_Q4_0, SRC_LOCAL, VT>(prm, s);
        default: return VMC_EINVAL;
    }
}

// workspace of the local prefill's prebuilt V^T tiles: 16 KB per (64-key
// tile, KV head), then one flag byte each
size_t vt_workspace_bytes(int64_t num_tokens, int64_t num_kv_heads) {
    const int64_t n = (num_tokens + BN - 1) / BN * num_kv_heads;
    return (size_t)(n * (kD * BN * 2) + ((n + 255) & ~(int64_t)255));
}

// workgroup shape shared by the local and paged entry points
void set_tiling(PrefillParams& prm, int num_tokens, int num_heads, int num_kv_heads, float scale) {
    prm.T = num_tokens;
    prm.Hq = num_heads;
    prm.Hkv = num_kv_heads;
    prm.G = num_heads / num_kv_heads;
    prm.scale_log2 = scale * kLog2e;
    // heads per workgroup: 4, 2 or 1, dividing G; 32-row blocks per head fill 8 waves
    prm.hw = prm.G % 4 == 0 ? 4 : (prm.G % 2 == 0 ? 2 : 1);
    prm.rb = NW / prm.hw;
    prm.qb = 32 * prm.rb;
    prm.hgroups = prm.G / prm.hw;
    prm.ntiles = (num_tokens + prm.qb - 1) / prm.qb;
}

}  // namespace

int tq_prefill_tiled(void* out, const void* query, const void* kv_cache, const int32_t* block_tables,
                     const int32_t* token_to_seq, const int32_t* token_positions, int num_tokens, int num_heads,
                     int num_kv_heads, float scale, int64_t max_blocks, const vmc_tq_config* cfg, int half_dtype,
                     hipStream_t stream) {
    if (!tq_config_valid(cfg) || cfg->head_dim != kD || cfg->group_size != 0) return VMC_EINVAL;
    if (half_dtype != VMC_DTYPE_F16 && half_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || max_blocks <= 0 ||
        max_blocks > 0x7fffffff)
        return VMC_EINVAL;
    if (num_tokens == 0) return VMC_OK;
    if (!out || !query || !kv_cache || !block_tables || !token_to_seq || !token_positions) return VMC_EINVAL;
    if (((uintptr_t)kv_cache & 3) != 0) return VMC_EINVAL;
    PrefillParams prm = {};
    prm.out = reinterpret_cast<uint16_t*>(out);
    prm.q = reinterpret_cast<const uint16_t*>(query);
    prm.pos = token_positions;
    set_tiling(prm, num_tokens, num_heads, num_kv_heads, scale);
    prm.kp = prm.vp = reinterpret_cast<const uint8_t*>(kv_cache);
    prm.bt = block_tables;
    prm.tok_seq = token_to_seq;
    prm.max_blocks = max_blocks;
    prm.num_seqs = 0x7fffffff;  // the rows' sequences are the caller's to keep in the table
    prm.E = cfg->slot_size_aligned;
    prm.page_bytes = (int64_t)kBsP * num_kv_heads * prm.E;
    prm.hnd = 0;
    prm.q_bf16 = half_dtype == VMC_DTYPE_BF16;
    if (!cfg->key_fp8) {
        const TQTables& tab = tq_tables(kD, cfg->key_quant_bits);
        for (int i = 0; i < 16; ++i) prm.cent[i] = i < tab.n_centroids ? tab.centroids[i] : 0.0f;
        prm.rot_c = tab.rot_c;
    }
    prm.fp8_e4b15 = cfg->fp8_e4b15 ? 1 : 0;
    prm.mse_bytes = cfg->mse_bytes;
    prm.key_packed = cfg->key_packed_size;
    prm.val_data = cfg->val_data_bytes;
    prm.norm_corr = cfg->norm_correction != 0;
    if ((int64_t)prm.ntiles * prm.Hkv * prm.hgroups > 0x7fffffffLL) return VMC_EINVAL;
    const int kb = cfg->key_quant_bits, vb = cfg->value_quant_bits;
    if (cfg->key_fp8) return vb == 4 ? launch_prefill<false, -1, SRC_K8>(prm, stream) : VMC_EINVAL;
    if (kb == 3 && vb == 3) return launch_prefill<false, -1, SRC_TQ33>(prm, stream);
    if (kb == 4 && vb == 4) return launch_prefill<false, -1, SRC_TQ44>(prm, stream);
    if (kb == 3 && vb == 4) return launch_prefill<false, -1, SRC_TQ34>(prm, stream);
    return VMC_EINVAL;
}

}  // namespace vmc

using namespace vmc;

extern "C" int vmc_flash_attention_prefill_v2(void* output, const void* query, const void* key_cache,
                                              const void* value_cache, int num_tokens, int num_heads,
                                              int num_kv_heads, int head_dim, float scale, int block_size,
                                              int max_num_blocks_per_req, const int32_t* block_tables,
                                              const int32_t* seq_lens, const int32_t* token_to_seq,
                                              const int32_t* token_positions, int num_reqs, int q_dtype,
                                              int kv_format, int layout, vmc_stream_t stream) {
    (void)seq_lens;  // a token's keys are positions 0 .. token_positions[t]
    if (generic_head_dim(head_dim)) {
        // head_dim 64 / 256: one wave per (token, query head), any block size
        if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
            block_size <= 0 || max_num_blocks_per_req <= 0 || num_reqs < 0)
            return VMC_EINVAL;
        if (q_dtype != VMC_DTYPE_F16 && q_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
        if (layout != VMC_LAYOUT_NHD && layout != VMC_LAYOUT_HND) return VMC_EINVAL;
        if (kv_format != VMC_KV_F16 && kv_format != VMC_KV_BF16 && kv_format != VMC_KV_Q8_0 &&
            kv_format != VMC_KV_Q4_0)
            return VMC_EINVAL;
        if (num_tokens == 0 || num_reqs == 0) return VMC_OK;
        if (!output || !query || !key_cache || !value_cache || !block_tables || !token_to_seq ||
            !token_positions)
            return VMC_EINVAL;
        GenArgs a = {};
        a.out = output;
        a.q = query;
        a.q_bf16 = q_dtype == VMC_DTYPE_BF16;
        a.src = kv_format == VMC_KV_F16 ? GEN_F16 : kv_format == VMC_KV_BF16 ? GEN_BF16
              : kv_format == VMC_KV_Q8_0 ? GEN_Q8 : GEN_Q4;
        a.kp = reinterpret_cast<const uint8_t*>(key_cache);
        a.vp = reinterpret_cast<const uint8_t*>(value_cache);
        a.entry = vmc_kv_entry_bytes(kv_format, head_dim);
        a.hnd = layout == VMC_LAYOUT_HND;
        a.bs = block_size;
        a.bt = block_tables;
        a.max_blocks = max_num_blocks_per_req;
        a.tok_seq = token_to_seq;
        a.pos = token_positions;
        a.num_seqs = num_reqs;
        a.rows = num_tokens;
        a.Hq = num_heads;
        a.Hkv = num_kv_heads;
        a.D = head_dim;
        a.scale = scale;
        return gen_attention(a, reinterpret_cast<hipStream_t>(stream));
    }
    if (head_dim != kD || block_size != kBsP || num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 ||
        num_heads % num_kv_heads != 0 || max_num_blocks_per_req <= 0 || num_reqs < 0)
        return VMC_EINVAL;
    if (q_dtype != VMC_DTYPE_F16 && q_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (layout != VMC_LAYOUT_NHD && layout != VMC_LAYOUT_HND) return VMC_EINVAL;
    if (kv_format != VMC_KV_F16 && kv_format != VMC_KV_BF16 && kv_format != VMC_KV_Q8_0 &&
        kv_format != VMC_KV_Q4_0)
        return VMC_EINVAL;
    if (num_tokens == 0 || num_reqs == 0) return VMC_OK;
    if (!output || !query || !key_cache || !value_cache || !block_tables || !token_to_seq ||
        !token_positions)
        return VMC_EINVAL;
    // pages are read in 16-byte (f16 / bf16) and 4-byte (q8_0 / q4_0) units
    if ((((uintptr_t)key_cache | (uintptr_t)value_cache) & 15) != 0) return VMC_EINVAL;
    PrefillParams prm = {};
    prm.out = reinterpret_cast<uint16_t*>(output);
    prm.q = reinterpret_cast<const uint16_t*>(query);
    prm.pos = token_positions;
    set_tiling(prm, num_tokens, num_heads, num_kv_heads, scale);
    prm.kp = reinterpret_cast<const uint8_t*>(key_cache);
    prm.vp = reinterpret_cast<const uint8_t*>(value_cache);
    prm.bt = block_tables;
    prm.tok_seq = token_to_seq;
    prm.max_blocks = max_num_blocks_per_req;
    prm.num_seqs = num_reqs;
    prm.E = vmc_kv_entry_bytes(kv_format, head_dim);
    prm.page_bytes = (int64_t)kBsP * num_kv_heads * prm.E;
    prm.hnd = layout == VMC_LAYOUT_HND;
    prm.q_bf16 = q_dtype == VMC_DTYPE_BF16;
    if ((int64_t)prm.ntiles * prm.Hkv * prm.hgroups > 0x7fffffffLL) return VMC_EINVAL;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (kv_format) {
        case VMC_KV_F16: return launch_prefill<false, -1, SRC_PAGED>(prm, s);
        case VMC_KV_BF16: return launch_prefill<true, -1, SRC_PAGED>(prm, s);
        case VMC_KV_Q8_0: return launch_prefill<false, -1, SRC_Q8>(prm, s);
        default: return launch_prefill<false, -1, SRC_Q4>(prm, s);
    }
}

namespace {
// the local prefill; with a workspace (ws != NULL) the V^T tiles are built
// once by vt_prep_kernel and the attention kernel fetches them
int local_prefill(void* output, const void* query, const void* key, const void* value, int num_tokens,
                  int num_heads, int num_kv_heads, int head_dim, float scale, const int32_t* token_positions,
                  int dtype, void* key_cache, void* value_cache, const int64_t* slot_mapping, int64_t block_size,
                  int kv_format, int layout, void* ws, size_t ws_bytes, vmc_stream_t stream) {
    if (generic_head_dim(head_dim)) {
        // head_dim 64 / 256: the append by vmc_reshape_and_cache, then one
        // wave per (token, query head) over this step's K/V
        if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
            return VMC_EINVAL;
        if (dtype != VMC_DTYPE_F16 && dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
        if (num_tokens == 0) return VMC_OK;
        if (!output || !query || !key || !value || !token_positions) return VMC_EINVAL;
        if (key_cache) {
            const int64_t E = vmc_kv_entry_bytes(kv_format, head_dim);
            if (E < 0 || block_size <= 0) return VMC_EINVAL;
            const int rc = vmc_reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, num_tokens,
                                                 num_kv_heads, head_dim, block_size,
                                                 block_size * num_kv_heads * E, kv_format, dtype, layout,
                                                 stream);
            if (rc != VMC_OK) return rc;
        }
        GenArgs a = {};
        a.out = output;
        a.q = query;
        a.q_bf16 = dtype == VMC_DTYPE_BF16;
        a.src = GEN_LOCAL;
        a.k = reinterpret_cast<const uint16_t*>(key);
        a.v = reinterpret_cast<const uint16_t*>(value);
        a.pos = token_positions;
        a.num_seqs = -1;
        a.rows = num_tokens;
        a.Hq = num_heads;
        a.Hkv = num_kv_heads;
        a.D = head_dim;
        a.scale = scale;
        return gen_attention(a, reinterpret_cast<hipStream_t>(stream));
    }
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
    set_tiling(prm, num_tokens, num_heads, num_kv_heads, scale);
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
    if ((int64_t)prm.ntiles * prm.Hkv * prm.hgroups > 0x7fffffffLL) return VMC_EINVAL;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool bf = dtype == VMC_DTYPE_BF16;
    if (!ws) return bf ? dispatch_fmt<true, false>(prm, fmt, s) : dispatch_fmt<false, false>(prm, fmt, s);
    if (ws_bytes < vt_workspace_bytes(num_tokens, num_kv_heads)) return VMC_ENOMEM;
    if (((uintptr_t)ws & 15) != 0) return VMC_EINVAL;
    const int ntT = (num_tokens + BN - 1) / BN;
    prm.vt = reinterpret_cast<const uint8_t*>(ws);
    prm.vt_flag = prm.vt + (int64_t)ntT * num_kv_heads * (kD * BN * 2);
    prm.vt_tiles = ntT;
    uint8_t* vt = reinterpret_cast<uint8_t*>(ws);
    uint8_t* flag = vt + (int64_t)ntT * num_kv_heads * (kD * BN * 2);
    const dim3 vgrid((unsigned)ntT, (unsigned)num_kv_heads);
    if (bf)
        hipLaunchKernelGGL(vt_prep_kernel<true>, vgrid, dim3(256), 0, s, prm.v, vt, flag, num_tokens, num_kv_heads, ntT);
    else
        hipLaunchKernelGGL(vt_prep_kernel<false>, vgrid, dim3(256), 0, s, prm.v, vt, flag, num_tokens, num_kv_heads,
                           ntT);
    VMC_LAUNCH_CHECK();
    return bf ? dispatch_fmt<true, true>(prm, fmt, s) : dispatch_fmt<false, true>(prm, fmt, s);
}
}  // namespace

extern "C" int vmc_flash_attention_prefill(void* output, const void* query, const void* key,
                                           const void* value, int num_tokens, int num_heads,
                                           int num_kv_heads, int head_dim, float scale,
                                           const int32_t* token_positions, int dtype,
                                           void* key_cache, void* value_cache,
                                           const int64_t* slot_mapping, int64_t block_size,
                                           int kv_format, int layout, vmc_stream_t stream) {
    return local_prefill(output, query, key, value, num_tokens, num_heads, num_kv_heads, head_dim, scale,
                         token_positions, dtype, key_cache, value_cache, slot_mapping, block_size, kv_format,
                         layout, nullptr, 0, stream);
}

extern "C" size_t vmc_flash_attention_prefill_workspace_size(int num_tokens, int num_kv_heads, int head_dim) {
    if (head_dim != kD || num_tokens <= 0 || num_kv_heads <= 0) return 0;
    return vt_workspace_bytes(num_tokens, num_kv_heads);
}

extern "C" int vmc_flash_attention_prefill_ws(void* output, const void* query, const void* key,
                                              const void* value, int num_tokens, int num_heads,
                                              int num_kv_heads, int head_dim, float scale,
                                              const int32_t* token_positions, int dtype, void* key_cache,
                                              void* value_cache, const int64_t* slot_mapping,
                                              int64_t block_size, int kv_format, int layout,
                                              void* workspace, size_t workspace_bytes, vmc_stream_t stream) {
    // head_dim 64 / 256 take no workspace (their kernel has no tiles)
    if (head_dim == kD && num_tokens > 0 && !workspace) return VMC_EINVAL;
    return local_prefill(output, query, key, value, num_tokens, num_heads, num_kv_heads, head_dim, scale,
                         token_positions, dtype, key_cache, value_cache, slot_mapping, block_size, kv_format,
                         layout, head_dim == kD ? workspace : nullptr, workspace_bytes, stream);
}
