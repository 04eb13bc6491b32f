// paged_decode.hip -- split-KV paged decode attention for gfx950.
//
// Replaces vm_c::paged_attention_v1/_v2 (src/cuda/attention_kernels.cu:438-473)
// and vm_c::turboquant_decode_attention (src/cuda/turboquant_kernels.cu:
// 939-1007).  Semantics: softmax(q k^T * scale) v per query head over the
// sequence's tokens, read through the block table, GQA kv head = q head /
// (Hq / Hkv) (ggml flash_attn_ext broadcast, ggml-cpu/ops.cpp:8260-8265).
//
// Work decomposition.  A work item is (sequence, split): a contiguous run of
// pages of one sequence.  Every workgroup recomputes the same plan from
// seq_lens (pages_b = ceil(L_b / bs); pages per split = max(pps_min,
// ceil(total / target_items)); splits_b = min(max_splits, ...)) so no host
// round trip or extra launch is needed; items beyond the plan exit.  The
// workgroup has one wave per KV head; a page of the reference layout holds
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
//
// Partials (multi-split sequences) are fp32 (o, m, l) per (item, head) in the
// caller's workspace; vmc_decode_merge_kernel combines them.
#include "vmc_common.hpp"
#include "vmc_tq.hpp"

#include <utility>

namespace vmc {
namespace {

constexpr int kD = 128;
constexpr int kBs = 16;
constexpr int kMaxItemPages = 1024;  // block-table slice of one work item, staged in LDS
constexpr float kNegInf = -__builtin_inff();

enum { FMT_F16 = 0, FMT_BF16 = 1, FMT_Q8_0 = 2, FMT_Q4_0 = 3, FMT_TQ = 4 };

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Register staging of LDS-staged formats: SPP 16-byte chunks per thread per
// page (= ceil(bytes per token-head / 64) for one wave per KV head) and PF
// pages in flight per workgroup.
template <int FMT, int KB, int VB>
struct StagePlan {
    static constexpr int entry = FMT == FMT_TQ ? (16 * KB + 2 + 16 * VB + 4 + 1) / 2 * 2
                                 : FMT == FMT_Q8_0 ? 2 * 136 : FMT == FMT_Q4_0 ? 2 * 72 : 0;
    static constexpr int spp = entry > 0 ? (entry + 63) / 64 : 1;
    static constexpr int pf = entry == 0 ? 1 : (spp <= 2 ? 4 : (spp <= 3 ? 3 : 2));
};

struct DecodeParams {
    void* out;
    const uint16_t* q;
    const uint8_t* kc;
    const uint8_t* vc;
    const int32_t* bt;
    const int32_t* seq_lens;
    float* part;       // [items][Hq][D + 2]
    int32_t* seqinfo;  // [B][2]: first item, number of splits
    int B, Hq, Hkv, G, max_blocks;
    float scale_log2;
    int64_t page_bytes;  // one page of one cache, all heads
    int entry_bytes;     // one (token, head) entry (TQ: the aligned slot)
    int hnd;
    int target_items, pps_min, max_splits;
    int q_bf16;
    // TurboQuant
    int mse_bytes, key_packed, val_data;
    TQTables tab;
};

struct Plan {
    int b, s, nsp, first_item, p0, p1, L;
};

// Identical in every workgroup (and in the merge kernel): a pure function of
// seq_lens.  Executed by one wave; lanes stride over sequences.
__device__ void compute_plan(const DecodeParams& p, int item, Plan* out) {
    const int lane = threadIdx.x & 63;
    int total = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
        const int b = b0 + lane;
        const int L = b < p.B ? min(p.seq_lens[b], p.max_blocks * kBs) : 0;
        int pages = L > 0 ? (L + kBs - 1) / kBs : 0;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) pages += __shfl_xor(pages, m, 64);
        total += pages;
    }
    const int pps = max(p.pps_min, (total + p.target_items - 1) / p.target_items);
    int carry = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
        const int b = b0 + lane;
        const int L = b < p.B ? min(p.seq_lens[b], p.max_blocks * kBs) : 0;
        const int pages = L > 0 ? (L + kBs - 1) / kBs : 0;
        int nsp = 0, ppsb = 0;
        if (b < p.B) {
            nsp = pages > 0 ? min(p.max_splits, (pages + pps - 1) / pps) : 1;
            ppsb = pages > 0 ? min(kMaxItemPages, (pages + nsp - 1) / nsp) : 0;
            nsp = pages > 0 ? (pages + ppsb - 1) / ppsb : 1;
        }
        int incl = nsp;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) {
            const int v = __shfl_up(incl, m, 64);
            if (lane >= m) incl += v;
        }
        const int first = carry + incl - nsp;
        const bool mine = b < p.B && item >= first && item < first + nsp;
        const unsigned long long bal = __ballot(mine);
        if (bal) {
            const int src = __builtin_ctzll(bal);
            if (lane == src) {
                const int s = item - first;
                out->b = b;
                out->s = s;
                out->nsp = nsp;
                out->first_item = first;
                out->p0 = s * ppsb;
                out->p1 = min(pages, (s + 1) * ppsb);
                out->L = L;
            }
            return;
        }
        carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) out->b = -1;
}

// ------------------------------------------------------------------ operands

// pair table for the TurboQuant key codebook: entry (c0 | c1 << KB) =
// fp16(C[c0]) | fp16(C[c1]) << 16, i.e. one dword of an f16x8 MFMA operand.
template <int KB>
__device__ __forceinline__ void build_pair_lut(uint32_t* lut, const TQTables& tab) {
    constexpr int N = 1 << KB;
    for (int e = threadIdx.x; e < N * N; e += blockDim.x) {
        const int c0 = e & (N - 1), c1 = e >> KB;
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int c = 0; c < N; ++c) {
            a = c == c0 ? tab.centroids[c] : a;
            b = c == c1 ? tab.centroids[c] : b;
        }
        lut[e] = (uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
    }
}

__device__ __forceinline__ uint32_t lds16(const uint8_t* p) {
    return (uint32_t)*reinterpret_cast<const uint16_t*>(p);
}

// int codes (0..15) -> exact fp16 via the 1024 + c bit trick
__device__ __forceinline__ _Float16 code_f16(uint32_t c) {
    return __builtin_bit_cast(_Float16, (uint16_t)(0x6400u | c)) - (_Float16)1024.0f;
}

template <int FMT>
__device__ __forceinline__ int entry_off(int tok, int g, int Hkv, int E, int hnd) {
    return hnd ? (g * kBs + tok) * E : (tok * Hkv + g) * E;
}

// ------------------------------------------------------------------ kernel

template <int FMT, int KB, int VB, bool MBF16>
__global__ void __launch_bounds__(512)
paged_decode_kernel(DecodeParams p) {
    using AT = typename std::conditional<MBF16, bf16x8, f16x8>::type;
    using PT = typename std::conditional<MBF16, s16x4, f16x4>::type;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ Plan plan;
    __shared__ __attribute__((aligned(16))) float wscr_all[8][48];  // per-wave exchange
    __shared__ int32_t bt_lds[kMaxItemPages];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int r16 = lane & 15, grp = lane >> 4;
    const int item = blockIdx.x;

    if (wave == 0) compute_plan(p, item, &plan);
    constexpr bool kStaged = FMT >= FMT_Q8_0;
    // static LDS: the LUT's address is a compile-time offset of each read
    __shared__ uint32_t lut[FMT == FMT_TQ ? 256 : 1];
    uint8_t* pagebuf = smem;
    if constexpr (FMT == FMT_TQ) build_pair_lut<KB>(lut, p.tab);
    __syncthreads();
    const int b = __builtin_amdgcn_readfirstlane(plan.b);
    if (b < 0) return;
    // wave-uniform: keep them in SGPRs so block-table reads are scalar loads
    const int s = __builtin_amdgcn_readfirstlane(plan.s);
    const int nsp = __builtin_amdgcn_readfirstlane(plan.nsp);
    const int L = __builtin_amdgcn_readfirstlane(plan.L);
    const int p0 = __builtin_amdgcn_readfirstlane(plan.p0);
    const int p1 = __builtin_amdgcn_readfirstlane(plan.p1);
    if (s == 0 && tid == 0) {
        p.seqinfo[2 * b] = plan.first_item;
        p.seqinfo[2 * b + 1] = nsp;
    }

    const int g = wave;  // kv head of this wave
    float* wscr = wscr_all[wave];
    const int G = p.G;
    const int hq0 = g * G;
    const int64_t qrow = ((int64_t)b * p.Hq + hq0 + r16) * kD;
    const bool head_ok = r16 < G;

    // ---- Q operand: lane (r16 = head, grp) holds dims 32*grp + 8*j + e, j = MFMA index
    AT qb[4];
    if constexpr (FMT == FMT_TQ) {
        float y[32];
        if (head_ok) {
            const u32x4* src = reinterpret_cast<const u32x4*>(p.q + qrow + 32 * grp);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const u32x4 w = src[c];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint16_t lo = (uint16_t)(w[e] & 0xffff), hi = (uint16_t)(w[e] >> 16);
                    y[8 * c + 2 * e] = p.q_bf16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
                    y[8 * c + 2 * e + 1] = p.q_bf16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 32; ++e) y[e] = 0.0f;
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
            u32x4 w = {0u, 0u, 0u, 0u};
            if (head_ok) w = *reinterpret_cast<const u32x4*>(p.q + qrow + 32 * grp + 8 * j);
            const bool qbf = p.q_bf16 != 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint16_t lo = (uint16_t)(w[e] & 0xffff), hi = (uint16_t)(w[e] >> 16);
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

    // ---- running state
    f32x4 oacc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) oacc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = kNegInf;  // per head r16 (log2 domain), replicated over grp
    float l_part = 0.0f;    // partial over this lane's tokens
    float z_part = 0.0f;    // TurboQuant: partial sum of p * zero

    const int Hkv = p.Hkv, E = p.entry_bytes, hnd = p.hnd;
    const int64_t page_bytes = p.page_bytes;
    // this item's block-table slice -> LDS, so the page loop issues no vector
    // loads besides the page prefetch (keeps the load counter exact)
    {
        const int32_t* bt_row = p.bt + (int64_t)b * p.max_blocks;
        for (int i = tid; i < p1 - p0; i += blockDim.x) bt_lds[i] = bt_row[p0 + i];
        __syncthreads();
    }
    const int nthreads = blockDim.x;

    // staged formats: PF pages in flight in registers -> LDS double buffer
    using SP = StagePlan<FMT, KB, VB>;
    constexpr int SPP = SP::spp, PF = SP::pf;
    const int n16_k = (int)(page_bytes / 16);
    const int n16 = (FMT == FMT_TQ) ? n16_k : 2 * n16_k;
    const int lds_page = (FMT == FMT_TQ) ? (int)page_bytes : 2 * (int)page_bytes;
    u32x4 stage[PF][SPP];
    auto stage_load = [&](auto slot_c, int pg) __attribute__((always_inline)) {
        constexpr int S = decltype(slot_c)::value;
        // Branch-free so the compiler can count outstanding loads exactly (a
        // hole reads page 0, whose tokens are then masked; chunks past the
        // page re-read its last chunk and are not stored).
        const int32_t blk = max(bt_lds[pg - p0], 0);
        const u32x4* ks = reinterpret_cast<const u32x4*>(p.kc + (int64_t)blk * page_bytes);
        const u32x4* vs = reinterpret_cast<const u32x4*>(p.vc + (int64_t)blk * page_bytes);
#pragma unroll
        for (int c = 0; c < SPP; ++c) {
            const int idx = min(tid + c * nthreads, n16 - 1);
            const u32x4* src = (FMT == FMT_TQ || idx < n16_k) ? ks + idx : vs + (idx - n16_k);
            stage[S][c] = *src;
        }
    };
    auto stage_store = [&](auto slot_c, uint8_t* dstb) __attribute__((always_inline)) {
        constexpr int S = decltype(slot_c)::value;
        u32x4* dst = reinterpret_cast<u32x4*>(dstb);
#pragma unroll
        for (int c = 0; c < SPP; ++c) {
            const int idx = tid + c * nthreads;
            if (idx < n16) dst[idx] = stage[S][c];
        }
    };

    // direct formats: per-lane operand registers for one page
    u32x4 kreg[4], vreg[4];
    auto direct_load = [&](int pg) __attribute__((always_inline)) {
        const int32_t blk = bt_lds[pg - p0];
        const int tok0 = pg * kBs;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            kreg[c] = u32x4{0u, 0u, 0u, 0u};
            vreg[c] = u32x4{0u, 0u, 0u, 0u};
        }
        if (blk < 0) return;
        const uint8_t* kp = p.kc + (int64_t)blk * page_bytes;
        const uint8_t* vp = p.vc + (int64_t)blk * page_bytes;
        if (tok0 + r16 < L) {
            const u32x4* src = reinterpret_cast<const u32x4*>(kp + entry_off<FMT>(r16, g, Hkv, E, hnd) + 64 * grp);
#pragma unroll
            for (int c = 0; c < 4; ++c) kreg[c] = src[c];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = 4 * grp + i;
            if (tok0 + tok < L)
                vreg[i] = *reinterpret_cast<const u32x4*>(vp + entry_off<FMT>(tok, g, Hkv, E, hnd) + 16 * r16);
        }
    };

    auto process = [&](int pg, const uint8_t* kpage, const uint8_t* vpage) __attribute__((always_inline)) {
        const int32_t blk = bt_lds[pg - p0];
        const int nv = blk < 0 ? 0 : min(kBs, L - pg * kBs);  // valid tokens in this page
        AT a[4];
        float rowf = p.scale_log2;  // factor of S row r16 (token r16)
        // V operand pieces (tokens 4*grp + i, dims 8*r16 .. +7) as fp16/bf16 bits
        uint32_t vw[4][4];  // [token i][dword e] = dims (2e, 2e+1)
        uint32_t bop[8][2];  // PV B operands: dim 8*r16 + c, tokens {0,1} / {2,3}
        float vsc[4] = {1.f, 1.f, 1.f, 1.f}, vzr[4] = {0.f, 0.f, 0.f, 0.f};

        if constexpr (kStaged) {
            // ---- K operand for token r16
            const uint8_t* ke = kpage + entry_off<FMT>(r16, g, Hkv, E, hnd);
            if constexpr (FMT == FMT_TQ) {
                // K: lane group grp owns dims 32*grp .. +31 of token r16; each
                // code pair indexes the LUT of packed fp16 centroid pairs.
                u32x4 aw[4];
                if constexpr (KB == 4) {
                    const uint8_t* cb = ke + 16 * grp;  // 16 bytes, 2-byte aligned
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t w = lds16(cb + 4 * j) | (lds16(cb + 4 * j + 2) << 16);
#pragma unroll
                        for (int e = 0; e < 4; ++e) aw[j][e] = lut[(w >> (8 * e)) & 0xffu];
                    }
                } else {
                    const uint8_t* cb = ke + 12 * grp;  // 12 bytes = four 8-code groups
                    uint32_t h[6];
#pragma unroll
                    for (int q = 0; q < 6; ++q) h[q] = lds16(cb + 2 * q);
                    const uint32_t g24[4] = {h[0] | ((h[1] & 0xffu) << 16), (h[1] >> 8) | (h[2] << 8),
                                             h[3] | ((h[4] & 0xffu) << 16), (h[4] >> 8) | (h[5] << 8)};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int e = 0; e < 4; ++e) aw[j][e] = lut[(g24[j] >> (6 * e)) & 63u];
                }
                // sum of squared centroids (one mixed-precision fma per value;
                // v_dot2 with a squared operand gave wrong sums on this toolchain)
                float csq = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    a[j] = __builtin_bit_cast(AT, aw[j]);
#pragma unroll
                    for (int e = 0; e < 8; ++e) csq = __builtin_fmaf((float)a[j][e], (float)a[j][e], csq);
                }
                csq = sum_over_groups(csq);
                const float nrm = f16_bits_to_f32((uint16_t)lds16(ke + p.mse_bytes));
                rowf = p.scale_log2 * nrm * __builtin_amdgcn_rsqf(csq + 1e-16f);
                // V: codes of tokens 4*grp + i, dims 8*r16 .. +7, scale and zero
                uint32_t cw[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tok = 4 * grp + i;
                    const uint8_t* ve = kpage + entry_off<FMT>(tok, g, Hkv, E, hnd) + p.key_packed;
                    if constexpr (VB == 4) {
                        cw[i] = lds16(ve + 4 * r16) | (lds16(ve + 4 * r16 + 2) << 16);
                    } else {
                        // ve is even, so ve + 3*r16 is odd exactly when r16 is:
                        // read the two aligned 16-bit words around it
                        const uint8_t* al2 = ve + 3 * r16 - (r16 & 1);
                        const uint32_t w = lds16(al2) | (lds16(al2 + 2) << 16);
                        cw[i] = (w >> (8 * (r16 & 1))) & 0xffffffu;
                    }
                    const bool ok = tok < nv;
                    vsc[i] = ok ? f16_bits_to_f32((uint16_t)lds16(ve + p.val_data)) : 0.0f;
                    vzr[i] = ok ? f16_bits_to_f32((uint16_t)lds16(ve + p.val_data + 2)) : 0.0f;
                }
                // B operands {token a, token b} per dim, exact fp16 codes via 1024 + c
#pragma unroll
                for (int c = 0; c < 8; ++c) {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        uint32_t x;
                        if constexpr (VB == 4) {
                            const uint32_t t = __builtin_amdgcn_perm(cw[2 * hh + 1], cw[2 * hh],
                                                                     (uint32_t)(c >> 1) | 0x0c00u |
                                                                         ((uint32_t)(4 + (c >> 1)) << 16) | 0x0c000000u);
                            x = (c & 1) ? (t >> 4) : t;
                            x = (x & 0x000f000fu) | 0x64006400u;
                        } else {
                            const uint32_t c0 = (cw[2 * hh] >> (3 * c)) & 7u;
                            const uint32_t c1 = (cw[2 * hh + 1] >> (3 * c)) & 7u;
                            x = (c0 | (c1 << 16)) | 0x64006400u;
                        }
                        const f16x2 v2 = __builtin_bit_cast(f16x2, x) - f16x2{(_Float16)1024.0f, (_Float16)1024.0f};
                        bop[c][hh] = __builtin_bit_cast(uint32_t, v2);
                    }
                }
            } else {
                // GGUF blocks: lane group grp owns block grp (dims 32*grp .. +31)
                constexpr int BE = FMT == FMT_Q8_0 ? 34 : 18;
                const uint8_t* kb = ke + BE * grp;
                const float d = f16_bits_to_f32((uint16_t)lds16(kb));
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int e = 0; e < 8; e += 2) {
                        const int jj = 8 * j + e;  // index inside the 32-block
                        float x0, x1;
                        if constexpr (FMT == FMT_Q8_0) {
                            const uint32_t w = lds16(kb + 2 + jj);
                            x0 = (float)(int8_t)(w & 0xff);
                            x1 = (float)(int8_t)(w >> 8);
                        } else {
                            const int bi = jj & 15;
                            const uint32_t w = lds16(kb + 2 + bi);
                            const int sh = jj < 16 ? 0 : 4;
                            x0 = (float)((int)((w >> sh) & 0xf) - 8);
                            x1 = (float)((int)((w >> (8 + sh)) & 0xf) - 8);
                        }
                        a[j][e] = (_Float16)(x0 * d);
                        a[j][e + 1] = (_Float16)(x1 * d);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tok = 4 * grp + i;
                    const bool ok = tok < nv;
                    const uint8_t* vb = vpage + entry_off<FMT>(tok, g, Hkv, E, hnd) + BE * (r16 >> 2);
                    const float dv = ok ? f16_bits_to_f32((uint16_t)lds16(vb)) : 0.0f;
                    const int q0 = 8 * (r16 & 3);  // index inside the block
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float x0, x1;
                        if constexpr (FMT == FMT_Q8_0) {
                            const uint32_t w = lds16(vb + 2 + q0 + 2 * e);
                            x0 = (float)(int8_t)(w & 0xff);
                            x1 = (float)(int8_t)(w >> 8);
                        } else {
                            const int jj = q0 + 2 * e;
                            const int bi = jj & 15;
                            const int sh = jj < 16 ? 0 : 4;
                            const uint32_t w = lds16(vb + 2 + bi);
                            x0 = (float)((int)((w >> sh) & 0xf) - 8);
                            x1 = (float)((int)((w >> (8 + sh)) & 0xf) - 8);
                        }
                        vw[i][e] = (uint32_t)f32_to_f16_bits(ok ? x0 * dv : 0.0f) |
                                   ((uint32_t)f32_to_f16_bits(ok ? x1 * dv : 0.0f) << 16);
                    }
                }
            }
        } else {
            // f16 / bf16: operands straight from the registers loaded last iteration
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4 w = kreg[j];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (MBF16) {
                        a[j][2 * e] = __builtin_bit_cast(__bf16, (uint16_t)(w[e] & 0xffff));
                        a[j][2 * e + 1] = __builtin_bit_cast(__bf16, (uint16_t)(w[e] >> 16));
                    } else {
                        a[j][2 * e] = __builtin_bit_cast(_Float16, (uint16_t)(w[e] & 0xffff));
                        a[j][2 * e + 1] = __builtin_bit_cast(_Float16, (uint16_t)(w[e] >> 16));
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) vw[i][e] = vreg[i][e];
            if (pg + 1 < p1) direct_load(pg + 1);
        }

        // ---- S^T = K . Q^T
        f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) sacc = mfma16x16x32(a[j], qb[j], sacc);

        f32x4 rf = {rowf, rowf, rowf, rowf};
        if constexpr (FMT == FMT_TQ) rf = gather4_from_row0(rowf, wscr, r16, grp);
        float sv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = 4 * grp + i;
            sv[i] = tok < nv ? sacc[i] * rf[i] : kNegInf;
        }
        float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        mx = max_over_groups(mx);
        // Lazy reference max: m_run moves only when a head's max exceeds it by
        // more than 8 (log2 units), so p <= 256 and most pages skip the O
        // rescale.  Every term of l, z and O uses the same reference: exact.
        const bool upd = mx > m_run + 8.0f;
        if (__ballot(upd)) {  // wave-uniform
            const float m_new = upd ? mx : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 when m_run = -inf
            l_part *= alpha;
            if constexpr (FMT == FMT_TQ) z_part *= alpha;
            const f32x4 al = gather4_from_row0(alpha, wscr + 16, r16, grp);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int c = 0; c < 8; ++c) oacc[c][i] *= al[i];
            m_run = m_new;
        }
        const float m_use = m_run == kNegInf ? 0.0f : m_run;
        float pv[4], psum = 0.0f, zsum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pv[i] = __builtin_amdgcn_exp2f(sv[i] - m_use);
            psum += pv[i];
            if constexpr (FMT == FMT_TQ) zsum = __builtin_fmaf(pv[i], vzr[i], zsum);
        }
        l_part += psum;
        if constexpr (FMT == FMT_TQ) z_part += zsum;

        // ---- O += P . V
        PT pa;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float pw = (FMT == FMT_TQ) ? pv[i] * vsc[i] : pv[i];
            if constexpr (MBF16) pa[i] = (short)f32_to_bf16_bits(pw);
            else pa[i] = (_Float16)pw;
        }
        if constexpr (FMT != FMT_TQ) {
            // {token 0,1} and {token 2,3} halves of dims (2e, 2e+1)
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
                bop[c][0] = __builtin_amdgcn_perm(vw[1][c >> 1], vw[0][c >> 1], sel);
                bop[c][1] = __builtin_amdgcn_perm(vw[3][c >> 1], vw[2][c >> 1], sel);
            }
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const PT vb = __builtin_bit_cast(PT, u32x2{bop[c][0], bop[c][1]});
            oacc[c] = mfma16x16x16(pa, vb, oacc[c]);
        }
    };

    if constexpr (kStaged) {
        // Ring of PF register slots: slot S holds page base+S+PF while page
        // base+S is computed from LDS.  Loads and LDS stores are unconditional
        // (tail pages clamp to the last page), so the only branch holds no
        // memory loads and the compiler keeps exact load counters: each LDS
        // store waits only for its own slot, PF-1 pages stay in flight.
        const int npg = p1 - p0;
        if (npg > 0) {
            static_for<PF>([&](auto sc) __attribute__((always_inline)) {
                stage_load(sc, p0 + min((int)decltype(sc)::value, npg - 1));
            });
            stage_store(std::integral_constant<int, 0>{}, pagebuf);
            __syncthreads();
            for (int base = 0; base < npg; base += PF) {
                static_for<PF>([&](auto sc) __attribute__((always_inline)) {
                    constexpr int S = decltype(sc)::value;
                    const int i = base + S;
                    const int cur = i & 1;
                    if (i < npg) {  // uniform over the workgroup
                        const uint8_t* kp = pagebuf + cur * lds_page;
                        process(p0 + i, kp, kp + page_bytes);
                    }
                    stage_load(sc, p0 + min(i + PF, npg - 1));
                    stage_store(std::integral_constant<int, (S + 1) % PF>{}, pagebuf + (cur ^ 1) * lds_page);
                    __syncthreads();
                });
            }
        }
    } else {
        if (p0 < p1) direct_load(p0);
        for (int pg = p0; pg < p1; ++pg) process(pg, nullptr, nullptr);
    }

    // ---- finalize: per-head sums live in lanes r16 = head; O rows in 4*grp + i
    const float l_tot = sum_over_groups(l_part);
    const float z_tot = (FMT == FMT_TQ) ? sum_over_groups(z_part) : 0.0f;
    const bool single = nsp == 1;
    const f32x4 lh4 = gather4_from_row0(l_tot, wscr, r16, grp);
    const f32x4 zh4 = gather4_from_row0(z_tot, wscr + 16, r16, grp);
    const f32x4 mh4 = gather4_from_row0(m_run, wscr + 32, r16, grp);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int hh = 4 * grp + i;
        const float lh = lh4[i], zh = zh4[i], mh = mh4[i];
        if (hh >= G) continue;
        const int hq = hq0 + hh;
        if (single) {
            const float inv = lh > 0.0f ? 1.0f / lh : 0.0f;
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v0 = (oacc[2 * e][i] + zh) * inv;
                const float v1 = (oacc[2 * e + 1][i] + zh) * inv;
                const uint16_t b0 = p.q_bf16 ? f32_to_bf16_bits(v0) : f32_to_f16_bits(v0);
                const uint16_t b1 = p.q_bf16 ? f32_to_bf16_bits(v1) : f32_to_f16_bits(v1);
                w[e] = (uint32_t)b0 | ((uint32_t)b1 << 16);
            }
            uint16_t* o = reinterpret_cast<uint16_t*>(p.out) + ((int64_t)b * p.Hq + hq) * kD + 8 * r16;
            *reinterpret_cast<u32x4*>(o) = u32x4{w[0], w[1], w[2], w[3]};
        } else {
            float* o = p.part + ((int64_t)item * p.Hq + hq) * (kD + 2);
            f32x4 lo = {oacc[0][i] + zh, oacc[1][i] + zh, oacc[2][i] + zh, oacc[3][i] + zh};
            f32x4 hi = {oacc[4][i] + zh, oacc[5][i] + zh, oacc[6][i] + zh, oacc[7][i] + zh};
            // (D + 2) floats per row: 8-byte aligned only, store as float2
            float* od = o + 8 * r16;
            *reinterpret_cast<float2*>(od + 0) = make_float2(lo[0], lo[1]);
            *reinterpret_cast<float2*>(od + 2) = make_float2(lo[2], lo[3]);
            *reinterpret_cast<float2*>(od + 4) = make_float2(hi[0], hi[1]);
            *reinterpret_cast<float2*>(od + 6) = make_float2(hi[2], hi[3]);
            if (r16 == 0) *reinterpret_cast<float2*>(o + kD) = make_float2(mh, lh);
        }
    }
}

// Combines the split partials of every multi-split sequence, one workgroup
// per (sequence, head), one thread per dim:
// out = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M)   (M = max_s m_s)
__global__ void __launch_bounds__(kD)
decode_merge_kernel(void* out, const float* __restrict__ part, const int32_t* __restrict__ seqinfo,
                    int Hq, int q_bf16) {
    const int b = blockIdx.x / Hq, h = blockIdx.x % Hq;
    const int first = seqinfo[2 * b], nsp = seqinfo[2 * b + 1];
    if (nsp <= 1) return;
    const int d = threadIdx.x;
    const float* base = part + ((int64_t)first * Hq + h) * (kD + 2);
    const int64_t stride = (int64_t)Hq * (kD + 2);
    float M = kNegInf;
    for (int s = 0; s < nsp; ++s) M = fmaxf(M, base[s * stride + kD]);
    const float Mu = M == kNegInf ? 0.0f : M;
    float acc = 0.0f, lsum = 0.0f;
    for (int s = 0; s < nsp; ++s) {
        const float* r = base + s * stride;
        const float w = exp2f(r[kD] - Mu);
        lsum = __builtin_fmaf(r[kD + 1], w, lsum);
        acc = __builtin_fmaf(r[d], w, acc);
    }
    const float v = lsum > 0.0f ? acc / lsum : 0.0f;
    uint16_t* o = reinterpret_cast<uint16_t*>(out) + ((int64_t)b * Hq + h) * kD + d;
    *o = q_bf16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

// ------------------------------------------------------------------ host

constexpr int kTargetItems = 1024;
constexpr int kPpsMin = 4;
constexpr int kDefaultMaxSplits = 64;

// upper bound of the plan's item count: sum_b ceil(pages_b / min(pps, cap))
// <= target + B (+ B * ceil(max_blocks / cap) when the per-item page cap binds)
int max_items(int B, int max_blocks) {
    return kTargetItems + B + B * ((max_blocks + kMaxItemPages - 1) / kMaxItemPages);
}

size_t workspace_bytes_for(int B, int Hq, int max_blocks) {
    const size_t seqinfo = ((size_t)B * 2 * sizeof(int32_t) + 255) / 256 * 256;
    return seqinfo + (size_t)max_items(B, max_blocks) * Hq * (kD + 2) * sizeof(float);
}

template <int FMT, int KB, int VB, bool MBF16>
int launch_decode(DecodeParams& prm, size_t lds, hipStream_t stream) {
    const int items = max_items(prm.B, prm.max_blocks);
    auto kern = paged_decode_kernel<FMT, KB, VB, MBF16>;
    if (lds > 64 * 1024) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return VMC_EIO;
    }
    hipLaunchKernelGGL(kern, dim3(items), dim3(64 * prm.Hkv), lds, stream, prm);
    VMC_LAUNCH_CHECK();
    hipLaunchKernelGGL(decode_merge_kernel, dim3(prm.B * prm.Hq), dim3(kD), 0, stream, prm.out, prm.part,
                       prm.seqinfo, prm.Hq, prm.q_bf16);
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}

int setup_common(DecodeParams& prm, void* out, const void* query, const int32_t* bt,
                 const int32_t* seq_lens, int B, int Hq, int Hkv, int D, int bs, int max_blocks,
                 float scale, int max_splits, void* ws, size_t ws_bytes) {
    if (D != kD || bs != kBs) return VMC_EINVAL;
    if (B < 0 || Hq <= 0 || Hkv <= 0 || Hkv > 8 || Hq % Hkv != 0 || Hq / Hkv > 16) return VMC_EINVAL;
    if (max_blocks <= 0) return VMC_EINVAL;
    if (B > 0 && (!out || !query || !bt || !seq_lens || !ws)) return VMC_EINVAL;
    if (ws_bytes < workspace_bytes_for(B, Hq, max_blocks)) return VMC_ENOMEM;
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
    const size_t seqinfo = ((size_t)B * 2 * sizeof(int32_t) + 255) / 256 * 256;
    prm.seqinfo = reinterpret_cast<int32_t*>(ws);
    prm.part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ws) + seqinfo);
    prm.target_items = kTargetItems;
    prm.pps_min = kPpsMin;
    prm.max_splits = max_splits > 0 ? max_splits : kDefaultMaxSplits;
    return VMC_OK;
}

}  // namespace
}  // namespace vmc

using namespace vmc;

extern "C" size_t vmc_paged_decode_workspace_size(int batch_size, int num_heads, int head_dim,
                                                  int max_num_blocks_per_req, int block_size,
                                                  int max_num_kv_splits) {
    (void)head_dim;
    (void)block_size;
    (void)max_num_kv_splits;
    if (batch_size < 0 || num_heads <= 0) return 0;
    return workspace_bytes_for(batch_size, num_heads, max_num_blocks_per_req);
}

extern "C" size_t vmc_turboquant_decode_workspace_size(int batch_size, int num_heads, int head_dim,
                                                       int64_t max_num_blocks_per_req,
                                                       int64_t block_size, int max_num_kv_splits) {
    return vmc_paged_decode_workspace_size(batch_size, num_heads, head_dim,
                                           (int)max_num_blocks_per_req, (int)block_size,
                                           max_num_kv_splits);
}

extern "C" int vmc_paged_attention_decode(void* out, const void* query, const void* key_cache,
                                          const void* value_cache, const int32_t* block_tables,
                                          const int32_t* seq_lens, int batch_size, int num_heads,
                                          int num_kv_heads, int head_dim, int block_size,
                                          int max_num_blocks_per_req, float scale, int q_dtype,
                                          int kv_format, int layout, int max_num_kv_splits,
                                          void* workspace, size_t workspace_bytes,
                                          vmc_stream_t stream) {
    DecodeParams prm = {};
    int rc = setup_common(prm, out, query, block_tables, seq_lens, batch_size, num_heads,
                          num_kv_heads, head_dim, block_size, max_num_blocks_per_req, scale,
                          max_num_kv_splits, workspace, workspace_bytes);
    if (rc != VMC_OK) return rc;
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
        const int n16 = (int)(2 * prm.page_bytes / 16);
        (void)n16;
        if ((prm.page_bytes % 16) != 0) return VMC_EINVAL;
    }
    const size_t lds_q = (size_t)4 * prm.page_bytes;  // K+V, double buffered
    switch (kv_format) {
        case VMC_KV_F16: return launch_decode<FMT_F16, 0, 0, false>(prm, 0, s);
        case VMC_KV_BF16: return launch_decode<FMT_BF16, 0, 0, true>(prm, 0, s);
        case VMC_KV_Q8_0: return launch_decode<FMT_Q8_0, 0, 0, false>(prm, lds_q, s);
        case VMC_KV_Q4_0: return launch_decode<FMT_Q4_0, 0, 0, false>(prm, lds_q, s);
        default: return VMC_EINVAL;
    }
}

extern "C" int vmc_turboquant_decode_attention(void* output, const void* query, const void* kv_cache,
                                               const int32_t* block_tables, const int32_t* seq_lens,
                                               int batch_size, int num_heads, int num_kv_heads,
                                               int head_dim, float scale, int64_t block_size,
                                               int64_t max_num_blocks_per_req,
                                               const vmc_tq_config* cfg, int half_dtype,
                                               int max_num_kv_splits, void* workspace,
                                               size_t workspace_bytes, vmc_stream_t stream) {
    if (!tq_config_valid(cfg) || cfg->head_dim != head_dim) return VMC_EINVAL;
    if (half_dtype != VMC_DTYPE_F16 && half_dtype != VMC_DTYPE_BF16) return VMC_EINVAL;
    if (max_num_blocks_per_req > 0x7fffffff) return VMC_EINVAL;
    DecodeParams prm = {};
    int rc = setup_common(prm, output, query, block_tables, seq_lens, batch_size, num_heads,
                          num_kv_heads, head_dim, (int)block_size, (int)max_num_blocks_per_req,
                          scale, max_num_kv_splits, workspace, workspace_bytes);
    if (rc != VMC_OK) return rc;
    if (batch_size == 0) return VMC_OK;
    if (!kv_cache) return VMC_EINVAL;
    // stored norm/scale/zero are half_dtype; the kernel reads them as fp16
    if (half_dtype != VMC_DTYPE_F16) return VMC_EINVAL;
    prm.kc = reinterpret_cast<const uint8_t*>(kv_cache);
    prm.vc = prm.kc;
    prm.q_bf16 = 0;
    prm.entry_bytes = cfg->slot_size_aligned;
    prm.page_bytes = (int64_t)kBs * num_kv_heads * cfg->slot_size_aligned;
    prm.hnd = 0;
    prm.mse_bytes = cfg->mse_bytes;
    prm.key_packed = cfg->key_packed_size;
    prm.val_data = cfg->val_data_bytes;
    prm.tab = tq_tables(head_dim, cfg->key_quant_bits);
    if ((prm.page_bytes % 16) != 0)
        return VMC_EINVAL;
    const size_t lds = (size_t)2 * prm.page_bytes;  // double-buffered page
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int kb = cfg->key_quant_bits, vb = cfg->value_quant_bits;
    if (kb == 4 && vb == 4) return launch_decode<FMT_TQ, 4, 4, false>(prm, lds, s);
    if (kb == 3 && vb == 3) return launch_decode<FMT_TQ, 3, 3, false>(prm, lds, s);
    if (kb == 3 && vb == 4) return launch_decode<FMT_TQ, 3, 4, false>(prm, lds, s);
    return VMC_EINVAL;
}
