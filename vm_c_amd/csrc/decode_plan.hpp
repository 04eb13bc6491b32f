// decode_plan.hpp -- shared by the paged decode kernels (paged_decode.hip,
// tq_decode.hip): the kernel parameters, the page-range plan of a split-KV
// launch (every workgroup recomputes it from seq_lens), the TurboQuant key
// table builder, the merge kernel of cut sequences and the grid sizing.
#pragma once

#include "vmc_common.hpp"
#include "vmc_tq.hpp"

#include <algorithm>
#include <mutex>
#include <utility>

namespace vmc {

struct DecodeParams {
    void* out;
    const uint16_t* q;
    const uint8_t* kc;
    const uint8_t* vc;
    const int32_t* bt;
    const int32_t* seq_lens;
    float* part;  // [2 * grid][Hq][D + 2]: o, m, l of cut sequences
    int B, Hq, Hkv, G, max_blocks;
    float scale_log2;
    int64_t page_bytes;  // one page of one cache, all heads
    int entry_bytes;     // one (token, head) entry (TQ: the aligned slot)
    int hnd;
    int per_seq;         // 1: one workgroup per sequence
    int pps_min, max_splits;
    int grid;            // page ranges (flat) or sequences (per-sequence mode)
    // weighted split (flat mode with all grid ranges in use): ranges below
    // split_h take split_wa parts of the pages each, the others split_wb
    // (split_h 0: even ranges).  With the weighted split, each sequence
    // start after the first also counts as split_v pages (what a workgroup
    // spends switching sequences: the last piece's rows, the next q, a pair
    // computed twice), so that ranges holding a switch get fewer pages
    int split_h, split_wa, split_wb, split_v;
    int hgroups, hpw;    // KV-head groups per page (one workgroup each), heads per group
    int row_bytes;       // TurboQuant: one token's entries, all KV heads (Hkv * slot)
    int lds_pad;         // staged NHD pages: token rows padded in LDS (row a whole number of chunks)
    int lds_row;         // padded row bytes in LDS
    int row_chunks;      // 16-byte chunks of one token row in HBM
    int rc_inv;          // ceil(2^20 / row_chunks): chunk / row_chunks = chunk * rc_inv >> 20 (chunk * row_chunks < 2^20)
    int tq_nc;           // TurboQuant: 16-byte chunks fetched per token for one head group
    int q_bf16;
    // TurboQuant
    int mse_bytes, key_packed, val_data;
    int norm_corr;       // codebook keys: scaled by 1 / ||C[codes]|| (else by the stored norm alone)
    TQTables tab;
    uint32_t sgn[4];     // per-32-group variant: bit i set = rotation sign of dim i is -1
    int fp8_e4b15;       // turboquant_k8v4 keys: e4b15 (1) or e4m3 (0) codes
    // paged prefill: query row b is token b of sequence row_seq[b] at
    // position row_pos[b] (it attends positions 0 .. row_pos[b]); null =
    // row b is sequence b with seq_lens[b] tokens
    const int32_t* row_seq;
    const int32_t* row_pos;
};

namespace {

constexpr int kD = 128;
constexpr int kBs = 16;
// split partial rows: o[128], m, l, two floats of padding (528 B, so a row
// starts 16-byte aligned and takes 16-byte stores)
constexpr int kPartRow = kD + 4;
constexpr float kNegInf = -__builtin_inff();

// FMT_G4 / FMT_G3: the per-32-group variant (no reference counterpart): one
// slot per (token, head) holds the K part then the V part, each four 32-value
// blocks {fp16 d, fp16 m, 16 B of nibbles} (4-bit) or {fp16 d, 12 B of 3-bit
// codes} (3-bit) of the rotated vector
// FMT_K8: turboquant_k8v4 (kernels_turboquant.h:47-55): K as 128 fp8 bytes
// (the reference's own e4m3 / e4b15 codes), V as 4-bit codes + fp16 scale and
// zero, 196-byte slots; no rotation, no norm
enum { FMT_F16 = 0, FMT_BF16 = 1, FMT_Q8_0 = 2, FMT_Q4_0 = 3, FMT_TQ = 4, FMT_G4 = 5, FMT_G3 = 6, FMT_K8 = 7 };

// TurboQuant V codes enter the PV MFMA as fp16 subnormals: the code field of
// output chunk c is masked where it lies, at bit kVShift(c) of its 16-bit
// half (at most bit 9, so the pattern stays a subnormal), i.e. the value
// code * 2^(shift - 24).  kVScale(c) = 2^(24 - shift) undoes it; other formats
// enter as values.
template <int VB>
__device__ __forceinline__ constexpr int kVShift(int c) {
    return VB == 4 ? ((c & 1) ? 4 : 0) : (c == 0 ? 0 : c == 1 ? 3 : c == 2 ? 6 : c == 3 ? 1 : c == 4 ? 4 : c == 5 ? 7 : c == 6 ? 2 : 5);
}
template <int FMT, int VB>
__device__ __forceinline__ constexpr float kVScale(int c) {
    return FMT != FMT_TQ ? 1.0f : (float)(1 << (24 - kVShift<VB>(c)));
}

// fmax of scores (products, so never signalling NaNs: no quieting is added).
// Plain C++ rather than asm: the hazard checks that guard cross-lane reads
// (DPP, permlane) of a VGPR must see the instruction that wrote it.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_fmaxf(a, b); }
// bitwise select b where m is set, else a (v_bfi_b32).  Plain C++ so the
// compiler sees the operands: an asm consumer of an MFMA result would not get
// the wait states the MFMA's write requires.
__device__ __forceinline__ float sel_bits(float a, float b, uint32_t m) {
    return __builtin_bit_cast(float, (__builtin_bit_cast(uint32_t, b) & m) | (__builtin_bit_cast(uint32_t, a) & ~m));
}
// max over the four lane groups of a column (every lane gets its column's)
__device__ __forceinline__ float vmax_over_groups(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    swap_pair16(a, b);
    v = vmax(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    a = __builtin_bit_cast(uint32_t, v);
    b = a;
    swap_pair32(a, b);
    return vmax(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}



// ------------------------------------------------------------------ layout

__device__ __forceinline__ int seq_pages(const DecodeParams& p, int b, int* L_out) {
    const int L = min(p.row_seq ? p.row_pos[b] + 1 : p.seq_lens[b], p.max_blocks * kBs);
    *L_out = L;
    return L > 0 ? (L + kBs - 1) / kBs : 0;
}

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const int u = __shfl_up(v, m, 64);
        if (lane >= m) v += u;
    }
    return v;
}

// total pages of the batch (one wave, result in every lane)
__device__ __forceinline__ int total_pages(const DecodeParams& p, int lane) {
    int total = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
        int L = 0;
        int pg = b0 + lane < p.B ? seq_pages(p, b0 + lane, &L) : 0;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) pg += __shfl_xor(pg, m, 64);
        total += pg;
    }
    return total;
}

// workgroups that get pages: the launched grid, fewer when the batch is small
__device__ __forceinline__ int effective_wgs(const DecodeParams& p, int T, int grid) {
    int n = min(grid, max(1, (T + p.pps_min - 1) / p.pps_min));
    return max(1, min(n, T));
}

// workgroup whose range holds global page g: floor(((g + 1) n - 1) / T)
__device__ __forceinline__ int wg_of_page(int64_t g, int n, int T) {
    return (int)(((g + 1) * n - 1) / T);
}

// first page of range w of n: T w / n, or with the weighted split
// T C(w) / C(n), C(x) = wa min(x, h) + wb max(0, x - h)
__device__ __forceinline__ int range_lo(const DecodeParams& p, int w, int n, int T) {
    if (p.split_h <= 0 || n != p.grid) return (int)((int64_t)w * T / n);
    const int64_t h = p.split_h;
    const int64_t cw = (int64_t)p.split_wa * min((int64_t)w, h) + (int64_t)p.split_wb * max((int64_t)0, (int64_t)w - h);
    const int64_t cn = (int64_t)p.split_wa * min((int64_t)n, h) + (int64_t)p.split_wb * max((int64_t)0, (int64_t)n - h);
    return (int)((int64_t)T * cw / cn);
}

// range holding global page g under range_lo's split: the last w with
// floor(T C(w) / C(n)) <= g, i.e. with C(w) <= K = floor(((g + 1) C(n) - 1) / T)
__device__ __forceinline__ int range_of_page(const DecodeParams& p, int64_t g, int n, int T) {
    if (p.split_h <= 0 || n != p.grid) return wg_of_page(g, n, T);
    const int64_t h = min((int64_t)p.split_h, (int64_t)n), wa = p.split_wa, wb = p.split_wb;
    const int64_t cn = wa * h + wb * ((int64_t)n - h);
    const int64_t K = ((g + 1) * cn - 1) / T;
    const int64_t w = K < wa * h ? K / wa : h + (K - wa * h) / wb;
    return (int)min(w, (int64_t)n - 1);
}

__device__ __forceinline__ int plan_wave_sum(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}
__device__ __forceinline__ int plan_wave_max(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m, 64));
    return v;
}

// pages and non-empty sequences of the batch (one wave, results in every lane)
__device__ __forceinline__ void batch_pages(const DecodeParams& p, int lane, int* T_out, int* nz_out) {
    int total = 0, nz = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
        int L = 0;
        int pg = b0 + lane < p.B ? seq_pages(p, b0 + lane, &L) : 0;
        total += plan_wave_sum(pg);
        nz += __popcll(__ballot(pg > 0));
    }
    *T_out = total;
    *nz_out = nz;
}

// pages a sequence switch counts as under range_lo's split (0: none).  Only
// with the weighted split, and only when the ranges are long against it (an
// empty range then never falls inside a sequence's pieces).
__device__ __forceinline__ int switch_pages(const DecodeParams& p, int n, int T) {
    return p.split_h > 0 && n == p.grid && p.split_v > 0 && (int64_t)T >= (int64_t)8 * p.split_v * n ? p.split_v : 0;
}

// The page axis with V pages inserted before every non-empty sequence but
// the first: sequence b of rank r (non-empty sequences before it) starting
// at page ps holds virtual pages ps + V r ..; range boundaries are placed on
// this axis (range_lo over T + V (nz - 1)), and a boundary inside an
// inserted gap moves to the start of the sequence after it.  Real pages of
// the virtual boundaries v0 and v1 (one wave, results in every lane).
__device__ __forceinline__ void real_pages(const DecodeParams& p, int lane, int V, int v0, int v1, int* r0,
                                           int* r1) {
    int carry = 0, carry_nz = 0, best0 = 0, best1 = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
        const int b = b0 + lane;
        int L = 0;
        const int pg = b < p.B ? seq_pages(p, b, &L) : 0;
        const int nzf = pg > 0 ? 1 : 0;
        const int incl = wave_incl_scan(pg, lane), incl_nz = wave_incl_scan(nzf, lane);
        const int ps = carry + incl - pg, rank = carry_nz + incl_nz - nzf;
        const int vs = ps + V * rank, gs = vs - (rank > 0 ? V : 0);
        if (pg > 0 && gs <= v0) best0 = max(best0, v0 < vs ? ps : min(ps + (v0 - vs), ps + pg));
        if (pg > 0 && gs <= v1) best1 = max(best1, v1 < vs ? ps : min(ps + (v1 - vs), ps + pg));
        carry += __shfl(incl, 63, 64);
        carry_nz += __shfl(incl_nz, 63, 64);
    }
    *r0 = plan_wave_max(best0);
    *r1 = plan_wave_max(best1);
}

struct WGPlan {
    int p_lo, p_hi;        // global page range
    int first_b, last_b;   // sequences holding p_lo and p_hi - 1
    int first_cut, last_cut;  // first piece continues from before p_lo / last past p_hi
};

// Sequences with pages in [c_lo, c_hi), in order, into LDS (one wave).  In the
// same pass: the sequences holding p_lo and p_hi - 1.
__device__ __forceinline__ int collect_segments(const DecodeParams& p, int c_lo, int c_hi, int lane, int* seg_b,
                                int* seg_ps, int* seg_L, WGPlan* plan, bool plan_ends) {
    const int p_lo = plan->p_lo, p_hi = plan->p_hi;
    int carry = 0, ns = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
        const int b = b0 + lane;
        int L = 0;
        const int pg = b < p.B ? seq_pages(p, b, &L) : 0;
        const int incl = wave_incl_scan(pg, lane);
        const int ps = carry + incl - pg, pe = ps + pg;
        const bool hit = pg > 0 && ps < c_hi && pe > c_lo;
        const uint64_t bal = __ballot(hit);
        if (hit) {
            const int idx = ns + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                          __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
            seg_b[idx] = b;
            seg_ps[idx] = ps;
            seg_L[idx] = L;
        }
        // at most one lane holds each end page: it writes the shared plan
        if (plan_ends && pg > 0) {
            if (ps <= p_lo && p_lo < pe) {
                plan->first_b = b;
                plan->first_cut = ps < p_lo;
            }
            if (ps <= p_hi - 1 && p_hi - 1 < pe) {
                plan->last_b = b;
                plan->last_cut = pe > p_hi;
            }
        }
        ns += __popcll(bal);
        carry += __shfl(incl, 63, 64);
    }
    return ns;
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

__device__ __forceinline__ uint32_t lds32(const uint8_t* p) {
    return *reinterpret_cast<const uint32_t*>(p);
}
__device__ __forceinline__ uint32_t lds16(const uint8_t* p) {
    return (uint32_t)*reinterpret_cast<const uint16_t*>(p);
}

// ------------------------------------------------------------------ merge

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// Combines the pieces of every sequence that range boundaries cut.  Grid
// (B, Hkv), one wave per query head of the KV head.  Rows hold kPartRow floats:
// o unnormalised, m, l (log2 domain); out = sum_s o_s 2^(m_s - M) /
// sum_s l_s 2^(m_s - M), M = max_s m_s.  Pieces of sequence b: workgroups
// w0..w1 (those holding its first and last page); w0 wrote slot 2 w0 + 1,
// later ones slot 2 w.  Sequences without pages get zero rows.
__global__ void __launch_bounds__(1024) decode_merge_kernel(DecodeParams p) {
    const int b = blockIdx.x, g = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int hq = g * p.G + wave;
    __shared__ int sh[5];
    if (wave == 0) {
        int carry = 0, carry_nz = 0, ps_b = 0, pg_b = 0, rank_b = 0;
        for (int b0 = 0; b0 < p.B; b0 += 64) {
            int L = 0;
            const int pg = b0 + lane < p.B ? seq_pages(p, b0 + lane, &L) : 0;
            const int nzf = pg > 0 ? 1 : 0;
            const int incl = wave_incl_scan(pg, lane), incl_nz = wave_incl_scan(nzf, lane);
            if (b0 + lane == b) {
                ps_b = carry + incl - pg;
                pg_b = pg;
                rank_b = carry_nz + incl_nz - nzf;
            }
            carry += __shfl(incl, 63, 64);
            carry_nz += __shfl(incl_nz, 63, 64);
        }
        // the lane that held b publishes it
        if (lane == (b & 63)) {
            sh[0] = ps_b;
            sh[1] = pg_b;
            sh[2] = carry;
            sh[3] = rank_b;
            sh[4] = carry_nz;
        }
    }
    __syncthreads();
    const int ps = sh[0], pg = sh[1], T = sh[2], rank = sh[3], nz = sh[4];
    uint16_t* orow = reinterpret_cast<uint16_t*>(p.out) + ((int64_t)b * p.Hq + hq) * kD;
    if (pg == 0) {
        reinterpret_cast<uint32_t*>(orow)[lane] = 0u;
        return;
    }
    const int n = effective_wgs(p, T, p.grid);
    // pages on range_lo's axis (switch_pages: V pages before each sequence
    // after the first)
    const int V = switch_pages(p, n, T);
    const int Tv = T + V * max(nz - 1, 0), vs = ps + V * rank;
    const int w0 = range_of_page(p, vs, n, Tv), w1 = range_of_page(p, vs + pg - 1, n, Tv);
    if (w0 == w1) return;  // written by its workgroup
    const int nseg = w1 - w0 + 1;
    const int64_t rs = (int64_t)p.Hq * kPartRow;
    auto row = [&](int s) {  // piece s = workgroup w0 + s
        const int slot = s == 0 ? 2 * w0 + 1 : 2 * (w0 + s);
        return p.part + slot * rs + (int64_t)hq * kPartRow;
    };
    // one pass over the pieces, 64 at a time, with a running max: the m / l
    // pair of each piece and the first 16 pieces' o rows are loaded together,
    // so a sequence cut into at most 16 pieces costs one round of loads
    const int r16 = lane & 15, grp = lane >> 4;
    float M = kNegInf, L = 0.0f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < nseg; s0 += 64) {
        const int cnt = min(64, nseg - s0);
        float2 ml = make_float2(kNegInf, 0.0f);
        if (lane < cnt) ml = *reinterpret_cast<const float2*>(row(s0 + lane) + kD);
        // four 16-lane groups take pieces j = grp, grp + 4, ...; four in flight each
        float2 o[4][4];
        auto load_o = [&](int j0) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int jc = min(j0 + 4 * u + grp, cnt - 1);
                const float2* r = reinterpret_cast<const float2*>(row(s0 + jc) + 8 * r16);
#pragma unroll
                for (int e = 0; e < 4; ++e) o[u][e] = r[e];
            }
        };
        load_o(0);
        const float Mn = fmaxf(M, wave_max(ml.x));
        if (Mn > M && M != kNegInf) {  // wave-uniform
            const float f = __builtin_amdgcn_exp2f(M - Mn);
            L *= f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] *= f;
        }
        M = Mn;
        const float Mu = M == kNegInf ? 0.0f : M;
        float wt = 0.0f;
        if (lane < cnt) {
            wt = __builtin_amdgcn_exp2f(ml.x - Mu);
            L = __builtin_fmaf(ml.y, wt, L);
        }
        for (int j0 = 0; j0 < cnt; j0 += 16) {
            if (j0 > 0) load_o(j0);
            float ws[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = j0 + 4 * u + grp;
                ws[u] = __shfl(wt, min(j, cnt - 1), 64);
                ws[u] = j < cnt ? ws[u] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc[2 * e] = __builtin_fmaf(o[u][e].x, ws[u], acc[2 * e]);
                    acc[2 * e + 1] = __builtin_fmaf(o[u][e].y, ws[u], acc[2 * e + 1]);
                }
        }
    }
    L = wave_sum(L);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = sum_over_groups(acc[e]);
    if (grp != 0) return;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    uint32_t w4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint16_t b0 = p.q_bf16 ? f32_to_bf16_bits(acc[2 * e] * inv) : f32_to_f16_bits(acc[2 * e] * inv);
        const uint16_t b1 = p.q_bf16 ? f32_to_bf16_bits(acc[2 * e + 1] * inv) : f32_to_f16_bits(acc[2 * e + 1] * inv);
        w4[e] = (uint32_t)b0 | ((uint32_t)b1 << 16);
    }
    *reinterpret_cast<u32x4*>(orow + 8 * r16) = u32x4{w4[0], w4[1], w4[2], w4[3]};
}

}  // namespace

// ------------------------------------------------------------------ host

constexpr int kPpsMin = 2;

inline int num_cus() {
    static std::mutex mu;
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> lk(mu);
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

// Launched workgroups for the flat layout: one resident wave of them (a
// workgroup of Hkv waves at 2 waves per SIMD), fewer for small batches.
// Upper bound of the pages: B * max_blocks.
inline int flat_grid(int B, int Hkv, int max_blocks, int max_splits, int cus) {
    const int per_cu = max(1, 8 / Hkv);
    int64_t n = (int64_t)cus * per_cu;
    n = std::min<int64_t>(n, ((int64_t)B * max_blocks + kPpsMin - 1) / kPpsMin);
    if (max_splits > 1) n = std::min<int64_t>(n, (int64_t)B * max_splits);
    return (int)std::max<int64_t>(1, n);
}

// TurboQuant: KV heads per workgroup (one wave each) -- at most 4, so two
// workgroups fit a CU (LDS) and the two waves on each SIMD belong to
// different workgroups; 0 when Hkv cannot be split that way
inline int tq_heads_per_group(int Hkv) { return Hkv <= 4 ? Hkv : (Hkv % 2 == 0 && Hkv / 2 <= 4 ? Hkv / 2 : 1); }

// TurboQuant page ranges: two resident workgroups per CU, fewer for small
// batches; never more than flat_grid's count (the workspace is sized by it)
inline int tq_ranges(int B, int Hkv, int max_blocks, int max_splits, int cus) {
    const int hgroups = Hkv / tq_heads_per_group(Hkv);
    int64_t n = std::max<int64_t>(1, (int64_t)cus * 2 / hgroups);
    n = std::min<int64_t>(n, ((int64_t)B * max_blocks + kPpsMin - 1) / kPpsMin);
    if (max_splits > 1) n = std::min<int64_t>(n, (int64_t)B * max_splits);
    n = std::min<int64_t>(n, flat_grid(B, Hkv, max_blocks, max_splits, cus));
    return (int)std::max<int64_t>(1, n);
}

// Page ranges of the streaming TurboQuant decode (tq_stream.hip): two
// resident workgroups per CU, one per range (every KV head of its pages);
// fewer for small batches
inline int tq_stream_ranges(int B, int Hkv, int max_blocks, int max_splits, int cus) {
    (void)Hkv;
    int64_t n = std::max<int64_t>(1, (int64_t)cus * 2);
    n = std::min<int64_t>(n, ((int64_t)B * max_blocks + kPpsMin - 1) / kPpsMin);
    if (max_splits > 1) n = std::min<int64_t>(n, (int64_t)B * max_splits);
    return (int)std::max<int64_t>(1, n);
}

// Page ranges of the head_dim-256 TurboQuant decode (tq_decode_d256.hip):
// one workgroup of 8 / Hkv ranges (one per group of Hkv waves) per CU;
// fewer for small batches (the last workgroup's surplus streams idle)
inline int d256_ranges(int B, int Hkv, int max_blocks, int max_splits, int cus) {
    const int ns = std::max(1, 8 / Hkv);
    int64_t n = (int64_t)cus * ns;
    n = std::min<int64_t>(n, ((int64_t)B * max_blocks + kPpsMin - 1) / kPpsMin);
    if (max_splits > 1) n = std::min<int64_t>(n, (int64_t)B * max_splits);
    return (int)std::max<int64_t>(1, n);
}

// split partials of the head_dim-256 TurboQuant decode: two rows of 256 + 4
// floats per page range
inline size_t workspace_bytes_d256(int B, int Hq, int Hkv, int max_blocks, int max_splits, int cus) {
    if (max_splits == 1) return 0;
    return (size_t)2 * d256_ranges(B, Hkv, max_blocks, max_splits, cus) * Hq * (256 + 4) * sizeof(float);
}

// split partials: two rows per page range of the largest grid any decode
// kernel launches for the shape
inline size_t workspace_bytes_for(int B, int Hq, int Hkv, int max_blocks, int max_splits, int cus) {
    if (max_splits == 1) return 0;
    const int n = std::max(flat_grid(B, Hkv, max_blocks, max_splits, cus),
                           tq_stream_ranges(B, Hkv, max_blocks, max_splits, cus));
    return (size_t)2 * n * Hq * kPartRow * sizeof(float);
}

// The pipelined TurboQuant decode (tq_decode.hip): reference slot layout,
// at most 8 query heads per KV head; VMC_EINVAL for other shapes.
int launch_tq_decode_any(DecodeParams& prm, int key_bits, int value_bits, bool bf16, hipStream_t stream);
// The per-32-group variant (fp16, 3- or 4-bit codes) on the same kernel;
// VMC_EINVAL for shapes it does not take.
int launch_g32_decode(DecodeParams& prm, int bits, hipStream_t stream);
// The streaming TurboQuant decode (tq_stream.hip): reference slot layout,
// 8 KV heads, at most 8 query heads per KV head; VMC_EINVAL for other shapes.
int launch_tq_stream_any(DecodeParams& prm, int key_bits, int value_bits, bool bf16, hipStream_t stream);
// The head_dim-256 TurboQuant decode (tq_decode_d256.hip): reference slot
// layout, equal key and value bits (3 or 4), 1, 2 or 4 KV heads, at most 8
// query heads per KV head; VMC_EINVAL for other shapes.
int launch_tq_decode_d256(DecodeParams& prm, int bits, bool bf16, hipStream_t stream);

}  // namespace vmc
