// generic_attn.hpp -- head_dim 64 and 256: the TurboQuant store and one
// attention kernel behind every attention entry point (the head_dim 128
// kernels are tuned per format; these are written for any of the sources).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "vmc_attn.h"

namespace vmc {

inline bool generic_head_dim(int d) { return d == 64 || d == 256; }

// gen_attention also serves head_dim 128 where the tuned decode kernels do
// not: more than 8 KV heads or more than 16 query heads per KV head, and
// fp8-key TurboQuant slots with bf16 q, out and halves
inline bool beyond_tuned_decode(int d, int hq, int hkv) {
    return d == 128 && hkv > 0 && (hkv > 8 || hq / hkv > 16);
}

// K/V source of one attention call
enum GenSrc { GEN_F16 = 0, GEN_BF16 = 1, GEN_Q8 = 2, GEN_Q4 = 3, GEN_LOCAL = 4, GEN_TQ = 5 };

struct GenArgs {
    void* out;
    const void* q;
    int q_bf16;  // q / out dtype (local rows: also K / V)
    int src;     // GenSrc
    // pages: kp / vp pools (TurboQuant: both the slot pool), entry bytes per
    // (token, head), "hnd" placement, tokens per page, block tables
    const uint8_t* kp;
    const uint8_t* vp;
    int64_t entry;
    int hnd;
    int64_t bs;
    const int32_t* bt;
    int64_t max_blocks;
    // rows: with tok_seq null, row b is sequence b and attends positions
    // 0 .. seq_lens[b] - 1; else row t is a token of sequence tok_seq[t] and
    // attends positions 0 .. pos[t].  A row whose sequence is outside
    // [0, num_seqs) (num_seqs >= 0) or that has no keys gets zeros.
    const int32_t* seq_lens;
    const int32_t* tok_seq;
    const int32_t* pos;
    int num_seqs;
    // local rows (prefill over this step's K/V [T][Hkv][D]): token t attends
    // tokens t - pos[t] .. t
    const uint16_t* k;
    const uint16_t* v;
    int rows, Hq, Hkv, D;
    float scale;
    // TurboQuant slot fields
    int kb, vb, key_fp8, fp8_e4b15, mse_bytes, key_packed, val_data, norm_correction;
};

int gen_attention(const GenArgs& a, hipStream_t stream);
int gen_tq_store(const void* key, const void* value, void* cache, const int64_t* slots, int T, int Hkv,
                 int D, int64_t bs, const vmc_tq_config* c, bool bf16, hipStream_t stream);

}  // namespace vmc
