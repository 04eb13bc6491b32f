// prefill_api.hpp -- the tiled prefill over paged TurboQuant slots, for the
// entry point that serves TurboQuant prefill rows (paged_decode.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "vmc_attn.h"

namespace vmc {

// Chunked prefill over TurboQuant slots of the reference layout (codebook
// keys, 3/3, 4/4 or 3/4 bits, or fp8 keys with 4-bit values; head_dim 128,
// block size 16): token t attends
// positions 0 .. token_positions[t] of sequence token_to_seq[t] through its
// block-table row.  q, out and the stored halves are half_dtype.
int tq_prefill_tiled(void* out, const void* query, const void* kv_cache, const int32_t* block_tables,
                     const int32_t* token_to_seq, const int32_t* token_positions, int num_tokens, int num_heads,
                     int num_kv_heads, float scale, int64_t max_blocks, const vmc_tq_config* cfg, int half_dtype,
                     hipStream_t stream);

}  // namespace vmc
