// prefill.hip -- causal flash-attention prefill (MFMA), fused q8_0 append.
#include "vmc_common.hpp"

extern "C" int vmc_flash_attention_prefill(void* output, const void* query, const void* key,
                                           const void* value, int num_tokens, int num_heads,
                                           int num_kv_heads, int head_dim, float scale,
                                           const int32_t* token_positions, int dtype,
                                           void* key_cache, void* value_cache,
                                           const int64_t* slot_mapping, int64_t block_size,
                                           int kv_format, int layout, vmc_stream_t stream) {
    (void)output; (void)query; (void)key; (void)value; (void)num_tokens; (void)num_heads;
    (void)num_kv_heads; (void)head_dim; (void)scale; (void)token_positions; (void)dtype;
    (void)key_cache; (void)value_cache; (void)slot_mapping; (void)block_size; (void)kv_format;
    (void)layout; (void)stream;
    return VMC_EINVAL;
}
